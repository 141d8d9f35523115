"""Shared fixtures: the plugin package, the CPU oracle, seeded generators."""
from __future__ import annotations

import importlib
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

SEED = 20261002


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session", autouse=True)
def _references_without_miopen():
    """The model modules that serve as FP16 references call F.conv3d.  Through MIOpen its first call per
    shape runs a solver search and kernel compile that takes minutes on a fresh box, so the references
    use torch's own vol2col + BLAS convolution instead.  The product path never calls F.conv3d."""
    import torch
    enabled = torch.backends.cudnn.enabled
    torch.backends.cudnn.enabled = False
    yield
    torch.backends.cudnn.enabled = enabled


@pytest.fixture(scope="session")
def pkg():
    import __graft_entry__
    return __graft_entry__.load_package()


@pytest.fixture(scope="session")
def ops(pkg):
    """Namespace with every operator module of the package."""
    names = ["kitchen_int8", "int8_swiglu_fused", "int8_ffn_up_fused", "int8_norm_quant", "int8_norm1_quant",
             "decoder_fused_qk_rope", "decoder_block0_norm", "decoder_final_norm", "encoder_int8",
             "encoder_int8_norm", "encoder_int8_integration", "fp16_finalize"]

    class _Ops:
        pass

    ns = _Ops()
    for name in names:
        setattr(ns, name, importlib.import_module(f"{pkg.__name__}.opt.{name}"))
    ns.hip = importlib.import_module(f"{pkg.__name__}._hip")
    return ns


@pytest.fixture(scope="session")
def oracle():
    import oracle as _oracle
    _oracle.lib()
    return _oracle
