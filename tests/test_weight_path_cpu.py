"""Load-time weight path on the CPU: the runtime's strict checkpoint load (only the latent statistics may be
extra keys; safetensors and weights-only torch files) and the offload semantics of the static INT8 wrappers
(a module.to(dtype) move keeps INT8 weights, FP32 scales and FP16 biases)."""
from __future__ import annotations

import importlib

import pytest
import torch
import torch.nn as nn

import h3_arch


@pytest.fixture(scope="module")
def rt(pkg):
    return importlib.import_module(f"{pkg.__name__}.h3vae_runtime")


class _Opaque:
    """An arbitrary pickled class: the weights-only loader must refuse it."""


class _Core(nn.Module):
    def __init__(self):
        super().__init__()
        self.conv = nn.Conv3d(4, 8, 3)
        self.norm = nn.GroupNorm(2, 8)


def _state(core):
    return {k: v.detach().clone() for k, v in core.state_dict().items()}


def test_strict_load_safetensors_and_latent_statistics(rt, tmp_path):
    import safetensors.torch
    src, dst = _Core(), _Core()
    sd = _state(src)
    sd["latents_mean"] = torch.zeros(24)
    sd["latents_std"] = torch.ones(24)
    path = tmp_path / "vae.safetensors"
    safetensors.torch.save_file(sd, str(path))
    rt._load_weights(dst, str(path))
    for k, v in src.state_dict().items():
        assert torch.equal(dst.state_dict()[k], v)


def test_strict_load_rejects_missing_and_unknown_keys(rt, tmp_path):
    import safetensors.torch
    sd = _state(_Core())
    missing = dict(sd)
    del missing["conv.bias"]
    safetensors.torch.save_file(missing, str(tmp_path / "missing.safetensors"))
    with pytest.raises(RuntimeError, match="missing=\\['conv.bias'\\]"):
        rt._load_weights(_Core(), str(tmp_path / "missing.safetensors"))
    extra = dict(sd)
    extra["decoder.extra"] = torch.zeros(3)
    safetensors.torch.save_file(extra, str(tmp_path / "extra.safetensors"))
    with pytest.raises(RuntimeError, match="decoder.extra"):
        rt._load_weights(_Core(), str(tmp_path / "extra.safetensors"))
    with pytest.raises(FileNotFoundError):
        rt._load_weights(_Core(), str(tmp_path / "absent.safetensors"))
    with pytest.raises(ValueError):
        rt._load_weights(_Core(), "")


def test_torch_checkpoint_loaded_weights_only(rt, tmp_path):
    src, dst = _Core(), _Core()
    torch.save(_state(src), str(tmp_path / "vae.pt"))
    rt._load_weights(dst, str(tmp_path / "vae.pt"))
    assert torch.equal(dst.conv.weight, src.conv.weight)
    # a pickled object that is not plain tensors is refused by the weights-only loader
    torch.save({"conv.weight": _Opaque()}, str(tmp_path / "opaque.pt"))
    with pytest.raises(Exception):
        rt._load_weights(_Core(), str(tmp_path / "opaque.pt"))


def test_int8_encoder_wrapper_offload_keeps_quantization_dtypes(pkg):
    integ = importlib.import_module(f"{pkg.__name__}.opt.encoder_int8_integration")
    torch.manual_seed(0)
    conv = h3_arch.CausalConv3d(32, 64).half().eval()
    wrapper = integ.Int8FusedValidConv3d(conv, apply_bias=True)
    q, s, b = wrapper.qweight.detach().clone(), wrapper.weight_scale.clone(), wrapper.bias.detach().clone()
    assert q.dtype == torch.int8 and s.dtype == torch.float32 and b.dtype == torch.float16
    for dtype in (torch.float32, torch.bfloat16, torch.float16):
        wrapper.to(dtype=dtype)
        assert wrapper.qweight.dtype == torch.int8 and torch.equal(wrapper.qweight, q)
        assert wrapper.weight_scale.dtype == torch.float32 and torch.equal(wrapper.weight_scale, s)
        assert wrapper.bias.dtype == torch.float16 and torch.equal(wrapper.bias, b)
    # the source module is untouched
    assert conv.weight.dtype == torch.float16
