"""Small helpers shared by the tests."""
from __future__ import annotations

import numpy as np
import torch


def bits16(a) -> np.ndarray:
    """fp16 array/tensor -> uint16 bit patterns (for bitwise comparison)."""
    if isinstance(a, torch.Tensor):
        a = a.detach().cpu().contiguous().numpy()
    return np.ascontiguousarray(a).view(np.uint16)


def np_(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().numpy()


def ndhwc(t: torch.Tensor) -> np.ndarray:
    """[B, C, D, H, W] tensor -> numpy NDHWC [B, D, H, W, C]."""
    return t.detach().cpu().permute(0, 2, 3, 4, 1).contiguous().numpy()


def assert_bitwise(got, want, what=""):
    g = bits16(got) if (isinstance(got, torch.Tensor) and got.dtype == torch.float16) or (
        isinstance(got, np.ndarray) and got.dtype == np.float16) else np.asarray(got if not isinstance(got, torch.Tensor) else np_(got))
    w = bits16(want) if isinstance(want, np.ndarray) and want.dtype == np.float16 else np.asarray(want)
    assert g.shape == w.shape, f"{what}: shape {g.shape} != {w.shape}"
    bad = np.flatnonzero(g.reshape(-1) != w.reshape(-1))
    assert bad.size == 0, f"{what}: {bad.size} of {g.size} elements differ; first at {bad[:5].tolist()}: got {g.reshape(-1)[bad[:5]].tolist()} want {w.reshape(-1)[bad[:5]].tolist()}"


def rand_fp16(gen, *shape, scale=1.0):
    return (torch.randn(*shape, generator=gen) * scale).half()
