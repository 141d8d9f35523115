"""GPU parity: decoder pixel finalisation (opt/fp16_finalize.py) vs the CPU oracle, bit for bit."""
from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
STD = torch.tensor([0.229, 0.224, 0.225], dtype=torch.float32)
MEAN = torch.tensor([0.485, 0.456, 0.406], dtype=torch.float32)


def _check(ops, oracle, x, out=None):
    xd = x.to(DEV)
    std, mean = STD.to(DEV), MEAN.to(DEV)
    with torch.inference_mode():
        got = ops.fp16_finalize.finalize_pixels(xd, std, mean, out)
    torch.cuda.synchronize()
    if out is not None:
        assert got is out
    want = oracle.finalize_pixels(x.contiguous().numpy(), STD.numpy(), MEAN.numpy())
    g = got.cpu().numpy()
    assert g.shape == want.shape and got.is_contiguous()
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(g), nan)
    assert np.array_equal(g[~nan].view(np.uint32), want[~nan].view(np.uint32))


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("shape", [(1, 3, 28, 256, 256), (4, 3, 5, 16, 24), (2, 3, 3, 5, 7)])
def test_finalize_matches_oracle(ops, oracle, dtype, shape):
    """H3 decode tile output [1,3,28,256,256], a batched tile and a T*H*W not divisible by 8 (strided path)."""
    gen = torch.Generator().manual_seed(sum(shape))
    x = (torch.randn(shape, generator=gen) * 2.5).to(dtype)
    _check(ops, oracle, x)


def test_finalize_special_values_and_strided_input(ops, oracle):
    gen = torch.Generator().manual_seed(7)
    x = torch.randn((2, 8, 3, 4, 3), generator=gen).half()     # [B, W, C, T, H] storage
    flat = x.view(-1)
    flat[:9] = torch.tensor([float("nan"), float("inf"), -float("inf"), -0.0, 0.0, 65504.0, -65504.0, 1e-7, 6e-5])
    xs = x.permute(0, 2, 3, 4, 1)                               # [B, 3, T, H, W] view, not contiguous
    assert not xs.is_contiguous()
    _check(ops, oracle, xs)


def test_finalize_writes_the_given_buffer(ops, oracle):
    gen = torch.Generator().manual_seed(9)
    x = torch.randn((1, 3, 4, 8, 16), generator=gen).half()
    out = torch.full(x.shape, 7.0, dtype=torch.float32, device=DEV)
    _check(ops, oracle, x, out)
