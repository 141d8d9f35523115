"""GPU parity: decoder row producers and the fused QK-RMSNorm-RoPE vs the CPU oracle."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from _util import assert_bitwise, np_

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
SHAPES = [(1, 2048), (17, 2048), (129, 1024), (7188, 2048), (16384, 1024), (3, 4096)]


def _inputs(m, k, seed):
    gen = torch.Generator().manual_seed(seed)
    h = torch.randn(m, k, generator=gen).half()
    o = torch.randn(m, k, generator=gen).half()
    g = (0.1 * torch.randn(k, generator=gen)).half()
    w = (1 + 0.1 * torch.randn(k, generator=gen)).half()
    return h, o, g, w


@pytest.mark.parametrize("m,k", SHAPES)
@pytest.mark.parametrize("entry,recipe", [("h3v_residual_norm1_quant", 0), ("h3v_residual_rms_quant", 1)])
def test_residual_rms_quant_matches_oracle(ops, oracle, m, k, entry, recipe):
    h, o, g, w = _inputs(m, k, m + k + recipe)
    if m > 2:
        o[1] = 0
        h[1] = 0                                      # zero row -> q=-128, s=1e-30
    hd, od, gd, wd = (t.to(DEV) for t in (h, o, g, w))
    q = torch.empty((m, k), dtype=torch.int8, device=DEV)
    s = torch.empty(m, dtype=torch.float32, device=DEV)
    out_h = hd if recipe == 0 else torch.empty_like(hd)   # norm1 runs in place
    ops.hip.call(entry, ops.hip.ptr(hd), ops.hip.ptr(od), ops.hip.ptr(gd), ops.hip.ptr(wd), 1e-5, m, k,
                 ops.hip.ptr(out_h), ops.hip.ptr(q), ops.hip.ptr(s), ops.hip.stream(DEV))
    torch.cuda.synchronize()
    rh, rq, rs = oracle.residual_rms_quant(h.numpy(), o.numpy(), g.numpy(), w.numpy(), 1e-5, recipe)
    assert_bitwise(np_(out_h), rh, "h")
    assert_bitwise(np_(q), rq, "q")
    assert_bitwise(np_(s).view(np.uint32), rs.view(np.uint32), "s")


@pytest.mark.parametrize("m,k", SHAPES)
def test_rms_fp16_matches_oracle(ops, oracle, m, k):
    x, _, _, gamma = _inputs(m, k, 5 + m)
    out = torch.empty((m, k), dtype=torch.float16, device=DEV)
    xd, gd = x.to(DEV), gamma.to(DEV)
    ops.hip.call("h3v_rms_fp16", ops.hip.ptr(xd), ops.hip.ptr(gd), 9.999999747378752e-06, m, k, ops.hip.ptr(out),
                 ops.hip.stream(DEV))
    torch.cuda.synchronize()
    assert_bitwise(np_(out), oracle.rms_fp16(x.numpy(), gamma.numpy(), 9.999999747378752e-06), "rms")


@pytest.mark.parametrize("m,k", SHAPES)
def test_residual_layernorm_matches_oracle(ops, oracle, m, k):
    h, o, gate, gamma = _inputs(m, k, 9 + m)
    beta = (0.02 * torch.randn(k, generator=torch.Generator().manual_seed(m))).half()
    out = torch.empty((m, k), dtype=torch.float16, device=DEV)
    dev = [t.to(DEV) for t in (h, o, gate, gamma, beta)]
    ops.hip.call("h3v_residual_layernorm", *[ops.hip.ptr(t) for t in dev], 9.999999747378752e-06, m, k,
                 ops.hip.ptr(out), ops.hip.stream(DEV))
    torch.cuda.synchronize()
    want = oracle.residual_layernorm(h.numpy(), o.numpy(), gate.numpy(), gamma.numpy(), beta.numpy(),
                                     9.999999747378752e-06)
    assert_bitwise(np_(out), want, "ln")


def _rope_tables(n, seed):
    gen = torch.Generator().manual_seed(seed)
    ang = torch.rand(n, 48, generator=gen) * 6.2831853
    return torch.cos(ang).half(), torch.sin(ang).half()


@pytest.mark.parametrize("b,n,heads", [(1, 16384, 16), (4, 1797, 32), (1, 3, 2), (2, 5, 1)])
def test_qk_rope_matches_oracle(ops, oracle, b, n, heads):
    gen = torch.Generator().manual_seed(b * n + heads)
    x = torch.randn(b, n, heads * 192, generator=gen).half()
    cos, sin = _rope_tables(b * n, heads)
    cos = cos.reshape(b, n, 1, 48).contiguous()
    sin = sin.reshape(b, n, 1, 48).contiguous()
    with torch.inference_mode():
        q, k = ops.decoder_fused_qk_rope.qk_rope(x.to(DEV), cos.to(DEV), sin.to(DEV), heads, 1e-6, 8)
    torch.cuda.synchronize()
    rq, rk = oracle.qk_rope(x.numpy(), cos.numpy(), sin.numpy(), heads, 1e-6)
    assert_bitwise(np_(q), rq, "q")
    assert_bitwise(np_(k), rk, "k")
