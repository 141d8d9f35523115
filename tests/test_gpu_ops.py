"""GPU: the reference-named torch custom ops end to end (through libh3vae_hip.so)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from _util import assert_bitwise, np_

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _ffn_weights(gen, d, n):
    up = torch.randint(-31, 32, (2 * n, d), generator=gen, dtype=torch.int8)
    us = torch.full((2 * n,), 0.001, dtype=torch.float32)
    ub = (torch.randn(2 * n, generator=gen) * 0.01).half()
    down = torch.randint(-31, 32, (d, n), generator=gen, dtype=torch.int8)
    ds = torch.full((d,), 0.001, dtype=torch.float32)
    db = (torch.randn(d, generator=gen) * 0.01).half()
    return up, us, ub, down, ds, db


@pytest.mark.parametrize("d,n,shape", [(2048, 8192, (2, 3)), (1024, 4096, (1, 129))])
def test_fused_residual_ffn_matches_registered_ops_and_oracle(ops, oracle, d, n, shape):
    """Reference tests/test_int8_ffn_up_fused_gpu.py:48-64 plus the oracle chain."""
    gen = torch.Generator().manual_seed(d + n)
    x = torch.randn(*shape, d, generator=gen).half()
    a = torch.randn_like(x)
    g = torch.full((d,), 0.1, dtype=torch.float16)
    norm = torch.ones(d, dtype=torch.float16)
    up, us, ub, down, ds, db = _ffn_weights(gen, d, n)
    dv = [t.to(DEV) for t in (x, a, g, norm, up, us, ub, down, ds, db)]
    with torch.inference_mode():
        rh, hidden = ops.int8_norm_quant.residual_rms_linear(*dv[:4], dv[4], dv[5], dv[6], 1e-5, 8)
        rout = ops.int8_swiglu_fused.swiglu_int8_linear(hidden, dv[7], dv[8], dv[9], 16)
        ch, cout = ops.int8_ffn_up_fused.fused_residual_ffn(*dv, 1e-5, 8)
    torch.cuda.synchronize()
    assert torch.equal(ch, rh)
    assert torch.equal(cout, rout)
    oh, oq, osc = oracle.residual_rms_quant(x.numpy().reshape(-1, d), a.numpy().reshape(-1, d), g.numpy(),
                                            norm.numpy(), 1e-5, 1)
    act = oracle.gemm_swiglu(oracle.gemm_acc(oq, up.numpy()), osc, us.numpy(), ub.numpy())
    aq, asc = oracle.row_quant(act)
    want = oracle.gemm_dequant(oracle.gemm_acc(aq, down.numpy()), asc, ds.numpy(), db.numpy())
    assert_bitwise(np_(ch).reshape(-1, d), oh, "h")
    assert_bitwise(np_(cout).reshape(-1, d), want, "out")


def test_residual_qkv_mutates_h_and_matches_oracle(ops, oracle):
    gen = torch.Generator().manual_seed(3)
    h = torch.randn(4, 37, 2048, generator=gen).half()
    o = torch.randn_like(h)
    g = (0.1 * torch.randn(2048, generator=gen)).half()
    w = (1 + 0.1 * torch.randn(2048, generator=gen)).half()
    qw = torch.randint(-127, 128, (6144, 2048), generator=gen, dtype=torch.int8)
    ws = (torch.rand(6144, generator=gen) * 0.001 + 1e-4).float()
    bias = (0.02 * torch.randn(6144, generator=gen)).half()
    hd = h.to(DEV)
    with torch.inference_mode():
        qkv = ops.int8_norm1_quant.residual_qkv(hd, o.to(DEV), g.to(DEV), w.to(DEV), qw.to(DEV), ws.to(DEV),
                                                bias.to(DEV))
    torch.cuda.synchronize()
    rh, rq, rs = oracle.residual_rms_quant(h.numpy().reshape(-1, 2048), o.numpy().reshape(-1, 2048), g.numpy(),
                                           w.numpy(), 1e-5, 0)
    assert_bitwise(np_(hd).reshape(-1, 2048), rh, "h mutated in place")
    want = oracle.gemm_dequant(oracle.gemm_acc(rq, qw.numpy()), rs, ws.numpy(), bias.numpy())
    assert qkv.shape == (4, 37, 6144)
    assert_bitwise(np_(qkv).reshape(-1, 6144), want, "qkv")


def test_int8_linear_op_matches_oracle(ops, oracle):
    gen = torch.Generator().manual_seed(4)
    x = torch.randn(3, 129, 1024, generator=gen).half()
    w = (torch.randn(1024, 1024, generator=gen) * 0.02).half()
    w[5] = 0                                          # zero weight row -> q=0, s=1
    b = (0.02 * torch.randn(1024, generator=gen)).half()
    lin = torch.nn.Linear(1024, 1024).half().eval()
    with torch.no_grad():
        lin.weight.copy_(w)
        lin.bias.copy_(b)
    lin = lin.to(DEV)
    with torch.no_grad():
        mod = ops.kitchen_int8.KitchenInt8Linear(lin, require_cuda=True).eval()
        y = mod(x.to(DEV))
    torch.cuda.synchronize()
    rqw, rsw = oracle.row_quant(w.numpy())
    rqw[5] = 0
    rsw[5] = 1.0
    assert_bitwise(np_(mod.qweight), rqw, "qweight")
    assert_bitwise(np_(mod.weight_scale).view(np.uint32), rsw.view(np.uint32), "weight scale")
    want = oracle.int8_linear(x.numpy().reshape(-1, 1024), rqw, rsw, b.numpy())
    assert_bitwise(np_(y).reshape(-1, 1024), want, "y")


def test_block0_and_final_norm_ops(ops, oracle):
    gen = torch.Generator().manual_seed(6)
    x = torch.randn(4, 1797, 2048, generator=gen).half()
    o = torch.randn_like(x)
    gate = (0.1 * torch.randn(2048, generator=gen)).half()
    gamma = (1 + 0.1 * torch.randn(2048, generator=gen)).half()
    beta = (0.02 * torch.randn(2048, generator=gen)).half()
    with torch.inference_mode():
        y0 = ops.decoder_block0_norm.rms_fp16_x2_w16(x.to(DEV), gamma.to(DEV))
        y1 = ops.decoder_final_norm.final_residual_ln_w8(x.to(DEV), o.to(DEV), gate.to(DEV), gamma.to(DEV),
                                                         beta.to(DEV))
    torch.cuda.synchronize()
    eps = 9.999999747378752e-06
    assert_bitwise(np_(y0).reshape(-1, 2048), oracle.rms_fp16(x.numpy().reshape(-1, 2048), gamma.numpy(), eps), "b0")
    want = oracle.residual_layernorm(x.numpy().reshape(-1, 2048), o.numpy().reshape(-1, 2048), gate.numpy(),
                                     gamma.numpy(), beta.numpy(), eps)
    assert_bitwise(np_(y1).reshape(-1, 2048), want, "final ln")
    # within tolerance of an fp64 LayerNorm of the same residual (the reference's rounding is unpinned)
    raw = (o.double() * gate.double() + x.double()).reshape(-1, 2048)
    ref = torch.nn.functional.layer_norm(raw, (2048,), gamma.double(), beta.double(), eps)
    assert (y1.cpu().double().reshape(-1, 2048) - ref).abs().max().item() < 8e-3


def test_ops_reject_bad_inputs_before_launch(ops):
    x = torch.randn(2, 3, 2047, device=DEV).half()
    with pytest.raises(ValueError):
        ops.int8_norm_quant.residual_quant(x, x, x[0, 0], x[0, 0], 1e-5)
    q = torch.zeros((3, 2048), dtype=torch.int8, device=DEV)
    with pytest.raises(ValueError):
        ops.int8_swiglu_fused.prequantized_linear(q, torch.ones(3, 1, device=DEV), q.t().contiguous(),
                                                  torch.ones(3, device=DEV))
