"""GPU parity: the fp16-output GroupNorm/SiLU/pad producer of the encoder suffix and FP16 mode
(h3v_gn_norm_pack_f16, `batched_temporal_norm_pack`) against the CPU oracle, bit for bit, and the
clip-batched residual block against the model's own block run clip by clip."""
from __future__ import annotations

import importlib

import numpy as np
import pytest
import torch

import h3_arch
from _util import assert_bitwise, np_

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _inputs(b, c, d, h, w, pre_bias, seed):
    gen = torch.Generator().manual_seed(seed)
    x = (torch.randn(b * d, h, w, c, generator=gen) * 1.7 + 0.3).half()      # NDHWC, batch x time frames
    gamma = (1 + 0.2 * torch.randn(c, generator=gen)).half()
    beta = (0.1 * torch.randn(c, generator=gen)).half()
    pb = (0.1 * torch.randn(c, generator=gen)).half() if pre_bias else None
    return x, gamma, beta, pb


def _oracle(oracle, x, gamma, beta, pb, b, eps):
    frames = x.shape[0] // b
    ys, ss = [], []
    for i in range(b):
        xi = x[i * frames:(i + 1) * frames].numpy()
        st = oracle.gn_stats(xi, eps, None if pb is None else pb.numpy())
        y, _, _ = oracle.norm_pack(xi, gamma.numpy(), beta.numpy(), st, None if pb is None else pb.numpy())
        ys.append(y)
        ss.append(st)
    return np.stack(ys), np.concatenate(ss)


@pytest.mark.parametrize("c,b,d,h,w,pb", [(128, 1, 3, 6, 9, False), (256, 3, 2, 5, 7, True), (512, 1, 3, 8, 8, False),
                                          (512, 4, 2, 7, 5, True), (1024, 3, 2, 6, 6, False), (1024, 1, 5, 9, 4, True),
                                          (256, 4, 9, 64, 64, False), (512, 4, 5, 32, 32, True)])
def test_norm_pack_f16_matches_oracle(ops, oracle, c, b, d, h, w, pb):
    print(f"norm_pack_f16 C={c} B={b} D={d} {h}x{w} pre_bias={pb}", flush=True)
    x, gamma, beta, pre = _inputs(b, c, d, h, w, pb, seed=c + b + d + h + w)
    eps = 1e-6
    xd, gd, bd = x.to(DEV), gamma.to(DEV), beta.to(DEV)
    pd = None if pre is None else pre.to(DEV)
    y = torch.empty((b, d + 2, h + 2, w + 2, c), dtype=torch.float16, device=DEV)
    stats = torch.empty((b * d, 32, 2), dtype=torch.float32, device=DEV)
    ws = torch.empty(int(ops.hip.lib().h3v_gn_norm_pack_f16_workspace_floats(b, c, d, h, w)), device=DEV)
    ops.hip.call("h3v_gn_norm_pack_f16", ops.hip.ptr(xd), ops.hip.ptr(pd), ops.hip.ptr(gd), ops.hip.ptr(bd), eps, b, c,
                 d, h, w, ops.hip.ptr(y), ops.hip.ptr(stats), ops.hip.ptr(ws), ops.hip.stream(DEV))
    torch.cuda.synchronize()
    want_y, want_s = _oracle(oracle, x, gamma, beta, pre, b, eps)
    assert_bitwise(np_(stats), want_s, "stats")
    assert_bitwise(np_(y), want_y, "y")


@pytest.fixture(scope="module")
def bn(pkg):
    return importlib.import_module(f"{pkg.__name__}.opt.encoder_fused_batched_norm")


def test_batched_op_layouts_and_guards(bn, oracle):
    b, c, d, h, w = 4, 256, 3, 10, 12
    x, gamma, beta, _ = _inputs(b, c, d, h, w, False, seed=11)
    # [B*D, H, W, C] storage viewed as a channels-last-3d [B, C, D, H, W] tensor
    xd = x.to(DEV).view(b, d, h, w, c).permute(0, 4, 1, 2, 3)
    assert xd.is_contiguous(memory_format=torch.channels_last_3d)
    with torch.inference_mode():
        y = bn.batched_temporal_norm_pack(xd, None, gamma.to(DEV), beta.to(DEV), 1e-6)
    torch.cuda.synchronize()
    assert y.shape == (b, c, d + 2, h + 2, w + 2) and y.is_contiguous(memory_format=torch.channels_last_3d)
    want, _ = _oracle(oracle, x, gamma, beta, None, b, 1e-6)
    assert_bitwise(np_(y.permute(0, 2, 3, 4, 1)), want, "batched op")
    g, be = gamma.to(DEV), beta.to(DEV)
    with pytest.raises(ValueError, match="B=1..4"):
        bn.batched_temporal_norm_pack(torch.cat([xd, xd[:1]]), None, g, be, 1e-6)
    # two clips (the reference rejects B = 2, which its own staged encode produces)
    with torch.inference_mode():
        y2 = bn.batched_temporal_norm_pack(xd[:2], None, g, be, 1e-6)
    torch.cuda.synchronize()
    assert_bitwise(np_(y2.permute(0, 2, 3, 4, 1)), want[:2], "batched op, two clips")
    with pytest.raises(ValueError, match="adjacent"):
        bn.batched_temporal_norm_pack(xd.contiguous(), None, g, be, 1e-6)     # NCDHW: time not adjacent to batch
    with pytest.raises(ValueError, match="channel vectors"):
        bn.batched_temporal_norm_pack(xd, None, g.float(), be, 1e-6)


@pytest.mark.parametrize("cin,cout", [(256, 256), (256, 512)])
def test_batched_residual_block_matches_model_per_clip(bn, cin, cout):
    """Three clips batched through BatchedResidualBlock == the model's ResnetBlock3D clip by clip (FP16 tolerance:
    the model's GroupNorm statistics use torch's reduction order, the convs are the same FP16 convs)."""
    torch.manual_seed(cin + cout)
    block = h3_arch.ResnetBlock3D(cin, cout).half().to(DEV).eval()
    gen = torch.Generator().manual_seed(3)
    x = torch.randn(3, cin, 5, 16, 16, generator=gen).half().to(DEV).contiguous(memory_format=torch.channels_last_3d)
    with torch.inference_mode():
        ref = torch.cat([block(x[i:i + 1]) for i in range(3)])
        y = bn.BatchedResidualBlock(block)(x)
        torch.cuda.synchronize()
    rel = (y.float() - ref.float()).norm() / ref.float().norm()
    assert rel < 5e-3, float(rel)
