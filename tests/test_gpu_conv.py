"""GPU parity: encoder INT8 implicit-GEMM conv3d and the fused norm producer vs the CPU oracle."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from _util import assert_bitwise, ndhwc, np_

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def _conv_i32_gpu(ops, qx_ndhwc, qw, kernel, stride, causal_skip=False):
    b, d, h, w, c = qx_ndhwc.shape
    o = qw.shape[0]
    kd, kh, kw = kernel
    sd, sh, sw = stride
    do, ho, wo = (d - kd) // sd + 1, (h - kh) // sh + 1, (w - kw) // sw + 1
    acc = torch.empty((b, do, ho, wo, o), dtype=torch.int32, device=DEV)
    xd, wd = qx_ndhwc.to(DEV).contiguous(), qw.to(DEV).contiguous()
    ops.hip.call("h3v_conv3d_i8_i32", ops.hip.ptr(xd), ops.hip.ptr(wd), ops.hip.ptr(acc), b, c, d, h, w, o, kd, kh, kw,
                 sd, sh, sw, int(causal_skip), ops.hip.stream(DEV))
    torch.cuda.synchronize()
    return np_(acc)


# reference tests/test_encoder_int8_gpu.py:74-80 and :95-106 geometries (NCDHW shapes)
CASES = [
    (128, 128, (1, 128, 3, 19, 23), (3, 3, 3), (1, 1, 1)),
    (128, 256, (1, 128, 19, 17, 19), (3, 3, 3), (1, 1, 1)),
    (256, 256, (1, 256, 19, 17, 19), (3, 3, 3), (1, 1, 1)),
    (7, 19, (2, 7, 5, 9, 11), (3, 3, 3), (1, 2, 2)),
    (128, 128, (1, 128, 3, 10, 18), (3, 3, 3), (1, 1, 1)),
    (128, 256, (1, 128, 4, 10, 18), (3, 3, 3), (1, 1, 1)),
    (256, 129, (1, 256, 19, 10, 18), (3, 3, 3), (1, 1, 1)),
    (128, 128, (1, 128, 3, 7, 9), (3, 3, 3), (1, 1, 1)),
    (7, 19, (1, 7, 5, 10, 18), (3, 3, 3), (1, 1, 1)),
    (128, 128, (1, 128, 5, 17, 33), (3, 3, 3), (1, 2, 2)),
    (128, 128, (1, 128, 3, 10, 18), (1, 3, 3), (1, 1, 1)),
    (64, 128, (2, 64, 4, 6, 70), (3, 3, 3), (1, 1, 1)),
    # window-in-LDS kernel (stride 1, C % 64 == 0, N % 128 == 0, Wo in {32, 64, 128, 256})
    (64, 128, (1, 64, 4, 4, 258), (3, 3, 3), (1, 1, 1)),
    (128, 256, (2, 128, 4, 10, 66), (3, 3, 3), (1, 1, 1)),
    (128, 128, (1, 128, 5, 6, 130), (3, 3, 3), (1, 1, 1)),
    (256, 128, (1, 256, 3, 6, 130), (3, 3, 3), (1, 1, 1)),
    (128, 128, (1, 128, 4, 18, 34), (3, 3, 3), (1, 1, 1)),     # output width 32
    (256, 256, (3, 256, 5, 18, 34), (3, 3, 3), (1, 1, 1)),
    # one padded 9 x 64 x 64 clip at 128 -> 128: 72 window tiles, so it runs on 256 x 128 implicit-GEMM tiles
    (128, 128, (1, 128, 11, 66, 66), (3, 3, 3), (1, 1, 1)),
]


@pytest.mark.parametrize("ci,co,shape,kernel,stride", CASES)
def test_conv_int32_exact_and_causal_skip_equal(ops, oracle, ci, co, shape, kernel, stride):
    gen = _gen(ci * 7 + co + sum(shape))
    b, c, d, h, w = shape
    qx = torch.randint(-127, 128, (b, d, h, w, c), generator=gen, dtype=torch.int8)
    qx[:, :2] = 0                                    # the producer's causal zero planes
    k = kernel[0] * kernel[1] * kernel[2] * ci
    qw = torch.randint(-127, 128, (co, k), generator=gen, dtype=torch.int8)
    full = _conv_i32_gpu(ops, qx, qw, kernel, stride, False)
    skip = _conv_i32_gpu(ops, qx, qw, kernel, stride, True)
    want = oracle.conv3d_acc(qx.numpy(), qw.numpy(), kernel, stride)
    assert np.array_equal(full, want)
    assert np.array_equal(skip, want)


def test_conv_all_ones_kat(ops):
    """Reference tests/test_encoder_int8_gpu.py:153-165: all-ones 128-channel conv -> 27*128."""
    x = torch.ones((1, 3, 10, 18, 128), dtype=torch.int8)
    qw = torch.ones((128, 27 * 128), dtype=torch.int8)
    acc = _conv_i32_gpu(ops, x, qw, (3, 3, 3), (1, 1, 1))
    assert (acc == 3456).all()


@pytest.mark.parametrize("b,c,d,h,w,co,samples", [
    # 12 channel slices (the strided-pixel kernel runs its stages in groups of four), Wo 128: 128 tiles
    (1, 384, 10, 66, 130, 128, [(0, 0), (0, 1), (0, 7)]),
    # Wo 256, three weight tiles, two batch items: 192 tiles
    (2, 128, 4, 34, 258, 384, [(0, 0), (1, 1)]),
])
def test_conv_strided_pixel_shapes_sampled(ops, oracle, b, c, d, h, w, co, samples):
    """Window convs large enough (at least 128 tiles) to run the strided-pixel window kernel rather than
    the small-conv implicit GEMM: exact int32 against the oracle on the first output rows of sampled
    (batch, frame) pairs, with the causal skip."""
    gen = _gen(c + co + w)
    qx = torch.randint(-127, 128, (b, d, h, w, c), generator=gen, dtype=torch.int8)
    qx[:, :2] = 0
    qw = torch.randint(-127, 128, (co, 27 * c), generator=gen, dtype=torch.int8)
    print(f"strided-pixel window conv {b}x{c}x{d}x{h}x{w} -> {co}", flush=True)
    acc = _conv_i32_gpu(ops, qx, qw, (3, 3, 3), (1, 1, 1), True)
    rows = 512 // (w - 2)                                        # output rows of one tile
    for bi, t in samples:
        want = oracle.conv3d_acc(qx[bi:bi + 1, t:t + 3, :2 * rows + 2].numpy(), qw.numpy(), (3, 3, 3), (1, 1, 1))
        assert np.array_equal(acc[bi:bi + 1, t:t + 1, :2 * rows], want), f"batch {bi} frame {t}"


def test_conv_strided_pixel_partial_row_group(ops, oracle):
    """The window kernel walks its tiles in groups of 8 / (weight tiles) row blocks; an output height of 40
    (5 row blocks of 8 rows) leaves one partial group.  Exact int32 against the oracle on the first and the
    last row block of sampled frames (130 tiles: the strided-pixel window kernel)."""
    gen = _gen(4242)
    qx = torch.randint(-127, 128, (1, 15, 42, 130, 128), generator=gen, dtype=torch.int8)
    qx[:, :2] = 0
    qw = torch.randint(-127, 128, (128, 3456), generator=gen, dtype=torch.int8)
    print("strided-pixel window conv 1x128x15x42x130 -> 128 (partial row group)", flush=True)
    acc = _conv_i32_gpu(ops, qx, qw, (3, 3, 3), (1, 1, 1), True)
    for t in (0, 5, 12):
        for r0 in (0, 32):
            want = oracle.conv3d_acc(qx[:, t:t + 3, r0:r0 + 10].numpy(), qw.numpy(), (3, 3, 3), (1, 1, 1))
            assert np.array_equal(acc[:, t:t + 1, r0:r0 + 8], want), f"frame {t} rows {r0}.."


def test_conv_h3_stage0_shape_sampled(ops, oracle):
    """Real stage-0 layer: [1,128,19,258,258] int8 -> [1,17,256,256,128], causal skip; frames sampled."""
    gen = _gen(11)
    qx = torch.randint(-127, 128, (1, 19, 258, 258, 128), generator=gen, dtype=torch.int8)
    qx[:, :2] = 0
    qw = torch.randint(-127, 128, (128, 3456), generator=gen, dtype=torch.int8)
    acc = _conv_i32_gpu(ops, qx, qw, (3, 3, 3), (1, 1, 1), True)
    for t in (0, 1, 2, 16):
        want = oracle.conv3d_acc(qx[:, t:t + 3, :34].numpy(), qw.numpy(), (3, 3, 3), (1, 1, 1))
        assert np.array_equal(acc[:, t:t + 1, :32], want), f"frame {t}"


# (d, h, w, c): implicit-GEMM tiles (the second one a window-kernel geometry too small for the window kernel:
# 4 tiles), then the window kernel's strided-pixel form on 128-column blocks of Wo 256 (128 tiles)
@pytest.mark.parametrize("d,h,w,c", [(5, 12, 20, 256), (4, 6, 130, 128), (6, 34, 258, 128)])
@pytest.mark.parametrize("with_bias", [False, True])
def test_conv_dequant_epilogue(ops, oracle, with_bias, d, h, w, c):
    gen = _gen(5)
    qx = torch.randint(-127, 128, (1, d, h, w, c), generator=gen, dtype=torch.int8)
    qw = torch.randint(-127, 128, (256, 27 * c), generator=gen, dtype=torch.int8)
    xs = torch.tensor([0.013], dtype=torch.float32)
    ws = (torch.rand(256, generator=gen) * 0.001 + 1e-4).float()
    bias = torch.randn(256, generator=gen).half() if with_bias else None
    out = torch.empty((1, d - 2, h - 2, w - 2, 256), dtype=torch.float16, device=DEV)
    dev = [t.to(DEV) if t is not None else None for t in (qx, xs, qw, ws, bias)]
    ops.hip.call("h3v_conv3d_i8", *[ops.hip.ptr(t) for t in dev], ops.hip.ptr(out), 1, c, d, h, w, 256, 3, 3, 3, 1,
                 1, 1, 0, ops.hip.stream(DEV))
    torch.cuda.synchronize()
    acc = oracle.conv3d_acc(qx.numpy(), qw.numpy(), (3, 3, 3), (1, 1, 1))
    want = oracle.gemm_dequant(acc.reshape(-1, 256), xs.numpy(), ws.numpy(),
                               None if bias is None else bias.numpy()).reshape(acc.shape)
    assert_bitwise(np_(out), want, "conv out")


# the residual block's closing add fused into the epilogue: implicit GEMM (a small window geometry and a
# plain one), scalar fallback, and the window kernel (128 tiles at Wo 256)
@pytest.mark.parametrize("d,h,w,c,n", [(4, 6, 130, 128, 128), (5, 12, 20, 256, 256), (4, 7, 9, 7, 19),
                                       (6, 66, 258, 128, 128)])
def test_conv_residual_epilogue(ops, oracle, d, h, w, c, n):
    print(f"conv residual epilogue D={d} {h}x{w} C={c} N={n}", flush=True)
    gen = _gen(9 + c)
    qx = torch.randint(-127, 128, (1, d, h, w, c), generator=gen, dtype=torch.int8)
    qx[:, :2] = 0                                    # the producer's causal zero planes (causal_skip below)
    qw = torch.randint(-127, 128, (n, 27 * c), generator=gen, dtype=torch.int8)
    xs = torch.tensor([0.013], dtype=torch.float32)
    ws = (torch.rand(n, generator=gen) * 0.001 + 1e-4).float()
    bias = torch.randn(n, generator=gen).half()
    res = (torch.randn(1, d - 2, h - 2, w - 2, n, generator=gen) * 3).half()
    out = torch.empty((1, d - 2, h - 2, w - 2, n), dtype=torch.float16, device=DEV)
    dev = [t.to(DEV) for t in (qx, xs, qw, ws, bias)]
    rd = res.to(DEV)
    ops.hip.call("h3v_conv3d_i8_residual", *[ops.hip.ptr(t) for t in dev], ops.hip.ptr(rd), ops.hip.ptr(out), 1, c, d,
                 h, w, n, 3, 3, 3, 1, 1, 1, 1, ops.hip.stream(DEV))
    torch.cuda.synchronize()
    acc = oracle.conv3d_acc(qx.numpy(), qw.numpy(), (3, 3, 3), (1, 1, 1))
    conv = oracle.gemm_dequant(acc.reshape(-1, n), xs.numpy(), ws.numpy(), bias.numpy()).reshape(acc.shape)
    want = (res.numpy().astype(np.float32) + conv.astype(np.float32)).astype(np.float16)   # torch's fp16 add
    assert_bitwise(np_(out), want, "conv + residual")
    with pytest.raises(ValueError, match="alias"):
        ops.hip.call("h3v_conv3d_i8_residual", *[ops.hip.ptr(t) for t in dev], ops.hip.ptr(out), ops.hip.ptr(out), 1,
                     c, d, h, w, n, 3, 3, 3, 1, 1, 1, 1, ops.hip.stream(DEV))


# reference tests/test_encoder_int8_norm.py:38 (seed, c, d, h, w) plus a full-resolution frame set
NORM_CASES = [(41, 128, 1, 2, 3), (42, 256, 3, 13, 19), (43, 128, 3, 256, 256), (44, 256, 17, 32, 48)]


@pytest.mark.parametrize("seed,c,d,h,w", NORM_CASES)
@pytest.mark.parametrize("with_pre_bias", [False, True])
def test_norm_pack_matches_oracle(ops, oracle, seed, c, d, h, w, with_pre_bias):
    gen = _gen(seed)
    x = torch.randn((1, c, d, h, w), generator=gen).half()
    weight = torch.randn(c, generator=gen).half()
    bias = torch.randn(c, generator=gen).half()
    pre_bias = bias if with_pre_bias else None
    qy, scale, stats = ops.encoder_int8_norm.quantized_temporal_norm_pad(
        x.to(DEV), weight.to(DEV), bias.to(DEV), 1e-6, pre_bias=None if pre_bias is None else pre_bias.to(DEV),
        return_stats=True)
    torch.cuda.synchronize()
    xn = ndhwc(x)[0]
    rstats = oracle.gn_stats(xn, 1e-6, None if pre_bias is None else pre_bias.numpy())
    assert_bitwise(np_(stats).view(np.uint32), rstats.view(np.uint32), "stats")
    _, _, amax = oracle.norm_pack(xn, weight.numpy(), bias.numpy(), rstats,
                                  None if pre_bias is None else pre_bias.numpy(), want_fp16=False)
    rs = oracle.scale_from_amax(amax)
    assert np.float32(scale.item()).view(np.uint32) == rs.view(np.uint32)
    _, rq, _ = oracle.norm_pack(xn, weight.numpy(), bias.numpy(), rstats,
                                None if pre_bias is None else pre_bias.numpy(), scale=rs, want_fp16=False)
    assert qy.is_contiguous(memory_format=torch.channels_last_3d)
    assert_bitwise(ndhwc(qy)[0], rq, "q")
    assert (ndhwc(qy)[0, :2] == 0).all()


@pytest.mark.parametrize("value", [0.0, 2.0 ** -24, 2.0 ** -14, -10.0, 2.0])
def test_norm_pack_constant_inputs(ops, oracle, value):
    """Reference tests/test_encoder_int8_norm.py:61-69: zero input, constant beta."""
    x = torch.zeros((1, 128, 1, 3, 5), dtype=torch.float16)
    weight = torch.ones(128, dtype=torch.float16)
    bias = torch.full((128,), value, dtype=torch.float16)
    qy, scale = ops.encoder_int8_norm.quantized_temporal_norm_pad(x.to(DEV), weight.to(DEV), bias.to(DEV), 1e-6)
    torch.cuda.synchronize()
    xn = ndhwc(x)[0]
    st = oracle.gn_stats(xn, 1e-6)
    _, _, amax = oracle.norm_pack(xn, weight.numpy(), bias.numpy(), st, want_fp16=False)
    rs = oracle.scale_from_amax(amax)
    _, rq, _ = oracle.norm_pack(xn, weight.numpy(), bias.numpy(), st, scale=rs, want_fp16=False)
    assert np.float32(scale.item()) == rs
    assert_bitwise(ndhwc(qy)[0], rq, "q")


@pytest.mark.parametrize("c,d,pre,cb", [(128, 1, False, False), (128, 2, True, True), (256, 17, True, False),
                                        (128, 3, False, True)])
def test_norm_conv3d_op_matches_oracle(ops, oracle, c, d, pre, cb):
    """Reference tests/test_encoder_int8_norm.py:94-121 geometries through the custom op."""
    gen = _gen(45 + d)
    x = torch.randn((1, c, d, 8, 16), generator=gen).half()
    weight = torch.randn(c, generator=gen).half()
    bias = torch.randn(c, generator=gen).half()
    conv = (torch.randn((256, c, 3, 3, 3), generator=gen) / 64).half()
    qw, ws, _ = ops.encoder_int8.prepare_int8_weight(conv)
    conv_bias = torch.randn(256, generator=gen).half() if cb else None
    with torch.inference_mode():
        y = ops.encoder_int8_integration.int8_norm_conv3d(
            x.to(DEV), weight.to(DEV), bias.to(DEV), bias.to(DEV) if pre else None, 1e-6, qw.to(DEV), ws.to(DEV),
            None if conv_bias is None else conv_bias.to(DEV))
    torch.cuda.synchronize()
    ry, _, _ = oracle.norm_conv3d(ndhwc(x)[0], weight.numpy(), bias.numpy(), 1e-6, qw.numpy(), ws.numpy(),
                                  None if conv_bias is None else conv_bias.numpy(), bias.numpy() if pre else None)
    assert y.is_contiguous(memory_format=torch.channels_last_3d)
    assert_bitwise(ndhwc(y)[0], ry, "norm conv")


def test_prepare_weight_on_gpu_matches_oracle(ops, oracle):
    gen = _gen(3)
    w = (torch.randn((256, 128, 3, 3, 3), generator=gen) / 64).half()
    q_gpu, s_gpu, _ = ops.encoder_int8.prepare_int8_weight(w.to(DEV))
    rq, rs = oracle.prepare_conv_weight(w.float().numpy())
    assert_bitwise(np_(s_gpu).view(np.uint32), rs.view(np.uint32), "scale")
    assert_bitwise(np_(q_gpu), rq, "q")


def test_valid_conv_generic_entry(ops, oracle):
    """int8_valid_conv3d: per-tensor quant + conv, stride (1,2,2), odd channels, bias."""
    gen = _gen(9)
    x = torch.randn((2, 7, 5, 9, 11), generator=gen).half()
    w = (torch.randn((19, 7, 3, 3, 3), generator=gen) / (7 * 27) ** 0.5).half()
    bias = torch.randn(19, generator=gen).half()
    qw, ws, cfg = ops.encoder_int8.prepare_int8_weight(w, stride=(1, 2, 2))
    with torch.inference_mode():
        y = ops.encoder_int8.int8_valid_conv3d(x.to(DEV), qw.to(DEV), ws.to(DEV), config=cfg, bias=bias.to(DEV))
    torch.cuda.synchronize()
    xn = ndhwc(x)
    s = oracle.tensor_scale(xn)
    qx = oracle.tensor_quant(xn, s)
    acc = oracle.conv3d_acc(qx, qw.numpy(), (3, 3, 3), (1, 2, 2))
    want = oracle.gemm_dequant(acc.reshape(-1, 19), np.array([s], np.float32), ws.numpy(), bias.numpy())
    assert_bitwise(ndhwc(y), want.reshape(acc.shape), "conv")
