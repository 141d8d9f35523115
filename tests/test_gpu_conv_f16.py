"""GPU parity: the FP16 window-in-LDS 3x3x3 convolution (h3v_conv3d_f16, ``conv3d_f16``) of the encoder
suffix against a float64 CPU convolution of the same fp16 operands.

Tolerance: the kernel multiplies fp16 operands exactly, sums in fp32 on the matrix cores, adds the fp16
bias in fp32 and rounds once to fp16, so |y - ref| <= ulp16(ref) + 2^-20 * sum|x * w| per output (one
fp16 rounding plus the fp32 summation error with a 16x margin).  A dropped or misplaced tap moves an
output by about one product |x * w| ~ sum|x * w| / K, far outside that bound."""
from __future__ import annotations

import importlib

import pytest
import torch
import torch.nn.functional as F

import h3_arch

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


@pytest.fixture(scope="module")
def bn(pkg):
    return importlib.import_module(f"{pkg.__name__}.opt.encoder_fused_batched_norm")


@pytest.fixture(scope="module")
def fc(pkg):
    return importlib.import_module(f"{pkg.__name__}.opt.encoder_fp16_conv")


def _operands(b, c, d, h, w, cout, with_bias, seed, causal_zero=True):
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(b, c, d, h, w, generator=gen).half()
    if causal_zero:
        x[:, :, :2] = 0                                # the producer's two causal zero frames per item
    wt = (torch.randn(cout, c, 3, 3, 3, generator=gen) * (27 * c) ** -0.5).half()
    bias = (0.5 * torch.randn(cout, generator=gen)).half() if with_bias else None
    return x, wt, bias


def _reference(x, wt, bias):
    ref = F.conv3d(x.double(), wt.double(), None if bias is None else bias.double())
    mag = F.conv3d(x.double().abs(), wt.double().abs())
    return ref, mag


def _assert_close(y, ref, mag):
    y = y.detach().cpu().double()
    exp = torch.floor(torch.log2(ref.abs().clamp_min(2.0 ** -14)))
    ulp = torch.pow(2.0, exp - 10)
    bound = ulp + 2.0 ** -20 * mag
    err = (y - ref).abs()
    bad = err > bound
    assert not bool(bad.any()), (f"{int(bad.sum())} of {bad.numel()} outputs outside the bound; worst excess "
                                 f"{float((err - bound).max()):.3e}")


def _run(fc, x, wt, bias, causal_skip, stride=(1, 1, 1)):
    xd = x.to(DEV).contiguous(memory_format=torch.channels_last_3d)
    wp = fc.pack_conv_weight_f16(wt.to(DEV))
    bd = None if bias is None else bias.to(DEV)
    with torch.inference_mode():
        y = fc.conv3d_f16(xd, wp, bd, list(wt.shape[2:]), list(stride), causal_skip)
    torch.cuda.synchronize()
    return y


# (batch, Cin, D, H, W, Cout): output widths 32 / 64 / 128 / 256, one and several items, Cin 32..512
CASES = [
    (1, 32, 4, 18, 34, 128, True),
    (3, 256, 5, 10, 66, 128, True),
    (2, 128, 4, 6, 130, 256, False),
    (1, 64, 3, 4, 258, 128, True),
    (4, 512, 3, 18, 34, 256, True),
    (4, 256, 6, 34, 34, 512, False),
]


@pytest.mark.parametrize("b,c,d,h,w,cout,with_bias", CASES)
def test_conv3d_f16_matches_float64(fc, b, c, d, h, w, cout, with_bias):
    print(f"conv3d_f16 B={b} C={c} D={d} {h}x{w} Cout={cout} bias={with_bias}", flush=True)
    x, wt, bias = _operands(b, c, d, h, w, cout, with_bias, seed=b * 1000 + c + d + h + w + cout)
    y = _run(fc, x, wt, bias, causal_skip=True)
    assert y.shape == (b, cout, d - 2, h - 2, w - 2) and y.dtype == torch.float16
    assert y.is_contiguous(memory_format=torch.channels_last_3d)
    ref, mag = _reference(x, wt, bias)
    _assert_close(y, ref, mag)
    # the causal skip drops only taps on zero frames: the full reduction gives the same values
    y_full = _run(fc, x, wt, bias, causal_skip=False)
    assert torch.equal(y_full, y)


def test_conv3d_f16_nonzero_leading_frames_without_skip(fc):
    """causal_skip=False reads every depth tap: leading frames that are not zero take part."""
    x, wt, bias = _operands(2, 64, 5, 10, 66, 128, True, seed=5, causal_zero=False)
    y = _run(fc, x, wt, bias, causal_skip=False)
    ref, mag = _reference(x, wt, bias)
    _assert_close(y, ref, mag)


def test_conv3d_f16_matches_torch_fp16(fc):
    """Same operands through the model's FP16 F.conv3d on the GPU (its own accumulation order)."""
    x, wt, bias = _operands(3, 256, 6, 18, 66, 256, True, seed=17)
    y = _run(fc, x, wt, bias, causal_skip=True).float()
    ref = F.conv3d(x.to(DEV), wt.to(DEV), bias.to(DEV)).float()
    rel = (y - ref).norm() / ref.norm()
    assert rel < 1e-3, float(rel)


def test_conv3d_f16_rejects_unfit_shapes(fc):
    x = torch.zeros(1, 16, 3, 6, 66, dtype=torch.float16, device=DEV).contiguous(memory_format=torch.channels_last_3d)
    w = torch.zeros(128, 27 * 16, dtype=torch.float16, device=DEV)
    with pytest.raises(ValueError, match="Cin % 32"):
        fc.conv3d_f16(x, w, None, [3, 3, 3], [1, 1, 1], True)
    x2 = torch.zeros(1, 64, 3, 6, 66, dtype=torch.float16, device=DEV).contiguous(memory_format=torch.channels_last_3d)
    with pytest.raises(ValueError, match="packed"):
        fc.conv3d_f16(x2, w[:, :100].contiguous(), None, [3, 3, 3], [1, 1, 1], True)


# implicit-GEMM path: (batch, Cin, D, H, W, Cout, kernel, stride) -- strides, 1x1x1, Cout not a multiple of
# 128, widths the window kernel does not take, Cin 32 (64-byte reduction steps) and Cout > 128 (256 x 256 tiles)
GEMM_CASES = [
    (1, 128, 19, 34, 34, 128, (3, 3, 3), (1, 2, 2)),       # stage-0 downsample geometry, reduced
    (1, 256, 19, 17, 17, 256, (3, 3, 3), (2, 2, 2)),       # stage-1 downsample after the residual pack
    (2, 64, 5, 10, 50, 64, (3, 3, 3), (1, 1, 1)),          # Wo 48, Cout 64
    (1, 32, 4, 9, 21, 96, (3, 3, 3), (1, 1, 1)),
    (3, 256, 4, 8, 8, 512, (1, 1, 1), (1, 1, 1)),          # nin_shortcut
    (1, 128, 3, 20, 20, 200, (3, 3, 3), (1, 1, 1)),
    (1, 96, 4, 12, 12, 256, (3, 3, 3), (1, 1, 1)),          # 64-byte steps on 256 x 128 tiles (few tiles)
    (1, 256, 3, 18, 18, 1024, (3, 3, 3), (1, 1, 1)),        # 16^2 width, Cout 1024 on 256 x 128 tiles
]


@pytest.mark.parametrize("b,c,d,h,w,cout,kernel,stride", GEMM_CASES)
def test_conv3d_f16_implicit_gemm_matches_float64(fc, b, c, d, h, w, cout, kernel, stride):
    print(f"conv3d_f16 implicit GEMM B={b} C={c} D={d} {h}x{w} Cout={cout} k={kernel} s={stride}", flush=True)
    gen = torch.Generator().manual_seed(c + d + h + w + cout + sum(stride))
    x = torch.randn(b, c, d, h, w, generator=gen).half()
    wt = (torch.randn(cout, c, *kernel, generator=gen) * (c * kernel[0] * kernel[1] * kernel[2]) ** -0.5).half()
    bias = (0.5 * torch.randn(cout, generator=gen)).half()
    y = _run(fc, x, wt, bias, causal_skip=False, stride=stride)
    ref = F.conv3d(x.double(), wt.double(), bias.double(), stride=stride)
    mag = F.conv3d(x.double().abs(), wt.double().abs(), stride=stride)
    assert y.shape == ref.shape
    _assert_close(y, ref, mag)


# K split over a workspace: (batch, Cin, D, H, W, Cout, causal zero frames, residual); tiles fill under half
# a round, so S workgroups per tile write fp32 partial sums that a second kernel adds
SPLIT_CASES = [
    (1, 1024, 7, 18, 18, 48, False, False),     # conv_out-like: Cout 48 on 256 x 128 tiles, 16 splits
    (1, 256, 7, 18, 18, 256, False, True),      # 256 x 256 tiles, 12 splits, with a residual
    (2, 256, 5, 18, 18, 256, True, False),      # causal skip: frames 0 / 1 leave whole splits empty
]


@pytest.mark.parametrize("b,c,d,h,w,cout,causal,with_res", SPLIT_CASES)
def test_conv3d_f16_split_reduction_matches_float64(fc, b, c, d, h, w, cout, causal, with_res):
    print(f"conv3d_f16 split-K B={b} C={c} D={d} {h}x{w} Cout={cout} causal={causal} residual={with_res}", flush=True)
    lib = fc._hip.lib()
    floats = int(lib.h3v_conv3d_f16_workspace_floats(b, c, d, h, w, cout, 3, 3, 3, 1, 1, 1))
    m = b * (d - 2) * (h - 2) * (w - 2)
    assert floats > 0 and floats % (m * cout) == 0 and floats // (m * cout) >= 2   # the geometry splits
    x, wt, bias = _operands(b, c, d, h, w, cout, True, seed=c + cout + d, causal_zero=causal)
    gen = torch.Generator().manual_seed(cout)
    res = (torch.randn(b, cout, d - 2, h - 2, w - 2, generator=gen) * 2).half() if with_res else None
    xd = x.to(DEV).contiguous(memory_format=torch.channels_last_3d)
    wp = fc.pack_conv_weight_f16(wt.to(DEV))
    rd = None if res is None else res.to(DEV).contiguous(memory_format=torch.channels_last_3d)
    with torch.inference_mode():
        y = fc.conv3d_f16(xd, wp, bias.to(DEV), [3, 3, 3], [1, 1, 1], causal)
        fused = fc.conv3d_f16(xd, wp, bias.to(DEV), [3, 3, 3], [1, 1, 1], causal, rd) if with_res else None
        torch.cuda.synchronize()
    ref, mag = _reference(x, wt, bias)
    _assert_close(y, ref, mag)
    if with_res:
        assert torch.equal(fused, rd + y)                  # the reduction's residual add == torch's fp16 add
    # the unsplit entry (no workspace) gives values within the same bound
    out = torch.empty_like(y)
    fc._hip.call("h3v_conv3d_f16", fc._hip.ptr(xd), fc._hip.ptr(wp), fc._hip.ptr(bias.to(DEV)), None,
                 fc._hip.ptr(out), b, c, d, h, w, cout, 3, 3, 3, 1, 1, 1, int(causal), fc._hip.stream(DEV))
    torch.cuda.synchronize()
    _assert_close(out, ref, mag)
    # a workspace one float short is refused before anything runs
    ws = torch.empty(floats, device=DEV, dtype=torch.float32)
    with pytest.raises(ValueError, match="workspace"):
        fc._hip.call("h3v_conv3d_f16_ws", fc._hip.ptr(xd), fc._hip.ptr(wp), fc._hip.ptr(bias.to(DEV)), None,
                     fc._hip.ptr(out), b, c, d, h, w, cout, 3, 3, 3, 1, 1, 1, int(causal), fc._hip.ptr(ws),
                     floats - 1, fc._hip.stream(DEV))


@pytest.mark.parametrize("d,cout", [(18, 32), (10, 48)])
def test_conv3d_f16_row_tile_choice_sampled_frames(fc, d, cout):
    """Cout <= 128 implicit GEMM at full size: 16 output frames of 64 x 128 (131072 rows) fill whole rounds
    with 512-row tiles, 8 frames (65536 rows, half a round) take 256-row tiles; output frames sampled
    against float64 convs of their own three input frames."""
    print(f"conv3d_f16 row-tile choice D={d} Cout={cout}", flush=True)
    x, wt, bias = _operands(1, 64, d, 130, 258, cout, True, seed=d + cout, causal_zero=False)
    y = _run(fc, x, wt, bias, causal_skip=False, stride=(1, 2, 2))
    assert y.shape == (1, cout, d - 2, 64, 128)
    for t in (0, (d - 2) // 2, d - 3):
        xs = x[:, :, t:t + 3].double()
        ref = F.conv3d(xs, wt.double(), bias.double(), stride=(1, 2, 2))
        mag = F.conv3d(xs.abs(), wt.double().abs(), stride=(1, 2, 2))
        _assert_close(y[:, :, t:t + 1], ref, mag)


@pytest.mark.parametrize("b,c,d,h,w,cout,kernel", [(2, 64, 5, 10, 66, 128, (3, 3, 3)), (1, 64, 4, 10, 50, 96, (3, 3, 3)),
                                                   (3, 256, 4, 8, 8, 256, (1, 1, 1)),
                                                   (1, 64, 4, 10, 50, 100, (3, 3, 3))])   # scalar output rows
def test_conv3d_f16_residual_equals_separate_add(fc, b, c, d, h, w, cout, kernel):
    """The fused residual (window kernel, implicit GEMM, 1x1x1) == the conv followed by torch's fp16 add."""
    gen = torch.Generator().manual_seed(c + cout + d)
    x = torch.randn(b, c, d, h, w, generator=gen).half()
    x[:, :, :2] = 0
    wt = (torch.randn(cout, c, *kernel, generator=gen) * (c * kernel[0] ** 3) ** -0.5).half()
    bias = (0.5 * torch.randn(cout, generator=gen)).half()
    do, ho, wo = d - kernel[0] + 1, h - kernel[1] + 1, w - kernel[2] + 1
    res = (torch.randn(b, cout, do, ho, wo, generator=gen) * 2).half().to(DEV).contiguous(
        memory_format=torch.channels_last_3d)
    xd = x.to(DEV).contiguous(memory_format=torch.channels_last_3d)
    wp = fc.pack_conv_weight_f16(wt.to(DEV))
    with torch.inference_mode():
        plain = fc.conv3d_f16(xd, wp, bias.to(DEV), list(kernel), [1, 1, 1], kernel[0] == 3)
        fused = fc.conv3d_f16(xd, wp, bias.to(DEV), list(kernel), [1, 1, 1], kernel[0] == 3, res)
        strided = fc.conv3d_f16(xd, wp, bias.to(DEV), list(kernel), [1, 1, 1], kernel[0] == 3, res.contiguous())
        torch.cuda.synchronize()
    assert torch.equal(fused, res + plain)
    assert torch.equal(strided, fused)                           # an NCDHW residual is made channels-last first


def test_conv3d_f16_implicit_gemm_causal_skip(fc):
    """Stride-1 convs outside the window kernel skip the zero depth taps per tile with the same values."""
    x, wt, bias = _operands(2, 64, 6, 10, 50, 64, True, seed=9)
    y = _run(fc, x, wt, bias, causal_skip=True)
    assert torch.equal(y, _run(fc, x, wt, bias, causal_skip=False))
    ref, mag = _reference(x, wt, bias)
    _assert_close(y, ref, mag)


@pytest.mark.parametrize("shape,pads", [((1, 128, 5, 16, 16), (2, 1, 1, 1, 1)), ((4, 256, 3, 7, 9), (2, 0, 1, 0, 1)),
                                        ((2, 64, 1, 3, 4), (0, 2, 2, 3, 3))])
def test_causal_reflect_pack_matches_torch_pad(fc, shape, pads):
    front, top, bottom, left, right = pads
    gen = torch.Generator().manual_seed(sum(shape))
    x = torch.randn(*shape, generator=gen).half()
    with torch.inference_mode():
        y = fc.causal_reflect_pack(x.to(DEV).contiguous(memory_format=torch.channels_last_3d), *pads)
        torch.cuda.synchronize()
    want = F.pad(F.pad(x.float(), (left, right, top, bottom, 0, 0), mode="reflect"), (0, 0, 0, 0, front, 0)).half()
    assert y.is_contiguous(memory_format=torch.channels_last_3d)
    assert torch.equal(y.cpu(), want)


@pytest.mark.parametrize("c,b,d,h,w,front", [(3, 1, 5, 16, 20, 2), (1, 2, 3, 6, 9, 2), (2, 1, 1, 4, 4, 0)])
def test_tap_fold_pack_matches_torch(fc, c, b, d, h, w, front):
    gen = torch.Generator().manual_seed(c + d + h)
    x = torch.randn(b, c, d, h, w, generator=gen).half()
    with torch.inference_mode():
        y = fc.tap_fold_pack(x.to(DEV).contiguous(memory_format=torch.channels_last_3d), front)
        torch.cuda.synchronize()
    xp = F.pad(F.pad(x.float(), (1, 1, 1, 1, 0, 0), mode="reflect"), (0, 0, 0, 0, front, 0))
    want = torch.zeros(b, 32, d + front, h, w)
    for kh in range(3):
        for kw in range(3):
            want[:, (kh * 3 + kw) * c:(kh * 3 + kw + 1) * c] = xp[:, :, :, kh:kh + h, kw:kw + w]
    assert y.is_contiguous(memory_format=torch.channels_last_3d)
    assert torch.equal(y.cpu(), want.half())


@pytest.mark.parametrize("d,hw", [(17, 64), (1, 32), (5, 40)])
def test_conv_in_through_internal_padding_matches_float64(pkg, d, hw):
    """conv_in (3 -> 128) via ImplicitTemporalPadConv3d: tap-folded pack + 3x1x1 conv3d_f16, against a float64
    run of the model's padding and 3x3x3 conv (one image frame: two zero frames in front, as the model pads)."""
    ip = importlib.import_module(f"{pkg.__name__}.opt.encoder_internal_padding")
    torch.manual_seed(d + hw)
    conv = h3_arch.CausalConv3d(3, 128).half().to(DEV).eval()
    wrapped = ip.ImplicitTemporalPadConv3d(conv)
    gen = torch.Generator().manual_seed(hw)
    x = (torch.rand(1, 3, d, hw, hw, generator=gen) * 4 - 2).half()
    with torch.inference_mode():
        y = wrapped(x.to(DEV).contiguous(memory_format=torch.channels_last_3d))
        model = conv(x.to(DEV))
        torch.cuda.synchronize()
    xp = F.pad(F.pad(x.double(), (1, 1, 1, 1, 0, 0), mode="reflect"), (0, 0, 0, 0, 2, 0))
    w64, b64 = conv.weight.detach().cpu().double(), conv.bias.detach().cpu().double()
    ref = F.conv3d(xp, w64, b64)
    mag = F.conv3d(xp.abs(), w64.abs())
    assert y.shape == ref.shape == model.shape == (1, 128, d, hw, hw)
    _assert_close(y, ref, mag)


def test_stage0_downsample_matches_model(pkg, fc):
    """down.0.downsample.conv through ImplicitTemporalPadConv3d (pack + conv3d_f16) == the model's CausalConv3d
    within the fp16 bound, against a float64 run of the model's own padding."""
    ip = importlib.import_module(f"{pkg.__name__}.opt.encoder_internal_padding")
    torch.manual_seed(3)
    down = h3_arch.Downsample(128, (1, 2, 2), (1, 1, 1)).half().to(DEV).eval()
    conv = ip.ImplicitTemporalPadConv3d(down.conv)
    gen = torch.Generator().manual_seed(4)
    x = torch.randn(1, 128, 5, 32, 32, generator=gen).half()
    with torch.inference_mode():
        y = conv(x.to(DEV).contiguous(memory_format=torch.channels_last_3d))
        torch.cuda.synchronize()
    xp = F.pad(F.pad(x.double(), (1, 1, 1, 1, 0, 0), mode="reflect"), (0, 0, 0, 0, 2, 0))
    w64, b64 = down.conv.weight.detach().cpu().double(), down.conv.bias.detach().cpu().double()
    ref = F.conv3d(xp, w64, b64, stride=(1, 2, 2))
    mag = F.conv3d(xp.abs(), w64.abs(), stride=(1, 2, 2))
    assert y.shape == ref.shape == (1, 128, 5, 16, 16)
    _assert_close(y, ref, mag)


@pytest.mark.parametrize("cin,cout,hw", [(256, 256, 32), (256, 512, 64)])
def test_batched_residual_block_with_native_convs(bn, fc, cin, cout, hw):
    """Clips batched through BatchedResidualBlock, whose convs now fit h3v_conv3d_f16, == the model's
    ResnetBlock3D clip by clip (FP16 tolerance: different reduction orders for statistics and convs)."""
    torch.manual_seed(cin + cout + hw)
    block = h3_arch.ResnetBlock3D(cin, cout).half().to(DEV).eval()
    gen = torch.Generator().manual_seed(hw)
    x = torch.randn(4, cin, 5, hw, hw, generator=gen).half().to(DEV).contiguous(memory_format=torch.channels_last_3d)
    batched = bn.BatchedResidualBlock(block)
    probe = torch.zeros(1, cin, 7, hw + 2, hw + 2, dtype=torch.float16, device=DEV)
    assert fc.conv3d_f16_fits(probe, block.conv1.weight, (1, 1, 1))
    with torch.inference_mode():
        ref = torch.cat([block(x[i:i + 1]) for i in range(4)])
        y = batched(x)
        torch.cuda.synchronize()
    rel = (y.float() - ref.float()).norm() / ref.float().norm()
    assert rel < 5e-3, float(rel)


def test_batched_suffix_all_stages_matches_model_suffix(pkg, bn):
    """The runtime's suffix (BatchedSuffix over every suffix stage of the H3 encoder: its residual blocks,
    stride-(2,2,2) and (1,2,2) downsamples, norm_out, conv_out and quant_conv) on a staged batch of 4 clips ==
    the model's own suffix modules clip by clip, at the tile-256 suffix shape [4, 256, 9, 64, 64]."""
    staged = importlib.import_module(f"{pkg.__name__}.opt.encoder_staged_batch")
    torch.manual_seed(7)
    enc = h3_arch.H3Encoder(h3_arch.H3_ENCODER_STAGES).half().to(DEV).eval().to(memory_format=torch.channels_last_3d)
    quant = torch.nn.Conv3d(48, 48, 1).half().to(DEV).eval().to(memory_format=torch.channels_last_3d)
    gen = torch.Generator().manual_seed(8)
    x = torch.randn(4, 256, 9, 64, 64, generator=gen).half().to(DEV).contiguous(memory_format=torch.channels_last_3d)
    model = staged.EncoderSuffix(enc, quant, 2)
    fused = bn.fused_suffix(enc, quant, all_stages=True)
    with torch.inference_mode():
        ref = torch.cat([model(x[i:i + 1]) for i in range(4)])
        y = fused(x)
        torch.cuda.synchronize()
    assert y.shape == ref.shape == (4, 48, 5, 16, 16)
    rel = (y.float() - ref.float()).norm() / ref.float().norm()
    assert rel < 5e-3, float(rel)
