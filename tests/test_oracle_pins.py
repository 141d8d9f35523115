"""Pin the CPU oracle before trusting it (CPU only).

Every oracle function is checked against something that does not restate its
own formula: the reference's known-answer vectors, closed forms derived by
hand from exact arithmetic, numpy's independent implementations (float16
conversion, int64 matmul, float64 math) with stated error bounds, and
structural invariants of the padding/packing.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

RNG = np.random.default_rng(20261002)


# ---------------------------------------------------------------------------
# binary16 conversion and exp
# ---------------------------------------------------------------------------

def test_h2f_exhaustive_against_numpy(oracle):
    codes = np.arange(65536, dtype=np.uint16)
    ref = codes.view(np.float16).astype(np.float32)
    got = np.array([oracle.h2f(int(c)) for c in codes], np.float32)
    nan = np.isnan(ref)
    assert np.isnan(got[nan]).all()
    assert np.array_equal(ref[~nan].view(np.uint32), got[~nan].view(np.uint32))


def test_f2h_round_to_nearest_even_against_numpy(oracle):
    bits = RNG.integers(0, 2 ** 32, size=100000, dtype=np.uint64).astype(np.uint32)
    f = bits.view(np.float32)
    f = f[np.isfinite(f)]
    codes = np.arange(0, 0x7c00, dtype=np.uint16)
    v = codes.view(np.float16).astype(np.float64)
    mid = ((v[:-1] + v[1:]) / 2).astype(np.float32)            # exact ties
    probe = np.concatenate([f, mid, -mid, np.nextafter(mid, np.float32(np.inf)),
                            np.nextafter(mid, np.float32(0)), np.float32([65504, 65519.99, 65520, 1e9, 2.0 ** -25,
                                                                          2.0 ** -26, 0.0, -0.0])])
    with np.errstate(over="ignore"):
        ref = probe.astype(np.float16).view(np.uint16)
    got = np.array([oracle.f2h_bits(float(x)) for x in probe], np.uint16)
    assert np.array_equal(ref, got)


def test_exp_error_bound_and_special_values(oracle):
    xs = np.linspace(-87.0, 88.7, 100001).astype(np.float32)
    got = np.array([oracle.expf(float(x)) for x in xs], np.float64)
    ref = np.exp(xs.astype(np.float64))
    ulp = np.spacing(ref.astype(np.float32)).astype(np.float64)
    assert (np.abs(got - ref) / ulp).max() <= 2.0
    assert oracle.expf(0.0) == 1.0
    assert oracle.expf(float("inf")) == float("inf")
    assert oracle.expf(float("-inf")) == 0.0
    assert math.isnan(oracle.expf(float("nan")))
    assert oracle.expf(89.0) == float("inf")


# ---------------------------------------------------------------------------
# Q1 row quantizer (comfy-kitchen contract as restated by the reference)
# ---------------------------------------------------------------------------

def test_q1_zero_row_quirk(oracle):
    """opt/kitchen_int8.py:131-133: an all-zero row gives q=-128, s=1e-30."""
    q, s = oracle.row_quant(np.zeros((2, 64), np.float16))
    assert (q == -128).all()
    assert (s == np.float32(1e-30)).all()


@pytest.mark.parametrize("e", [-6, 0, 3])
def test_q1_closed_form_power_of_two_scale(oracle, e):
    """amax = 127*2^e -> s = 2^e exactly (127 * fp32(1/127) rounds to 1), so q = rint(a * 2^-e), ties to even."""
    base = np.array([127, 2.5, -2.5, 0.5, 1.5, -0.5, 3.5, 126.5, -127, 0, 64.5, -64.5], np.float64)
    row = (base * 2.0 ** e).astype(np.float16)[None]
    q, s = oracle.row_quant(row)
    assert s[0] == np.float32(2.0 ** e)
    assert q[0].tolist() == [127, 2, -2, 0, 2, 0, 4, 126, -127, 0, 64, -64]


def test_q1_zero_divisor_saturates_and_nan(oracle):
    """amax = 2^-24: s = 2^-24/127 rounds to fp16 0, so +x/0 -> 127, -x/0 -> -128, 0/0 -> NaN -> -128."""
    row = np.array([[2.0 ** -24, -(2.0 ** -24), 0.0, 2.0 ** -24]], np.float16)
    q, s = oracle.row_quant(row)
    assert q[0].tolist() == [127, -128, -128, 127]
    assert s[0] == np.float32(2.0 ** -24) * np.float32(1.0 / 127.0)
    row = np.array([[1.0, np.nan, -1.0]], np.float16)
    q, _ = oracle.row_quant(row)
    assert q[0, 1] == -128 and q[0, 0] == 127 and q[0, 2] == -127


def test_q1_dequant_error_bound(oracle):
    x = (RNG.standard_normal((64, 1024)) * RNG.uniform(0.01, 100, (64, 1))).astype(np.float16)
    q, s = oracle.row_quant(x)
    d = s.astype(np.float16).astype(np.float64)[:, None]
    err = np.abs(q.astype(np.float64) * d - x.astype(np.float64))
    # rint(fp16(x/d)): fp16 spacing below 128 is at most 1/16, so |q*d - x| <= (1/2 + 1/32) d
    assert (err <= (0.5 + 1.0 / 32) * d * (1 + 1e-6) + 1e-12).all()
    assert np.abs(q).max() <= 127 and (np.abs(q).max(axis=1) >= 126).all()


# ---------------------------------------------------------------------------
# encoder per-tensor quantizer (reference KATs)
# ---------------------------------------------------------------------------

def test_e3_reference_half_away_vector(oracle):
    """tests/test_encoder_int8_gpu.py:65-72 of the reference."""
    x = np.array([-127.0, -0.5, -1.5, 0.0, 0.5, 1.5, 127.0], np.float16)
    s = oracle.tensor_scale(x)
    assert s == np.float32(1.0)
    assert oracle.tensor_quant(x, s).tolist() == [-127, -1, -2, 0, 1, 2, 127]


@pytest.mark.parametrize("maximum", [0.0, 2.0 ** -24, 2.0 ** -14, 0.5, 127.0, 65504.0])
def test_e3_reference_extremes(oracle, maximum):
    """tests/test_encoder_int8_gpu.py:57-64: [-m, m, ..., m] -> [-127, 127, ...]; zero tensor -> s = 1, q = 0."""
    x = np.full(9, maximum, np.float16)
    x[0] = -maximum
    s = oracle.tensor_scale(x)
    q = oracle.tensor_quant(x, s)
    if maximum == 0:
        assert s == 1.0 and (q == 0).all()
    else:
        assert s == np.float32(maximum) * np.float32(1.0 / 127.0)
        assert q[0] == -127 and (q[1:] == 127).all()


# ---------------------------------------------------------------------------
# integer GEMM / conv accumulators and epilogues
# ---------------------------------------------------------------------------

def test_gemm_acc_matches_numpy_int64(oracle):
    a = RNG.integers(-128, 128, (37, 200), dtype=np.int8)
    w = RNG.integers(-128, 128, (53, 200), dtype=np.int8)
    assert np.array_equal(oracle.gemm_acc(a, w), a.astype(np.int64) @ w.astype(np.int64).T)


def test_dequant_zero_accumulator_is_bias_and_fp64_bound(oracle):
    """Zero products leave exactly the bias (reference tests/test_encoder_int8.py:44-50)."""
    bias = RNG.standard_normal(40).astype(np.float16)
    out = oracle.gemm_dequant(np.zeros((3, 40), np.int32), np.ones(3, np.float32), np.ones(40, np.float32), bias)
    assert np.array_equal(out.view(np.uint16), np.broadcast_to(bias, (3, 40)).view(np.uint16))
    acc = RNG.integers(-2 ** 20, 2 ** 20, (64, 48)).astype(np.int32)
    sx = RNG.uniform(1e-4, 1e-2, 64).astype(np.float32)
    sw = RNG.uniform(1e-4, 1e-2, 48).astype(np.float32)
    b = RNG.standard_normal(48).astype(np.float16)
    got = oracle.gemm_dequant(acc, sx, sw, b).astype(np.float64)
    ref = acc.astype(np.float64) * sx[:, None].astype(np.float64) * sw[None].astype(np.float64) + b.astype(np.float64)
    ulp16 = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64)
    assert (np.abs(got - ref) <= ulp16 * 0.5 + np.abs(ref) * 2e-7 + 1e-7).all()


def test_swiglu_epilogue_equals_dequant_then_swiglu(oracle):
    """Reference tests/test_int8_ffn_up_fused_gpu.py:21-33: fused == G1 then quantize_swiglu."""
    acc = RNG.integers(-200000, 200000, (9, 64)).astype(np.int32)
    sx = RNG.uniform(1e-4, 1e-3, 9).astype(np.float32)
    sw = RNG.uniform(1e-3, 1e-2, 64).astype(np.float32)
    b = RNG.standard_normal(64).astype(np.float16)
    act = oracle.gemm_swiglu(acc, sx, sw, b)
    hidden = oracle.gemm_dequant(acc, sx, sw, b)
    q1, s1 = oracle.row_quant(act)
    q2, s2 = oracle.swiglu_row_quant(hidden)
    assert np.array_equal(q1, q2) and np.array_equal(s1, s2)
    g = hidden[:, :32].astype(np.float64)
    u = hidden[:, 32:].astype(np.float64)
    ref = g / (1 + np.exp(-g)) * u
    assert np.allclose(act.astype(np.float64), ref, rtol=2e-3, atol=1e-4)


@pytest.mark.parametrize("magnitude", [0.0, 2.0 ** -14, 1.0])
def test_swiglu_zero_input_bias_kat(oracle, magnitude):
    """Reference tests/test_int8_ffn_up_fused_gpu.py:35-46: zero GEMM, bias only."""
    acc = np.zeros((3, 16), np.int32)
    b = np.full(16, magnitude, np.float16)
    act = oracle.gemm_swiglu(acc, np.ones(3, np.float32), np.ones(16, np.float32), b)
    q, s = oracle.row_quant(act)
    m = np.float64(magnitude)
    expect = np.float16(m / (1 + np.exp(-m)) * m)      # 2^-14: ~2^-29 underflows fp16 to zero
    assert np.allclose(act.astype(np.float64), np.float64(expect), rtol=1e-3)
    if expect == 0:
        assert (q == -128).all() and (s == np.float32(1e-30)).all()
    else:
        assert (q == 127).all()


def _conv_ref(qx, qw, kernel, stride):
    """Independent int64 direct convolution via numpy slicing (NDHWC, [O, (kd,kh,kw,c)] weights)."""
    b, d, h, w, c = qx.shape
    o = qw.shape[0]
    kd, kh, kw = kernel
    sd, sh, sw = stride
    wt = qw.reshape(o, kd, kh, kw, c).astype(np.int64)
    do, ho, wo = (d - kd) // sd + 1, (h - kh) // sh + 1, (w - kw) // sw + 1
    out = np.zeros((b, do, ho, wo, o), np.int64)
    x = qx.astype(np.int64)
    for a in range(kd):
        for bb in range(kh):
            for e in range(kw):
                patch = x[:, a:a + sd * (do - 1) + 1:sd, bb:bb + sh * (ho - 1) + 1:sh, e:e + sw * (wo - 1) + 1:sw]
                out += np.einsum("bdhwc,oc->bdhwo", patch, wt[:, a, bb, e])
    return out


@pytest.mark.parametrize("shape,o,kernel,stride", [((1, 5, 9, 11, 7), 19, (3, 3, 3), (1, 2, 2)),
                                                   ((2, 4, 6, 6, 16), 8, (3, 3, 3), (1, 1, 1)),
                                                   ((1, 5, 8, 10, 3), 4, (3, 1, 3), (2, 1, 2))])
def test_conv_acc_matches_independent_reference(oracle, shape, o, kernel, stride):
    qx = RNG.integers(-127, 128, shape, dtype=np.int8)
    qw = RNG.integers(-127, 128, (o, kernel[0] * kernel[1] * kernel[2] * shape[-1]), dtype=np.int8)
    got = oracle.conv3d_acc(qx, qw, kernel, stride)
    assert np.array_equal(got, _conv_ref(qx, qw, kernel, stride))


def test_conv_all_ones_kat_and_output_shape(oracle):
    """Reference KAT: all-ones 128-channel 3x3x3 conv -> 27*128 = 3456; stride-2 shape (1,4,2,8,4)."""
    acc = oracle.conv3d_acc(np.ones((1, 3, 10, 18, 128), np.int8), np.ones((128, 3456), np.int8), (3, 3, 3),
                            (1, 1, 1))
    assert (acc == 3456).all()
    acc = oracle.conv3d_acc(np.zeros((1, 5, 8, 10, 3), np.int8), np.zeros((4, 27), np.int8), (3, 1, 3), (2, 1, 2))
    assert acc.shape[1:4] == (2, 8, 4)


def test_prepare_weight_shape_scale_and_error_bound(oracle):
    """Reference tests/test_encoder_int8.py:20-30: [5,3,3,1,3] packs to (5, 27); scales positive."""
    w = RNG.standard_normal((5, 3, 3, 1, 3)).astype(np.float32)
    w[2] = 0
    q, s = oracle.prepare_conv_weight(w)
    assert q.shape == (5, 27) and (s > 0).all() and s[2] == 1.0 and (q[2] == 0).all()
    assert np.abs(q).max() <= 127
    packed = w.transpose(0, 2, 3, 4, 1).reshape(5, 27)
    err = np.abs(q.astype(np.float64) * s[:, None] - packed)
    assert (err <= 0.5 * s[:, None] * (1 + 1e-6)).all()


# ---------------------------------------------------------------------------
# encoder GroupNorm producer
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("c,d,h,w,pre", [(128, 2, 20, 30, False), (256, 3, 13, 19, True), (128, 1, 2, 3, True)])
def test_gn_stats_against_float64(oracle, c, d, h, w, pre):
    x = (RNG.standard_normal((d, h, w, c)) * 2 + 0.3).astype(np.float16)
    pb = RNG.standard_normal(c).astype(np.float16) if pre else None
    st = oracle.gn_stats(x, 1e-6, pb)
    v = x.astype(np.float32)
    if pre:
        v = (v + pb.astype(np.float32)).astype(np.float16)
    g = v.astype(np.float64).reshape(d, h * w, 32, c // 32)
    mean = g.mean(axis=(1, 3))
    var = g.var(axis=(1, 3))
    assert np.allclose(st[..., 0], mean, rtol=1e-5, atol=1e-6)
    assert np.allclose(st[..., 1], 1 / np.sqrt(var + 1e-6), rtol=1e-5)


@pytest.mark.parametrize("c,d,h,w,pre", [(128, 2, 16, 128, False), (256, 1, 24, 64, True), (128, 1, 8, 192, True)])
def test_gn_tiled_partials_against_float64(oracle, c, d, h, w, pre):
    """Tile statistics of the window conv's 8 x 64 output tiles: per (frame, tile, channel) max / min
    exactly numpy's over that tile's pixels (pins the tile geometry and the chunk numbering
    rb * (W / 64) + cb), per (frame, group, tile) avg and M2 within float32 rounding of float64."""
    x = (RNG.standard_normal((d, h, w, c)) * 2 + 0.3).astype(np.float16)
    pb = RNG.standard_normal(c).astype(np.float16) if pre else None
    avg, m2, ext = oracle.gn_partials_tiled(x, pb)
    v = x.astype(np.float32)
    if pre:
        v = (v + pb.astype(np.float32)).astype(np.float16)
    v = v.astype(np.float64)
    ncb = w // 64
    nchunk = (h // 8) * ncb
    assert avg.shape == m2.shape == (d, 32, nchunk) and ext.shape == (d, nchunk, c)
    # tiles[t, j, pixel, channel] with j = rb * ncb + cb
    tiles = v.reshape(d, h // 8, 8, ncb, 64, c).transpose(0, 1, 3, 2, 4, 5).reshape(d, nchunk, 512, c)
    mx = tiles.max(axis=2).astype(np.float16).view(np.uint16).astype(np.uint32)
    mn = tiles.min(axis=2).astype(np.float16).view(np.uint16).astype(np.uint32)
    assert np.array_equal(ext, mx | (mn << 16))
    g = tiles.reshape(d, nchunk, 512, 32, c // 32)
    mean = g.mean(axis=(2, 4)).transpose(0, 2, 1)                         # [d, 32, nchunk]
    assert np.allclose(avg, mean, rtol=1e-5, atol=2e-6)
    dev = g - avg.transpose(0, 2, 1)[:, :, None, :, None].astype(np.float64)
    ss = (dev ** 2).sum(axis=(2, 4)).transpose(0, 2, 1)
    assert np.allclose(m2, ss, rtol=1e-5)
    st = oracle.gn_stats_tiled(x, 1e-6, pb)
    gf = v.reshape(d, h * w, 32, c // 32)
    assert np.allclose(st[..., 0], gf.mean(axis=(1, 3)), rtol=1e-5, atol=1e-6)
    assert np.allclose(st[..., 1], 1 / np.sqrt(gf.var(axis=(1, 3)) + 1e-6), rtol=1e-5)
    # the 256-pixel row chunks of the producer's own pass sum the same values in another order
    assert np.allclose(st, oracle.gn_stats(x, 1e-6, pb), rtol=2e-6, atol=1e-7)


def test_gn_tiled_lane_order(oracle):
    """The documented order inside a tile, on values where the fp32 addition order shows.  One 8 x 64
    tile, group 0 (channels 0-3): tile pixel 0 sums to B = 4 x 2048 = 2^13 (ulp 2^-10), tile pixels 16
    and 17 hold d = 2^-11 in channel 0, half an ulp of B.  Documented: lanes pl = pixel % 32, so the
    two d sit in lanes 16 and 17, whose adjacent-tree sum 2^-10 reaches lane 0 at the last level:
    S = B + 2^-10 exactly, avg = S / 2048 = 4 + 2^-21.  Adding the pixels in raster order, a halving
    tree (lane 0 + lane 16 first) or 16 pixel lanes (pixel 16 in lane 0 after B) each meets B + d
    alone, a tie that rounds to B: avg = 4."""
    x = np.zeros((1, 8, 64, 128), np.float16)
    x[0, 0, 0, 0:4] = np.float16(2048.0)
    x[0, 0, 16, 0] = x[0, 0, 17, 0] = np.float16(2.0 ** -11)
    avg, m2, _ = oracle.gn_partials_tiled(x)
    assert avg[0, 0, 0] == np.float32(4.0 + 2.0 ** -21)
    assert (avg[0, 1:, 0] == 0).all() and (m2[0, 1:, 0] == 0).all()


def test_norm_pack_structure_and_float64(oracle):
    d, h, w, c = 3, 6, 7, 128
    x = RNG.standard_normal((d, h, w, c)).astype(np.float16)
    gamma = (1 + 0.2 * RNG.standard_normal(c)).astype(np.float16)
    beta = (0.2 * RNG.standard_normal(c)).astype(np.float16)
    st = oracle.gn_stats(x, 1e-6)
    y, _, amax = oracle.norm_pack(x, gamma, beta, st)
    assert y.shape == (d + 2, h + 2, w + 2, c)
    assert (y[:2] == 0).all()                                    # causal zero planes
    assert np.array_equal(y[2:, 0], y[2:, 2]) and np.array_equal(y[2:, -1], y[2:, -3])   # reflect rows
    assert np.array_equal(y[2:, :, 0], y[2:, :, 2]) and np.array_equal(y[2:, :, -1], y[2:, :, -3])
    assert amax == np.abs(y.astype(np.float32)).max()
    mean = np.repeat(st[..., 0], c // 32, axis=1)[:, None, None, :].astype(np.float64)
    rstd = np.repeat(st[..., 1], c // 32, axis=1)[:, None, None, :].astype(np.float64)
    z = (x.astype(np.float64) - mean) * rstd * gamma.astype(np.float64) + beta.astype(np.float64)
    z = z.astype(np.float16).astype(np.float64)
    ref = z / (1 + np.exp(-z))
    inner = y[2:, 1:-1, 1:-1].astype(np.float64)
    assert np.allclose(inner, ref, rtol=2e-3, atol=2e-4)
    s = oracle.scale_from_amax(amax)
    _, q, _ = oracle.norm_pack(x, gamma, beta, st, scale=s, want_fp16=False)
    assert np.array_equal(q, oracle.tensor_quant(y, s))         # pass 2 == E3 quant of pass-1 values


# ---------------------------------------------------------------------------
# decoder producers
# ---------------------------------------------------------------------------

def test_w16_tree_order_closed_form(oracle):
    """The published W16 tree: lanes combine inside 32-lane groups first, then across groups.

    Partials 2^24 (lane 0) and 1, 1 at lanes 1 and 17: the in-group level 16 adds
    lanes 1 and 17 exactly (2) before lane 0 absorbs it -> 2^24 + 2.  Ones at lanes
    1 and 33 (different groups) are each absorbed into 2^24 separately (ties to
    even) -> 2^24.  A sequential sum gives 2^24 for the first case and a single
    halving tree over all 512 partials gives 2^24 + 2 for the second.
    """
    x = np.zeros(2048, np.float32)
    x[0], x[4], x[68] = 2.0 ** 12, 1.0, 1.0
    assert oracle.tree_sumsq_w16(x) == np.float32(2.0 ** 24 + 2)
    x = np.zeros(2048, np.float32)
    x[0], x[4], x[132] = 2.0 ** 12, 1.0, 1.0
    assert oracle.tree_sumsq_w16(x) == np.float32(2.0 ** 24)
    # the per-lane fma chain: x0^2 + x1^2 with x1^2 absorbed by the fma
    x = np.zeros(2048, np.float32)
    x[0], x[1] = 2.0 ** 12, 1.0
    assert oracle.tree_sumsq_w16(x) == np.float32(2.0 ** 24)    # fma(2^12,2^12,1) ties to even
    v = RNG.standard_normal(2048).astype(np.float32)
    assert np.isclose(oracle.tree_sumsq_w16(v), np.sum(v.astype(np.float64) ** 2), rtol=1e-6)
    assert np.isclose(oracle.tree_sum_plain(v), np.sum(v.astype(np.float64)), rtol=1e-5, atol=1e-4)


@pytest.mark.parametrize("recipe", [0, 1])
def test_residual_rms_quant_against_float64(oracle, recipe):
    m, k = 33, 2048
    h = RNG.standard_normal((m, k)).astype(np.float16)
    o = RNG.standard_normal((m, k)).astype(np.float16)
    g = (0.1 * RNG.standard_normal(k)).astype(np.float16)
    w = (1 + 0.1 * RNG.standard_normal(k)).astype(np.float16)
    h_out, q, s = oracle.residual_rms_quant(h, o, g, w, 1e-5, recipe)
    raw = o.astype(np.float64) * g.astype(np.float64) + h.astype(np.float64)      # exact for fp16 inputs
    assert np.array_equal(h_out.view(np.uint16), raw.astype(np.float32).astype(np.float16).view(np.uint16))
    inv = 1 / np.sqrt((raw ** 2).mean(axis=1, keepdims=True) + 1e-5)
    n = h_out.astype(np.float64) * inv * w.astype(np.float64)
    d = s.astype(np.float16).astype(np.float64)[:, None]
    assert np.allclose(s, np.abs(n).max(axis=1) / 127, rtol=2e-3)
    assert (np.abs(q * d - n) <= 0.5 * d + 2e-3 * np.abs(n) + 1e-6).all()


def test_rms_and_layernorm_against_float64(oracle):
    m, k = 17, 1024
    x = RNG.standard_normal((m, k)).astype(np.float16)
    o = RNG.standard_normal((m, k)).astype(np.float16)
    gate = (0.1 * RNG.standard_normal(k)).astype(np.float16)
    gamma = (1 + 0.1 * RNG.standard_normal(k)).astype(np.float16)
    beta = (0.1 * RNG.standard_normal(k)).astype(np.float16)
    xd = x.astype(np.float64)
    ref = xd / np.sqrt((xd ** 2).mean(1, keepdims=True) + 1e-5) * gamma.astype(np.float64)
    assert np.allclose(oracle.rms_fp16(x, gamma, 1e-5).astype(np.float64), ref, rtol=2e-3, atol=2e-3)
    raw = o.astype(np.float64) * gate.astype(np.float64) + xd
    mu = raw.mean(1, keepdims=True)
    ln = (raw - mu) / np.sqrt(raw.var(1, keepdims=True) + 1e-5) * gamma.astype(np.float64) + beta.astype(np.float64)
    got = oracle.residual_layernorm(x, o, gate, gamma, beta, 1e-5).astype(np.float64)
    assert np.allclose(got, ln, rtol=2e-3, atol=2e-3)


def test_qk_rope_closed_forms(oracle):
    """cos=1, sin=0 returns the normalised rows; cos=0, sin=1 is the exact rotate-half permutation."""
    tokens, heads = 5, 3
    x = RNG.standard_normal((1, tokens, heads * 192)).astype(np.float16)
    ones = np.ones((1, tokens, 1, 48), np.float16)
    zeros = np.zeros((1, tokens, 1, 48), np.float16)
    q_id, k_id = oracle.qk_rope(x, ones, zeros, heads, 1e-6)
    xr = x.reshape(tokens, heads, 3, 64).astype(np.float64)
    for part, got in ((0, q_id), (1, k_id)):
        v = xr[:, :, part]
        ref = v / np.sqrt((v ** 2).mean(-1, keepdims=True) + 1e-6)
        assert np.allclose(got[0].astype(np.float64), ref, rtol=2e-3, atol=2e-3)
    q_rot, _ = oracle.qk_rope(x, zeros, ones, heads, 1e-6)
    q0 = q_id[0].astype(np.float32)
    want = q0.copy()
    want[..., :24] = -q0[..., 24:48]
    want[..., 24:48] = q0[..., :24]
    assert np.array_equal(q_rot[0].astype(np.float32), want)


# ---------------------------------------------------------------------------
# E9 residual + bias downsample pack (opt/encoder_fused_residual_pack.py:12-33)
# ---------------------------------------------------------------------------

def test_residual_pack_layout_and_exact_sums(oracle):
    d, h, w, c = 3, 5, 4, 16
    # small integers: every sum is exact in fp16, so the values pin the index mapping alone
    x = RNG.integers(-8, 8, size=(d, h, w, c)).astype(np.float16)
    r = RNG.integers(-8, 8, size=(d, h, w, c)).astype(np.float16)
    b = RNG.integers(-4, 4, size=(c,)).astype(np.float16)
    y = oracle.residual_downsample_pack(x, r, b)
    assert y.shape == (d + 2, h + 1, w + 1, c)
    assert not y[:2].any()                                        # two causal zero frames
    body = (x.astype(np.float64) + r + b).astype(np.float16)
    assert np.array_equal(y[2:, :h, :w], body)
    assert np.array_equal(y[2:, h, :w], body[:, h - 2])           # bottom row reflects row h-2
    assert np.array_equal(y[2:, :h, w], body[:, :, w - 2])        # right column reflects column w-2
    assert np.array_equal(y[2:, h, w], body[:, h - 2, w - 2])


def test_residual_pack_single_fp16_rounding(oracle):
    # x + b + r = 1 + 2^-11 + 2^-11 = 1 + 2^-10 exactly in fp32.  One rounding at the store keeps it;
    # rounding x + b to fp16 first (a tie, to even = 1.0) would give 1.0.
    x = np.full((1, 2, 2, 8), 1.0, np.float16)
    r = np.full((1, 2, 2, 8), 2.0 ** -11, np.float16)
    b = np.full((8,), 2.0 ** -11, np.float16)
    y = oracle.residual_downsample_pack(x, r, b)
    assert (y[2:] == np.float16(1.0 + 2.0 ** -10)).all()


# ---------------------------------------------------------------------------
# decoder pixel finalisation (opt/fp16_finalize.py)
# ---------------------------------------------------------------------------

def test_finalize_channel_mapping_exact(oracle):
    # small integers x power-of-two scales are exact: the values pin the channel index alone
    b, t, h, w = 2, 3, 2, 5
    x = RNG.integers(0, 4, size=(b, 3, t, h, w)).astype(np.float16)
    std = np.float32([2.0 ** -3, 2.0 ** -4, 2.0 ** -5])
    y = oracle.finalize_pixels(x, std, np.zeros(3, np.float32))
    assert np.array_equal(y, x.astype(np.float32) * std.reshape(1, 3, 1, 1, 1))


def test_finalize_two_roundings_not_fma(oracle):
    # x*s = 1 + 2^-10 + 2^-14 + 2^-23 + 2^-24 + 2^-33 rounds up to 1 + 2^-10 + 2^-14 + 2^-22 in fp32;
    # adding m = -1 then gives 2^-10 + 2^-14 + 2^-22.  A fused multiply-add would keep
    # 2^-10 + 2^-14 + 2^-23 + 2^-24 + 2^-33 (exact in fp32).
    x = np.full((1, 3, 1, 1, 8), 1.0 + 2.0 ** -10, np.float16)
    s = np.float32(1.0 + 2.0 ** -14 + 2.0 ** -23)
    std = np.full(3, s, np.float32)
    mean = np.full(3, -1.0, np.float32)
    y = oracle.finalize_pixels(x, std, mean)
    two = 2.0 ** -10 + 2.0 ** -14 + 2.0 ** -22
    fused = 2.0 ** -10 + 2.0 ** -14 + 2.0 ** -23 + 2.0 ** -24 + 2.0 ** -33
    assert (y == np.float32(two)).all() and np.float32(fused) != np.float32(two)


def test_finalize_clamp_nan_and_signed_zero(oracle):
    vals = np.float32([-5.0, -0.0, 0.0, 0.25, 1.0, 1.5, np.inf, -np.inf, np.nan, 2.0 ** -149])
    x = np.zeros((1, 3, 1, 1, vals.size), np.float32)
    x[0, :, 0, 0, :] = vals
    # mean = -0 keeps every product unchanged (-0 + -0 = -0, x + -0 = x), so the clamp's own
    # treatment of -0 shows; the comparisons must neither flip it nor swallow NaN
    y = oracle.finalize_pixels(x, np.ones(3, np.float32), np.full(3, -0.0, np.float32))[0, 0, 0, 0]
    expect = np.float32([0.0, -0.0, 0.0, 0.25, 1.0, 1.0, 1.0, 0.0, np.nan, 2.0 ** -149])
    assert np.isnan(y[8]) and np.array_equal(np.delete(y, 8).view(np.uint32), np.delete(expect, 8).view(np.uint32))


@pytest.mark.parametrize("dtype", [np.float16, np.float32])
def test_finalize_against_numpy_float32(oracle, dtype):
    x = (RNG.standard_normal((2, 3, 3, 4, 7)) * 2).astype(dtype)
    std = np.float32([0.229, 0.224, 0.225])
    mean = np.float32([0.485, 0.456, 0.406])
    prod = x.astype(np.float32) * std.reshape(1, 3, 1, 1, 1)        # numpy rounds each float32 op once
    v = prod + mean.reshape(1, 3, 1, 1, 1)
    expect = np.where(v < 0, np.float32(0), np.where(v > 1, np.float32(1), v)).astype(np.float32)
    assert np.array_equal(oracle.finalize_pixels(x, std, mean), expect)


# ---------------------------------------------------------------------------
# decoder attention (float64 restatement)
# ---------------------------------------------------------------------------

def test_attention_uniform_weights_closed_form(oracle):
    # q = 0: every key gets weight 1/N, so the output is the mean of the values
    b, n, h, d = 2, 37, 3, 64
    q = np.zeros((b, n, h, d))
    k = RNG.standard_normal((b, n, h, d))
    v = RNG.standard_normal((b, n, h, d))
    o = oracle.attention(q, k, v, 0.125)
    assert np.allclose(o, np.broadcast_to(v.mean(axis=1, keepdims=True), o.shape), rtol=0, atol=1e-12)


def test_attention_one_hot_selects_a_value_row(oracle):
    # orthogonal keys, query = 40 x key j: weight of j is 1 / (1 + 15 e^-40) -> v[j] to 1e-15
    n, d = 16, 64
    k = np.zeros((1, n, 1, d))
    k[0, np.arange(n), 0, np.arange(n)] = 1.0
    v = RNG.standard_normal((1, n, 1, d))
    q = 40.0 * k[:, [5, 11]]
    o = oracle.attention(q, k, v, 1.0)
    assert np.allclose(o[0, :, 0], v[0, [5, 11], 0], rtol=0, atol=1e-12)


def test_attention_against_torch_sdpa_float64(oracle):
    torch = pytest.importorskip("torch")
    b, n, h, d = 2, 29, 4, 64
    q, k, v = (RNG.standard_normal((b, n, h, d)) for _ in range(3))
    ref = torch.nn.functional.scaled_dot_product_attention(
        *(torch.from_numpy(t).permute(0, 2, 1, 3) for t in (q, k, v)), scale=0.125).permute(0, 2, 1, 3).numpy()
    assert np.allclose(oracle.attention(q, k, v, 0.125), ref, rtol=1e-12, atol=1e-12)
    sub = oracle.attention(q, k, v, 0.125, queries=[0, 7, 28])
    assert np.array_equal(sub, oracle.attention(q, k, v, 0.125)[:, [0, 7, 28]])


# ---------------------------------------------------------------------------
# one fused multiply-add in the G1 / F2 epilogue: closed-form cases where it differs from two roundings
# ---------------------------------------------------------------------------

# acc = 3, sx = 1, sw = 5616981 * 2^-24, b = 2^-23: the exact value a*sw + b = 1 + 9*2^-11 + 2^-24 lies
# half an fp32 ulp above an fp16 midpoint.  One rounding (fma) lands on that midpoint, which ties to the
# even fp16 1 + 4*2^-10; rounding the product first (1 + 9*2^-11 - 2^-24 ties up to the midpoint) and
# then adding b lands one fp32 ulp above it, which rounds to 1 + 5*2^-10.  (Found by exact rational
# search over fp16 midpoints near 1; the same values drive the GPU epilogue tests.)
FMA_ACC, FMA_SW, FMA_B = 3, np.float32(5616981 * 2.0 ** -24), np.float16(2.0 ** -23)
FMA_ONE, TWO_ROUNDINGS = np.float16(1 + 4 * 2.0 ** -10), np.float16(1 + 5 * 2.0 ** -10)


def _exact(x):
    from fractions import Fraction
    return Fraction(float(x))


def test_fma_case_is_what_the_comment_says():
    from fractions import Fraction
    exact = _exact(FMA_ACC) * _exact(FMA_SW) + _exact(FMA_B)
    assert exact == 1 + Fraction(9, 2 ** 11) + Fraction(1, 2 ** 24)
    assert FMA_SW == np.float32(5616981 * 2.0 ** -24) and float(FMA_SW) * 2 ** 24 == 5616981
    two = np.float16(np.float32(np.float32(FMA_ACC) * FMA_SW) + np.float32(FMA_B))
    assert two == TWO_ROUNDINGS != FMA_ONE


def test_gemm_dequant_rounds_once(oracle):
    acc = np.full((2, 3), FMA_ACC, np.int32)
    out = oracle.gemm_dequant(acc, np.ones(2, np.float32), np.full(3, FMA_SW, np.float32), np.full(3, FMA_B))
    assert (out == FMA_ONE).all()
    # without a bias the epilogue is (acc * sx) * sw, one rounding per product
    plain = oracle.gemm_dequant(acc, np.ones(2, np.float32), np.full(3, FMA_SW, np.float32), None)
    assert (plain == np.float16(np.float32(FMA_ACC) * FMA_SW)).all()


def _silu64(g):
    g = float(g)
    return g / (1.0 + np.exp(-g))


def test_gemm_swiglu_gate_and_up_round_once(oracle):
    """[gate | up] columns in weight-row order; gate 32 makes SiLU(gate) exactly 32, so act = fp16(32 * up)
    carries the up column's rounding unchanged; up 1.0 leaves act = fp16(SiLU(gate))."""
    nh = 2
    acc = np.zeros((1, 2 * nh), np.int32)
    sw = np.ones(2 * nh, np.float32)
    b = np.zeros(2 * nh, np.float16)
    # pair 0: gate = 32 (bias only), up = the fma case
    b[0], acc[0, nh], sw[nh], b[nh] = 32.0, FMA_ACC, FMA_SW, FMA_B
    # pair 1: gate = the fma case, up = 1 (bias only)
    acc[0, 1], sw[1], b[1], b[nh + 1] = FMA_ACC, FMA_SW, FMA_B, 1.0
    act = oracle.gemm_swiglu(acc, np.ones(1, np.float32), sw, b)[0]
    assert act[0] == np.float16(32 * float(FMA_ONE)) != np.float16(32 * float(TWO_ROUNDINGS))
    # SiLU(1 + 4*2^-10) = 0.73468... lies over a thousand fp32 ulps from an fp16 rounding boundary, so any
    # SiLU within a few fp32 ulps rounds to the same fp16 value; the two-rounding gate gives another one
    want, wrong = np.float16(_silu64(FMA_ONE)), np.float16(_silu64(TWO_ROUNDINGS))
    ulps = _silu64(FMA_ONE) / 2.0 ** -11
    assert abs(ulps - np.floor(ulps) - 0.5) * 2.0 ** -11 > 64 * 2.0 ** -24
    assert want != wrong and act[1] == want
