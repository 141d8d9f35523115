"""GPU parity: row quantizers and INT8 GEMMs (through the C ABI) vs the CPU oracle.

Integer outputs (int8 codes, int32 accumulators) and the fp16 epilogues must
match bit for bit: the kernels and the oracle implement the same IEEE
operation sequence.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from _util import assert_bitwise, bits16, np_

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _gen(seed=20261002):
    return torch.Generator().manual_seed(seed)


def _row_quant_gpu(ops, x):
    q = torch.empty(x.shape, dtype=torch.int8, device=DEV)
    s = torch.empty(x.shape[0], dtype=torch.float32, device=DEV)
    xd = x.to(DEV)
    ops.hip.call("h3v_row_quant", ops.hip.ptr(xd), x.shape[0], x.shape[1], ops.hip.ptr(q), ops.hip.ptr(s),
                 ops.hip.stream(DEV))
    torch.cuda.synchronize()
    return np_(q), np_(s)


@pytest.mark.parametrize("m,k", [(1, 2048), (17, 2048), (129, 1024), (7188, 2048), (33, 8192), (5, 5), (3, 40),
                                 (2, 16384), (6, 4096), (9, 512)])
def test_row_quant_matches_oracle(ops, oracle, m, k):
    gen = _gen(m * 31 + k)
    x = torch.randn(m, k, generator=gen).half()
    if m > 2:
        x[1] = 0                                    # zero row: q=-128, s=1e-30
        x[2] = x[2] * 2.0 ** -20                    # rows whose fp16 scale is subnormal / zero
    if m > 4:
        x[3, 0] = 65504.0
        x[4] = torch.tensor(2.0 ** -24).half()
    q, s = _row_quant_gpu(ops, x)
    rq, rs = oracle.row_quant(x.numpy())
    assert_bitwise(q, rq, "q")
    assert_bitwise(s.view(np.uint32), rs.view(np.uint32), "scale")
    if m > 2:
        assert (q[1] == -128).all() and s[1] == np.float32(1e-30)


@pytest.mark.parametrize("m,k,scale", [(1, 8192, 3.0), (17, 4096, 3.0), (129, 8192, 3.0), (4, 5, 3.0), (6, 1024, 3.0),
                                       (7, 2048, 400.0)])
def test_swiglu_row_quant_matches_oracle(ops, oracle, m, k, scale):
    # scale 400: |gate| > 80 takes the IEEE SiLU path and products overflow to inf (amax inf rows)
    gen = _gen(k + m)
    x = (torch.randn(m, 2 * k, generator=gen) * scale).half()
    q = torch.empty((m, k), dtype=torch.int8, device=DEV)
    s = torch.empty(m, dtype=torch.float32, device=DEV)
    xd = x.to(DEV)
    ops.hip.call("h3v_swiglu_row_quant", ops.hip.ptr(xd), m, k, ops.hip.ptr(q), ops.hip.ptr(s), ops.hip.stream(DEV))
    torch.cuda.synchronize()
    rq, rs = oracle.swiglu_row_quant(x.numpy())
    assert_bitwise(np_(q), rq, "q")
    assert_bitwise(np_(s).view(np.uint32), rs.view(np.uint32), "scale")


def _swiglu_gpu(ops, x):
    m, k = x.shape[0], x.shape[1] // 2
    q = torch.empty((m, k), dtype=torch.int8, device=DEV)
    s = torch.empty(m, dtype=torch.float32, device=DEV)
    xd = x.to(DEV)
    ops.hip.call("h3v_swiglu_row_quant", ops.hip.ptr(xd), m, k, ops.hip.ptr(q), ops.hip.ptr(s), ops.hip.stream(DEV))
    torch.cuda.synchronize()
    return np_(q), np_(s)


def test_swiglu_row_quant_every_gate_code(ops, oracle):
    """Every fp16 gate code through the SwiGLU quantizer: every finite code (both zeros, subnormals,
    +-65504; |gate| > 80 takes the IEEE SiLU path) appears as a gate in eight shuffled rows, the infinities
    and NaNs in a ninth; up ~ N(0, 1)."""
    codes = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    special = (codes & 0x7C00) == 0x7C00
    rng = np.random.default_rng(8192)
    finite = rng.permutation(codes[~special])
    k = 8192
    gate = np.zeros((9, k), np.uint16)
    pad = rng.standard_normal(9 * k).astype(np.float16).view(np.uint16)
    gate.reshape(-1)[:] = pad
    per = (finite.size + 7) // 8
    for r in range(8):
        part = finite[r * per:(r + 1) * per]
        gate[r, :part.size] = part
    gate[8, :special.sum()] = codes[special]
    up = rng.standard_normal((9, k)).astype(np.float16)
    x = torch.from_numpy(np.concatenate([gate.view(np.float16), up], axis=1).copy())
    q, s = _swiglu_gpu(ops, x)
    rq, rs = oracle.swiglu_row_quant(x.numpy())
    assert_bitwise(q, rq, "q")
    assert_bitwise(s.view(np.uint32), rs.view(np.uint32), "scale")


@pytest.mark.parametrize("m,k", [(257, 4096), (1031, 4096), (333, 1024), (70, 2048), (515, 8192)])
def test_swiglu_row_quant_odd_rows_large_gates(ops, oracle, m, k):
    """Odd row counts at every vector width (1024-8192) with large gates ~ N(0, 6)."""
    x = (torch.randn(m, 2 * k, generator=_gen(m + k)) * 6.0).half()
    q, s = _swiglu_gpu(ops, x)
    rq, rs = oracle.swiglu_row_quant(x.numpy())
    assert_bitwise(q, rq, "q")
    assert_bitwise(s.view(np.uint32), rs.view(np.uint32), "scale")


def test_swiglu_row_quant_h3_shape_bitwise(ops, oracle):
    """The decoder FFN's SwiGLU quantizer at the H3 shape (7188 rows of [gate | up] 2 x 8192), every row
    against the oracle; gates ~ N(0, 4)."""
    print("swiglu row quant [7188, 2 x 8192]", flush=True)
    x = (torch.randn(7188, 2 * 8192, generator=_gen(7188)) * 4.0).half()
    q, s = _swiglu_gpu(ops, x)
    rq, rs = oracle.swiglu_row_quant(x.numpy())
    assert_bitwise(q, rq, "q")
    assert_bitwise(s.view(np.uint32), rs.view(np.uint32), "scale")


def _i32_gpu(ops, a, w):
    m, k = a.shape
    n = w.shape[0]
    acc = torch.empty((m, n), dtype=torch.int32, device=DEV)
    ad, wd = a.to(DEV), w.to(DEV)
    ops.hip.call("h3v_gemm_i8_i32", ops.hip.ptr(ad), ops.hip.ptr(wd), ops.hip.ptr(acc), m, n, k, ops.hip.stream(DEV))
    torch.cuda.synchronize()
    return np_(acc)


@pytest.mark.parametrize("m,n,k", [(1, 256, 2048), (17, 6144, 2048), (129, 512, 1024), (300, 200, 192),
                                   (256, 256, 64), (5, 7, 33), (2, 3, 5),
                                   # one, two, three and many K steps of 128, ragged M and N (13: scalar stores)
                                   (257, 300, 128), (70, 13, 256), (300, 520, 384), (515, 264, 8192)])
def test_gemm_int32_accumulators_exact(ops, oracle, m, n, k):
    gen = _gen(m + n + k)
    a = torch.randint(-128, 128, (m, k), generator=gen, dtype=torch.int8)
    w = torch.randint(-128, 128, (n, k), generator=gen, dtype=torch.int8)
    got = _i32_gpu(ops, a, w)
    want = a.numpy().astype(np.int64) @ w.numpy().astype(np.int64).T
    assert np.array_equal(got, want)


def test_gemm_int32_full_size_sampled_rows(ops):
    """H3 QKV shape M=7188, N=6144, K=2048: every tile position, rows sampled across all M tiles."""
    gen = _gen(7)
    m, n, k = 7188, 6144, 2048
    a = torch.randint(-128, 128, (m, k), generator=gen, dtype=torch.int8)
    w = torch.randint(-128, 128, (n, k), generator=gen, dtype=torch.int8)
    got = _i32_gpu(ops, a, w)
    rows = np.unique(np.concatenate([np.arange(0, m, 97), np.arange(m - 20, m), np.arange(0, 256, 7)]))
    want = a.numpy()[rows].astype(np.int64) @ w.numpy().astype(np.int64).T
    assert np.array_equal(got[rows], want)
    # and a column checksum over all rows (checksum of checksums)
    col = w.numpy().astype(np.int64)[:: 61]
    assert np.array_equal(got[:, ::61].astype(np.int64).sum(0), (a.numpy().astype(np.int64).sum(0) @ col.T))


@pytest.mark.parametrize("m,n,k,with_bias", [(1, 6144, 2048, True), (17, 2048, 2048, False), (129, 1024, 4096, True),
                                             (300, 200, 192, True), (5, 7, 33, False), (257, 300, 128, True),
                                             (70, 13, 256, True), (300, 520, 384, False), (515, 264, 8192, True)])
def test_gemm_dequant_matches_oracle(ops, oracle, m, n, k, with_bias):
    gen = _gen(m * 3 + n)
    a = torch.randint(-128, 128, (m, k), generator=gen, dtype=torch.int8)
    w = torch.randint(-31, 32, (n, k), generator=gen, dtype=torch.int8)
    sx = (torch.rand(m, generator=gen) * 0.02 + 0.001).float()
    sw = (torch.rand(n, generator=gen) * 0.02 + 0.001).float()
    bias = torch.randn(n, generator=gen).half() if with_bias else None
    out = torch.empty((m, n), dtype=torch.float16, device=DEV)
    dev = [t.to(DEV) if t is not None else None for t in (a, sx, w, sw, bias)]
    ops.hip.call("h3v_gemm_i8_dequant", *[ops.hip.ptr(t) for t in dev], ops.hip.ptr(out), m, n, k, ops.hip.stream(DEV))
    torch.cuda.synchronize()
    want = oracle.gemm_dequant(oracle.gemm_acc(a.numpy(), w.numpy()), sx.numpy(), sw.numpy(),
                               None if bias is None else bias.numpy())
    assert_bitwise(np_(out), want, "out")


@pytest.mark.parametrize("rows,bias", [(1, None), (17, True), (129, True)])
def test_swiglu_gemm_matches_oracle(ops, oracle, rows, bias):
    """Reference fixture tests/test_int8_ffn_up_fused_gpu.py:21-33 (K2048, 16384 weight rows)."""
    gen = _gen(rows)
    w = torch.randint(-31, 32, (16384, 2048), generator=gen, dtype=torch.int8)
    ws = (torch.rand(16384, generator=gen) * 0.02 + 0.001).float()
    q = torch.randint(-31, 32, (rows, 2048), generator=gen, dtype=torch.int8)
    scale = (torch.rand(rows, 1, generator=gen) * 0.02 + 0.001).float()
    b = torch.randn(16384, generator=gen).half() if bias else None
    act = torch.empty((rows, 8192), dtype=torch.float16, device=DEV)
    dev = [t.to(DEV) if t is not None else None for t in (q, scale, w, ws, b)]
    ops.hip.call("h3v_gemm_i8_swiglu", *[ops.hip.ptr(t) for t in dev], ops.hip.ptr(act), rows, 8192, 2048,
                 ops.hip.stream(DEV))
    torch.cuda.synchronize()
    want = oracle.gemm_swiglu(oracle.gemm_acc(q.numpy(), w.numpy()), scale.numpy(), ws.numpy(),
                              None if b is None else b.numpy())
    assert_bitwise(np_(act), want, "act")
    # fused (GEMM+SwiGLU then row quant) == unfused (dequant GEMM then SwiGLU+quant)
    hidden = oracle.gemm_dequant(oracle.gemm_acc(q.numpy(), w.numpy()), scale.numpy(), ws.numpy(),
                                 None if b is None else b.numpy())
    rq, rs = oracle.swiglu_row_quant(hidden)
    gq, gs = _row_quant_gpu(ops, act.cpu())
    assert_bitwise(gq, rq, "requant q")
    assert_bitwise(gs.view(np.uint32), rs.view(np.uint32), "requant scale")


@pytest.mark.parametrize("magnitude", [0.0, 2.0 ** -14, 1.0])
def test_swiglu_gemm_zero_input_bias_contract(ops, oracle, magnitude):
    """Reference fixture tests/test_int8_ffn_up_fused_gpu.py:35-46."""
    q = torch.zeros((3, 2048), dtype=torch.int8)
    s = torch.ones((3, 1), dtype=torch.float32)
    w = torch.zeros((16384, 2048), dtype=torch.int8)
    ws = torch.ones(16384, dtype=torch.float32)
    b = torch.full((16384,), magnitude, dtype=torch.float16)
    act = torch.empty((3, 8192), dtype=torch.float16, device=DEV)
    dev = [t.to(DEV) for t in (q, s, w, ws, b)]
    ops.hip.call("h3v_gemm_i8_swiglu", *[ops.hip.ptr(t) for t in dev], ops.hip.ptr(act), 3, 8192, 2048,
                 ops.hip.stream(DEV))
    torch.cuda.synchronize()
    gq, gs = _row_quant_gpu(ops, act.cpu())
    rq, rs = oracle.swiglu_row_quant(np.full((3, 16384), magnitude, np.float16))
    assert_bitwise(gq, rq, "q")
    assert_bitwise(gs.view(np.uint32), rs.view(np.uint32), "s")
    if magnitude == 0.0:
        assert (gq == -128).all() and (gs == np.float32(1e-30)).all()


# one fused multiply-add in the G1 / F2 epilogues: acc = 3, sx = 1, sw = 5616981 * 2^-24, b = 2^-23 gives
# fp16 1 + 4*2^-10 with one rounding and 1 + 5*2^-10 with the product rounded first (closed form in
# tests/test_oracle_pins.py, test_fma_case_is_what_the_comment_says)
FMA_SW, FMA_B = 5616981 * 2.0 ** -24, 2.0 ** -23
FMA_ONE, TWO_ROUNDINGS = 1 + 4 * 2.0 ** -10, 1 + 5 * 2.0 ** -10


def _ones_prefix(rows, k, width=3):
    t = torch.zeros((rows, k), dtype=torch.int8)
    t[:, :width] = 1
    return t


@pytest.mark.parametrize("m,n,k", [(300, 256, 1024), (7188, 2048, 2048), (64, 6144, 2048)])
def test_gemm_dequant_epilogue_is_one_fma(ops, m, n, k):
    print(f"dequant epilogue fma m={m} n={n} k={k}", flush=True)
    a, w = _ones_prefix(m, k), _ones_prefix(n, k)
    sx = torch.ones(m, dtype=torch.float32)
    sw = torch.full((n,), FMA_SW, dtype=torch.float32)
    b = torch.full((n,), FMA_B, dtype=torch.float16)
    out = torch.empty((m, n), dtype=torch.float16, device=DEV)
    dev = [t.to(DEV) for t in (a, sx, w, sw, b)]
    ops.hip.call("h3v_gemm_i8_dequant", *[ops.hip.ptr(t) for t in dev], ops.hip.ptr(out), m, n, k, ops.hip.stream(DEV))
    torch.cuda.synchronize()
    got = np_(out)
    assert (got == np.float16(FMA_ONE)).all(), np.unique(got)[:5]


def test_swiglu_gemm_epilogue_is_one_fma_per_column(ops):
    """Gate / up weight rows in reference order: pairs c < 128 have gate = 32 (bias only, SiLU(32) = 32
    exactly) and up = the fma case, so act = 32 * (1 + 4*2^-10); pairs c >= 128 have gate = the fma case and
    up = 1, so act = fp16(SiLU(1 + 4*2^-10)) = 0.735 (over a thousand fp32 ulps from an fp16 boundary)."""
    m, nh, k = 129, 256, 2048
    q = _ones_prefix(m, k)
    w = torch.zeros((2 * nh, k), dtype=torch.int8)
    w[nh:nh + 128, :3] = 1            # up rows of pairs 0..127
    w[128:nh, :3] = 1                 # gate rows of pairs 128..255
    sw = torch.ones(2 * nh, dtype=torch.float32)
    sw[nh:nh + 128] = FMA_SW
    sw[128:nh] = FMA_SW
    b = torch.zeros(2 * nh, dtype=torch.float16)
    b[:128], b[nh:nh + 128] = 32.0, FMA_B
    b[128:nh], b[nh + 128:] = FMA_B, 1.0
    scale = torch.ones((m, 1), dtype=torch.float32)
    act = torch.empty((m, nh), dtype=torch.float16, device=DEV)
    dev = [t.to(DEV) for t in (q, scale, w, sw, b)]
    ops.hip.call("h3v_gemm_i8_swiglu", *[ops.hip.ptr(t) for t in dev], ops.hip.ptr(act), m, nh, k, ops.hip.stream(DEV))
    torch.cuda.synchronize()
    got = np_(act)
    assert (got[:, :128] == np.float16(32 * FMA_ONE)).all(), np.unique(got[:, :128])[:5]
    silu_one = np.float16(FMA_ONE / (1 + np.exp(-FMA_ONE)))
    assert silu_one != np.float16(TWO_ROUNDINGS / (1 + np.exp(-TWO_ROUNDINGS)))
    assert (got[:, 128:] == silu_one).all(), np.unique(got[:, 128:])[:5]


@pytest.mark.parametrize("name,m,n,k", [("cfg2 qkv", 16384, 3072, 1024), ("cfg3 up", 16384, 8192, 1024),
                                        ("cfg3 down", 16384, 1024, 4096), ("cfg4 out", 16384, 1024, 1024),
                                        ("H3 ffn-up", 7188, 16384, 2048)])
def test_gemm_dequant_full_size_sampled_rows(ops, oracle, name, m, n, k):
    """BASELINE.json configs 2-4 (and the H3 FFN-up) at full M: the fp16 epilogue of sampled rows (every M tile,
    the first and last rows) bit for bit against the oracle."""
    print(f"dequant full size {name}: {m} x {n} x {k}", flush=True)
    gen = _gen(m + n + k)
    a = torch.randint(-127, 128, (m, k), generator=gen, dtype=torch.int8)
    w = torch.randint(-31, 32, (n, k), generator=gen, dtype=torch.int8)
    sx = (torch.rand(m, generator=gen) * 0.02 + 0.001).float()
    sw = (torch.rand(n, generator=gen) * 0.002 + 0.0001).float()
    bias = (0.02 * torch.randn(n, generator=gen)).half()
    out = torch.empty((m, n), dtype=torch.float16, device=DEV)
    dev = [t.to(DEV) for t in (a, sx, w, sw, bias)]
    ops.hip.call("h3v_gemm_i8_dequant", *[ops.hip.ptr(t) for t in dev], ops.hip.ptr(out), m, n, k, ops.hip.stream(DEV))
    torch.cuda.synchronize()
    rows = np.unique(np.concatenate([np.arange(0, m, 257), np.arange(m - 8, m), np.arange(0, 8)]))
    got = np_(out)[rows]
    want = oracle.gemm_dequant(oracle.gemm_acc(a.numpy()[rows], w.numpy()), sx.numpy()[rows], sw.numpy(),
                               bias.numpy())
    assert_bitwise(got, want, name)


def _tensor_quant_gpu(ops, x):
    xd = x.to(DEV).contiguous()
    q = torch.empty(x.shape, dtype=torch.int8, device=DEV)
    s = torch.empty((), dtype=torch.float32, device=DEV)
    words = int(ops.hip.lib().h3v_tensor_quant_scratch_words())
    scratch = torch.full((words,), -1, dtype=torch.int32, device=DEV)
    ops.hip.call("h3v_tensor_quant_i8", ops.hip.ptr(xd), x.numel(), ops.hip.ptr(q), ops.hip.ptr(s),
                 ops.hip.ptr(scratch), words, ops.hip.stream(DEV))
    torch.cuda.synchronize()
    return np_(q), np.float32(s.item())


@pytest.mark.parametrize("shape", [(2, 3, 5, 7, 11), (1, 128, 11, 66, 66), (1, 256, 19, 130, 130), (7,)])
def test_tensor_quant_matches_oracle(ops, oracle, shape):
    gen = _gen(sum(shape))
    x = torch.randn(*shape, generator=gen).half()
    q, s = _tensor_quant_gpu(ops, x)
    rs = oracle.tensor_scale(x.numpy())
    assert np.float32(s).view(np.uint32) == rs.view(np.uint32)
    assert_bitwise(q, oracle.tensor_quant(x.numpy(), rs), "q")


def test_tensor_quant_reference_kats(ops):
    """Reference tests/test_encoder_int8_gpu.py:57-72: extremes and half-away rounding."""
    for maximum in [0.0, 2 ** -24, 2 ** -14, 0.5, 127.0, 65504.0]:
        x = torch.full((9,), maximum, dtype=torch.float16)
        x[0] = -maximum
        q, s = _tensor_quant_gpu(ops, x)
        expect_s = np.float32(maximum) * np.float32(1.0 / 127.0) if maximum else np.float32(1.0)
        assert s == expect_s
        if maximum:
            assert q[0] == -127 and (q[1:] == 127).all()
        else:
            assert (q == 0).all()
    x = torch.tensor([-127.0, -0.5, -1.5, 0.0, 0.5, 1.5, 127.0], dtype=torch.float16)
    q, s = _tensor_quant_gpu(ops, x)
    assert s == 1.0
    assert q.tolist() == [-127, -1, -2, 0, 1, 2, 127]


def test_fast_quotients_match_ieee_division_exhaustively(ops):
    """The quantizers' reciprocal + Newton quotient equals IEEE division on every operand they see."""
    counts = torch.full((3,), 7, dtype=torch.int32, device=DEV)
    ops.hip.call("h3v_selftest_fast_div", ops.hip.ptr(counts), ops.hip.stream(DEV))
    torch.cuda.synchronize()
    assert counts.tolist() == [0, 0, 0], f"fast quotient mismatches (div, q, silu): {counts.tolist()}"


def test_mfma_ceiling_probe_counts_and_clock(ops):
    """The MFMA ceiling probe multiplies what it is given: all-ones operands give 32 per MFMA
    output, so after `iters` iterations of 4 operand sets every lane's sum of its 8 blocks x 16
    accumulators is iters * 4 * 32 * 128; the clock it reports is a plausible shader clock."""
    blocks, iters = 4, 3
    a = torch.ones(4096, dtype=torch.int8, device=DEV)
    b = torch.ones(2048, dtype=torch.int8, device=DEV)
    sink = torch.zeros(blocks * 512, dtype=torch.int32, device=DEV)
    clocks = torch.zeros(2 * blocks, dtype=torch.int64, device=DEV)
    ops.hip.call("h3v_probe_mfma_rate", ops.hip.ptr(a), a.numel(), ops.hip.ptr(b), b.numel(), blocks, iters,
                 ops.hip.ptr(sink), ops.hip.ptr(clocks), ops.hip.stream(DEV))
    torch.cuda.synchronize()
    assert (sink == iters * 4 * 32 * 128).all()
    ticks = clocks.view(blocks, 2).double()
    assert (ticks > 0).all()
    mhz = ticks[:, 0].sum().item() / ticks[:, 1].sum().item() * 100.0
    assert 300.0 < mhz < 3500.0, mhz
