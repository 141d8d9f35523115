"""CPU oracle for the H3 VAE INT8 hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker (or the timed
CPU baseline).  The product package never imports it.

The arithmetic lives in ``h3v_oracle.c`` (plain scalar binary32 C, FMA
contraction off, explicit ``fmaf`` only where the reference contract names a
fused multiply-add).  This module loads the compiled library with ctypes and
exposes numpy-facing wrappers.  FP16 arrays are passed as ``np.float16`` and
reinterpreted as raw ``uint16`` bit patterns.

Every function here is pinned by ``tests/test_oracle_pins.py``: the
reference's own known-answer vectors, closed forms, invariants or an
independent float64 / integer computation, chosen so that a dropped term, a
wrong sign or index, or a transposed operand fails one of them.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "_build" / "libh3v_oracle.so"
_lib = None

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
_F = ctypes.c_float

_SIGNATURES = {
    "ora_h2f": (_F, [ctypes.c_uint16]),
    "ora_f2h": (ctypes.c_uint16, [_F]),
    "ora_expf": (_F, [_F]),
    "ora_row_quant": (None, [_P, _I64, _I64, _P, _P]),
    "ora_swiglu_row_quant": (None, [_P, _I64, _I64, _P, _P]),
    "ora_gemm_i8_acc": (None, [_P, _P, _P, _I64, _I64, _I64]),
    "ora_gemm_dequant": (None, [_P, _P, _I64, _P, _P, _P, _I64, _I64]),
    "ora_gemm_swiglu": (None, [_P, _P, _P, _P, _P, _I64, _I64]),
    "ora_prepare_conv_weight": (None, [_P, _I, _I, _I, _I, _I, _P, _P]),
    "ora_tensor_scale_from_amax": (_F, [_F]),
    "ora_tensor_amax": (_F, [_P, _I64]),
    "ora_tensor_quant": (None, [_P, _I64, _F, _P]),
    "ora_conv3d_acc": (None, [_P, _P, _P] + [_I] * 12),
    "ora_gn_stats": (None, [_P, _P, _I, _I, _I, _I, _F, _P]),
    "ora_gn_partials_tiled": (None, [_P, _P, _I, _I, _I, _I, _P, _P, _P]),
    "ora_gn_merge_equal": (None, [_P, _P, _I, _I, _I, _I, _F, _P]),
    "ora_norm_pack": (_F, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _P, _P, _F]),
    "ora_residual_rms_quant": (None, [_P, _P, _P, _P, _F, _I64, _I, _I, _P, _P, _P]),
    "ora_rms_fp16": (None, [_P, _P, _F, _I64, _I, _P]),
    "ora_residual_layernorm": (None, [_P, _P, _P, _P, _P, _F, _I64, _I, _P]),
    "ora_qk_rope": (None, [_P, _P, _P, _I64, _I, _I, _I, _F, _P, _P]),
    "ora_residual_downsample_pack": (None, [_P, _P, _P, _P, _I, _I, _I, _I]),
    "ora_finalize_pixels": (None, [_P, _I, _I64, _I64, _P, _P, _P]),
    "ora_tree_sumsq_w16": (_F, [_P, _I]),
    "ora_tree_sum_plain": (_F, [_P, _I]),
    "ora_num_threads": (_I, []),
    "ora_set_num_threads": (None, [_I]),
}


def build() -> Path:
    """Compile the oracle with its Makefile (gcc, no GPU needed)."""
    subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            build()
        handle = ctypes.CDLL(str(_LIB_PATH))
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def _ptr(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data


def _f16(a) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float16)
    return a


def _opt16(a):
    return None if a is None else _f16(a)


def set_threads(n: int) -> None:
    lib().ora_set_num_threads(int(n))


def num_threads() -> int:
    return int(lib().ora_num_threads())


# -- scalar helpers ---------------------------------------------------------

def f2h_bits(x: float) -> int:
    return int(lib().ora_f2h(float(x)))


def h2f(bits: int) -> float:
    return float(lib().ora_h2f(int(bits)))


def expf(x: float) -> float:
    return float(lib().ora_expf(float(x)))


def tree_sumsq_w16(x) -> np.float32:
    """Published norm1 W16 sum of squares of one fp32 row (test pin)."""
    x = np.ascontiguousarray(x, np.float32)
    return np.float32(lib().ora_tree_sumsq_w16(_ptr(x), x.size))


def tree_sum_plain(terms) -> np.float32:
    """Plain fixed-tree sum of one fp32 row of terms (test pin)."""
    t = np.ascontiguousarray(terms, np.float32)
    return np.float32(lib().ora_tree_sum_plain(_ptr(t), t.size))


# -- Q1 / F6 ------------------------------------------------------------------

def row_quant(x):
    """Q1 row quantization of fp16 rows [M, K] -> (int8 [M, K], fp32 [M])."""
    x = _f16(x)
    m, k = x.reshape(-1, x.shape[-1]).shape
    q = np.empty((m, k), np.int8)
    s = np.empty((m,), np.float32)
    lib().ora_row_quant(_ptr(x), m, k, _ptr(q), _ptr(s))
    return q, s


def swiglu_row_quant(x):
    """F6: SiLU(gate)*up over fp16 [M, 2K] rows then Q1 -> (int8 [M, K], fp32 [M])."""
    x = _f16(x)
    m = x.size // x.shape[-1]
    k = x.shape[-1] // 2
    q = np.empty((m, k), np.int8)
    s = np.empty((m,), np.float32)
    lib().ora_swiglu_row_quant(_ptr(x), m, k, _ptr(q), _ptr(s))
    return q, s


# -- GEMM -----------------------------------------------------------------------

def gemm_acc(a, w):
    """int32 accumulators of int8 A[M,K] . W[N,K]^T."""
    a = np.ascontiguousarray(a, np.int8)
    w = np.ascontiguousarray(w, np.int8)
    m, k = a.shape
    n = w.shape[0]
    acc = np.empty((m, n), np.int32)
    lib().ora_gemm_i8_acc(_ptr(a), _ptr(w), _ptr(acc), m, n, k)
    return acc


def gemm_dequant(acc, sx, sw, bias=None):
    """G1 epilogue: fp16(fma(fp32(acc)*sx[m], sw[n], b[n])) (or without bias)."""
    acc = np.ascontiguousarray(acc, np.int32)
    m, n = acc.shape
    sx = np.ascontiguousarray(np.asarray(sx, np.float32).reshape(-1))
    stride = 0 if sx.size == 1 else 1
    sw = np.ascontiguousarray(sw, np.float32)
    b = _opt16(bias)
    out = np.empty((m, n), np.float16)
    lib().ora_gemm_dequant(_ptr(acc), _ptr(sx), stride, _ptr(sw), _ptr(b), _ptr(out), m, n)
    return out


def gemm_swiglu(acc, sx, sw, bias=None):
    """F2 epilogue over [M, 2*Nh] accumulators in weight-row order -> fp16 [M, Nh]."""
    acc = np.ascontiguousarray(acc, np.int32)
    m, n2 = acc.shape
    sx = np.ascontiguousarray(np.asarray(sx, np.float32).reshape(-1))
    sw = np.ascontiguousarray(sw, np.float32)
    b = _opt16(bias)
    out = np.empty((m, n2 // 2), np.float16)
    lib().ora_gemm_swiglu(_ptr(acc), _ptr(sx), _ptr(sw), _ptr(b), _ptr(out), m, n2 // 2)
    return out


def int8_linear(x, qw, ws, bias=None):
    """Q2 + G1: dynamic row quant of fp16 x then the dequant GEMM."""
    q, s = row_quant(x)
    return gemm_dequant(gemm_acc(q, qw), s, ws, bias)


# -- encoder ---------------------------------------------------------------------

def prepare_conv_weight(w):
    """E1: fp32 [O,C,kd,kh,kw] -> (int8 [O, kd*kh*kw*C], fp32 [O])."""
    w = np.ascontiguousarray(w, np.float32)
    o, c, kd, kh, kw = w.shape
    q = np.empty((o, kd * kh * kw * c), np.int8)
    s = np.empty((o,), np.float32)
    lib().ora_prepare_conv_weight(_ptr(w), o, c, kd, kh, kw, _ptr(q), _ptr(s))
    return q, s


def tensor_scale(x) -> np.float32:
    x = _f16(x)
    amax = lib().ora_tensor_amax(_ptr(x), x.size)
    return np.float32(lib().ora_tensor_scale_from_amax(amax))


def scale_from_amax(amax: float) -> np.float32:
    return np.float32(lib().ora_tensor_scale_from_amax(float(amax)))


def tensor_quant(x, s):
    x = _f16(x)
    q = np.empty(x.shape, np.int8)
    lib().ora_tensor_quant(_ptr(x), x.size, float(s), _ptr(q))
    return q


def conv3d_acc(qx, qw, kernel, stride):
    """int32 accumulators of a valid conv over int8 NDHWC [B,Dp,Hp,Wp,C] -> [B,Do,Ho,Wo,O]."""
    qx = np.ascontiguousarray(qx, np.int8)
    qw = np.ascontiguousarray(qw, np.int8)
    b, dp, hp, wp, c = qx.shape
    o = qw.shape[0]
    kd, kh, kw = kernel
    sd, sh, sw = stride
    do, ho, wo = (dp - kd) // sd + 1, (hp - kh) // sh + 1, (wp - kw) // sw + 1
    acc = np.empty((b, do, ho, wo, o), np.int32)
    lib().ora_conv3d_acc(_ptr(qx), _ptr(qw), _ptr(acc), b, c, dp, hp, wp, o, kd, kh, kw, sd, sh, sw)
    return acc


def gn_stats(x_ndhwc, eps, pre_bias=None):
    """Per-frame GroupNorm(32) (mean, rstd) of fp16 NDHWC [D,H,W,C] -> fp32 [D,32,2]."""
    x = _f16(x_ndhwc)
    d, h, w, c = x.shape
    pb = _opt16(pre_bias)
    stats = np.empty((d, 32, 2), np.float32)
    lib().ora_gn_stats(_ptr(x), _ptr(pb), d, h, w, c, float(eps), _ptr(stats))
    return stats


GN_TILE = (8, 64)   # rows x columns of the window conv's output tiles (512 pixels)


def gn_partials_tiled(x_ndhwc, pre_bias=None):
    """GroupNorm(32) partial statistics of fp16 NDHWC [D,H,W,C] over the window conv's 8 x 64 output
    tiles -> (avg [D,32,nchunk] fp32, m2 [D,32,nchunk] fp32, ext [D,nchunk,C] uint32 = fp16 max | min << 16),
    the producer workspace layout of h3v_conv3d_i8_gn.  H % 8 == 0, W % 64 == 0."""
    x = _f16(x_ndhwc)
    d, h, w, c = x.shape
    if h % GN_TILE[0] or w % GN_TILE[1]:
        raise ValueError("tiled statistics need H % 8 == 0 and W % 64 == 0")
    nchunk = (h // GN_TILE[0]) * (w // GN_TILE[1])
    avg = np.empty((d, 32, nchunk), np.float32)
    m2 = np.empty((d, 32, nchunk), np.float32)
    ext = np.empty((d, nchunk, c), np.uint32)
    lib().ora_gn_partials_tiled(_ptr(x), _ptr(_opt16(pre_bias)), d, h, w, c, _ptr(avg), _ptr(m2), _ptr(ext))
    return avg, m2, ext


def gn_merge_equal(avg, m2, chunk_pixels, c, eps):
    """Sequential Chan merge of equal chunks (ora_gn_stats' merge) -> fp32 [D,32,2] (mean, rstd)."""
    avg = np.ascontiguousarray(avg, np.float32)
    m2 = np.ascontiguousarray(m2, np.float32)
    d, _, nchunk = avg.shape
    stats = np.empty((d, 32, 2), np.float32)
    lib().ora_gn_merge_equal(_ptr(avg), _ptr(m2), d, nchunk, int(chunk_pixels), int(c), float(eps), _ptr(stats))
    return stats


def gn_stats_tiled(x_ndhwc, eps, pre_bias=None):
    """Per-frame GroupNorm(32) (mean, rstd) summed over the window conv's 512-pixel tiles."""
    avg, m2, _ = gn_partials_tiled(x_ndhwc, pre_bias)
    return gn_merge_equal(avg, m2, GN_TILE[0] * GN_TILE[1], np.asarray(x_ndhwc).shape[-1], eps)


def norm_pack(x_ndhwc, gamma, beta, stats, pre_bias=None, scale=None, want_fp16=True):
    """GroupNorm/SiLU/causal+reflect pack -> (fp16 y or None, int8 q or None, amax)."""
    x = _f16(x_ndhwc)
    d, h, w, c = x.shape
    shape = (d + 2, h + 2, w + 2, c)
    y = np.empty(shape, np.float16) if want_fp16 else None
    q = np.empty(shape, np.int8) if scale is not None else None
    amax = lib().ora_norm_pack(
        _ptr(x), _ptr(_opt16(pre_bias)), _ptr(_f16(gamma)), _ptr(_f16(beta)),
        _ptr(np.ascontiguousarray(stats, np.float32)), d, h, w, c,
        _ptr(y), _ptr(q), float(scale if scale is not None else 1.0))
    return y, q, np.float32(amax)


def norm_conv3d(x_ndhwc, gamma, beta, eps, qw, ws, bias=None, pre_bias=None, tiled=False):
    """E7: GN stats -> pack (absmax) -> scale -> INT8 pack -> conv -> fp16 NDHWC.  ``tiled``: the
    statistics summed over the window conv's 8 x 64 output tiles (an input written by h3v_conv3d_i8_gn)."""
    stats = gn_stats_tiled(x_ndhwc, eps, pre_bias) if tiled else gn_stats(x_ndhwc, eps, pre_bias)
    _, _, amax = norm_pack(x_ndhwc, gamma, beta, stats, pre_bias, want_fp16=False)
    s = scale_from_amax(amax)
    _, q, _ = norm_pack(x_ndhwc, gamma, beta, stats, pre_bias, scale=s, want_fp16=False)
    acc = conv3d_acc(q[None], qw, (3, 3, 3), (1, 1, 1))[0]
    d, h, w, o = acc.shape
    out = gemm_dequant(acc.reshape(-1, o), np.array([s], np.float32), ws, bias)
    return out.reshape(d, h, w, o), q, s


# -- decoder producers -----------------------------------------------------------

def residual_rms_quant(h, o, g, w, eps, recipe):
    """N1 (recipe 0, W16 tree) / F1 (recipe 1) -> (h_out fp16, q int8, s fp32)."""
    h = _f16(h)
    k = h.shape[-1]
    m = h.size // k
    h_out = np.empty(h.shape, np.float16)
    q = np.empty((m, k), np.int8)
    s = np.empty((m,), np.float32)
    lib().ora_residual_rms_quant(_ptr(h), _ptr(_f16(o)), _ptr(_f16(g)), _ptr(_f16(w)), float(eps),
                                 m, k, int(recipe), _ptr(h_out), _ptr(q), _ptr(s))
    return h_out, q, s


def rms_fp16(x, gamma, eps):
    x = _f16(x)
    k = x.shape[-1]
    out = np.empty(x.shape, np.float16)
    lib().ora_rms_fp16(_ptr(x), _ptr(_f16(gamma)), float(eps), x.size // k, k, _ptr(out))
    return out


def residual_layernorm(h, o, gate, gamma, beta, eps):
    h = _f16(h)
    k = h.shape[-1]
    out = np.empty(h.shape, np.float16)
    lib().ora_residual_layernorm(_ptr(h), _ptr(_f16(o)), _ptr(_f16(gate)), _ptr(_f16(gamma)),
                                 _ptr(_f16(beta)), float(eps), h.size // k, k, _ptr(out))
    return out


def qk_rope(x, cos, sin, heads, eps):
    """x fp16 [..., N, heads*3*dh]; cos/sin fp16 [..., N, 1, rot] -> q, k fp16 [..., N, heads, dh]."""
    x = _f16(x)
    dh = x.shape[-1] // (3 * heads)
    tokens = x.size // x.shape[-1]
    rot = cos.shape[-1]
    q = np.empty((*x.shape[:-1], heads, dh), np.float16)
    k = np.empty_like(q)
    lib().ora_qk_rope(_ptr(x), _ptr(_f16(cos)), _ptr(_f16(sin)), tokens, heads, dh, rot,
                      float(eps), _ptr(q), _ptr(k))
    return q, k


def residual_downsample_pack(x_ndhwc, residual_ndhwc, bias):
    """E9 pack: fp16 NDHWC [D,H,W,C] x2 + bias [C] -> fp16 [D+2, H+1, W+1, C]."""
    x = _f16(x_ndhwc)
    d, h, w, c = x.shape
    out = np.empty((d + 2, h + 1, w + 1, c), np.float16)
    lib().ora_residual_downsample_pack(_ptr(x), _ptr(_f16(residual_ndhwc)), _ptr(_f16(bias)), _ptr(out), c, d, h, w)
    return out


def finalize_pixels(x, std, mean):
    """Decoder pixel finalisation: [B,3,T,H,W] fp16/fp32 -> fp32 clamp(x*std[c] + mean[c], 0, 1), NaN kept."""
    x = np.ascontiguousarray(x)
    if x.dtype not in (np.float16, np.float32) or x.ndim != 5 or x.shape[1] != 3:
        raise ValueError("fp16/fp32 [B,3,T,H,W] pixels required")
    b, _, t, h, w = x.shape
    out = np.empty(x.shape, np.float32)
    lib().ora_finalize_pixels(_ptr(x), int(x.dtype == np.float16), b, t * h * w,
                              _ptr(np.ascontiguousarray(std, np.float32)), _ptr(np.ascontiguousarray(mean, np.float32)),
                              _ptr(out))
    return out


def attention(q, k, v, scale, queries=None):
    """Decoder attention in float64: softmax(scale * q k^T) v per (batch, head).

    q, k, v: [B, N, H, D] (any float dtype, converted exactly to float64).  `queries` optionally
    selects query token indices (all keys are always used).  Returns float64 [B, len(queries), H, D].
    The kernels' fp16 softmax weights and fp32 accumulation are compared against it with a tolerance.
    """
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    if queries is not None:
        q = q[:, np.asarray(queries)]
    s = np.einsum("bqhd,bkhd->bhqk", q, k) * float(scale)
    s -= s.max(axis=-1, keepdims=True)
    w = np.exp(s)
    w /= w.sum(axis=-1, keepdims=True)
    return np.einsum("bhqk,bkhd->bqhd", w, v)


__all__ = [name for name in dir() if not name.startswith("_")]
