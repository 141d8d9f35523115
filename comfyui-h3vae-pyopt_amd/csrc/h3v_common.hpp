// Shared device helpers for the H3 VAE INT8 hot-path kernels (gfx950 / CDNA4).
//
// Numerics contract: every kernel is compiled with -ffp-contract=off, so a*b+c
// is two roundings unless written as __builtin_fmaf.  Division and sqrtf are
// IEEE correctly rounded (hipcc default -fhip-fp32-correctly-rounded-divide-sqrt).
// FP16 conversion is round-to-nearest-even with subnormals kept.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace h3v {

typedef _Float16 f16;
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));
typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float h2f(uint16_t b) { return (float)__builtin_bit_cast(f16, b); }
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (f16)f); }
__device__ __forceinline__ float rt16(float f) { return (float)(f16)f; }
// Four fp32 values to fp16 (round to nearest even, as f2h) with two v_cvt_pk_f16_f32; element-wise f2h
// into a u16x4 compiles to single conversions plus packing instructions.
__device__ __forceinline__ u16x4 f2h4(float a, float b, float c, float d) {
    const f16x2 lo = __builtin_convertvector((f32x2){a, b}, f16x2);
    const f16x2 hi = __builtin_convertvector((f32x2){c, d}, f16x2);
    const uint2 w = {__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi)};
    return __builtin_bit_cast(u16x4, w);
}

// A 16-byte load marked non-temporal (global_load ... nt): for streams read once whose lines need
// not stay in the caches.  A large activation read this way (the GroupNorm producers' input, 285 MB
// at stage 0) streams at about 7 TB/s instead of 6.3.
__device__ __forceinline__ u16x8 load_nt(const uint16_t* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u16x8*>(p));
}

// Eight IEEE fp16 sums a + b (four v_pk_add_f16).  For fp16 operands this is bit for bit
// fp16(float(a) + float(b)), the fp32 sum rounded to fp16: the fp32 sum of two fp16 values
// rounds once and fp32's 24-bit significand is at least 2 * 11 + 2 bits, so rounding it again
// to fp16 gives the correctly rounded sum (the double rounding is innocuous; checked over all
// 2^32 pairs of finite fp16 values, overflow to infinity included).  A NaN stays a NaN.
__device__ __forceinline__ u16x8 add_f16x8(u16x8 a, u16x8 b) {
    return __builtin_bit_cast(u16x8, __builtin_bit_cast(f16x8, a) + __builtin_bit_cast(f16x8, b));
}

// exp(x) by Cody-Waite reduction and a degree-7 Taylor polynomial in Horner
// form with fused multiply-adds:  n = rint(x*log2 e),
// r = fma(-n, LN2_LO, fma(-n, LN2_HI, x)),  exp(x) = 2^n * P(r).
// LN2_HI has 15 significant bits so n*LN2_HI is exact; |r| <= 0.35 keeps the
// truncation error below 6e-9 relative; error <= 2 ulp against float64.
// The same operation sequence is the CPU oracle's ora_expf.
__device__ __forceinline__ float exp_f32_core(float x) {   // finite x in [-103.97, 88.72]
    const float LOG2E = 0x1.715476p+0f;
    const float LN2_HI = 0x1.62e4p-1f;
    const float LN2_LO = 0x1.7f7d1cp-20f;
    float n = __builtin_rintf(x * LOG2E);
    float r = __builtin_fmaf(-n, LN2_HI, x);
    r = __builtin_fmaf(-n, LN2_LO, r);
    float p = 0x1.a01a02p-13f;
    p = __builtin_fmaf(p, r, 0x1.6c16c2p-10f);
    p = __builtin_fmaf(p, r, 0x1.111112p-7f);
    p = __builtin_fmaf(p, r, 0x1.555556p-5f);
    p = __builtin_fmaf(p, r, 0x1.555556p-3f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    return __builtin_amdgcn_ldexpf(p, (int)n);
}
__device__ __forceinline__ float exp_f32(float x) {
    if (x != x) return x;
    if (x > 88.72283935546875f) return __builtin_inff();
    if (x < -103.972084045410156f) return 0.0f;
    return exp_f32_core(x);
}

// SiLU written as the reference writes it: z / (1 + exp(-z)).
__device__ __forceinline__ float silu(float z) { return z / (1.0f + exp_f32(-z)); }

// Quotient a / b (b > 0) through the hardware reciprocal and one fused Newton
// correction of the quotient: q0 = a * r, e = a - q0 * b (exact), q = q0 + e * r,
// with the sign of q0 (which is the quotient's sign; it keeps -0 / b = -0).  The
// error is within a tiny fraction of an ulp beyond 1/2, so q is the IEEE quotient
// unless a / b lies almost exactly on a rounding boundary.  Used only where that
// never happens for the operands that occur; h3v_selftest_fast_div checks every
// case on the device (all fp16 numerators against all finite positive fp16
// divisors, and every fp16 SiLU argument).
__device__ __forceinline__ float div_newton(float a, float b, float r) {
    const float q0 = a * r;
    const float e = __builtin_fmaf(-q0, b, a);
    return __builtin_copysignf(__builtin_fmaf(e, r, q0), q0);
}

// SiLU of an fp16-valued z with the fast quotient where the denominator is a
// finite normal number; the IEEE path keeps the special cases (|z| large, inf, NaN).
__device__ __forceinline__ float silu_fast(float z) {
    if (__builtin_fabsf(z) <= 80.0f) {
        const float den = 1.0f + exp_f32_core(-z);
        return div_newton(z, den, __builtin_amdgcn_rcpf(den));
    }
    return silu(z);
}

// 1/sqrt as two correctly rounded operations.
__device__ __forceinline__ float rsqrt_rn(float x) { return 1.0f / __builtin_sqrtf(x); }

// Row scale of the comfy-kitchen row quantizer: max(amax * fp32(1/127), 1e-30).
__device__ __forceinline__ float q1_scale(float amax) {
    float s = amax * (1.0f / 127.0f);
    return s >= 1.0e-30f ? s : 1.0e-30f;
}

// One element of the row quantizer, d = fp32(fp16(scale)):
// v = fp16(a / d); v = rint(v); NaN -> -128; clamp [-128, 127].
__device__ __forceinline__ int q1_quant(float a, float d) {
    float v = rt16(a / d);
    v = __builtin_rintf(v);
    if (v != v) return -128;
    v = __builtin_fminf(127.0f, __builtin_fmaxf(-128.0f, v));
    return (int)v;
}

// The row quantizer's divisor d = fp32(fp16(scale)) with its reciprocal.  When d is
// finite and positive, every finite fp16 numerator goes through the fast quotient
// (both operands have 11-bit significands, so their quotient never sits near an
// fp32 rounding boundary without being on it); otherwise the IEEE division runs.
struct Q1Div {
    float d, r, rr;   // divisor, hardware reciprocal, correctly rounded reciprocal
    bool fast;
};
__device__ __forceinline__ Q1Div q1_div(float d) {
    Q1Div q;
    q.d = d;
    q.r = __builtin_amdgcn_rcpf(d);
    q.rr = 1.0f / d;
    q.fast = d > 0.0f && d <= 65504.0f;
    return q;
}
// q1_quant with the divisor prepared once per row; identical results.  A row whose
// divisor is finite and positive holds no infinite value (its amax would be infinite).
__device__ __forceinline__ int q1_quant(float a, const Q1Div& q) {
    float v = rt16(q.fast ? div_newton(a, q.d, q.r) : a / q.d);
    v = __builtin_rintf(v);
    if (v != v) return -128;
    v = __builtin_fminf(127.0f, __builtin_fmaxf(-128.0f, v));
    return (int)v;
}

// A stand-in for q1_quant's quotient a / d that gives the same int8 code through q1_codes4 (not
// always the same fp32 value), the divisor's path chosen by the caller: FAST must equal q.fast.
// FAST: a * fl(1 / d), the correctly rounded reciprocal.  For an fp16 value a and a finite positive
// fp16 divisor d the product differs from fl(a / d) by at most 2^-23 relative; rounded to fp16 it
// differs in 2990 of the 2.0e9 (finite a, d) pairs, never across a rounding boundary of the code
// (checked exhaustively on the CPU, and on the device by h3v_selftest_fast_div).
template <bool FAST>
__device__ __forceinline__ float q1_quot(float a, const Q1Div& q) {
    return FAST ? a * q.rr : a / q.d;
}

// q1_quant's code chain for four quotients x, packed as four int8 codes (x0 in the low byte):
// fp16(x) rounded to nearest even, that fp16 value rounded to the nearest integer (ties to even),
// NaN -> -128, clamp [-128, 127].  Done in packed fp16: max(h, -128) sends a quotient's (quiet) NaN
// to -128 (IEEE maxNum) and min(., 127) clamps; clamping before the integer rounding gives the same
// codes at +-127.5 and -128.5.  Adding 1536 then moves [-128, 127] into [1408, 1663], where fp16
// values are one apart, so the add itself rounds to the nearest integer, ties to even, and the low
// byte of the sum's bit pattern is the code in two's complement.  Equal to q1_quant's chain for
// every fp16 value h (all 65536 checked, NaN and infinities included).
__device__ __forceinline__ uint32_t q1_codes4(float x0, float x1, float x2, float x3) {
    const f16x2 lo = __builtin_convertvector((f32x2){x0, x1}, f16x2);
    const f16x2 hi = __builtin_convertvector((f32x2){x2, x3}, f16x2);
    const f16x2 vmin = {(f16)-128.0f, (f16)-128.0f}, vmax = {(f16)127.0f, (f16)127.0f};
    const f16x2 mag = {(f16)1536.0f, (f16)1536.0f};
    const f16x2 a = __builtin_elementwise_min(__builtin_elementwise_max(lo, vmin), vmax) + mag;
    const f16x2 b = __builtin_elementwise_min(__builtin_elementwise_max(hi, vmin), vmax) + mag;
    // bytes 0 and 2 of a (codes 0, 1), then bytes 0 and 2 of b (codes 2, 3)
    return __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, b), __builtin_bit_cast(uint32_t, a), 0x06040200u);
}

// Per-tensor scale of the encoder activation quantizer: amax * fp32(1/127), 0 -> 1.
__device__ __forceinline__ float e3_scale(float amax) {
    float s = amax * (1.0f / 127.0f);
    return s > 0.0f ? s : 1.0f;
}

// Encoder activation rounding: half away from zero as floor(t + 0.5), clamp +-127.
__device__ __forceinline__ int e3_quant(float v, float s) {
    float t = v / s;
    float r = t >= 0.0f ? __builtin_floorf(t + 0.5f) : -__builtin_floorf(-t + 0.5f);
    r = __builtin_fminf(127.0f, __builtin_fmaxf(-127.0f, r));
    return (int)r;
}

// Pack four int8 values (low byte first) into one 32-bit word.
__device__ __forceinline__ uint32_t pack4(int a, int b, int c, int d) {
    return (uint32_t)(a & 0xff) | ((uint32_t)(b & 0xff) << 8) |
           ((uint32_t)(c & 0xff) << 16) | ((uint32_t)(d & 0xff) << 24);
}

// Wave-wide (64 lanes) max of a non-negative float.
__device__ __forceinline__ float wave_max(float v) {
    for (int off = 32; off >= 1; off >>= 1) v = __builtin_fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

// Workspace of the INT8 encoder producer (h3v_gn_norm_pack_i8) for an fp16 [D, H, W, C] input whose
// GroupNorm(32) statistics are summed over chunks of `chunk` pixels of a frame: the average and M2 of
// every (frame, group, chunk) ([D][32][nchunk] each), the packed fp16 (max, min) of every (frame, chunk,
// channel) ([D][nchunk][C], with room for C = 256), the int8 quantize table (64 KB), 64 words whose first
// two are absmax_lut's counters, and the absmax candidate of every (frame, group).  The producer's own
// statistics pass uses 256-pixel chunks, which sizes the workspace (h3v_gn_norm_pack_workspace_floats);
// the window conv's statistics epilogue uses its 512-pixel tiles, whose layout fits inside.
constexpr int kGnGroups = 32;
constexpr int kGnMaxC = 256;
constexpr int kGnSizingChunk = 256;
constexpr int kGnTileChunk = 512;   // pixels of a window-conv output tile (8 rows of a 64-pixel column block)
constexpr int kGnLutFloats = 65536 / 4;

struct GnWorkspace {
    float* avg;
    float* m2;
    uint32_t* ext;
    int8_t* lut;
    uint32_t* done;
    uint32_t* cands;
    int nchunk;
};

__host__ __device__ inline GnWorkspace gn_workspace(float* ws, int d, int hw, int chunk) {
    GnWorkspace g;
    g.nchunk = (hw + chunk - 1) / chunk;
    const int64_t stat = (int64_t)d * g.nchunk * kGnGroups;
    g.avg = ws;
    g.m2 = ws + stat;
    g.ext = reinterpret_cast<uint32_t*>(ws + 2 * stat);
    float* const tail = ws + 2 * stat + (int64_t)d * g.nchunk * kGnMaxC;
    g.lut = reinterpret_cast<int8_t*>(tail);
    g.done = reinterpret_cast<uint32_t*>(tail + kGnLutFloats);
    g.cands = g.done + 64;
    return g;
}

// floats of the producer workspace for [D, H, W] (the 256-pixel layout, the larger one)
inline int64_t gn_workspace_floats(int d, int h, int w) {
    const int64_t nchunk = ((int64_t)h * w + kGnSizingChunk - 1) / kGnSizingChunk;
    return 2 * (int64_t)d * nchunk * kGnGroups + (int64_t)d * nchunk * kGnMaxC + kGnLutFloats + 64 +
           (int64_t)d * kGnGroups;
}

}  // namespace h3v
