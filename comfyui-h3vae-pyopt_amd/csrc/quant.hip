// Quantizers of the H3 VAE INT8 hot path.
//
//  * row quantizer (comfy-kitchen 0.2.34 contract as restated in
//    opt/int8_swiglu_fused.py:29-37 and opt/int8_ffn_up_fused.py:91-104):
//    one wave per row for widths 512 * {1, 2, 4, 8, 16} (one workgroup per
//    row otherwise and for SwiGLU), the row stays in registers between the
//    amax and the quantize step, 16-byte loads and 8-byte stores, the division
//    by the row divisor through the verified fast quotient (h3v_common.hpp);
//  * SwiGLU + row quantizer (opt/int8_swiglu_fused.py:22-38);
//  * per-tensor encoder activation quantizer (opt/encoder_int8.py:343-378):
//    an absmax pass writing one partial per workgroup (no atomics, nothing to
//    clear), then a quantize pass whose workgroups each fold the partials and
//    derive the scale on the fly: two launches.
#include "h3v_common.hpp"
#include "h3v_abi.hpp"

namespace h3v {
namespace {

constexpr int kRowThreads = 256;

__device__ __forceinline__ float block_max(float v, float* red) {
    v = wave_max(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float m = red[0];
    for (int i = 1; i < (int)(blockDim.x >> 6); ++i) m = __builtin_fmaxf(m, red[i]);
    return m;
}

// Quantize 8 values against the row divisor and store them as two 32-bit words.  The divisor is the
// same in every lane of the row: one uniform branch picks the quotient path.
__device__ __forceinline__ void store_q8(int8_t* dst, const float* v, const Q1Div& d) {
    uint32_t lo, hi;
    if (__builtin_amdgcn_readfirstlane((int)d.fast)) {
        lo = q1_codes4(q1_quot<true>(v[0], d), q1_quot<true>(v[1], d), q1_quot<true>(v[2], d), q1_quot<true>(v[3], d));
        hi = q1_codes4(q1_quot<true>(v[4], d), q1_quot<true>(v[5], d), q1_quot<true>(v[6], d), q1_quot<true>(v[7], d));
    } else {
        lo = q1_codes4(q1_quot<false>(v[0], d), q1_quot<false>(v[1], d), q1_quot<false>(v[2], d),
                       q1_quot<false>(v[3], d));
        hi = q1_codes4(q1_quot<false>(v[4], d), q1_quot<false>(v[5], d), q1_quot<false>(v[6], d),
                       q1_quot<false>(v[7], d));
    }
    *reinterpret_cast<uint2*>(dst) = make_uint2(lo, hi);
}

__device__ __forceinline__ float swiglu_value(uint16_t g, uint16_t u) { return rt16(silu_fast(h2f(g)) * h2f(u)); }

// One wave per row of K = NCH * 512 values, blockDim/64 rows per workgroup, no
// LDS: lane L holds the eight values [c*512 + 8L, c*512 + 8L + 8) of chunk c.
// SWIGLU: the row of K outputs comes from a [gate | up] input row of 2K; the
// fp16-rounded products are kept as fp16 pairs until the scale is known.
template <int NCH, bool SWIGLU>
__global__ __launch_bounds__(kRowThreads) void row_quant_wave(const uint16_t* __restrict__ x, int64_t rows,
                                                              int8_t* __restrict__ q, float* __restrict__ s) {
    constexpr int K = NCH * 512;
    constexpr int64_t LDX = SWIGLU ? 2 * K : K;
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (row >= rows) return;
    const uint16_t* xr = x + row * LDX;
    u16x8 v[NCH];
    float amax = 0.0f;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const int col = c * 512 + lane * 8;
        v[c] = load_nt(xr + col);
        if constexpr (SWIGLU) {
            const u16x8 u = load_nt(xr + K + col);
#pragma unroll
            for (int e = 0; e < 8; ++e) v[c][e] = f2h(swiglu_value(v[c][e], u[e]));
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) amax = __builtin_fmaxf(amax, __builtin_fabsf(h2f(v[c][e])));
    }
    amax = wave_max(amax);
    const float sc = q1_scale(amax);
    const Q1Div d = q1_div(rt16(sc));
    int8_t* qr = q + row * (int64_t)K;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        float f[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) f[e] = h2f(v[c][e]);
        store_q8(qr + c * 512 + lane * 8, f, d);
    }
    if (lane == 0) s[row] = sc;
}

// SWIGLU=false: values are the fp16 row.  SWIGLU=true: values are
// fp16(silu(gate) * up) of a [gate | up] row of width 2K.
template <int CH, bool SWIGLU>
__global__ __launch_bounds__(kRowThreads) void row_quant_vec(const uint16_t* __restrict__ x, int64_t ldx, int K,
                                                             int8_t* __restrict__ q, float* __restrict__ s) {
    __shared__ float red[kRowThreads / 64];
    const int64_t row = blockIdx.x;
    const uint16_t* xr = x + row * ldx;
    float v[CH][8];
    float amax = 0.0f;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        int idx = (c * kRowThreads + (int)threadIdx.x) * 8;
        if (idx < K) {
            u16x8 a = load_nt(xr + idx);
            if constexpr (SWIGLU) {
                u16x8 b = load_nt(xr + K + idx);
#pragma unroll
                for (int e = 0; e < 8; ++e) v[c][e] = swiglu_value(a[e], b[e]);
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) v[c][e] = h2f(a[e]);
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) amax = __builtin_fmaxf(amax, __builtin_fabsf(v[c][e]));
        }
    }
    amax = block_max(amax, red);
    const float sc = q1_scale(amax);
    const Q1Div d = q1_div(rt16(sc));
    int8_t* qr = q + row * (int64_t)K;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        int idx = (c * kRowThreads + (int)threadIdx.x) * 8;
        if (idx < K) store_q8(qr + idx, v[c], d);
    }
    if (threadIdx.x == 0) s[row] = sc;
}

// Any width / alignment: two passes over global memory, scalar accesses.
template <bool SWIGLU>
__global__ __launch_bounds__(kRowThreads) void row_quant_scalar(const uint16_t* __restrict__ x, int64_t ldx, int K,
                                                                int8_t* __restrict__ q, float* __restrict__ s) {
    __shared__ float red[kRowThreads / 64];
    const int64_t row = blockIdx.x;
    const uint16_t* xr = x + row * ldx;
    auto value = [&](int i) {
        if constexpr (SWIGLU) return swiglu_value(xr[i], xr[K + i]);
        else return h2f(xr[i]);
    };
    float amax = 0.0f;
    for (int i = threadIdx.x; i < K; i += kRowThreads) amax = __builtin_fmaxf(amax, __builtin_fabsf(value(i)));
    amax = block_max(amax, red);
    const float sc = q1_scale(amax);
    const Q1Div d = q1_div(rt16(sc));
    for (int i = threadIdx.x; i < K; i += kRowThreads) q[row * (int64_t)K + i] = (int8_t)q1_quant(value(i), d);
    if (threadIdx.x == 0) s[row] = sc;
}

template <bool SWIGLU>
int launch_row_quant(const uint16_t* x, int64_t rows, int64_t k, int8_t* q, float* s, hipStream_t stream,
                     const char* what) {
    H3V_REQUIRE(x && q && s, "%s: null pointer argument", what);
    H3V_REQUIRE(rows > 0 && k > 0, "%s: rows and columns must be positive", what);
    H3V_REQUIRE(rows <= 0x7fffffff && k <= (1 << 20), "%s: shape out of range", what);
    const int64_t ldx = SWIGLU ? 2 * k : k;
    const bool vec = k % 8 == 0 && aligned(x, 16) && aligned(q, 8) && k <= 8 * 8 * kRowThreads;
    dim3 grid((unsigned)rows), block(kRowThreads);
    int K = (int)k;
    // One wave per row pays off for the plain quantizer; the SwiGLU rows carry
    // about 40 VALU operations per output and run better one workgroup per row,
    // where more waves per SIMD hide the loads (measured at 7188 x 8192: 65 us
    // against 114 us with one wave per row).
    if (!SWIGLU && k % 512 == 0 && k <= 8192 && aligned(x, 16) && aligned(q, 8)) {
        dim3 wgrid((unsigned)((rows + kRowThreads / 64 - 1) / (kRowThreads / 64)));
        bool launched = true;
        switch (k / 512) {
            case 1: hipLaunchKernelGGL((row_quant_wave<1, SWIGLU>), wgrid, block, 0, stream, x, rows, q, s); break;
            case 2: hipLaunchKernelGGL((row_quant_wave<2, SWIGLU>), wgrid, block, 0, stream, x, rows, q, s); break;
            case 4: hipLaunchKernelGGL((row_quant_wave<4, SWIGLU>), wgrid, block, 0, stream, x, rows, q, s); break;
            case 8: hipLaunchKernelGGL((row_quant_wave<8, SWIGLU>), wgrid, block, 0, stream, x, rows, q, s); break;
            case 16: hipLaunchKernelGGL((row_quant_wave<16, SWIGLU>), wgrid, block, 0, stream, x, rows, q, s); break;
            default: launched = false; break;
        }
        if (launched) return launch_status(what);
    }
    if (!vec) {
        hipLaunchKernelGGL((row_quant_scalar<SWIGLU>), grid, block, 0, stream, x, ldx, K, q, s);
    } else if (k <= 8 * kRowThreads) {
        hipLaunchKernelGGL((row_quant_vec<1, SWIGLU>), grid, block, 0, stream, x, ldx, K, q, s);
    } else if (k <= 2 * 8 * kRowThreads) {
        hipLaunchKernelGGL((row_quant_vec<2, SWIGLU>), grid, block, 0, stream, x, ldx, K, q, s);
    } else if (k <= 4 * 8 * kRowThreads) {
        hipLaunchKernelGGL((row_quant_vec<4, SWIGLU>), grid, block, 0, stream, x, ldx, K, q, s);
    } else {
        hipLaunchKernelGGL((row_quant_vec<8, SWIGLU>), grid, block, 0, stream, x, ldx, K, q, s);
    }
    return launch_status(what);
}

// ---------------------------------------------------------------------------
// Per-tensor encoder activation quantization.
// ---------------------------------------------------------------------------
constexpr int kTensorThreads = 256;
constexpr int kTensorPartials = 1024;   // at most this many absmax partials (one per workgroup of pass 1)

// Pass 1: each workgroup's absmax over a grid-strided share of the tensor, written to partial[block]
// (no atomics, nothing to clear first).  Four independent 16-byte loads in flight per lane.
__global__ __launch_bounds__(kTensorThreads) void tensor_absmax_partial(const uint16_t* __restrict__ x, int64_t n,
                                                                        bool vec, float* __restrict__ partial) {
    __shared__ float red[kTensorThreads / 64];
    float m = 0.0f;
    const int64_t stride = (int64_t)gridDim.x * kTensorThreads;
    const int64_t nvec = vec ? n / 8 : 0;
    int64_t i = (int64_t)blockIdx.x * kTensorThreads + threadIdx.x;
    for (; i + 3 * stride < nvec; i += 4 * stride) {
        u16x8 a[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) a[u] = *reinterpret_cast<const u16x8*>(x + (i + u * stride) * 8);
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int e = 0; e < 8; ++e) m = __builtin_fmaxf(m, __builtin_fabsf(h2f(a[u][e])));
    }
    for (; i < nvec; i += stride) {
        const u16x8 a = *reinterpret_cast<const u16x8*>(x + i * 8);
#pragma unroll
        for (int e = 0; e < 8; ++e) m = __builtin_fmaxf(m, __builtin_fabsf(h2f(a[e])));
    }
    for (int64_t j = nvec * 8 + (int64_t)blockIdx.x * kTensorThreads + threadIdx.x; j < n; j += stride)
        m = __builtin_fmaxf(m, __builtin_fabsf(h2f(x[j])));
    m = block_max(m, red);
    if (threadIdx.x == 0) partial[blockIdx.x] = m;
}

// Pass 2: every workgroup folds the partials into the tensor absmax (a few KB from L2), derives the
// scale, and quantizes its grid-strided share; workgroup 0 also stores the scale.
__global__ __launch_bounds__(kTensorThreads) void tensor_quantize(const uint16_t* __restrict__ x, int64_t n, bool vec,
                                                                  const float* __restrict__ partial, int nparts,
                                                                  int8_t* __restrict__ q, float* __restrict__ scale) {
    __shared__ float red[kTensorThreads / 64];
    float m = 0.0f;
    for (int p = threadIdx.x; p < nparts; p += kTensorThreads) m = __builtin_fmaxf(m, partial[p]);
    const float s = e3_scale(block_max(m, red));
    if (blockIdx.x == 0 && threadIdx.x == 0) *scale = s;
    const int64_t stride = (int64_t)gridDim.x * kTensorThreads;
    const int64_t nvec = vec ? n / 8 : 0;
    for (int64_t i = (int64_t)blockIdx.x * kTensorThreads + threadIdx.x; i < nvec; i += stride) {
        const u16x8 a = *reinterpret_cast<const u16x8*>(x + i * 8);
        uint32_t lo = pack4(e3_quant(h2f(a[0]), s), e3_quant(h2f(a[1]), s), e3_quant(h2f(a[2]), s), e3_quant(h2f(a[3]), s));
        uint32_t hi = pack4(e3_quant(h2f(a[4]), s), e3_quant(h2f(a[5]), s), e3_quant(h2f(a[6]), s), e3_quant(h2f(a[7]), s));
        *reinterpret_cast<uint2*>(q + i * 8) = make_uint2(lo, hi);
    }
    for (int64_t j = nvec * 8 + (int64_t)blockIdx.x * kTensorThreads + threadIdx.x; j < n; j += stride)
        q[j] = (int8_t)e3_quant(h2f(x[j]), s);
}

// ---------------------------------------------------------------------------
// Self-test of the fast quotients against IEEE division, over every operand the
// kernels can pass them: counts[0] = fp32 quotient mismatches and counts[1] =
// quantized-code mismatches (the fast quotient with the scalar code chain, and
// the kernels' path: a * fl(1 / d) with the packed-fp16 code chain) over all fp16 numerators
// (infinities excluded: a row holding one has an infinite divisor and takes the
// IEEE path) and all finite positive fp16 divisors; counts[2] = SiLU mismatches
// over all 65536 fp16 codes.
// ---------------------------------------------------------------------------
__global__ void zero_counts(uint32_t* c) {
    if (threadIdx.x < 3) c[threadIdx.x] = 0u;
}

__device__ __forceinline__ bool same_bits(float a, float b) {
    return __builtin_bit_cast(uint32_t, a) == __builtin_bit_cast(uint32_t, b) || (a != a && b != b);
}

constexpr int kDivChunk = 1024;
constexpr uint32_t kMaxFiniteHalf = 0x7BFFu;

__global__ __launch_bounds__(256) void selftest_q1_div(uint32_t* __restrict__ counts) {
    const uint32_t acode = blockIdx.x * 256 + threadIdx.x;
    const float a = h2f((uint16_t)acode);
    uint32_t bad_div = 0, bad_q = 0;
    if (__builtin_fabsf(a) != __builtin_inff()) {
        const uint32_t d0 = blockIdx.y * kDivChunk + 1;
        for (uint32_t dc = d0; dc < d0 + kDivChunk && dc <= kMaxFiniteHalf; ++dc) {
            const float d = h2f((uint16_t)dc);
            const Q1Div qd = q1_div(d);
            if (!same_bits(div_newton(a, d, qd.r), a / d)) ++bad_div;
            // the kernels' code path: the reciprocal-multiply quotient, then the packed-fp16 code chain
            const int ref = q1_quant(a, d);
            const int packed = (int)(int8_t)(q1_codes4(q1_quot<true>(a, qd), 0.0f, 0.0f, 0.0f) & 0xFFu);
            if (q1_quant(a, qd) != ref || packed != ref) ++bad_q;
        }
    }
    if (bad_div) atomicAdd(&counts[0], bad_div);
    if (bad_q) atomicAdd(&counts[1], bad_q);
}

__global__ __launch_bounds__(256) void selftest_silu(uint32_t* __restrict__ counts) {
    const uint32_t code = blockIdx.x * 256 + threadIdx.x;
    const float z = h2f((uint16_t)code);
    if (!same_bits(silu_fast(z), silu(z))) atomicAdd(&counts[2], 1u);
}

}  // namespace
}  // namespace h3v

using namespace h3v;

extern "C" {

int h3v_row_quant(const uint16_t* x, int64_t rows, int64_t cols, int8_t* q, float* scale, hipStream_t stream) {
    return launch_row_quant<false>(x, rows, cols, q, scale, stream, "h3v_row_quant");
}

int h3v_swiglu_row_quant(const uint16_t* x, int64_t rows, int64_t cols, int8_t* q, float* scale,
                         hipStream_t stream) {
    return launch_row_quant<true>(x, rows, cols, q, scale, stream, "h3v_swiglu_row_quant");
}

int h3v_selftest_fast_div(uint32_t* counts, hipStream_t stream) {
    const char* what = "h3v_selftest_fast_div";
    H3V_REQUIRE(counts, "%s: null pointer argument", what);
    hipLaunchKernelGGL(zero_counts, dim3(1), dim3(64), 0, stream, counts);
    hipLaunchKernelGGL(selftest_q1_div, dim3(65536 / 256, (kMaxFiniteHalf + kDivChunk - 1) / kDivChunk), dim3(256), 0,
                       stream, counts);
    hipLaunchKernelGGL(selftest_silu, dim3(65536 / 256), dim3(256), 0, stream, counts);
    return launch_status(what);
}

int64_t h3v_tensor_quant_scratch_words(void) { return kTensorPartials; }

int h3v_tensor_quant_i8(const uint16_t* x, int64_t n, int8_t* q, float* scale, uint32_t* scratch,
                        int64_t scratch_words, hipStream_t stream) {
    const char* what = "h3v_tensor_quant_i8";
    H3V_REQUIRE(x && q && scale && scratch, "%s: null pointer argument", what);
    H3V_REQUIRE(n > 0, "%s: activation quantization requires a nonempty tensor", what);
    H3V_REQUIRE(scratch_words >= kTensorPartials,
                "%s: scratch holds %lld words; h3v_tensor_quant_scratch_words() = %d are required", what,
                (long long)scratch_words, kTensorPartials);
    const bool vec = aligned(x, 16) && aligned(q, 8);
    const int64_t nvec = vec ? n / 8 : n / 8 + 1;
    // pass 1: at least 8 vectors per lane; pass 2: at least 4 (it also writes)
    const int64_t p1 = (nvec + 8 * kTensorThreads - 1) / (8 * kTensorThreads);
    const int64_t p2 = (nvec + 4 * kTensorThreads - 1) / (4 * kTensorThreads);
    const int parts = (int)(p1 < 1 ? 1 : (p1 > kTensorPartials ? kTensorPartials : p1));
    const unsigned blocks = (unsigned)(p2 < 1 ? 1 : (p2 > 2048 ? 2048 : p2));
    float* partial = reinterpret_cast<float*>(scratch);
    hipLaunchKernelGGL(tensor_absmax_partial, dim3(parts), dim3(kTensorThreads), 0, stream, x, n, vec, partial);
    hipLaunchKernelGGL(tensor_quantize, dim3(blocks), dim3(kTensorThreads), 0, stream, x, n, vec, partial, parts, q,
                       scale);
    return launch_status(what);
}

}  // extern "C"
