// Quantizers of the H3 VAE INT8 hot path.
//
//  * row quantizer (comfy-kitchen 0.2.34 contract as restated in
//    opt/int8_swiglu_fused.py:29-37 and opt/int8_ffn_up_fused.py:91-104):
//    one workgroup per row, the row stays in registers between the amax and
//    the quantize step, 16-byte loads and 8-byte stores;
//  * SwiGLU + row quantizer (opt/int8_swiglu_fused.py:22-38);
//  * per-tensor encoder activation quantizer (opt/encoder_int8.py:343-378):
//    absmax pass with one atomic max per workgroup, then a quantize pass that
//    derives the scale from the maximum on the fly.
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

// Quantize 8 values against d and store them as two 32-bit words.
__device__ __forceinline__ void store_q8(int8_t* dst, const float* v, float d) {
    uint32_t lo = pack4(q1_quant(v[0], d), q1_quant(v[1], d), q1_quant(v[2], d), q1_quant(v[3], d));
    uint32_t hi = pack4(q1_quant(v[4], d), q1_quant(v[5], d), q1_quant(v[6], d), q1_quant(v[7], d));
    *reinterpret_cast<uint2*>(dst) = make_uint2(lo, hi);
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
            u16x8 a = *reinterpret_cast<const u16x8*>(xr + idx);
            if constexpr (SWIGLU) {
                u16x8 b = *reinterpret_cast<const u16x8*>(xr + K + idx);
#pragma unroll
                for (int e = 0; e < 8; ++e) v[c][e] = rt16(silu(h2f(a[e])) * h2f(b[e]));
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
    const float d = rt16(sc);
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
        if constexpr (SWIGLU) return rt16(silu(h2f(xr[i])) * h2f(xr[K + i]));
        else return h2f(xr[i]);
    };
    float amax = 0.0f;
    for (int i = threadIdx.x; i < K; i += kRowThreads) amax = __builtin_fmaxf(amax, __builtin_fabsf(value(i)));
    amax = block_max(amax, red);
    const float sc = q1_scale(amax);
    const float d = rt16(sc);
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
__global__ void fill_u32(uint32_t* p, uint32_t v) { *p = v; }

constexpr int kTensorThreads = 256;

__global__ __launch_bounds__(kTensorThreads) void tensor_absmax(const uint16_t* __restrict__ x, int64_t n, bool vec,
                                                                uint32_t* __restrict__ amax_bits) {
    __shared__ float red[kTensorThreads / 64];
    float m = 0.0f;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    int64_t i0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    int64_t nvec = vec ? n / 8 : 0;
    for (int64_t i = i0; i < nvec; i += stride) {
        u16x8 a = *reinterpret_cast<const u16x8*>(x + i * 8);
#pragma unroll
        for (int e = 0; e < 8; ++e) m = __builtin_fmaxf(m, __builtin_fabsf(h2f(a[e])));
    }
    for (int64_t i = nvec * 8 + i0; i < n; i += stride) m = __builtin_fmaxf(m, __builtin_fabsf(h2f(x[i])));
    m = block_max(m, red);
    // non-negative floats order like their bit patterns
    if (threadIdx.x == 0) atomicMax(amax_bits, __builtin_bit_cast(uint32_t, m));
}

__global__ __launch_bounds__(kTensorThreads) void tensor_quantize(const uint16_t* __restrict__ x, int64_t n, bool vec,
                                                                  const uint32_t* __restrict__ amax_bits,
                                                                  int8_t* __restrict__ q, float* __restrict__ scale) {
    const float s = e3_scale(__builtin_bit_cast(float, *amax_bits));
    if (blockIdx.x == 0 && threadIdx.x == 0) *scale = s;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    int64_t i0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    int64_t nvec = vec ? n / 8 : 0;
    for (int64_t i = i0; i < nvec; i += stride) {
        u16x8 a = *reinterpret_cast<const u16x8*>(x + i * 8);
        uint32_t lo = pack4(e3_quant(h2f(a[0]), s), e3_quant(h2f(a[1]), s), e3_quant(h2f(a[2]), s), e3_quant(h2f(a[3]), s));
        uint32_t hi = pack4(e3_quant(h2f(a[4]), s), e3_quant(h2f(a[5]), s), e3_quant(h2f(a[6]), s), e3_quant(h2f(a[7]), s));
        *reinterpret_cast<uint2*>(q + i * 8) = make_uint2(lo, hi);
    }
    for (int64_t i = nvec * 8 + i0; i < n; i += stride) q[i] = (int8_t)e3_quant(h2f(x[i]), s);
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

int h3v_tensor_quant_i8(const uint16_t* x, int64_t n, int8_t* q, float* scale, uint32_t* amax_scratch,
                        hipStream_t stream) {
    const char* what = "h3v_tensor_quant_i8";
    H3V_REQUIRE(x && q && scale && amax_scratch, "%s: null pointer argument", what);
    H3V_REQUIRE(n > 0, "%s: activation quantization requires a nonempty tensor", what);
    const bool vec = aligned(x, 16) && aligned(q, 8);
    int64_t want = (n / 8 + kTensorThreads - 1) / kTensorThreads;
    unsigned blocks = (unsigned)(want < 1 ? 1 : (want > 8192 ? 8192 : want));
    hipLaunchKernelGGL(fill_u32, dim3(1), dim3(1), 0, stream, amax_scratch, 0u);
    hipLaunchKernelGGL(tensor_absmax, dim3(blocks), dim3(kTensorThreads), 0, stream, x, n, vec, amax_scratch);
    hipLaunchKernelGGL(tensor_quantize, dim3(blocks), dim3(kTensorThreads), 0, stream, x, n, vec, amax_scratch, q,
                       scale);
    return launch_status(what);
}

}  // extern "C"
