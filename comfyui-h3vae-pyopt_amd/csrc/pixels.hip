// Decoder edge: pixel finalisation of the decoded tiles.
//
// Reference: opt/fp16_finalize.py:24-54 (`finalize_pixels`), the FP32 step that
// turns the decoder's ImageNet-normalised output [B, 3, T, H, W] (fp16 or fp32,
// any strides) into contiguous fp32 pixels in [0, 1]:
//   v = fp32(x) * std[c] + mean[c]       (two roundings: built with -ffp-contract=off)
//   v < 0 -> 0, v > 1 -> 1               (comparisons: NaN and an in-range -0 pass through)
// Memory-bound: 2 or 4 bytes read and 4 written per element.  Contiguous
// inputs whose T*H*W is a multiple of 8 take the vector path (8 elements per
// thread and step, one channel each); anything else walks the strides.
#include "h3v_common.hpp"
#include "h3v_abi.hpp"

namespace h3v {
namespace {

__device__ __forceinline__ float finalize_one(float x, float s, float m) {
    const float v = x * s + m;
    return v < 0.0f ? 0.0f : (v > 1.0f ? 1.0f : v);
}

typedef float f32x4v __attribute__((ext_vector_type(4)));

template <bool F16>
__global__ __launch_bounds__(256) void finalize_vec(const void* __restrict__ x, int64_t n8, int64_t thw8,
                                                    const float* __restrict__ stdv, const float* __restrict__ meanv,
                                                    float* __restrict__ out) {
    const float s0 = stdv[0], s1 = stdv[1], s2 = stdv[2];
    const float m0 = meanv[0], m1 = meanv[1], m2 = meanv[2];
    for (int64_t v = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; v < n8; v += (int64_t)gridDim.x * blockDim.x) {
        const int c = (int)((v / thw8) % 3);
        const float s = c == 0 ? s0 : (c == 1 ? s1 : s2);
        const float m = c == 0 ? m0 : (c == 1 ? m1 : m2);
        float f[8];
        if constexpr (F16) {
            const u16x8 h = reinterpret_cast<const u16x8*>(x)[v];
#pragma unroll
            for (int e = 0; e < 8; ++e) f[e] = h2f(h[e]);
        } else {
            const f32x4v a = reinterpret_cast<const f32x4v*>(x)[2 * v];
            const f32x4v b = reinterpret_cast<const f32x4v*>(x)[2 * v + 1];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                f[e] = a[e];
                f[4 + e] = b[e];
            }
        }
        f32x4v lo, hi;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            lo[e] = finalize_one(f[e], s, m);
            hi[e] = finalize_one(f[4 + e], s, m);
        }
        reinterpret_cast<f32x4v*>(out)[2 * v] = lo;
        reinterpret_cast<f32x4v*>(out)[2 * v + 1] = hi;
    }
}

struct Strides5 {
    int64_t s[5];
};

template <bool F16>
__global__ __launch_bounds__(256) void finalize_strided(const void* __restrict__ x, int64_t n, int64_t t, int64_t h,
                                                        int64_t w, Strides5 st, const float* __restrict__ stdv,
                                                        const float* __restrict__ meanv, float* __restrict__ out) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        int64_t r = i;
        const int64_t iw = r % w;
        r /= w;
        const int64_t ih = r % h;
        r /= h;
        const int64_t it = r % t;
        r /= t;
        const int c = (int)(r % 3);
        const int64_t ib = r / 3;
        const int64_t off = ib * st.s[0] + c * st.s[1] + it * st.s[2] + ih * st.s[3] + iw * st.s[4];
        const float xv = F16 ? h2f(static_cast<const uint16_t*>(x)[off]) : static_cast<const float*>(x)[off];
        out[i] = finalize_one(xv, stdv[c], meanv[c]);
    }
}

}  // namespace
}  // namespace h3v

using namespace h3v;

extern "C" int h3v_finalize_pixels(const void* x, int x_is_f16, int64_t batch, int64_t frames, int64_t height,
                                   int64_t width, const int64_t* strides, const float* std, const float* mean,
                                   float* out, hipStream_t stream) {
    const char* what = "h3v_finalize_pixels";
    H3V_REQUIRE(x && strides && std && mean && out, "%s: null pointer argument", what);
    H3V_REQUIRE(batch > 0 && frames > 0 && height > 0 && width > 0, "%s: a nonempty [B,3,T,H,W] tensor is required",
                what);
    const int64_t thw = frames * height * width;
    H3V_REQUIRE(thw <= ((int64_t)1 << 40) && batch <= ((int64_t)1 << 20), "%s: shape out of range", what);
    const int64_t n = batch * 3 * thw;
    const int64_t cs[5] = {3 * thw, thw, height * width, width, 1};
    bool contiguous = true;
    for (int d = 0; d < 5; ++d) contiguous = contiguous && strides[d] == cs[d];
    const bool vec = contiguous && thw % 8 == 0 && aligned(x, 16) && aligned(out, 16);
    const int64_t work = vec ? n / 8 : n;
    const int64_t blocks = (work + 255) / 256 < 256 * 32 ? (work + 255) / 256 : 256 * 32;
    if (vec) {
        if (x_is_f16) hipLaunchKernelGGL((finalize_vec<true>), dim3((unsigned)blocks), dim3(256), 0, stream, x, n / 8,
                                         thw / 8, std, mean, out);
        else hipLaunchKernelGGL((finalize_vec<false>), dim3((unsigned)blocks), dim3(256), 0, stream, x, n / 8,
                                thw / 8, std, mean, out);
    } else {
        Strides5 st;
        for (int d = 0; d < 5; ++d) st.s[d] = strides[d];
        if (x_is_f16) hipLaunchKernelGGL((finalize_strided<true>), dim3((unsigned)blocks), dim3(256), 0, stream, x, n,
                                         frames, height, width, st, std, mean, out);
        else hipLaunchKernelGGL((finalize_strided<false>), dim3((unsigned)blocks), dim3(256), 0, stream, x, n, frames,
                                height, width, st, std, mean, out);
    }
    return launch_status(what);
}
