// Residual + bias pack ahead of the stride-2 downsample conv of the last
// encoder prefix block (opt/encoder_fused_residual_pack.py:12-55).
//
// x, residual: fp16 NDHWC [D, H, W, C] (batch one); bias fp16 [C].
// out: fp16 NDHWC [D+2, H+1, W+1, C]:
//   out[t', h', w', c] = 0                                   for t' < 2
//                      = fp16(r[t,h,w,c] + (x[t,h,w,c] + b[c]))  otherwise,
// with t = t'-2, h = h' (h' < H) or H-2 (h' == H), w likewise: one reflected
// row/column at the bottom/right.  Both adds are fp32 and the result is
// rounded to fp16 once.
//
// HBM-bound: 2 B read of x and r per source element, 2 B written per output
// element.  One thread owns 8 channels (16-byte loads and stores); consecutive
// threads walk channels, then pixels, so every wave touches contiguous memory.
#include "h3v_common.hpp"
#include "h3v_abi.hpp"

namespace h3v {
namespace {

constexpr int kThreads = 256;

__global__ __launch_bounds__(kThreads) void residual_downsample_pack_kernel(
    const u16x8* __restrict__ x, const u16x8* __restrict__ r, const uint16_t* __restrict__ bias,
    u16x8* __restrict__ out, uint32_t cv, uint32_t d, uint32_t h, uint32_t w, uint32_t nvec) {
    const uint32_t i = blockIdx.x * kThreads + threadIdx.x;
    if (i >= nvec) return;
    const uint32_t c8 = i % cv;
    uint32_t p = i / cv;
    const uint32_t wo = p % (w + 1);
    p /= (w + 1);
    const uint32_t ho = p % (h + 1);
    const uint32_t to = p / (h + 1);
    u16x8 y;
    if (to < 2) {
#pragma unroll
        for (int e = 0; e < 8; ++e) y[e] = 0;
    } else {
        const uint32_t t = to - 2;
        const uint32_t hs = ho == h ? h - 2 : ho;
        const uint32_t ws = wo == w ? w - 2 : wo;
        const uint32_t src = ((t * h + hs) * w + ws) * cv + c8;
        const u16x8 xv = x[src];
        const u16x8 rv = r[src];
        const u16x8 bv = *reinterpret_cast<const u16x8*>(bias + 8 * c8);
#pragma unroll
        for (int e = 0; e < 8; ++e) y[e] = f2h(h2f(rv[e]) + (h2f(xv[e]) + h2f(bv[e])));
    }
    out[i] = y;
}

// Causal/reflect pack of an fp16 NDHWC tensor [B, D, H, W, C] into
// [B, D + front, H + top + bottom, W + left + right, C]: `front` zero frames per
// item, then the frames with the spatial border reflected (index -p -> p,
// H - 1 + p -> H - 1 - p).  One thread per 8 channels of one output pixel.
__global__ __launch_bounds__(kThreads) void causal_reflect_pack_kernel(
    const u16x8* __restrict__ x, u16x8* __restrict__ out, uint32_t cv, uint32_t d, uint32_t h, uint32_t w,
    uint32_t front, uint32_t top, uint32_t left, uint32_t dp, uint32_t hp, uint32_t wp, uint64_t nvec) {
    const uint64_t i = (uint64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i >= nvec) return;
    const uint32_t c8 = (uint32_t)(i % cv);
    uint64_t p = i / cv;
    const uint32_t wo = (uint32_t)(p % wp);
    p /= wp;
    const uint32_t ho = (uint32_t)(p % hp);
    p /= hp;
    const uint32_t to = (uint32_t)(p % dp);
    const uint32_t b = (uint32_t)(p / dp);
    u16x8 y;
    if (to < front) {
#pragma unroll
        for (int e = 0; e < 8; ++e) y[e] = 0;
    } else {
        const int hs0 = (int)ho - (int)top, ws0 = (int)wo - (int)left;
        const int hs = hs0 < 0 ? -hs0 : (hs0 >= (int)h ? 2 * ((int)h - 1) - hs0 : hs0);
        const int ws = ws0 < 0 ? -ws0 : (ws0 >= (int)w ? 2 * ((int)w - 1) - ws0 : ws0);
        const uint64_t src = ((((uint64_t)b * d + (to - front)) * h + (uint32_t)hs) * w + (uint32_t)ws) * cv + c8;
        y = x[src];
    }
    out[i] = y;
}

// Tap-folded pack for a 3x3x3 convolution with few input channels (the encoder's conv_in, C = 3):
// out[b, t', h, w, (kh * 3 + kw) * C + c] = x[b, t' - front, reflect(h + kh - 1), reflect(w + kw - 1), c]
// for t' >= front, 0 for t' < front and for the channels 9C .. CF-1.  The 3x3x3 conv over x becomes a
// 3x1x1 conv over out (K = 3 * CF), which the matrix-core conv runs without padding C to 32 per tap.
// One thread per output pixel: CF / 8 16-byte stores.
template <int C, int CF>
__global__ __launch_bounds__(kThreads) void tap_fold_pack_kernel(const uint16_t* __restrict__ x,
                                                                 u16x8* __restrict__ out, uint32_t d, uint32_t h,
                                                                 uint32_t w, uint32_t front, uint32_t dp,
                                                                 uint64_t npix) {
    static_assert(9 * C <= CF && CF % 8 == 0, "folded channels");
    const uint64_t i = (uint64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i >= npix) return;
    const uint32_t wo = (uint32_t)(i % w);
    uint64_t p = i / w;
    const uint32_t ho = (uint32_t)(p % h);
    p /= h;
    const uint32_t to = (uint32_t)(p % dp);
    const uint32_t b = (uint32_t)(p / dp);
    uint16_t v[CF];
#pragma unroll
    for (int e = 0; e < CF; ++e) v[e] = 0;
    if (to >= front) {
        const uint64_t frame = ((uint64_t)b * d + (to - front)) * h;
#pragma unroll
        for (int kh = 0; kh < 3; ++kh) {
            const int hs0 = (int)ho + kh - 1;
            const int hs = hs0 < 0 ? -hs0 : (hs0 >= (int)h ? 2 * ((int)h - 1) - hs0 : hs0);
#pragma unroll
            for (int kw = 0; kw < 3; ++kw) {
                const int ws0 = (int)wo + kw - 1;
                const int ws = ws0 < 0 ? -ws0 : (ws0 >= (int)w ? 2 * ((int)w - 1) - ws0 : ws0);
                const uint16_t* src = x + ((frame + (uint32_t)hs) * w + (uint32_t)ws) * C;
#pragma unroll
                for (int ch = 0; ch < C; ++ch) v[(kh * 3 + kw) * C + ch] = src[ch];
            }
        }
    }
#pragma unroll
    for (int q = 0; q < CF / 8; ++q) {
        u16x8 y;
#pragma unroll
        for (int e = 0; e < 8; ++e) y[e] = v[q * 8 + e];
        out[i * (CF / 8) + q] = y;
    }
}

}  // namespace
}  // namespace h3v

using namespace h3v;

extern "C" int h3v_tap_fold_pack(const uint16_t* x, uint16_t* out, int batch, int c, int d, int h, int w, int front,
                                 int cf, hipStream_t stream) {
    const char* what = "tap_fold_pack";
    H3V_REQUIRE(x && out, "%s: null pointer", what);
    H3V_REQUIRE(cf == 32 && c >= 1 && c <= 3, "%s: needs C in 1..3 and 32 folded channels (got C %d, %d)", what, c,
                cf);
    H3V_REQUIRE(batch > 0 && d > 0 && h >= 2 && w >= 2 && front >= 0,
                "%s: need positive sizes and H, W >= 2 (got B %d, %dx%dx%d)", what, batch, d, h, w);
    H3V_REQUIRE(aligned(out, 16), "%s: output must be 16-byte aligned", what);
    const uint32_t dp = (uint32_t)(d + front);
    const uint64_t npix = (uint64_t)batch * dp * h * w;
    H3V_REQUIRE(npix < ((uint64_t)1 << 36), "%s: tensor too large", what);
    const uint64_t blocks = (npix + kThreads - 1) / kThreads;
    H3V_REQUIRE(blocks <= 0x7fffffffu, "%s: tensor too large", what);
    auto kernel = c == 1 ? tap_fold_pack_kernel<1, 32> : (c == 2 ? tap_fold_pack_kernel<2, 32> : tap_fold_pack_kernel<3, 32>);
    hipLaunchKernelGGL(kernel, dim3((unsigned)blocks), dim3(kThreads), 0, stream, x, reinterpret_cast<u16x8*>(out),
                       (uint32_t)d, (uint32_t)h, (uint32_t)w, (uint32_t)front, dp, npix);
    return launch_status(what);
}

extern "C" int h3v_causal_reflect_pack(const uint16_t* x, uint16_t* out, int batch, int c, int d, int h, int w,
                                       int front, int top, int bottom, int left, int right, hipStream_t stream) {
    const char* what = "causal_reflect_pack";
    H3V_REQUIRE(x && out, "%s: null pointer", what);
    H3V_REQUIRE(batch > 0 && c > 0 && c % 8 == 0 && d > 0 && h > 0 && w > 0,
                "%s: need positive sizes and channels a multiple of 8 (got B %d, C %d, %dx%dx%d)", what, batch, c, d,
                h, w);
    H3V_REQUIRE(front >= 0 && top >= 0 && bottom >= 0 && left >= 0 && right >= 0 && top < h && bottom < h &&
                left < w && right < w, "%s: reflect padding must be smaller than the padded dimension", what);
    H3V_REQUIRE(aligned(x, 16) && aligned(out, 16), "%s: buffers must be 16-byte aligned", what);
    const uint32_t dp = (uint32_t)(d + front), hp = (uint32_t)(h + top + bottom), wp = (uint32_t)(w + left + right);
    const uint64_t nvec = (uint64_t)batch * dp * hp * wp * (uint32_t)(c / 8);
    H3V_REQUIRE(nvec < ((uint64_t)1 << 40), "%s: tensor too large", what);
    const uint64_t blocks = (nvec + kThreads - 1) / kThreads;
    H3V_REQUIRE(blocks <= 0x7fffffffu, "%s: tensor too large", what);
    hipLaunchKernelGGL(causal_reflect_pack_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, stream,
                       reinterpret_cast<const u16x8*>(x), reinterpret_cast<u16x8*>(out), (uint32_t)(c / 8),
                       (uint32_t)d, (uint32_t)h, (uint32_t)w, (uint32_t)front, (uint32_t)top, (uint32_t)left, dp, hp,
                       wp, nvec);
    return launch_status(what);
}

extern "C" int h3v_residual_downsample_pack(const uint16_t* x, const uint16_t* residual, const uint16_t* bias,
                                            uint16_t* out, int c, int d, int h, int w, hipStream_t stream) {
    H3V_REQUIRE(x && residual && bias && out, "residual_downsample_pack: null pointer");
    H3V_REQUIRE(c > 0 && c % 8 == 0, "residual_downsample_pack: channels must be a positive multiple of 8, got %d", c);
    H3V_REQUIRE(d >= 1 && h >= 2 && w >= 2, "residual_downsample_pack: need D>=1 and H, W>=2 (got %d, %d, %d)", d, h,
                w);
    const int64_t total = (int64_t)c * (d + 2) * (h + 1) * (w + 1);
    H3V_REQUIRE(total < (int64_t{1} << 31), "residual_downsample_pack: output exceeds the int32 index range");
    H3V_REQUIRE(aligned(x, 16) && aligned(residual, 16) && aligned(bias, 16) && aligned(out, 16),
                "residual_downsample_pack: buffers must be 16-byte aligned");
    const uint32_t nvec = (uint32_t)(total / 8);
    const uint32_t blocks = (nvec + kThreads - 1) / kThreads;
    hipLaunchKernelGGL(residual_downsample_pack_kernel, dim3(blocks), dim3(kThreads), 0, stream,
                       reinterpret_cast<const u16x8*>(x), reinterpret_cast<const u16x8*>(residual), bias,
                       reinterpret_cast<u16x8*>(out), (uint32_t)(c / 8), (uint32_t)d, (uint32_t)h, (uint32_t)w, nvec);
    return launch_status("residual_downsample_pack");
}
