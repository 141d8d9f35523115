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

}  // namespace
}  // namespace h3v

using namespace h3v;

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
