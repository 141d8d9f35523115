// Measured MFMA ceiling of the part for a given int8 data set.
//
// The INT8 dense peak (256 CU x 8192 ops/clk x 2.4 GHz) assumes the top shader
// clock.  The clock the part sustains under a matrix load depends on the power
// the MFMAs draw, and that depends on the data they multiply (zeros toggle
// nothing; quantized Gaussian activations toggle a lot).  This kernel measures
// the ceiling for the caller's own operands: 8 waves per CU (2 per SIMD), each
// issuing back-to-back v_mfma_i32_32x32x32_i8 on a 4 x 2 block of independent
// accumulators with register-resident operands (four operand sets rotated per
// iteration, so successive MFMAs see different data), no memory traffic and
// no LDS in the timed loop.  Every workgroup records its shader-clock ticks
// (s_memtime) and 100 MHz reference ticks (s_memrealtime) over the loop, so
// the caller also gets the average clock the part held.
#include "h3v_common.hpp"
#include "h3v_abi.hpp"

namespace h3v {
namespace {

constexpr int kProbeSets = 4;
constexpr int kProbeWaves = 8;

__global__ __launch_bounds__(kProbeWaves * 64) void mfma_rate(const int8_t* __restrict__ a, int64_t a_vecs,
                                                              const int8_t* __restrict__ b, int64_t b_vecs,
                                                              int iters, int32_t* __restrict__ sink,
                                                              int64_t* __restrict__ clocks) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int64_t slot = (int64_t)blockIdx.x * kProbeWaves + wave;
    // operand fragments: 16 bytes per lane, taken from the caller's buffers at
    // offsets spread over them (a_vecs / b_vecs = number of 16-byte vectors)
    v4i fa[kProbeSets][4], fb[kProbeSets][2];
#pragma unroll
    for (int s = 0; s < kProbeSets; ++s) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int64_t v = ((slot * kProbeSets + s) * 4 + i) * 64 + lane;
            fa[s][i] = *reinterpret_cast<const v4i*>(a + (v * 7919 % a_vecs) * 16);
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int64_t v = ((slot * kProbeSets + s) * 2 + j) * 64 + lane;
            fb[s][j] = *reinterpret_cast<const v4i*>(b + (v * 7919 % b_vecs) * 16);
        }
    }
    v16i acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = v16i{};
    __syncthreads();
    const int64_t t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int s = 0; s < kProbeSets; ++s)
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fb[s][j], fa[s][i], acc[i][j], 0, 0, 0);
    }
    const int64_t t1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
    int32_t x = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) x += acc[i][j][e];
    sink[(int64_t)blockIdx.x * blockDim.x + threadIdx.x] = x;   // keeps the MFMAs live
    if (threadIdx.x == 0) {
        clocks[2 * (int64_t)blockIdx.x] = t1 - t0;
        clocks[2 * (int64_t)blockIdx.x + 1] = r1 - r0;
    }
}

}  // namespace
}  // namespace h3v

using namespace h3v;

extern "C" int h3v_probe_mfma_rate(const int8_t* a, int64_t a_bytes, const int8_t* b, int64_t b_bytes, int blocks,
                                   int iters, int32_t* sink, int64_t* clocks, hipStream_t stream) {
    const char* what = "h3v_probe_mfma_rate";
    H3V_REQUIRE(a && b && sink && clocks, "%s: null pointer argument", what);
    H3V_REQUIRE(aligned(a, 16) && aligned(b, 16), "%s: operand buffers must be 16-byte aligned", what);
    H3V_REQUIRE(a_bytes >= 16 && b_bytes >= 16, "%s: operand buffers must hold at least 16 bytes", what);
    H3V_REQUIRE(blocks > 0 && blocks <= 65536 && iters > 0, "%s: blocks in [1, 65536] and iters > 0 required", what);
    hipLaunchKernelGGL(mfma_rate, dim3((unsigned)blocks), dim3(kProbeWaves * 64), 0, stream, a, a_bytes / 16, b,
                       b_bytes / 16, iters, sink, clocks);
    return launch_status(what);
}

extern "C" int64_t h3v_probe_mfma_ops_per_block(int iters) {
    // sets x (4 x 2 MFMAs) x waves x 32*32*32 MACs x 2
    return (int64_t)iters * kProbeSets * 8 * kProbeWaves * 32 * 32 * 32 * 2;
}
