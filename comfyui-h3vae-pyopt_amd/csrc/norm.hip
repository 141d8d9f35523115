// Decoder row producers: residual + RMSNorm + row quantization (norm1 / norm2),
// the block-0 RMSNorm and the final residual + LayerNorm.
//
// One wave per row of width K = NCH * 512 (K in {1024, 2048, 4096}; the
// residual producers keep persistent waves that walk several rows); four waves
// per 256-thread workgroup, no LDS and no workgroup barrier (measured against
// one 256-thread workgroup per row: 20.7 vs 27.5 us at 16384 x 1024, equal at
// 7188 x 2048).  Lane L holds the
// eight consecutive values [c*512 + 8L, c*512 + 8L + 8) of each chunk c, read
// and written with 16-byte accesses.
//
// Reductions follow a fixed tree that does not depend on how lanes hold the
// row: the row is split into K/4 "virtual threads" of four consecutive values;
// each forms a partial, partials are combined by a butterfly over groups of 32
// (offsets 16, 8, 4, 2, 1) and the K/128 group results by the halving tree
// g[i] += g[i + off], off = K/256 .. 1.  Lane L holds virtual threads
// c*128 + 2L and c*128 + 2L + 1, so the butterfly offsets 16..2 are lane XORs
// 8..1 inside 16-lane segments and offset 1 is a lane-local add; group
// c*4 + L/16 sits in chunk c of segment L/16, so the halving tree is local
// across chunks for off >= 4 and lane XORs 32 and 16 for off = 2 and 1.
//
// Partial of four values:
//   W16 recipe (norm1, docs/decoder_norm1_contract_2026-10-03.md:57-70):
//       s1 = x1*x1; a = fma(x0,x0,s1); b = fma(x2,x2,a); s3 = x3*x3; p = s3 + b
//   plain recipe: p = ((t0 + t1) + t2) + t3 over already rounded terms.
#include <algorithm>
#include <mutex>
#include <type_traits>

#include "h3v_common.hpp"
#include "h3v_abi.hpp"


namespace h3v {
namespace {

constexpr int kNT = 256;
constexpr int kRowsPerBlock = kNT / 64;

enum class Recipe { W16, Plain };

__device__ __forceinline__ float partial_w16(const float* x) {
    float s1 = x[1] * x[1];
    float a = __builtin_fmaf(x[0], x[0], s1);
    float b = __builtin_fmaf(x[2], x[2], a);
    float s3 = x[3] * x[3];
    return s3 + b;
}

__device__ __forceinline__ float partial_plain(const float* t) { return ((t[0] + t[1]) + t[2]) + t[3]; }

// Tree sum of the row from the two partials p[c][0..1] every lane holds per chunk.
template <int NCH>
__device__ __forceinline__ float row_tree(float (&p)[NCH][2]) {
#pragma unroll
    for (int c = 0; c < NCH; ++c)
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int off = 8; off >= 1; off >>= 1) p[c][h] = p[c][h] + __shfl_xor(p[c][h], off, 64);
    float g[NCH];
#pragma unroll
    for (int c = 0; c < NCH; ++c) g[c] = p[c][0] + p[c][1];
#pragma unroll
    for (int off = NCH * 2; off >= 4; off >>= 1)
#pragma unroll
        for (int c = 0; c < off / 4; ++c) g[c] = g[c] + g[c + off / 4];
    g[0] = g[0] + __shfl_xor(g[0], 32, 64);
    g[0] = g[0] + __shfl_xor(g[0], 16, 64);
    return __shfl(g[0], 0, 64);
}

__device__ __forceinline__ void load8f(const uint16_t* p, float* v) {
    u16x8 a = *reinterpret_cast<const u16x8*>(p);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = h2f(a[e]);
}

__device__ __forceinline__ void store8h(uint16_t* p, const float* v) {
    u16x8 a;
#pragma unroll
    for (int e = 0; e < 8; ++e) a[e] = f2h(v[e]);
    *reinterpret_cast<u16x8*>(p) = a;
}

// N1 / F1: raw = fma(o, g, h); h_out = fp16(raw); ss = tree(raw^2);
// inv = 1/sqrt(ss/K + eps); n = fp16((fp32(h_out) * inv) * w); row-quantize n.
//
// Persistent waves: wave i of the grid takes rows i, i + W, i + 2W, ... (W waves in the grid), and the
// next row's h and o are loaded before the current row is reduced, so one row's loads overlap the
// previous row's arithmetic (about 30 VALU operations per element).  With one wave per row every load
// is issued at once and the arithmetic starts only when they have all arrived, which serialises the two.
// Two register buffers alternate in a loop unrolled by two, so the buffer carried over the loop edge is
// never copied (a copy would have to wait for its loads).  The gate and the norm weight are the same for
// every row and load once per wave.  Kernel time at 7188 x 2048: 21.1 us against 23.6 us with one wave
// per row, equal at 16384 x 1024 (same box); 4 or 16 persistent waves per CU were slower.
template <int NCH, Recipe R>
__global__ __launch_bounds__(kNT) void residual_rms_quant_kernel(const uint16_t* h, const uint16_t* __restrict__ o,
                                                                 const uint16_t* __restrict__ g, const uint16_t* __restrict__ w,
                                                                 float eps, uint16_t* h_out, int8_t* __restrict__ q,
                                                                 float* __restrict__ s, int64_t m) {
    constexpr int K = NCH * 512;
    const int lane = threadIdx.x & 63;
    const int64_t nw = (int64_t)gridDim.x * (kNT / 64);
    int64_t row = (int64_t)blockIdx.x * (kNT / 64) + (threadIdx.x >> 6);   // wave-uniform
    float gv[NCH][8];
    u16x8 wq[NCH];
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        load8f(g + c * 512 + lane * 8, gv[c]);
        wq[c] = *reinterpret_cast<const u16x8*>(w + c * 512 + lane * 8);
    }
    u16x8 ha[NCH], oa[NCH], hb[NCH], ob[NCH];
    auto load = [&](u16x8 (&hx)[NCH], u16x8 (&ox)[NCH], int64_t r) {
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            hx[c] = load_nt(h + r * K + c * 512 + lane * 8);
            ox[c] = load_nt(o + r * K + c * 512 + lane * 8);
        }
    };
    auto process = [&](const u16x8 (&hx)[NCH], const u16x8 (&ox)[NCH], int64_t r) {
        float raw[NCH][8];
        float part[NCH][2];
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
#pragma unroll
            for (int e = 0; e < 8; ++e) raw[c][e] = __builtin_fmaf(h2f(ox[c][e]), gv[c][e], h2f(hx[c][e]));
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                const float* x = &raw[c][hh * 4];
                if constexpr (R == Recipe::W16) {
                    part[c][hh] = partial_w16(x);
                } else {
                    float sq[4] = {x[0] * x[0], x[1] * x[1], x[2] * x[2], x[3] * x[3]};
                    part[c][hh] = partial_plain(sq);
                }
            }
        }
        // from here on only fp16-rounded values are used (h_out = fp16(raw), then n = fp16(...)): the row
        // is held as packed fp16
        u16x8 hv[NCH];
#pragma unroll
        for (int c = 0; c < NCH; ++c)
#pragma unroll
            for (int e = 0; e < 8; ++e) hv[c][e] = f2h(raw[c][e]);
        const float ss = row_tree<NCH>(part);
        const float inv = rsqrt_rn(ss / (float)K + eps);
        float amax = 0.0f;
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            const int col = c * 512 + lane * 8;
            *reinterpret_cast<u16x8*>(h_out + r * K + col) = hv[c];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float n = rt16((h2f(hv[c][e]) * inv) * h2f(wq[c][e]));
                amax = __builtin_fmaxf(amax, __builtin_fabsf(n));
                hv[c][e] = f2h(n);
            }
        }
        amax = wave_max(amax);
        const float sc = q1_scale(amax);
        const Q1Div qd = q1_div(rt16(sc));
        // the divisor is the same in every lane: one uniform branch per row picks the quotient path
        auto store_q = [&](auto fast) {
            constexpr bool F = decltype(fast)::value;
#pragma unroll
            for (int c = 0; c < NCH; ++c) {
                const int col = c * 512 + lane * 8;
                float v[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) v[e] = h2f(hv[c][e]);
                const uint32_t lo = q1_codes4(q1_quot<F>(v[0], qd), q1_quot<F>(v[1], qd), q1_quot<F>(v[2], qd),
                                              q1_quot<F>(v[3], qd));
                const uint32_t hi = q1_codes4(q1_quot<F>(v[4], qd), q1_quot<F>(v[5], qd), q1_quot<F>(v[6], qd),
                                              q1_quot<F>(v[7], qd));
                *reinterpret_cast<uint2*>(q + r * K + col) = make_uint2(lo, hi);
            }
        };
        if (__builtin_amdgcn_readfirstlane((int)qd.fast)) store_q(std::true_type{});
        else store_q(std::false_type{});
        if (lane == 0) s[r] = sc;
    };
    if (row >= m) return;
    load(ha, oa, row);
    for (; row < m; row += 2 * nw) {
        // Both loads are unconditional (a branch around one would make the compiler's wait counts wait
        // for it too); a wave without a next row re-reads its current row, which L2 still holds.
        const bool more = row + nw < m;        // wave-uniform
        load(hb, ob, more ? row + nw : row);
        __builtin_amdgcn_sched_barrier(0);   // keep the next row's loads ahead of this row's arithmetic
        process(ha, oa, row);
        load(ha, oa, row + 2 * nw < m ? row + 2 * nw : row);
        __builtin_amdgcn_sched_barrier(0);
        if (more) process(hb, ob, row + nw);
    }
}

// N3: out = fp16((x * inv) * gamma), inv = 1/sqrt(W16(x^2)/K + eps).
template <int NCH>
__global__ __launch_bounds__(kNT) void rms_fp16_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ gamma,
                                                       float eps, uint16_t* __restrict__ out, int64_t m) {
    constexpr int K = NCH * 512;
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (row >= m) return;
    float xv[NCH][8], part[NCH][2];
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        load8f(x + row * K + c * 512 + lane * 8, xv[c]);
        part[c][0] = partial_w16(&xv[c][0]);
        part[c][1] = partial_w16(&xv[c][4]);
    }
    const float inv = rsqrt_rn(row_tree<NCH>(part) / (float)K + eps);
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const int col = c * 512 + lane * 8;
        float gv[8], r[8];
        load8f(gamma + col, gv);
#pragma unroll
        for (int e = 0; e < 8; ++e) r[e] = (xv[c][e] * inv) * gv[e];
        store8h(out + row * K + col, r);
    }
}

// N4: raw = fma(o, gate, h); mean = plain(raw)/K; var = plain((raw-mean)^2)/K;
// y = fp16(fma((raw - mean) * inv, gamma, beta)).
template <int NCH>
__global__ __launch_bounds__(kNT) void residual_layernorm_kernel(const uint16_t* __restrict__ h, const uint16_t* __restrict__ o,
                                                                 const uint16_t* __restrict__ gate, const uint16_t* __restrict__ gamma,
                                                                 const uint16_t* __restrict__ beta, float eps,
                                                                 uint16_t* __restrict__ out, int64_t m) {
    constexpr int K = NCH * 512;
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (row >= m) return;
    float raw[NCH][8], part[NCH][2];
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const int col = c * 512 + lane * 8;
        float hv[8], ov[8], gv[8];
        load8f(h + row * K + col, hv);
        load8f(o + row * K + col, ov);
        load8f(gate + col, gv);
#pragma unroll
        for (int e = 0; e < 8; ++e) raw[c][e] = __builtin_fmaf(ov[e], gv[e], hv[e]);
        part[c][0] = partial_plain(&raw[c][0]);
        part[c][1] = partial_plain(&raw[c][4]);
    }
    const float mean = row_tree<NCH>(part) / (float)K;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        float sq[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            float dv = raw[c][e] - mean;
            sq[e] = dv * dv;
        }
        part[c][0] = partial_plain(&sq[0]);
        part[c][1] = partial_plain(&sq[4]);
    }
    const float inv = rsqrt_rn(row_tree<NCH>(part) / (float)K + eps);
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const int col = c * 512 + lane * 8;
        float gv[8], bv[8], r[8];
        load8f(gamma + col, gv);
        load8f(beta + col, bv);
#pragma unroll
        for (int e = 0; e < 8; ++e) r[e] = __builtin_fmaf((raw[c][e] - mean) * inv, gv[e], bv[e]);
        store8h(out + row * K + col, r);
    }
}

constexpr int kWavesPerCu = 8;    // persistent waves per CU of the residual producers

constexpr int kMaxDevices = 64;
std::mutex g_cu_mutex;
int g_cus[kMaxDevices] = {};

// CU count of the current device (looked up once per device).
int cu_count(const char* what, int* out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail(H3V_ELAUNCH, "%s: hipGetDevice failed: %s", what, hipGetErrorString(e));
    H3V_REQUIRE(dev >= 0 && dev < kMaxDevices, "%s: device index %d out of range", what, dev);
    std::lock_guard<std::mutex> lock(g_cu_mutex);
    if (!g_cus[dev]) {
        int n = 0;
        e = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev);
        if (e != hipSuccess || n <= 0) return fail(H3V_ELAUNCH, "%s: CU count query failed: %s", what, hipGetErrorString(e));
        g_cus[dev] = n;
    }
    *out = g_cus[dev];
    return H3V_OK;
}

int check_row_width(const char* what, int64_t rows, int64_t k) {
    if (rows <= 0 || rows > 0x7fffffff) return fail(H3V_EINVAL, "%s: row count must be in [1, 2^31)", what);
    if (k != 1024 && k != 2048 && k != 4096)
        return fail(H3V_EINVAL, "%s: row width must be 1024, 2048 or 4096 (got %lld)", what, (long long)k);
    return H3V_OK;
}

}  // namespace
}  // namespace h3v

using namespace h3v;

extern "C" {

static int residual_quant_common(const uint16_t* h, const uint16_t* o, const uint16_t* g, const uint16_t* w,
                                 float eps, int64_t m, int64_t k, uint16_t* h_out, int8_t* q, float* scale,
                                 hipStream_t stream, bool w16, const char* what) {
    H3V_REQUIRE(h && o && g && w && h_out && q && scale, "%s: null pointer argument", what);
    int rc = check_row_width(what, m, k);
    if (rc) return rc;
    H3V_REQUIRE(aligned(h, 16) && aligned(o, 16) && aligned(g, 16) && aligned(w, 16) && aligned(h_out, 16) && aligned(q, 8),
                "%s: fp16 pointers must be 16-byte and q 8-byte aligned", what);
    H3V_REQUIRE(h_out == h || (h_out + m * k <= o || o + m * k <= h_out),
                "%s: h_out must not overlap o", what);
    int cus = 0;
    rc = cu_count(what, &cus);
    if (rc) return rc;
    // persistent waves (kWavesPerCu per CU), at most one per row
    const int64_t blocks = std::min<int64_t>((m + kRowsPerBlock - 1) / kRowsPerBlock, (int64_t)cus * kWavesPerCu / kRowsPerBlock);
    dim3 grid((unsigned)blocks), block(kNT);
    if (w16) {
        if (k == 1024) hipLaunchKernelGGL((residual_rms_quant_kernel<2, Recipe::W16>), grid, block, 0, stream, h, o, g, w, eps, h_out, q, scale, m);
        else if (k == 2048) hipLaunchKernelGGL((residual_rms_quant_kernel<4, Recipe::W16>), grid, block, 0, stream, h, o, g, w, eps, h_out, q, scale, m);
        else hipLaunchKernelGGL((residual_rms_quant_kernel<8, Recipe::W16>), grid, block, 0, stream, h, o, g, w, eps, h_out, q, scale, m);
    } else {
        if (k == 1024) hipLaunchKernelGGL((residual_rms_quant_kernel<2, Recipe::Plain>), grid, block, 0, stream, h, o, g, w, eps, h_out, q, scale, m);
        else if (k == 2048) hipLaunchKernelGGL((residual_rms_quant_kernel<4, Recipe::Plain>), grid, block, 0, stream, h, o, g, w, eps, h_out, q, scale, m);
        else hipLaunchKernelGGL((residual_rms_quant_kernel<8, Recipe::Plain>), grid, block, 0, stream, h, o, g, w, eps, h_out, q, scale, m);
    }
    return launch_status(what);
}

int h3v_residual_norm1_quant(const uint16_t* h, const uint16_t* o, const uint16_t* g, const uint16_t* w, float eps,
                             int64_t m, int64_t k, uint16_t* h_out, int8_t* q, float* scale, hipStream_t stream) {
    return residual_quant_common(h, o, g, w, eps, m, k, h_out, q, scale, stream, true, "h3v_residual_norm1_quant");
}

int h3v_residual_rms_quant(const uint16_t* x, const uint16_t* a, const uint16_t* g, const uint16_t* w, float eps,
                           int64_t m, int64_t k, uint16_t* h_out, int8_t* q, float* scale, hipStream_t stream) {
    return residual_quant_common(x, a, g, w, eps, m, k, h_out, q, scale, stream, false, "h3v_residual_rms_quant");
}

int h3v_rms_fp16(const uint16_t* x, const uint16_t* gamma, float eps, int64_t m, int64_t k, uint16_t* out,
                 hipStream_t stream) {
    const char* what = "h3v_rms_fp16";
    H3V_REQUIRE(x && gamma && out, "%s: null pointer argument", what);
    int rc = check_row_width(what, m, k);
    if (rc) return rc;
    H3V_REQUIRE(aligned(x, 16) && aligned(gamma, 16) && aligned(out, 16), "%s: pointers must be 16-byte aligned", what);
    H3V_REQUIRE(out + m * k <= x || x + m * k <= out, "%s: output must own separate storage", what);
    dim3 grid((unsigned)((m + kRowsPerBlock - 1) / kRowsPerBlock)), block(kNT);
    if (k == 1024) hipLaunchKernelGGL((rms_fp16_kernel<2>), grid, block, 0, stream, x, gamma, eps, out, m);
    else if (k == 2048) hipLaunchKernelGGL((rms_fp16_kernel<4>), grid, block, 0, stream, x, gamma, eps, out, m);
    else hipLaunchKernelGGL((rms_fp16_kernel<8>), grid, block, 0, stream, x, gamma, eps, out, m);
    return launch_status(what);
}

int h3v_residual_layernorm(const uint16_t* h, const uint16_t* o, const uint16_t* gate, const uint16_t* gamma,
                           const uint16_t* beta, float eps, int64_t m, int64_t k, uint16_t* out,
                           hipStream_t stream) {
    const char* what = "h3v_residual_layernorm";
    H3V_REQUIRE(h && o && gate && gamma && beta && out, "%s: null pointer argument", what);
    int rc = check_row_width(what, m, k);
    if (rc) return rc;
    H3V_REQUIRE(aligned(h, 16) && aligned(o, 16) && aligned(gate, 16) && aligned(gamma, 16) && aligned(beta, 16) &&
                    aligned(out, 16),
                "%s: pointers must be 16-byte aligned", what);
    H3V_REQUIRE((out + m * k <= h || h + m * k <= out) && (out + m * k <= o || o + m * k <= out),
                "%s: output must own separate storage", what);
    dim3 grid((unsigned)((m + kRowsPerBlock - 1) / kRowsPerBlock)), block(kNT);
    if (k == 1024) hipLaunchKernelGGL((residual_layernorm_kernel<2>), grid, block, 0, stream, h, o, gate, gamma, beta, eps, out, m);
    else if (k == 2048) hipLaunchKernelGGL((residual_layernorm_kernel<4>), grid, block, 0, stream, h, o, gate, gamma, beta, eps, out, m);
    else hipLaunchKernelGGL((residual_layernorm_kernel<8>), grid, block, 0, stream, h, o, gate, gamma, beta, eps, out, m);
    return launch_status(what);
}

}  // extern "C"
