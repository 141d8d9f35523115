// Decoder row producers: residual + RMSNorm + row quantization (norm1 / norm2),
// the block-0 RMSNorm and the final residual + LayerNorm.
//
// One 256-thread workgroup per row of width K (K/4 a power of two, K <= 4096).
// Reductions follow a fixed tree that does not depend on the wave size: the
// row is split into K/4 "virtual threads" of four consecutive values; each
// forms a partial, partials are combined by a butterfly over groups of 32
// (offsets 16, 8, 4, 2, 1) and the group results by a butterfly over the
// groups.  Virtual thread v lives in real thread v % 256, so the 32-groups map
// onto 32-lane halves of a wave64 and the in-group butterfly is a lane shuffle.
//
// Partial of four values:
//   W16 recipe (norm1, docs/decoder_norm1_contract_2026-10-03.md:57-70):
//       s1 = x1*x1; a = fma(x0,x0,s1); b = fma(x2,x2,a); s3 = x3*x3; p = s3 + b
//   plain recipe: p = ((t0 + t1) + t2) + t3 over already rounded terms.
#include "h3v_common.hpp"
#include "h3v_abi.hpp"

namespace h3v {
namespace {

constexpr int kNT = 256;

enum class Recipe { W16, Plain };

template <int VPT>
struct RowTree {
    // partial of one virtual thread -> in-group butterfly -> group butterfly
    __device__ static float reduce(float (&p)[VPT], float* lds) {
        const int t = threadIdx.x;
#pragma unroll
        for (int j = 0; j < VPT; ++j)
#pragma unroll
            for (int off = 16; off >= 1; off >>= 1) p[j] = p[j] + __shfl_xor(p[j], off, 64);
        // group index of virtual thread t + j*256 is t/32 + j*8
        if ((t & 31) == 0) {
#pragma unroll
            for (int j = 0; j < VPT; ++j) lds[t / 32 + j * (kNT / 32)] = p[j];
        }
        __syncthreads();
        constexpr int NG = VPT * (kNT / 32);
        if (t == 0) {
            for (int off = NG / 2; off >= 1; off >>= 1)
                for (int i = 0; i < off; ++i) lds[i] = lds[i] + lds[i + off];
        }
        __syncthreads();
        float r = lds[0];
        __syncthreads();  // lds may be reused by the caller
        return r;
    }
};

__device__ __forceinline__ float partial_w16(const float* x) {
    float s1 = x[1] * x[1];
    float a = __builtin_fmaf(x[0], x[0], s1);
    float b = __builtin_fmaf(x[2], x[2], a);
    float s3 = x[3] * x[3];
    return s3 + b;
}

__device__ __forceinline__ float partial_plain(const float* t) { return ((t[0] + t[1]) + t[2]) + t[3]; }

__device__ __forceinline__ void load4(const uint16_t* p, float* v) {
    u16x4 a = *reinterpret_cast<const u16x4*>(p);
    v[0] = h2f(a[0]); v[1] = h2f(a[1]); v[2] = h2f(a[2]); v[3] = h2f(a[3]);
}

__device__ __forceinline__ void store4(uint16_t* p, const float* v) {
    u16x4 a = {f2h(v[0]), f2h(v[1]), f2h(v[2]), f2h(v[3])};
    *reinterpret_cast<u16x4*>(p) = a;
}

__device__ __forceinline__ float block_max(float v, float* red) {
    v = wave_max(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float m = red[0];
#pragma unroll
    for (int i = 1; i < kNT / 64; ++i) m = __builtin_fmaxf(m, red[i]);
    return m;
}

// N1 / F1: raw = fma(o, g, h); h_out = fp16(raw); ss = tree(raw^2);
// inv = 1/sqrt(ss/K + eps); n = fp16((fp32(h_out) * inv) * w); row-quantize n.
template <int VPT, Recipe R>
__global__ __launch_bounds__(kNT) void residual_rms_quant_kernel(const uint16_t* h, const uint16_t* __restrict__ o,
                                                                 const uint16_t* __restrict__ g, const uint16_t* __restrict__ w,
                                                                 float eps, uint16_t* h_out, int8_t* __restrict__ q,
                                                                 float* __restrict__ s) {
    constexpr int K = VPT * kNT * 4;
    __shared__ float lds[VPT * (kNT / 32)];
    __shared__ float red[kNT / 64];
    const int64_t row = blockIdx.x;
    const int t = threadIdx.x;
    float raw[VPT][4];
    float part[VPT];
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int col = (t + j * kNT) * 4;
        float hv[4], ov[4], gv[4];
        load4(h + row * K + col, hv);
        load4(o + row * K + col, ov);
        load4(g + col, gv);
#pragma unroll
        for (int e = 0; e < 4; ++e) raw[j][e] = __builtin_fmaf(ov[e], gv[e], hv[e]);
        if constexpr (R == Recipe::W16) {
            part[j] = partial_w16(raw[j]);
        } else {
            float sq[4] = {raw[j][0] * raw[j][0], raw[j][1] * raw[j][1], raw[j][2] * raw[j][2], raw[j][3] * raw[j][3]};
            part[j] = partial_plain(sq);
        }
    }
    const float ss = RowTree<VPT>::reduce(part, lds);
    const float inv = rsqrt_rn(ss / (float)K + eps);
    float nrm[VPT][4];
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int col = (t + j * kNT) * 4;
        float wv[4], hr[4];
        load4(w + col, wv);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            hr[e] = rt16(raw[j][e]);
            nrm[j][e] = rt16((hr[e] * inv) * wv[e]);
            amax = __builtin_fmaxf(amax, __builtin_fabsf(nrm[j][e]));
        }
        store4(h_out + row * K + col, hr);
    }
    amax = block_max(amax, red);
    const float sc = q1_scale(amax);
    const float d = rt16(sc);
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int col = (t + j * kNT) * 4;
        *reinterpret_cast<uint32_t*>(q + row * K + col) =
            pack4(q1_quant(nrm[j][0], d), q1_quant(nrm[j][1], d), q1_quant(nrm[j][2], d), q1_quant(nrm[j][3], d));
    }
    if (t == 0) s[row] = sc;
}

// N3: out = fp16((x * inv) * gamma), inv = 1/sqrt(W16(x^2)/K + eps).
template <int VPT>
__global__ __launch_bounds__(kNT) void rms_fp16_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ gamma,
                                                       float eps, uint16_t* __restrict__ out) {
    constexpr int K = VPT * kNT * 4;
    __shared__ float lds[VPT * (kNT / 32)];
    const int64_t row = blockIdx.x;
    const int t = threadIdx.x;
    float xv[VPT][4], part[VPT];
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        load4(x + row * K + (t + j * kNT) * 4, xv[j]);
        part[j] = partial_w16(xv[j]);
    }
    const float inv = rsqrt_rn(RowTree<VPT>::reduce(part, lds) / (float)K + eps);
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int col = (t + j * kNT) * 4;
        float gv[4], r[4];
        load4(gamma + col, gv);
#pragma unroll
        for (int e = 0; e < 4; ++e) r[e] = (xv[j][e] * inv) * gv[e];
        store4(out + row * K + col, r);
    }
}

// N4: raw = fma(o, gate, h); mean = plain(raw)/K; var = plain((raw-mean)^2)/K;
// y = fp16(fma((raw - mean) * inv, gamma, beta)).
template <int VPT>
__global__ __launch_bounds__(kNT) void residual_layernorm_kernel(const uint16_t* __restrict__ h, const uint16_t* __restrict__ o,
                                                                 const uint16_t* __restrict__ gate, const uint16_t* __restrict__ gamma,
                                                                 const uint16_t* __restrict__ beta, float eps,
                                                                 uint16_t* __restrict__ out) {
    constexpr int K = VPT * kNT * 4;
    __shared__ float lds[VPT * (kNT / 32)];
    const int64_t row = blockIdx.x;
    const int t = threadIdx.x;
    float raw[VPT][4], part[VPT];
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int col = (t + j * kNT) * 4;
        float hv[4], ov[4], gv[4];
        load4(h + row * K + col, hv);
        load4(o + row * K + col, ov);
        load4(gate + col, gv);
#pragma unroll
        for (int e = 0; e < 4; ++e) raw[j][e] = __builtin_fmaf(ov[e], gv[e], hv[e]);
        part[j] = partial_plain(raw[j]);
    }
    const float mean = RowTree<VPT>::reduce(part, lds) / (float)K;
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        float sq[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float dv = raw[j][e] - mean;
            sq[e] = dv * dv;
        }
        part[j] = partial_plain(sq);
    }
    const float inv = rsqrt_rn(RowTree<VPT>::reduce(part, lds) / (float)K + eps);
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int col = (t + j * kNT) * 4;
        float gv[4], bv[4], r[4];
        load4(gamma + col, gv);
        load4(beta + col, bv);
#pragma unroll
        for (int e = 0; e < 4; ++e) r[e] = __builtin_fmaf((raw[j][e] - mean) * inv, gv[e], bv[e]);
        store4(out + row * K + col, r);
    }
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
    H3V_REQUIRE(aligned(h, 8) && aligned(o, 8) && aligned(g, 8) && aligned(w, 8) && aligned(h_out, 8) && aligned(q, 4),
                "%s: pointers must be 8-byte aligned", what);
    H3V_REQUIRE(h_out == h || (h_out + m * k <= o || o + m * k <= h_out),
                "%s: h_out must not overlap o", what);
    dim3 grid((unsigned)m), block(kNT);
    if (w16) {
        if (k == 1024) hipLaunchKernelGGL((residual_rms_quant_kernel<1, Recipe::W16>), grid, block, 0, stream, h, o, g, w, eps, h_out, q, scale);
        else if (k == 2048) hipLaunchKernelGGL((residual_rms_quant_kernel<2, Recipe::W16>), grid, block, 0, stream, h, o, g, w, eps, h_out, q, scale);
        else hipLaunchKernelGGL((residual_rms_quant_kernel<4, Recipe::W16>), grid, block, 0, stream, h, o, g, w, eps, h_out, q, scale);
    } else {
        if (k == 1024) hipLaunchKernelGGL((residual_rms_quant_kernel<1, Recipe::Plain>), grid, block, 0, stream, h, o, g, w, eps, h_out, q, scale);
        else if (k == 2048) hipLaunchKernelGGL((residual_rms_quant_kernel<2, Recipe::Plain>), grid, block, 0, stream, h, o, g, w, eps, h_out, q, scale);
        else hipLaunchKernelGGL((residual_rms_quant_kernel<4, Recipe::Plain>), grid, block, 0, stream, h, o, g, w, eps, h_out, q, scale);
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
    H3V_REQUIRE(aligned(x, 8) && aligned(gamma, 8) && aligned(out, 8), "%s: pointers must be 8-byte aligned", what);
    H3V_REQUIRE(out + m * k <= x || x + m * k <= out, "%s: output must own separate storage", what);
    dim3 grid((unsigned)m), block(kNT);
    if (k == 1024) hipLaunchKernelGGL((rms_fp16_kernel<1>), grid, block, 0, stream, x, gamma, eps, out);
    else if (k == 2048) hipLaunchKernelGGL((rms_fp16_kernel<2>), grid, block, 0, stream, x, gamma, eps, out);
    else hipLaunchKernelGGL((rms_fp16_kernel<4>), grid, block, 0, stream, x, gamma, eps, out);
    return launch_status(what);
}

int h3v_residual_layernorm(const uint16_t* h, const uint16_t* o, const uint16_t* gate, const uint16_t* gamma,
                           const uint16_t* beta, float eps, int64_t m, int64_t k, uint16_t* out,
                           hipStream_t stream) {
    const char* what = "h3v_residual_layernorm";
    H3V_REQUIRE(h && o && gate && gamma && beta && out, "%s: null pointer argument", what);
    int rc = check_row_width(what, m, k);
    if (rc) return rc;
    H3V_REQUIRE(aligned(h, 8) && aligned(o, 8) && aligned(gate, 8) && aligned(gamma, 8) && aligned(beta, 8) &&
                    aligned(out, 8),
                "%s: pointers must be 8-byte aligned", what);
    H3V_REQUIRE((out + m * k <= h || h + m * k <= out) && (out + m * k <= o || o + m * k <= out),
                "%s: output must own separate storage", what);
    dim3 grid((unsigned)m), block(kNT);
    if (k == 1024) hipLaunchKernelGGL((residual_layernorm_kernel<1>), grid, block, 0, stream, h, o, gate, gamma, beta, eps, out);
    else if (k == 2048) hipLaunchKernelGGL((residual_layernorm_kernel<2>), grid, block, 0, stream, h, o, gate, gamma, beta, eps, out);
    else hipLaunchKernelGGL((residual_layernorm_kernel<4>), grid, block, 0, stream, h, o, gate, gamma, beta, eps, out);
    return launch_status(what);
}

}  // extern "C"
