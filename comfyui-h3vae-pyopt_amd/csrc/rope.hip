// Fused QK RMSNorm + partial rotate-half RoPE (opt/decoder_fused_qk_rope.py:12-35).
//
// qkv: fp16 [tokens, heads, 3*DH] with the per-head layout [q | k | v];
// cos/sin: fp16 [tokens, ROT] shared by all heads.  Output q, k: fp16
// [tokens, heads, DH].  DH = 64, ROT = 48 (the rotated prefix); dims >= ROT
// pass through after the norm.
//
// 16 lanes own one (token, head) row of 64 dims, 4 consecutive dims per lane,
// so a wave64 handles 4 rows and every load/store is an 8-byte vector.  The sum
// of squares is ((t0+t1)+t2)+t3 per lane followed by a butterfly over the 16
// lanes (offsets 8, 4, 2, 1).  The rotate-half partner of dim d (+-ROT/2 = 24)
// sits in lane +-6 at the same position, fetched with a lane shuffle.
#include "h3v_common.hpp"
#include "h3v_abi.hpp"

namespace h3v {
namespace {

constexpr int kDH = 64;
constexpr int kROT = 48;
constexpr int kNT = 256;

__device__ __forceinline__ void norm_rope(float (&v)[4], float eps, int li, const float (&c)[4], const float (&s)[4]) {
    float part = ((v[0] * v[0] + v[1] * v[1]) + v[2] * v[2]) + v[3] * v[3];
#pragma unroll
    for (int off = 8; off >= 1; off >>= 1) part = part + __shfl_xor(part, off, 16);
    const float inv = rsqrt_rn(part / (float)kDH + eps);
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = rt16(v[e] * inv);
    // partner lane for rotate-half over the first ROT dims: li<6 -> li+6, 6<=li<12 -> li-6
    const int lane = threadIdx.x & 63;
    const int base = lane & ~15;
    const int partner = li < 6 ? li + 6 : (li < 12 ? li - 6 : li);
    float r[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) r[e] = __shfl(v[e], base + partner, 64);
    if (li < kROT / 4) {
        const float sign = li < kROT / 8 ? -1.0f : 1.0f;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = rt16(v[e] * c[e]) + rt16((r[e] * sign) * s[e]);
    }
}

__global__ __launch_bounds__(kNT) void qk_rope_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ cosv,
                                                      const uint16_t* __restrict__ sinv, int64_t rows, int heads,
                                                      float eps, uint16_t* __restrict__ qo, uint16_t* __restrict__ ko) {
    const int64_t row = (int64_t)blockIdx.x * (kNT / 16) + (threadIdx.x >> 4);   // (token, head)
    const int li = threadIdx.x & 15;
    const bool valid = row < rows;
    const int64_t r = valid ? row : rows - 1;   // keep every lane in the shuffles
    const int64_t token = r / heads;
    const uint16_t* src = x + r * (3 * kDH) + li * 4;
    float q[4], k[4], c[4] = {1.f, 1.f, 1.f, 1.f}, s[4] = {0.f, 0.f, 0.f, 0.f};
    u16x4 a = *reinterpret_cast<const u16x4*>(src);
    u16x4 b = *reinterpret_cast<const u16x4*>(src + kDH);
#pragma unroll
    for (int e = 0; e < 4; ++e) { q[e] = h2f(a[e]); k[e] = h2f(b[e]); }
    if (li < kROT / 4) {
        u16x4 cc = *reinterpret_cast<const u16x4*>(cosv + token * kROT + li * 4);
        u16x4 ss = *reinterpret_cast<const u16x4*>(sinv + token * kROT + li * 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) { c[e] = h2f(cc[e]); s[e] = h2f(ss[e]); }
    }
    norm_rope(q, eps, li, c, s);
    norm_rope(k, eps, li, c, s);
    if (valid) {
        u16x4 oq = {f2h(q[0]), f2h(q[1]), f2h(q[2]), f2h(q[3])};
        u16x4 ok = {f2h(k[0]), f2h(k[1]), f2h(k[2]), f2h(k[3])};
        *reinterpret_cast<u16x4*>(qo + r * kDH + li * 4) = oq;
        *reinterpret_cast<u16x4*>(ko + r * kDH + li * 4) = ok;
    }
}

}  // namespace
}  // namespace h3v

using namespace h3v;

extern "C" {

int h3v_qk_rope(const uint16_t* qkv, const uint16_t* cosv, const uint16_t* sinv, int64_t tokens, int heads,
                int head_dim, int rot_dim, float eps, uint16_t* q, uint16_t* k, hipStream_t stream) {
    const char* what = "h3v_qk_rope";
    H3V_REQUIRE(qkv && cosv && sinv && q && k, "%s: null pointer argument", what);
    H3V_REQUIRE(head_dim == kDH && rot_dim == kROT, "%s: only head_dim 64 with a 48-dim rotary prefix is supported", what);
    H3V_REQUIRE(tokens > 0 && heads > 0, "%s: tokens and heads must be positive", what);
    H3V_REQUIRE(aligned(qkv, 8) && aligned(cosv, 8) && aligned(sinv, 8) && aligned(q, 8) && aligned(k, 8),
                "%s: pointers must be 8-byte aligned", what);
    const int64_t rows = tokens * heads;
    const int64_t blocks = (rows + kNT / 16 - 1) / (kNT / 16);
    H3V_REQUIRE(blocks <= 0x7fffffff, "%s: too many rows", what);
    hipLaunchKernelGGL(qk_rope_kernel, dim3((unsigned)blocks), dim3(kNT), 0, stream, qkv, cosv, sinv, rows, heads, eps,
                       q, k);
    return launch_status(what);
}

}  // extern "C"
