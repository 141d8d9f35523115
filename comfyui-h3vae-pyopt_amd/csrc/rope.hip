// Fused QK RMSNorm + partial rotate-half RoPE (opt/decoder_fused_qk_rope.py:12-35).
//
// qkv: fp16 [tokens, heads, 3*DH] with the per-head layout [q | k | v];
// cos/sin: fp16 [tokens, ROT] shared by all heads.  Output q, k: fp16
// [tokens, heads, DH].  DH = 64, ROT = 48 (the rotated prefix); dims >= ROT
// pass through after the norm.
//
// 8 lanes own one (token, head) row of 64 dims, 8 consecutive dims per lane,
// so a wave64 handles 8 rows and every load/store is a 16-byte vector.  The sum
// of squares is formed per "virtual thread" of 4 dims as ((t0+t1)+t2)+t3 and
// combined by a butterfly over the 16 virtual threads (offsets 8, 4, 2, 1);
// lane li holds virtual threads 2li and 2li+1, so offsets 8, 4, 2 are lane XORs
// 4, 2, 1 and offset 1 is a local add.  The rotate-half partner of dim d
// (+-ROT/2 = 24) sits in lane +-3 at the same position, fetched with a shuffle.
#include "h3v_common.hpp"
#include "h3v_abi.hpp"

namespace h3v {
namespace {

constexpr int kDH = 64;
constexpr int kROT = 48;
constexpr int kNT = 256;
constexpr int kLanesPerRow = 8;

// One (token, head) row of q or k held by 8 lanes: RMS normalisation, then the rotate-half RoPE on the
// first ROT dims.  Every product of the rotation multiplies two fp16 values; their fp32 product is exact
// (11-bit significands), so rounding it to fp16 is the IEEE fp16 product, and the products run as packed
// fp16 multiplies (two per instruction) on the normalised row kept as fp16 pairs.  The reference chain
// adds the two rounded products in fp32 and rounds the sum to fp16; for fp16 operands that is the IEEE
// fp16 sum (fp32 carries more than 2 * 11 + 2 significand bits), so the sum is a packed fp16 add too.
__device__ __forceinline__ u16x8 norm_rope(const u16x8& in, float eps, int li, const f16x2 (&c2)[4],
                                           const f16x2 (&s2)[4]) {
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = h2f(in[e]);
    float p0 = ((v[0] * v[0] + v[1] * v[1]) + v[2] * v[2]) + v[3] * v[3];
    float p1 = ((v[4] * v[4] + v[5] * v[5]) + v[6] * v[6]) + v[7] * v[7];
#pragma unroll
    for (int off = 4; off >= 1; off >>= 1) {
        p0 = p0 + __shfl_xor(p0, off, kLanesPerRow);
        p1 = p1 + __shfl_xor(p1, off, kLanesPerRow);
    }
    const float part = p0 + p1;
    const float inv = rsqrt_rn(part / (float)kDH + eps);
    // normalised row, fp16 pairs (v_cvt_pk_f16_f32 rounds each to nearest even, as fp16(x) does)
    uint32_t n2[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
        n2[j] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){v[2 * j] * inv, v[2 * j + 1] * inv}, f16x2));
    // rotate-half partner over the first ROT dims: li < 3 -> li + 3, 3 <= li < 6 -> li - 3
    const int lane = threadIdx.x & 63;
    const int base = lane & ~(kLanesPerRow - 1);
    const int partner = li < 3 ? li + 3 : (li < 6 ? li - 3 : li);
    uint32_t r2[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) r2[j] = (uint32_t)__shfl((int)n2[j], base + partner, 64);
    u16x8 out;
    if (li < kROT / 8) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const f16x2 a = __builtin_bit_cast(f16x2, n2[j]) * c2[j];   // fp16(n * cos)
            const f16x2 b = __builtin_bit_cast(f16x2, r2[j]) * s2[j];   // fp16(+-partner * sin)
            // the pair is bit-cast whole: clang's __builtin_bit_cast of one element of an ext_vector reads
            // element 0 whatever the index
            const uint32_t y = __builtin_bit_cast(uint32_t, a + b);
            out[2 * j] = (uint16_t)(y & 0xffffu);
            out[2 * j + 1] = (uint16_t)(y >> 16);
        }
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            out[2 * j] = (uint16_t)(n2[j] & 0xffffu);
            out[2 * j + 1] = (uint16_t)(n2[j] >> 16);
        }
    }
    return out;
}

__global__ __launch_bounds__(kNT) void qk_rope_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ cosv,
                                                      const uint16_t* __restrict__ sinv, int64_t rows, int heads,
                                                      float eps, uint16_t* __restrict__ qo, uint16_t* __restrict__ ko) {
    const int64_t row = (int64_t)blockIdx.x * (kNT / kLanesPerRow) + (threadIdx.x / kLanesPerRow);   // (token, head)
    const int li = threadIdx.x & (kLanesPerRow - 1);
    const bool valid = row < rows;
    const int64_t r = valid ? row : rows - 1;   // keep every lane in the shuffles
    const int64_t token = r / heads;
    const uint16_t* src = x + r * (3 * kDH) + li * 8;
    const u16x8 a = *reinterpret_cast<const u16x8*>(src);
    const u16x8 b = *reinterpret_cast<const u16x8*>(src + kDH);
    // cos and the signed sin of the lane's 8 dims as fp16 pairs: the rotate-half term is -partner * sin for
    // the first ROT/2 dims and +partner * sin for the next ROT/2 (the sign flip is exact)
    f16x2 c2[4], s2[4];
    if (li < kROT / 8) {
        const u16x8 cc = *reinterpret_cast<const u16x8*>(cosv + token * kROT + li * 8);
        u16x8 ss = *reinterpret_cast<const u16x8*>(sinv + token * kROT + li * 8);
        if (li < kROT / 16) {
#pragma unroll
            for (int e = 0; e < 8; ++e) ss[e] ^= 0x8000u;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            c2[j] = __builtin_bit_cast(f16x2, (uint32_t)cc[2 * j] | ((uint32_t)cc[2 * j + 1] << 16));
            s2[j] = __builtin_bit_cast(f16x2, (uint32_t)ss[2 * j] | ((uint32_t)ss[2 * j + 1] << 16));
        }
    }
    const u16x8 oq = norm_rope(a, eps, li, c2, s2);
    const u16x8 ok = norm_rope(b, eps, li, c2, s2);
    if (valid) {
        *reinterpret_cast<u16x8*>(qo + r * kDH + li * 8) = oq;
        *reinterpret_cast<u16x8*>(ko + r * kDH + li * 8) = ok;
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
    H3V_REQUIRE(aligned(qkv, 16) && aligned(cosv, 16) && aligned(sinv, 16) && aligned(q, 16) && aligned(k, 16),
                "%s: pointers must be 16-byte aligned", what);
    const int64_t rows = tokens * heads;
    const int64_t blocks = (rows + kNT / kLanesPerRow - 1) / (kNT / kLanesPerRow);
    H3V_REQUIRE(blocks <= 0x7fffffff, "%s: too many rows", what);
    hipLaunchKernelGGL(qk_rope_kernel, dim3((unsigned)blocks), dim3(kNT), 0, stream, qkv, cosv, sinv, rows, heads, eps,
                       q, k);
    return launch_status(what);
}

}  // extern "C"
