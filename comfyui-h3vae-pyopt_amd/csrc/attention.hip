// Scaled-dot-product attention for head_dim 64 (fp16 in and out, fp32 softmax
// and accumulation), non-causal, no mask: the decoder attention of the H3 VAE
// that the reference hands to the model's `perform_attention` (flash attention
// on NVIDIA) between the fused QK-RMSNorm-RoPE and the INT8 attention-out
// linear (opt/decoder_fused_qk_rope.py:66-74, `FusedQKAttention.forward`).
//
//   O[q, :] = sum_k softmax_k(scale * Q[q, :] . K[k, :]) V[k, :]
//
// q, k, v, o are [batch, tokens, heads, 64] with arbitrary token and head
// strides (in elements; the 64 dims contiguous), so v can be the strided
// slice of the QKV projection and q, k the QK-RoPE outputs, with no copies.
//
// One workgroup = 8 waves = 512 queries of one (batch, head); each wave owns
// two sets of 32 queries.  Keys and values stream in blocks of 64 through LDS:
//
//   S = K . Q^T   v_mfma_f32_32x32x16_f16, A = K rows from LDS, B = the wave's
//                 Q fragments (registers, loaded once).  In the 32 x 32 result
//                 layout lane l holds query l % 32 and keys 8g + 4(l / 32) + e
//                 (g, e = 0..3) of each 32-key half, so a query's 64 keys sit
//                 in lanes l and l ^ 32 (32 each): the row max and sum are
//                 in-lane reductions plus one exchange.
//   online softmax in fp32 (exp2 with the scale folded into log2 e) against a
//                 lazy reference maximum that moves only when a weight would
//                 exceed 2^8; the row sums add the fp16-rounded weights that the
//                 P.V product uses
//   O^T += V^T . P^T   A = V^T rows from LDS (V is written transposed), B = P
//                 in fp16: one v_permlane32_swap per dword pair turns the S
//                 layout into the MFMA's 8 consecutive keys per lane.
//
// LDS: three slots of K [64 keys][64 dims] and V^T [64 dims][64 keys] fp16,
// 128-byte rows whose 16-byte chunks are XOR-swizzled by (row >> 1) & 7, so the
// 16-lane fragment reads hit 16 distinct 4-bank groups.  K and V of block j + 2
// are loaded into registers while block j is computed and stored into their
// slot after the next barrier; waves 4-7 run one phase behind waves 0-3 (see
// the main loop).
#include "h3v_common.hpp"
#include "h3v_abi.hpp"

namespace h3v {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kD = 64;        // head dim
constexpr int kBK = 64;       // keys per block
// 32-query sets per wave: two share every K / V^T fragment read (246 VGPRs, 2 waves per SIMD);
// one set (152 VGPRs, 3 waves per SIMD) measured 5% slower on the H3 shape, 11% on [1, 16384, 16, 64]
constexpr int kQuerySets = 2;
constexpr int kThreads = 256;   // the K / V loading threads (waves 0-3); a workgroup has 8 waves
constexpr float kLazy = 8.0f;   // log2 margin of the lazy softmax maximum (weights stay <= 2^kLazy)
constexpr int kSlots = 3;       // K / V^T blocks resident in LDS (block j in slot j % 3)

struct AttnParams {
    const uint16_t* q;
    const uint16_t* k;
    const uint16_t* v;
    uint16_t* o;
    int64_t q_ts, q_hs, k_ts, k_hs, v_ts, v_hs, o_ts, o_hs;
    int tokens;
    float c;   // scale * log2(e)
};

__device__ __forceinline__ int swz(int row, int chunk) { return chunk ^ ((row >> 1) & 7); }

__device__ __forceinline__ float wave_pair_max(float v) { return __builtin_fmaxf(v, __shfl_xor(v, 32, 64)); }

// two fp32 -> packed fp16 (round to nearest even), one v_cvt_pk_f16_f32
__device__ __forceinline__ uint32_t pack_f16x2(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, f16x2));
}

// QS sets of 32 queries per wave, 8 waves (256 * QS queries per workgroup); every K and V^T
// fragment read from LDS feeds the MFMAs of all QS sets.  Waves 0-3 move each K / V block
// into LDS for all 8 (half the per-query load and transpose work of 4-wave workgroups).
template <int QS>
__global__ __launch_bounds__(2 * kThreads) void fmha_d64(AttnParams p) {
    constexpr int BQ = 256 * QS;
    constexpr int KV = kBK * kD;                                      // elements of one K or V^T block
    __shared__ __attribute__((aligned(16))) uint16_t ks[kSlots * KV];   // [slot][key][dim]
    __shared__ __attribute__((aligned(16))) uint16_t vt[kSlots * KV];   // [slot][dim][key]

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform (scalar)
    const int h = blockIdx.y, b = blockIdx.z;
    const int n = p.tokens;
    const int64_t row0 = (int64_t)b * n;                 // first token row of this batch item
    const int q0 = blockIdx.x * BQ + wave * 32 * QS;   // the wave's first query
    const int hi = lane >> 5;                           // which 8 of a 16-wide k chunk this lane holds
    const bool wave_active = q0 < n;                    // wave-uniform

    // the wave's Q fragments: query q0 + 32 qs + lane % 32, dims 16 kc + 8 hi .. + 7
    half8 qf[QS][4];
#pragma unroll
    for (int qs = 0; qs < QS; ++qs) {
        const int qi = q0 + 32 * qs + (lane & 31);
        const int qr = qi < n ? qi : n - 1;
        const uint16_t* src = p.q + (row0 + qr) * p.q_ts + h * p.q_hs + 8 * hi;
#pragma unroll
        for (int kc = 0; kc < 4; ++kc) qf[qs][kc] = *reinterpret_cast<const half8*>(src + 16 * kc);
    }

    // cooperative K / V block loads.  K: 64 keys x 8 chunks of 8 dims = 512 chunks, two per thread,
    // consecutive threads walking a key row.  V: each thread reads a 4-key x 4-dim block (four
    // 8-byte loads; 16 consecutive threads cover one 128-byte key row) and transposes it in
    // registers, so the V^T rows go to LDS as four 8-byte stores of 4 consecutive keys each.
    u32x4 kreg[2];
    uint32_t vreg[4][2];                                  // [key of the 4][dims 0-1, 2-3]
    const int vdg = tid & 15, vkg = tid >> 4;             // dims 4 vdg .. +3, keys 4 vkg .. +3
    // Per-thread source rows of block 0; a full block adds the uniform kb0 * stride (scalar),
    // only the last, partial block clamps rows past the end to the last token.
    const uint16_t* kbase[2];
    const uint16_t* vbase[4];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int c = tid + kThreads * i;
        kbase[i] = p.k + (row0 + (c >> 3)) * p.k_ts + h * p.k_hs + 8 * (c & 7);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) vbase[i] = p.v + (row0 + 4 * vkg + i) * p.v_ts + h * p.v_hs + 4 * vdg;
    auto load_block = [&](int kb0) {
        if (kb0 + kBK <= n) {
            const int64_t ko = (int64_t)kb0 * p.k_ts, vo = (int64_t)kb0 * p.v_ts;
#pragma unroll
            for (int i = 0; i < 2; ++i) kreg[i] = *reinterpret_cast<const u32x4*>(kbase[i] + ko);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint2 w = *reinterpret_cast<const uint2*>(vbase[i] + vo);
                vreg[i][0] = w.x;
                vreg[i][1] = w.y;
            }
            return;
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int c = tid + kThreads * i;
            const int key = c >> 3, dch = c & 7;
            const int kr = kb0 + key < n ? kb0 + key : n - 1;
            kreg[i] = *reinterpret_cast<const u32x4*>(p.k + (row0 + kr) * p.k_ts + h * p.k_hs + 8 * dch);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int key = 4 * vkg + i;
            const int vr = kb0 + key < n ? kb0 + key : n - 1;
            const uint2 w = *reinterpret_cast<const uint2*>(p.v + (row0 + vr) * p.v_ts + h * p.v_hs + 4 * vdg);
            vreg[i][0] = w.x;
            vreg[i][1] = w.y;
        }
    };
    auto store_block = [&](int slot) {
        uint16_t* const kd = ks + slot * KV;
        uint16_t* const vd = vt + slot * KV;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int c = tid + kThreads * i;
            const int key = c >> 3, dch = c & 7;
            *reinterpret_cast<u32x4*>(kd + key * kD + 8 * swz(key, dch)) = kreg[i];
        }
        // dim j of the 4: keys 0-1 from the low (j even) or high (j odd) halves of vreg[0..1][j >> 1],
        // keys 2-3 likewise from vreg[2..3]; v_perm_b32 picks the two halves into one dword
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
            const uint32_t lo = __builtin_amdgcn_perm(vreg[1][j >> 1], vreg[0][j >> 1], sel);
            const uint32_t hi = __builtin_amdgcn_perm(vreg[3][j >> 1], vreg[2][j >> 1], sel);
            const int d = 4 * vdg + j;
            *reinterpret_cast<uint2*>(vd + d * kBK + 8 * swz(d, vkg >> 1) + 4 * (vkg & 1)) = make_uint2(lo, hi);
        }
    };

    f32x16 oacc[QS][2];
    float m_ref[QS], mc[QS], l_run[QS];
#pragma unroll
    for (int qs = 0; qs < QS; ++qs) {
        oacc[qs][0] = f32x16{};
        oacc[qs][1] = f32x16{};
        m_ref[qs] = -__builtin_inff();
        mc[qs] = -__builtin_inff();
        l_run[qs] = 0.0f;
    }
    const float thr = kLazy / p.c;   // raw-score margin of the lazy maximum

    const int nblk = (n + kBK - 1) / kBK;
    const bool loader = tid < kThreads;                   // waves 0-3 (wave-uniform)

    // S = K . Q^T for the 64 keys of block j (two 32-key halves), each K fragment used by every set;
    // keys past the end (last block only) are -inf
    auto scores = [&](int j, int slot, f32x16 (&s)[QS][2]) {
        const int kb0 = j * kBK;
        const uint16_t* const kb = ks + slot * KV;
#pragma unroll
        for (int kh = 0; kh < 2; ++kh) {
#pragma unroll
            for (int qs = 0; qs < QS; ++qs) s[qs][kh] = f32x16{};
            const int row = 32 * kh + (lane & 31);
#pragma unroll
            for (int kc = 0; kc < 4; ++kc) {
                const half8 a = *reinterpret_cast<const half8*>(kb + row * kD + 8 * swz(row, 2 * kc + hi));
#pragma unroll
                for (int qs = 0; qs < QS; ++qs)
                    s[qs][kh] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qf[qs][kc], s[qs][kh], 0, 0, 0);
            }
        }
        if (kb0 + kBK > n) {
#pragma unroll
            for (int qs = 0; qs < QS; ++qs)
#pragma unroll
                for (int kh = 0; kh < 2; ++kh)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int key = kb0 + 32 * kh + 8 * (r >> 2) + 4 * hi + (r & 3);
                        if (key >= n) s[qs][kh][r] = -__builtin_inff();
                    }
        }
    };
    // online softmax per set in raw-score units (the exponent folds in scale * log2 e), with a lazy
    // reference maximum: the weights are exp2(s * c - m_ref * c), and m_ref moves (rescaling O and l by
    // exp2((m_old - m_ref) * c)) only when a score of the block exceeds it by more than kLazy / c, i.e.
    // when a weight would exceed 2^kLazy.  Every weight stays in [0, 256], where fp16 keeps the same
    // relative precision, and after the first block the 64 rescale multiplies almost never run (with
    // the exact running maximum some lane's maximum moves in nearly every block).  P in fp16.
    auto softmax = [&](const f32x16 (&s)[QS][2], uint32_t (&pk)[QS][2][8]) {
        bool up = false;
        float mblk[QS];
#pragma unroll
        for (int qs = 0; qs < QS; ++qs) {
            float mloc = s[qs][0][0];
#pragma unroll
            for (int kh = 0; kh < 2; ++kh)
#pragma unroll
                for (int r = 0; r < 16; ++r) mloc = __builtin_fmaxf(mloc, s[qs][kh][r]);
            mblk[qs] = wave_pair_max(mloc);
            up |= mblk[qs] > m_ref[qs] + thr;   // m_ref = -inf before the first block: true there
        }
        if (__ballot(up)) {
#pragma unroll
            for (int qs = 0; qs < QS; ++qs) {
                const float m_new = __builtin_fmaxf(m_ref[qs], mblk[qs]);
                const float alpha = __builtin_amdgcn_exp2f((m_ref[qs] - m_new) * p.c);   // 0 from -inf, 1 if unmoved
                m_ref[qs] = m_new;
                mc[qs] = m_new * p.c;
                l_run[qs] *= alpha;
#pragma unroll
                for (int db = 0; db < 2; ++db)
#pragma unroll
                    for (int r = 0; r < 16; ++r) oacc[qs][db][r] *= alpha;
            }
        }
#pragma unroll
        for (int qs = 0; qs < QS; ++qs) {
            float lsum = 0.0f;
#pragma unroll
            for (int kh = 0; kh < 2; ++kh)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    float e4[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        e4[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[qs][kh][4 * g + e], p.c, -mc[qs]));
                    pk[qs][kh][2 * g] = pack_f16x2(e4[0], e4[1]);
                    pk[qs][kh][2 * g + 1] = pack_f16x2(e4[2], e4[3]);
                    // the row sum adds the fp16 weights the P.V product uses, two per v_dot2_f32_f16
                    const f16x2 one = {(_Float16)1.0f, (_Float16)1.0f};
                    lsum = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, pk[qs][kh][2 * g]), one, lsum, false);
                    lsum = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, pk[qs][kh][2 * g + 1]), one, lsum, false);
                }
            l_run[qs] += lsum;
        }
    };
    // O^T += V^T . P^T over four 16-key chunks, each V^T fragment used by every set.  (With both wave
    // groups in one phase a raised issue priority for these MFMAs had paid, 153.7 -> 151.5 us on the H3
    // call; with the groups a phase apart it costs: 146.8 us without it against 149.5 us.)
    auto pv = [&](int slot, const uint32_t (&pk)[QS][2][8]) {
        const uint16_t* const vb = vt + slot * KV;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int kh = c >> 1, g0 = 2 * (c & 1);
            // lane < 32 needs keys 16c + 0..7 (its own group g0 + the partner's), lane >= 32
            // keys 16c + 8..15 (the partner's group g0 + 1 + its own)
            half8 bop[QS];
#pragma unroll
            for (int qs = 0; qs < QS; ++qs) {
                const auto x0 = __builtin_amdgcn_permlane32_swap(pk[qs][kh][2 * g0], pk[qs][kh][2 * g0 + 2], false, false);
                const auto x1 = __builtin_amdgcn_permlane32_swap(pk[qs][kh][2 * g0 + 1], pk[qs][kh][2 * g0 + 3], false,
                                                                 false);
                const u32x4 bw = {x0[0], x1[0], x0[1], x1[1]};
                bop[qs] = __builtin_bit_cast(half8, bw);
            }
#pragma unroll
            for (int db = 0; db < 2; ++db) {
                const int row = 32 * db + (lane & 31);
                const half8 a = *reinterpret_cast<const half8*>(vb + row * kBK + 8 * swz(row, 2 * c + hi));
#pragma unroll
                for (int qs = 0; qs < QS; ++qs)
                    oacc[qs][db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, bop[qs], oacc[qs][db], 0, 0, 0);
            }
        }
    };

    // One barrier per block, three LDS slots.  Waves 0-3 (the loaders) run block j as scores, softmax,
    // P.V after barrier j; waves 4-7 run the P.V of block j - 1 and then the scores and softmax of block
    // j, carrying the packed weights P over the barrier.  On each SIMD one wave's softmax VALU work then
    // runs beside its partner's MFMAs for two of the three phases instead of both waves running the
    // same phase; every query sees the same operations in the same order.  After barrier j the loaders
    // store block j + 1 into slot (j + 1) % 3, which last held block j - 2: its readers finished before
    // barrier j (waves 4-7 read it in their iteration j - 1); block j + 1 is read only after barrier
    // j + 1.  The two groups run separate loops with one barrier per iteration each.
    // The Q fragment loads complete here, once: otherwise the wait counters merged over the loop's back
    // edge keep them pending, and the first score MFMAs of every block wait for that block's K / V loads.
    __builtin_amdgcn_s_waitcnt(0);
    uint32_t pk[QS][2][8];                                // [set][half][g * 2 + dword]
    if (loader) {
        load_block(0);
        store_block(0);
        if (nblk > 1) load_block(kBK);
        int slot = 0;                                     // slot of block j
        for (int j = 0; j < nblk; ++j) {
            __syncthreads();                              // block j stored; blocks before j - 1 no longer read
            const int nslot = slot == kSlots - 1 ? 0 : slot + 1;
            if (j + 1 < nblk) {
                store_block(nslot);
                if (j + 2 < nblk) load_block((j + 2) * kBK);   // block j + 2 in flight during this one
            }
            // a wave whose 32 queries all lie past the end (the last workgroup of a head) only helps
            // with the shared K / V loads and barriers
            if (wave_active) {
                f32x16 s[QS][2];
                scores(j, slot, s);
                softmax(s, pk);
                pv(slot, pk);
            }
            slot = nslot;
        }
    } else {
        int slot = 0, pslot = 0;                          // slots of blocks j and j - 1
        for (int j = 0; j < nblk; ++j) {
            __syncthreads();
            if (wave_active) {
                if (j > 0) pv(pslot, pk);
                f32x16 s[QS][2];
                scores(j, slot, s);
                softmax(s, pk);
            }
            pslot = slot;
            slot = slot == kSlots - 1 ? 0 : slot + 1;
        }
        if (wave_active) pv(pslot, pk);                   // the last block (no store follows it)
    }

    // normalise and store: lane l holds query q0 + 32 qs + l % 32, dims 32 db + 8 g + 4 hi + e
#pragma unroll
    for (int qs = 0; qs < QS; ++qs) {
        const int qi = q0 + 32 * qs + (lane & 31);
        const float l_tot = l_run[qs] + __shfl_xor(l_run[qs], 32, 64);
        const float inv = 1.0f / l_tot;
        if (qi < n) {
            uint16_t* dst = p.o + (row0 + qi) * p.o_ts + h * p.o_hs + 4 * hi;
#pragma unroll
            for (int db = 0; db < 2; ++db)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    u16x4 v;
#pragma unroll
                    for (int e = 0; e < 4; ++e) v[e] = f2h(oacc[qs][db][4 * g + e] * inv);
                    *reinterpret_cast<u16x4*>(dst + 32 * db + 8 * g) = v;
                }
        }
    }
}

}  // namespace
}  // namespace h3v

using namespace h3v;

extern "C" int h3v_attention_d64(const uint16_t* q, int64_t q_token_stride, int64_t q_head_stride, const uint16_t* k,
                                 int64_t k_token_stride, int64_t k_head_stride, const uint16_t* v,
                                 int64_t v_token_stride, int64_t v_head_stride, uint16_t* o, int64_t o_token_stride,
                                 int64_t o_head_stride, int64_t batch, int64_t tokens, int64_t heads, float scale,
                                 hipStream_t stream) {
    const char* what = "h3v_attention_d64";
    H3V_REQUIRE(q && k && v && o, "%s: null pointer argument", what);
    H3V_REQUIRE(batch > 0 && tokens > 0 && heads > 0, "%s: batch, tokens and heads must be positive", what);
    H3V_REQUIRE(batch <= 65535 && heads <= 65535 && tokens <= (1 << 24), "%s: shape out of range", what);
    H3V_REQUIRE(scale > 0.0f && scale < 1e30f, "%s: scale must be positive and finite", what);
    const int64_t strides[8] = {q_token_stride, q_head_stride, k_token_stride, k_head_stride,
                                v_token_stride, v_head_stride, o_token_stride, o_head_stride};
    for (int i = 0; i < 8; ++i)
        H3V_REQUIRE(strides[i] > 0 && strides[i] % 8 == 0, "%s: token/head strides must be positive multiples of 8 "
                    "elements (16-byte rows)", what);
    H3V_REQUIRE(aligned(q, 16) && aligned(k, 16) && aligned(v, 16) && aligned(o, 8),
                "%s: q, k, v must be 16-byte and o 8-byte aligned", what);
    AttnParams p;
    p.q = q; p.k = k; p.v = v; p.o = o;
    p.q_ts = q_token_stride; p.q_hs = q_head_stride;
    p.k_ts = k_token_stride; p.k_hs = k_head_stride;
    p.v_ts = v_token_stride; p.v_hs = v_head_stride;
    p.o_ts = o_token_stride; p.o_hs = o_head_stride;
    p.tokens = (int)tokens;
    p.c = scale * 1.4426950408889634f;
    constexpr int QS = kQuerySets;
    dim3 grid((unsigned)((tokens + 256 * QS - 1) / (256 * QS)), (unsigned)heads, (unsigned)batch);
    hipLaunchKernelGGL(fmha_d64<QS>, grid, dim3(2 * kThreads), 0, stream, p);
    return launch_status(what);
}
