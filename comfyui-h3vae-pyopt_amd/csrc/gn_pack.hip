// Encoder INT8 producer: per-frame GroupNorm(32) statistics, then a norm /
// SiLU / causal + reflect pad recompute that writes padded INT8 directly
// (opt/encoder_int8_norm.py:16-110, opt/encoder_fused_temporal_norm.py:12-51,
// opt/encoder_fused_norm_bias.py:14-39, opt/encoder_int8_norm_recompute.py:11-48).
//
// x: fp16 NDHWC [D, H, W, C] (batch one, C in {128, 256}).  Output q: int8 NDHWC
// [D+2, H+2, W+2, C], frames 0 and 1 zero, spatial reflect padding of 1.
//
// Launch sequence (all on the caller's stream, no host synchronisation, no atomic
// counters to clear beforehand):
//   gn_partial    grid (chunks, D): per 256-pixel chunk and group, avg and M2;
//                 per chunk and channel max and min of the (pre-biased) input
//                 (fp16, exact).  Skipped by h3v_gn_norm_pack_i8_partials, whose
//                 caller's conv already wrote the same three arrays: the window
//                 conv (h3v_conv3d_i8_gn) for its 512-pixel output tiles, or the
//                 FP16 implicit-GEMM conv (h3v_conv3d_f16_gn) for 256-pixel
//                 chunks in this pass's own order
//   gn_merge      grid (32, D): Chan merge of the chunks -> (mean, rstd); the
//                 per-channel extremes over the chunks give the group's absmax
//                 candidate (below), one word per (frame, group); block (0, 0)
//                 also zeroes the two counters of absmax_lut
//   absmax_lut    reduces the candidates, then builds the int8 code of every
//                 fp16 pre-activation z under the final scale; when the candidate
//                 cannot be proven exact it first runs the full absmax pass and
//                 the last block to finish builds the table
//   norm_pack_lut every padded value -> int8 through that table; writes the scale
//
// Quantize table.  After the normalisation rounds z to fp16, the rest of the
// chain (SiLU, fp16 rounding, division by the tensor scale, half-away
// rounding, clamp) is a fixed function of z's 16-bit code for one call, so it
// is evaluated once per code (65536 entries, 64 KB) and each block looks the
// codes up from LDS: no exp and no division per element.  Every entry is the
// same scalar code path as the direct evaluation, so the output is bitwise
// identical (NaN codes included).
//
// Absmax shortcut.  z = fp16(((v - mean) * rstd) * gamma + beta) is monotone in
// v for each channel (every rounding step is monotone; the direction is the
// sign of gamma), so the largest z of a (frame, channel) is z(vmax) or z(vmin)
// exactly.  SiLU is increasing for z above its minimum (|SiLU| <= 0.2785 below
// z = 0.43), so if the largest fp16(SiLU(zmax)) over all (frame, channel) is at
// least 0.5, it is the absmax of the whole padded tensor and the full pass
// exits at once; otherwise the full pass runs.  The result is bitwise the same.
//
// Fixed reduction order (shared with the CPU oracle): a chunk has PL = 256/(C/8)
// pixel lanes; lane pl owns pixels pl, pl+PL, ...; per pixel the group's
// channels are summed left to right and added to the lane's running sum; the
// lanes combine by the halving tree off = PL/2 .. 1; chunks merge sequentially.
// The window conv's epilogue partials follow their own fixed order (32 pixel
// lanes of a 512-pixel tile, adjacent-pair tree), also restated by the oracle;
// the FP16 implicit-GEMM conv's (h3v_conv3d_f16_gn) follow this pass's order on
// 256-pixel chunks, so its partials are this pass's bit for bit.
#include "h3v_common.hpp"
#include "h3v_abi.hpp"

#include <mutex>

// ---------------------------------------------------------------------------
// Static scratch of h3v_gn_norm_pack_i8_noalloc, for callers that cannot
// allocate device memory.  Each GPU holds its own copy of this array for the
// life of the process (8 MiB + 256 bytes): 64 head floats (word 0 is the absmax
// key) then the workspace, which covers every [D, H, W] whose
// workspace_floats() fits (at 256 x 256 frames up to D = 25).  Every call on a
// GPU reuses that GPU's copy; every word a call reads was written earlier in
// the same call, so nothing carries over, but calls that overlap on one GPU (two streams, two threads)
// race on it.  The name `scratch` is a host-side stand-in: host code uses only
// the device address hipGetSymbolAddress returns, looked up once per device.
constexpr int64_t kScratchHeadFloats = 64;
constexpr int64_t kScratchWorkspaceFloats = (int64_t)1 << 21;
static __device__ __align__(256) float scratch[kScratchHeadFloats + kScratchWorkspaceFloats];

namespace h3v {
namespace {

constexpr int kGroups = 32;
constexpr int kChunk = 256;
constexpr int kNT = 256;
constexpr int kMaxC = 256;
constexpr float kShortcutFloor = 0.5f;

__device__ __forceinline__ void load8(const uint16_t* p, float* v) {
    u16x8 a = *reinterpret_cast<const u16x8*>(p);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = h2f(a[e]);
}

// C channels, cg = C/32 channels per group, TPP = C/8 threads per pixel.
template <int C, bool PRE_BIAS>
__global__ __launch_bounds__(kNT) void gn_partial(const uint16_t* __restrict__ x, const uint16_t* __restrict__ pre_bias,
                                                  int hw, int nchunk, float* __restrict__ part_avg,
                                                  float* __restrict__ part_m2, uint32_t* __restrict__ ext) {
    constexpr int CG = C / kGroups;
    constexpr int TPP = C / 8;
    constexpr int PL = kNT / TPP;
    constexpr int STEPS = kChunk / PL;
    constexpr int GPT = 8 / CG;                 // groups inside one thread's 8 channels
    __shared__ float red[PL][kGroups];
    __shared__ float avg_s[kGroups];
    __shared__ float mx_s[PL][C];
    __shared__ float mn_s[PL][C];

    const int j = blockIdx.x, t = blockIdx.y;
    const int tid = threadIdx.x;
    const int cv = tid % TPP, pl = tid / TPP;
    const int p0 = j * kChunk;
    const int npix = hw - p0 < kChunk ? hw - p0 : kChunk;
    const uint16_t* base = x + ((int64_t)t * hw + p0) * C + cv * 8;

    u16x8 pb{};
    if constexpr (PRE_BIAS) pb = *reinterpret_cast<const u16x8*>(pre_bias + cv * 8);
    // The thread's whole slice of the chunk stays in registers for both passes:
    // every load is issued up front and the data is read from memory once.  The
    // first pass replaces it by the pre-biased fp16 values.
    u16x8 xr[STEPS];
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
        const int p = pl + s * PL;
        if (p < npix) xr[s] = load_nt(base + (int64_t)p * C);
    }
    auto load = [&](int s, float* v) {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = h2f(xr[s][e]);
    };

    float ls[GPT], vmx[8], vmn[8];
#pragma unroll
    for (int gi = 0; gi < GPT; ++gi) ls[gi] = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) { vmx[e] = -__builtin_inff(); vmn[e] = __builtin_inff(); }
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
        int p = pl + s * PL;
        if (p >= npix) break;
        if constexpr (PRE_BIAS) xr[s] = add_f16x8(xr[s], pb);   // fp16(x + b), one rounding
        float v[8];
        load(s, v);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            vmx[e] = __builtin_fmaxf(vmx[e], v[e]);
            vmn[e] = __builtin_fminf(vmn[e], v[e]);
        }
#pragma unroll
        for (int gi = 0; gi < GPT; ++gi) {
            float ps = v[gi * CG];
#pragma unroll
            for (int i = 1; i < CG; ++i) ps = ps + v[gi * CG + i];
            ls[gi] = ls[gi] + ps;
        }
    }
#pragma unroll
    for (int gi = 0; gi < GPT; ++gi) red[pl][cv * GPT + gi] = ls[gi];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        mx_s[pl][cv * 8 + e] = vmx[e];
        mn_s[pl][cv * 8 + e] = vmn[e];
    }
    __syncthreads();
    if (tid < kGroups) {
        for (int off = PL / 2; off >= 1; off >>= 1)
            for (int i = 0; i < off; ++i) red[i][tid] = red[i][tid] + red[i + off][tid];
        avg_s[tid] = red[0][tid] / (float)(npix * CG);
    }
    if (tid < C) {
        float a = mx_s[0][tid], b = mn_s[0][tid];
        for (int i = 1; i < PL; ++i) {
            a = __builtin_fmaxf(a, mx_s[i][tid]);
            b = __builtin_fminf(b, mn_s[i][tid]);
        }
        // the extremes are input values (fp16, or fp16-rounded with the pre-bias): exact as fp16
        ext[((int64_t)t * nchunk + j) * C + tid] = (uint32_t)f2h(a) | ((uint32_t)f2h(b) << 16);
    }
    __syncthreads();

    float a[GPT], lm[GPT];
#pragma unroll
    for (int gi = 0; gi < GPT; ++gi) { a[gi] = avg_s[cv * GPT + gi]; lm[gi] = 0.0f; }
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
        int p = pl + s * PL;
        if (p >= npix) break;
        float v[8];
        load(s, v);
#pragma unroll
        for (int gi = 0; gi < GPT; ++gi) {
            float dv = v[gi * CG] - a[gi];
            float pm = dv * dv;
#pragma unroll
            for (int i = 1; i < CG; ++i) {
                dv = v[gi * CG + i] - a[gi];
                pm = pm + dv * dv;
            }
            lm[gi] = lm[gi] + pm;
        }
    }
    __syncthreads();
#pragma unroll
    for (int gi = 0; gi < GPT; ++gi) red[pl][cv * GPT + gi] = lm[gi];
    __syncthreads();
    if (tid < kGroups) {
        for (int off = PL / 2; off >= 1; off >>= 1)
            for (int i = 0; i < off; ++i) red[i][tid] = red[i][tid] + red[i + off][tid];
        // group-major [frame][group][chunk]: each merge reads one contiguous run
        int64_t dst = ((int64_t)t * kGroups + tid) * nchunk + j;
        part_avg[dst] = avg_s[tid];
        part_m2[dst] = red[0][tid];
    }
}

// One wave per (group, frame).  lane 0 merges the group's chunk partials
// sequentially as in _merge; the lanes of the group's channels then form the
// absmax candidates.  Up to kMergeRegs * 64 chunks the partials are read once,
// into registers, for both sums; more go through LDS in batches of kMergeBatch.
constexpr int kMergeRegs = 4;
constexpr int kMergeBatch = 1024;

// LDS hand-off between the lanes of a one-wave workgroup: waits for the LDS
// accesses only (__syncthreads() would also wait for loads still in flight).
__device__ __forceinline__ void wave_lds_sync() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Chan merge of one group's chunk partials (chunks of `chunk` pixels, the last
// one short) by one wave: the terms of both sums are formed by all lanes and
// lane 0 adds them in chunk order, so the result is the sequential merge of
// _merge.  `issue_loads()` runs right after the partials' loads are issued, so
// that loads it issues stay in flight during the sums.  ms[0] = mean,
// ms[1] = rstd on return (after a barrier).
template <typename F>
__device__ void gn_merge_group(const float* __restrict__ pa, const float* __restrict__ pm, int hw, int nchunk,
                               int chunk, int cg, float eps, float* sa, float* sm, float* ms, F&& issue_loads) {
    const int tid = threadIdx.x;
    const float total = (float)(hw * cg);
    auto weight = [&](int jj) { return (float)((hw - jj * chunk < chunk ? hw - jj * chunk : chunk) * cg); };
    float san = 0.0f, sv = 0.0f;
    if (nchunk <= 64 * kMergeRegs) {
        // unconditional loads (an index past the last chunk re-reads it, and that value is not used), so
        // that no branch separates them and the waits before the sums leave `issue_loads`' loads in flight
        float a[kMergeRegs], m[kMergeRegs];
#pragma unroll
        for (int r = 0; r < kMergeRegs; ++r) {
            const int jj = min(tid + 64 * r, nchunk - 1);
            a[r] = pa[jj];
            m[r] = pm[jj];
        }
        issue_loads();
        // pass 1: mean = (sum_j avg_j * n_j) / N
#pragma unroll
        for (int r = 0; r < kMergeRegs; ++r) {
            const int jj = tid + 64 * r;
            if (jj < nchunk) sa[jj] = a[r] * weight(jj);
        }
        wave_lds_sync();
        if (tid == 0) {
#pragma unroll 16
            for (int j = 0; j < nchunk; ++j) san = san + sa[j];
            ms[0] = san / total;
        }
        wave_lds_sync();
        const float mean = ms[0];
        // pass 2: var = (sum_j (m2_j + (n_j * d_j) * d_j)) / N
#pragma unroll
        for (int r = 0; r < kMergeRegs; ++r) {
            const int jj = tid + 64 * r;
            if (jj < nchunk) {
                const float dl = a[r] - mean;
                sm[jj] = m[r] + (weight(jj) * dl) * dl;
            }
        }
        wave_lds_sync();
        if (tid == 0) {
#pragma unroll 16
            for (int j = 0; j < nchunk; ++j) sv = sv + sm[j];
        }
    } else {
        issue_loads();
        for (int j0 = 0; j0 < nchunk; j0 += kMergeBatch) {
            const int nb = nchunk - j0 < kMergeBatch ? nchunk - j0 : kMergeBatch;
            wave_lds_sync();
            for (int i = tid; i < nb; i += 64) sa[i] = pa[j0 + i] * weight(j0 + i);
            wave_lds_sync();
            if (tid == 0) {
#pragma unroll 16
                for (int j = 0; j < nb; ++j) san = san + sa[j];
            }
        }
        if (tid == 0) ms[0] = san / total;
        wave_lds_sync();
        const float mean = ms[0];
        for (int j0 = 0; j0 < nchunk; j0 += kMergeBatch) {
            const int nb = nchunk - j0 < kMergeBatch ? nchunk - j0 : kMergeBatch;
            wave_lds_sync();
            for (int i = tid; i < nb; i += 64) {
                const float dl = pa[j0 + i] - mean;
                sm[i] = pm[j0 + i] + (weight(j0 + i) * dl) * dl;
            }
            wave_lds_sync();
            if (tid == 0) {
#pragma unroll 16
                for (int j = 0; j < nb; ++j) sv = sv + sm[j];
            }
        }
    }
    if (tid == 0) {
        float var = sv / total;
        if (var < 0.0f) var = 0.0f;
        ms[1] = rsqrt_rn(var + eps);
    }
    wave_lds_sync();
}

__global__ __launch_bounds__(64) void gn_merge(const float* __restrict__ part_avg, const float* __restrict__ part_m2,
                                               const uint32_t* __restrict__ ext,
                                               const uint16_t* __restrict__ gamma, const uint16_t* __restrict__ beta,
                                               int hw, int nchunk, int chunk, int c, float eps,
                                               float* __restrict__ stats, uint32_t* __restrict__ cands,
                                               uint32_t* __restrict__ done) {
    __shared__ float sa[kMergeBatch];
    __shared__ float sm[kMergeBatch];
    __shared__ float ms[2];
    const int g = blockIdx.x, t = blockIdx.y, tid = threadIdx.x;
    if (g == 0 && t == 0 && tid == 0) {   // absmax_lut's counters (it runs after this kernel)
        done[0] = 0u;
        done[1] = 0u;
    }
    const int cg = c / kGroups;
    const float* pa = part_avg + ((int64_t)t * kGroups + g) * nchunk;
    const float* pm = part_m2 + ((int64_t)t * kGroups + g) * nchunk;

    // absmax candidate: fp16(silu(zmax)) per channel, zmax from the monotone map of the channel's
    // extreme over all chunks.  Lane l takes channel l % cg and every (64 / cg)-th chunk from l / cg,
    // so all of the group's extreme loads are in flight at once (issued with the merge's own loads and
    // read after the merge); lanes of one channel then combine by shuffles, and the cg candidates are
    // evaluated in parallel lanes.  Max and min are exact in any order, so the candidate is the same as
    // any other reduction order gives.
    const int lpc = 64 / cg;                                  // lanes per channel (cg = 4 or 8)
    const int e = tid % cg;
    const int ch = g * cg + e;
    const uint32_t* ep = ext + (int64_t)t * nchunk * c + ch;
    constexpr int kExtRegs = 64 * kMergeRegs / 8;             // chunks per lane at cg = 8
    const bool held = nchunk <= 64 * kMergeRegs;
    uint32_t ek[kExtRegs];
    gn_merge_group(pa, pm, hw, nchunk, chunk, cg, eps, sa, sm, ms, [&] {
        if (held) {
#pragma unroll
            for (int r = 0; r < kExtRegs; ++r)   // a clamped index re-reads the last chunk: max / min unchanged
                ek[r] = ep[(int64_t)min(tid / cg + r * lpc, nchunk - 1) * c];
        }
    });
    if (tid == 0) {
        stats[(t * kGroups + g) * 2] = ms[0];
        stats[(t * kGroups + g) * 2 + 1] = ms[1];
    }
    const float mean = ms[0], rstd = ms[1];
    float vmx = -__builtin_inff(), vmn = __builtin_inff();
    if (held) {
#pragma unroll
        for (int r = 0; r < kExtRegs; ++r) {
            vmx = __builtin_fmaxf(vmx, h2f((uint16_t)(ek[r] & 0xffffu)));
            vmn = __builtin_fminf(vmn, h2f((uint16_t)(ek[r] >> 16)));
        }
    } else {
#pragma unroll 8
        for (int j = tid / cg; j < nchunk; j += lpc) {
            const uint32_t k = ep[(int64_t)j * c];
            vmx = __builtin_fmaxf(vmx, h2f((uint16_t)(k & 0xffffu)));
            vmn = __builtin_fminf(vmn, h2f((uint16_t)(k >> 16)));
        }
    }
    for (int off = cg; off < 64; off <<= 1) {
        vmx = __builtin_fmaxf(vmx, __shfl_xor(vmx, off, 64));
        vmn = __builtin_fminf(vmn, __shfl_xor(vmn, off, 64));
    }
    float cand = 0.0f;
    if (tid < cg) {
        const float gm = h2f(gamma[ch]), bt = h2f(beta[ch]);
        const float v = gm >= 0.0f ? vmx : vmn;
        const float z = rt16(((v - mean) * rstd) * gm + bt);
        cand = __builtin_fabsf(rt16(silu(z)));
    }
    for (int off = 1; off < cg; off <<= 1) cand = __builtin_fmaxf(cand, __shfl_xor(cand, off, 64));
    // every candidate is the |value| of a real element, so it never exceeds the true absmax
    // one word per (frame, group), reduced by absmax_lut: a plain store where a single atomic word would
    // serialise every workgroup of the launch
    if (tid == 0) cands[t * kGroups + g] = __builtin_bit_cast(uint32_t, cand);
}

__device__ __forceinline__ int reflect(int i, int n) { return i < 0 ? -i : (i >= n ? 2 * n - 2 - i : i); }

// q code of table entries [first, first + count) under the scale of the final absmax.
__device__ __forceinline__ void build_lut_range(float amax, int8_t* __restrict__ lut, int first, int count) {
    const float s = e3_scale(amax);
    for (int code = first + (int)threadIdx.x; code < first + count; code += kNT)
        lut[code] = (int8_t)e3_quant(rt16(silu(h2f((uint16_t)code))), s);
}

// The quantize table of norm_pack_lut.  Every block first reduces gn_merge's (frame, group) candidates
// to the absmax candidate (unsigned max of the bit patterns: non-negative floats order as their bits and
// a NaN candidate ranks above every number, so it forces the full pass).  When the candidate is exact
// (almost always) the final scale is known at once: block 0 stores it and the first 256 blocks build 256
// table entries each.  Otherwise every block runs its share of the full absmax pass into done[1]; the
// last block to finish (counter done[0]) stores the final absmax and builds the whole table from it.
// All blocks compute the same candidate, so all take the same branch.  gn_merge zeroed both counters.
// Grid: at least 256 blocks.
template <int C, bool PRE_BIAS>
__global__ __launch_bounds__(kNT) void absmax_lut(const uint16_t* __restrict__ x, const uint16_t* __restrict__ pre_bias,
                                                  const uint16_t* __restrict__ gamma, const uint16_t* __restrict__ beta,
                                                  const float* __restrict__ stats, int d, int h, int w,
                                                  const uint32_t* __restrict__ cands,
                                                  uint32_t* __restrict__ amax_bits, uint32_t* __restrict__ done,
                                                  int8_t* __restrict__ lut) {
    constexpr int CG = C / kGroups;
    constexpr int TPP = C / 8;
    __shared__ uint32_t cred[kNT / 64];
    uint32_t cb = 0u;
    for (int i = threadIdx.x; i < d * kGroups; i += kNT) cb = cands[i] > cb ? cands[i] : cb;
    for (int off = 32; off >= 1; off >>= 1) {
        const uint32_t o = (uint32_t)__shfl_xor((int)cb, off, 64);
        cb = o > cb ? o : cb;
    }
    if ((threadIdx.x & 63) == 0) cred[threadIdx.x >> 6] = cb;
    __syncthreads();
    cb = cred[0];
#pragma unroll
    for (int i = 1; i < kNT / 64; ++i) cb = cred[i] > cb ? cred[i] : cb;
    const float cand = __builtin_bit_cast(float, cb);
    if (cand >= kShortcutFloor) {
        if (blockIdx.x == 0 && threadIdx.x == 0) *amax_bits = cb;
        if (blockIdx.x < 65536 / kNT) build_lut_range(cand, lut, blockIdx.x * kNT, kNT);
        return;
    }
    const int hp = h + 2, wp = w + 2;
    const int64_t nvec = (int64_t)(d + 2) * hp * wp * TPP;
    float amax = 0.0f;
    const int64_t stride = (int64_t)gridDim.x * kNT;
    for (int64_t vi = (int64_t)blockIdx.x * kNT + threadIdx.x; vi < nvec; vi += stride) {
        const int cv = (int)(vi % TPP);
        const int64_t pix = vi / TPP;
        const int jj = (int)(pix % wp);
        const int64_t r = pix / wp;
        const int ii = (int)(r % hp);
        const int t = (int)(r / hp) - 2;
        if (t < 0) continue;   // causal zero frames
        const int si = reflect(ii - 1, h), sj = reflect(jj - 1, w);
        float v[8], gm[8], bt[8];
        u16x8 xv = *reinterpret_cast<const u16x8*>(x + (((int64_t)t * h + si) * w + sj) * C + cv * 8);
        if constexpr (PRE_BIAS) xv = add_f16x8(xv, *reinterpret_cast<const u16x8*>(pre_bias + cv * 8));
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = h2f(xv[e]);
        load8(gamma + cv * 8, gm);
        load8(beta + cv * 8, bt);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int g = (cv * 8 + e) / CG;
            const float mean = stats[(t * kGroups + g) * 2];
            const float rstd = stats[(t * kGroups + g) * 2 + 1];
            const float zz = rt16(((v[e] - mean) * rstd) * gm[e] + bt[e]);
            amax = __builtin_fmaxf(amax, __builtin_fabsf(rt16(silu(zz))));
        }
    }
    __shared__ float red[kNT / 64];
    __shared__ int last;
    __shared__ float fin;
    amax = wave_max(amax);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
    __syncthreads();
    if (threadIdx.x == 0) {
        float m = red[0];
        for (int i = 1; i < kNT / 64; ++i) m = __builtin_fmaxf(m, red[i]);
        atomicMax(&done[1], __builtin_bit_cast(uint32_t, m));   // non-negative floats order as their bits
        __threadfence();
        last = atomicAdd(&done[0], 1u) == gridDim.x - 1;
        if (last) {
            __threadfence();
            const float full = __builtin_bit_cast(float, __hip_atomic_load(&done[1], __ATOMIC_RELAXED,
                                                                           __HIP_MEMORY_SCOPE_AGENT));
            fin = __builtin_fmaxf(cand, full);
            *amax_bits = __builtin_bit_cast(uint32_t, fin);
        }
    }
    __syncthreads();
    if (last) build_lut_range(fin, lut, 0, 65536);
}

static_assert(kGnGroups == kGroups && kGnMaxC == kMaxC && kGnSizingChunk == kChunk, "producer workspace layout");

int64_t workspace_floats(int d, int h, int w) { return gn_workspace_floats(d, h, w); }

// PASS 1 through the table.  Each block walks whole padded output rows
// (frame, padded row): the source row follows from the row index alone, so the
// only per-vector index arithmetic is a shift by C/8 and a reflect of the
// column.  256 threads stride a row in steps that are a multiple of C/8, so each
// thread keeps one 8-channel slice (gamma, beta, pre-bias, groups) for the whole
// kernel; the (mean, rstd) pairs are reloaded when the frame changes.
template <int C, bool PRE_BIAS>
__global__ __launch_bounds__(kNT) void norm_pack_lut(const uint16_t* __restrict__ x,
                                                     const uint16_t* __restrict__ pre_bias,
                                                     const uint16_t* __restrict__ gamma,
                                                     const uint16_t* __restrict__ beta, const float* __restrict__ stats,
                                                     int d, int h, int w, const uint32_t* __restrict__ amax_bits,
                                                     const int8_t* __restrict__ lut_g, int8_t* __restrict__ q,
                                                     float* __restrict__ scale) {
    constexpr int CG = C / kGroups;
    constexpr int TPP = C / 8;
    constexpr int LOG_TPP = TPP == 16 ? 4 : 5;
    static_assert((1 << LOG_TPP) == TPP, "C/8 is a power of two");
    constexpr int NG = 8 / CG > 1 ? 8 / CG : 1;    // groups touched by one 8-channel slice
    __shared__ __attribute__((aligned(16))) int8_t lut[65536];
    for (int i = threadIdx.x; i < 65536 / 16; i += kNT)
        reinterpret_cast<u16x8*>(lut)[i] = reinterpret_cast<const u16x8*>(lut_g)[i];
    if (blockIdx.x == 0 && threadIdx.x == 0) *scale = e3_scale(__builtin_bit_cast(float, *amax_bits));
    __syncthreads();

    const int hp = h + 2, wp = w + 2;
    const int nrow = (d + 2) * hp;
    const int rowvec = wp * TPP;                    // 8-channel vectors per padded row
    const int cv = threadIdx.x & (TPP - 1);
    float gm[8], bt[8];
    u16x8 pb{};
    load8(gamma + cv * 8, gm);
    load8(beta + cv * 8, bt);
    if constexpr (PRE_BIAS) pb = *reinterpret_cast<const u16x8*>(pre_bias + cv * 8);
    const int g0 = cv * 8 / CG;
    int tcur = -1;
    float mean[NG], rstd[NG];
    constexpr int U = 4;   // independent 16-byte loads in flight per lane
    for (int row = blockIdx.x; row < nrow; row += gridDim.x) {
        const int t = row / hp - 2;
        const int ii = row - (t + 2) * hp;
        int8_t* dst = q + (int64_t)row * rowvec * 8;
        if (t < 0) {   // causal zero frames
            for (int j = threadIdx.x; j < rowvec; j += kNT) *reinterpret_cast<uint2*>(dst + (int64_t)j * 8) = make_uint2(0u, 0u);
            continue;
        }
        if (t != tcur) {
            tcur = t;
#pragma unroll
            for (int k = 0; k < NG; ++k) {
                mean[k] = stats[(t * kGroups + g0 + k) * 2];
                rstd[k] = stats[(t * kGroups + g0 + k) * 2 + 1];
            }
        }
        const uint16_t* src = x + ((int64_t)t * h + reflect(ii - 1, h)) * w * C + cv * 8;
        for (int j0 = threadIdx.x; j0 < rowvec; j0 += U * kNT) {
            u16x8 xv[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int j = j0 + u * kNT;
                if (j < rowvec) xv[u] = load_nt(src + (int64_t)reflect((j >> LOG_TPP) - 1, w) * C);
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int j = j0 + u * kNT;
                if (j >= rowvec) break;
                int code[8];
                const u16x8 xs = PRE_BIAS ? add_f16x8(xv[u], pb) : xv[u];   // fp16(x + b), one rounding
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float ve = h2f(xs[e]);
                    const int k = (NG > 1) ? e / CG : 0;
                    code[e] = f2h(((ve - mean[k]) * rstd[k]) * gm[e] + bt[e]);
                }
                const uint32_t lo = pack4(lut[code[0]], lut[code[1]], lut[code[2]], lut[code[3]]);
                const uint32_t hi = pack4(lut[code[4]], lut[code[5]], lut[code[6]], lut[code[7]]);
                *reinterpret_cast<uint2*>(dst + (int64_t)j * 8) = make_uint2(lo, hi);
            }
        }
    }
}

// chunk = kChunk: the statistics pass runs here; chunk = kGnTileChunk: the workspace already holds the
// partial statistics of 512-pixel tiles, written by the window conv that produced x (h3v_conv3d_i8_gn).
template <int C, bool PB>
void launch_all(const uint16_t* x, const uint16_t* pre_bias, const uint16_t* gamma, const uint16_t* beta, float eps,
                int d, int h, int w, int chunk, bool own_stats, int8_t* q, float* scale, float* stats, float* ws,
                uint32_t* amax_bits, hipStream_t stream) {
    const int hw = h * w;
    const GnWorkspace g = gn_workspace(ws, d, hw, chunk);
    if (own_stats)
        hipLaunchKernelGGL((gn_partial<C, PB>), dim3(g.nchunk, d), dim3(kNT), 0, stream, x, pre_bias, hw, g.nchunk,
                           g.avg, g.m2, g.ext);
    // block (0, 0) zeroes absmax_lut's counters; every candidate word is written
    hipLaunchKernelGGL(gn_merge, dim3(kGroups, d), dim3(64), 0, stream, g.avg, g.m2, g.ext, gamma, beta, hw,
                       g.nchunk, chunk, C, eps, stats, g.cands, g.done);
    const int64_t nvec = (int64_t)(d + 2) * (h + 2) * (w + 2) * (C / 8);
    int64_t want = (nvec + kNT - 1) / kNT;
    // grid-strided full pass (rarely run) with at least one block per 256 table entries
    unsigned blocks = (unsigned)(want > 1024 ? 1024 : (want < 256 ? 256 : want));
    hipLaunchKernelGGL((absmax_lut<C, PB>), dim3(blocks), dim3(kNT), 0, stream, x, pre_bias, gamma, beta, stats, d, h,
                       w, g.cands, amax_bits, g.done, g.lut);
    // 64 KB of LDS per block: two blocks per CU; each block walks many vectors
    unsigned lut_blocks = (unsigned)(want > 512 ? 512 : want);
    hipLaunchKernelGGL((norm_pack_lut<C, PB>), dim3(lut_blocks), dim3(kNT), 0, stream, x, pre_bias, gamma, beta, stats,
                       d, h, w, amax_bits, g.lut, q, scale);
}

// ---------------------------------------------------------------------------
// fp16-output producer of the encoder suffix (opt/encoder_fused_batched_norm.py
// :15-66, `batched_temporal_norm_pack`): per-frame GroupNorm(32) statistics of
// every (batch item, frame), then y = fp16(SiLU(fp16(((v - mean) * rstd) *
// gamma + beta))) into fp16 NDHWC [B, D+2, H+2, W+2, C], two zero frames and a
// reflect border per batch item.  C in {128, 256, 512, 1024}.
//
// Statistics order (shared with the CPU oracle's gn_stats): TPP threads per
// pixel, C/8 of them up to C = 256 and one per group above; each thread covers
// CPT = C/TPP channels (GPT whole groups), sums a group's channels left to
// right per pixel and adds the pixel sums of its pixels pl, pl+PL, ... of the
// chunk (PL = 256/TPP); lanes combine by the halving tree.  Chunks hold 256
// pixels up to C = 256 and 65536/C above, so a thread's slice of a chunk stays
// in 64-128 VGPRs for both passes.  For C <= 256 this is gn_partial's order.
// ---------------------------------------------------------------------------
template <int C>
struct GnGeom {
    static constexpr int CG = C / kGroups;
    static constexpr int CPT = C <= 256 ? 8 : CG;
    static constexpr int TPP = C / CPT;
    static constexpr int PL = kNT / TPP;
    static constexpr int CHUNK = C <= 256 ? kChunk : 65536 / C;
    static constexpr int STEPS = CHUNK / PL;
    static constexpr int GPT = CPT / CG;
    static constexpr int NV = CPT / 8;
    static_assert(TPP * PL == kNT && STEPS * PL == CHUNK && GPT >= 1, "statistics geometry");
};

int gn_chunk(int c) { return c <= 256 ? kChunk : 65536 / c; }

template <int C, bool PRE_BIAS>
__global__ __launch_bounds__(kNT) void gn_stats_partial(const uint16_t* __restrict__ x,
                                                        const uint16_t* __restrict__ pre_bias, int hw, int nchunk,
                                                        float* __restrict__ part_avg, float* __restrict__ part_m2) {
    using G = GnGeom<C>;
    __shared__ float red[G::PL][kGroups];
    __shared__ float avg_s[kGroups];
    const int j = blockIdx.x, t = blockIdx.y;
    const int tid = threadIdx.x;
    const int cv = tid % G::TPP, pl = tid / G::TPP;
    const int p0 = j * G::CHUNK;
    const int npix = hw - p0 < G::CHUNK ? hw - p0 : G::CHUNK;
    const uint16_t* base = x + ((int64_t)t * hw + p0) * C + cv * G::CPT;

    u16x8 pb[G::NV] = {};
    if constexpr (PRE_BIAS)
#pragma unroll
        for (int u = 0; u < G::NV; ++u) pb[u] = *reinterpret_cast<const u16x8*>(pre_bias + cv * G::CPT + 8 * u);
    u16x8 xr[G::STEPS][G::NV];
#pragma unroll
    for (int s = 0; s < G::STEPS; ++s) {
        const int p = pl + s * G::PL;
        if (p < npix)
#pragma unroll
            for (int u = 0; u < G::NV; ++u) xr[s][u] = load_nt(base + (int64_t)p * C + 8 * u);
    }
    auto load = [&](int s, float* v) {
#pragma unroll
        for (int u = 0; u < G::NV; ++u)
#pragma unroll
            for (int e = 0; e < 8; ++e) v[8 * u + e] = h2f(xr[s][u][e]);
    };
    float ls[G::GPT];
#pragma unroll
    for (int gi = 0; gi < G::GPT; ++gi) ls[gi] = 0.0f;
#pragma unroll
    for (int s = 0; s < G::STEPS; ++s) {
        const int p = pl + s * G::PL;
        if (p >= npix) break;
        if constexpr (PRE_BIAS)   // fp16(x + b), one rounding; the second pass reads the biased values
#pragma unroll
            for (int u = 0; u < G::NV; ++u) xr[s][u] = add_f16x8(xr[s][u], pb[u]);
        float v[G::CPT];
        load(s, v);
#pragma unroll
        for (int gi = 0; gi < G::GPT; ++gi) {
            float ps = v[gi * G::CG];
#pragma unroll
            for (int i = 1; i < G::CG; ++i) ps = ps + v[gi * G::CG + i];
            ls[gi] = ls[gi] + ps;
        }
    }
#pragma unroll
    for (int gi = 0; gi < G::GPT; ++gi) red[pl][cv * G::GPT + gi] = ls[gi];
    __syncthreads();
    if (tid < kGroups) {
        for (int off = G::PL / 2; off >= 1; off >>= 1)
            for (int i = 0; i < off; ++i) red[i][tid] = red[i][tid] + red[i + off][tid];
        avg_s[tid] = red[0][tid] / (float)(npix * G::CG);
    }
    __syncthreads();
    float a[G::GPT], lm[G::GPT];
#pragma unroll
    for (int gi = 0; gi < G::GPT; ++gi) {
        a[gi] = avg_s[cv * G::GPT + gi];
        lm[gi] = 0.0f;
    }
#pragma unroll
    for (int s = 0; s < G::STEPS; ++s) {
        const int p = pl + s * G::PL;
        if (p >= npix) break;
        float v[G::CPT];
        load(s, v);
#pragma unroll
        for (int gi = 0; gi < G::GPT; ++gi) {
            float dv = v[gi * G::CG] - a[gi];
            float pm = dv * dv;
#pragma unroll
            for (int i = 1; i < G::CG; ++i) {
                dv = v[gi * G::CG + i] - a[gi];
                pm = pm + dv * dv;
            }
            lm[gi] = lm[gi] + pm;
        }
    }
    __syncthreads();
#pragma unroll
    for (int gi = 0; gi < G::GPT; ++gi) red[pl][cv * G::GPT + gi] = lm[gi];
    __syncthreads();
    if (tid < kGroups) {
        for (int off = G::PL / 2; off >= 1; off >>= 1)
            for (int i = 0; i < off; ++i) red[i][tid] = red[i][tid] + red[i + off][tid];
        const int64_t dst = ((int64_t)t * kGroups + tid) * nchunk + j;
        part_avg[dst] = avg_s[tid];
        part_m2[dst] = red[0][tid];
    }
}

__global__ __launch_bounds__(64) void gn_stats_merge(const float* __restrict__ part_avg, const float* __restrict__ part_m2,
                                                     int hw, int nchunk, int chunk, int c, float eps,
                                                     float* __restrict__ stats) {
    __shared__ float sa[kMergeBatch];
    __shared__ float sm[kMergeBatch];
    __shared__ float ms[2];
    const int g = blockIdx.x, t = blockIdx.y;
    const float* pa = part_avg + ((int64_t)t * kGroups + g) * nchunk;
    const float* pm = part_m2 + ((int64_t)t * kGroups + g) * nchunk;
    gn_merge_group(pa, pm, hw, nchunk, chunk, c / kGroups, eps, sa, sm, ms, [] {});
    if (threadIdx.x == 0) {
        stats[(t * kGroups + g) * 2] = ms[0];
        stats[(t * kGroups + g) * 2 + 1] = ms[1];
    }
}

// One block per padded output row (batch item, padded frame, padded row): the
// source row follows from the row index alone; the 256 threads stride the row
// in steps that are a multiple of C/8, so each keeps one 8-channel slice.
template <int C, bool PRE_BIAS>
__global__ __launch_bounds__(kNT) void norm_pack_f16(const uint16_t* __restrict__ x,
                                                     const uint16_t* __restrict__ pre_bias,
                                                     const uint16_t* __restrict__ gamma,
                                                     const uint16_t* __restrict__ beta, const float* __restrict__ stats,
                                                     int d, int h, int w, uint16_t* __restrict__ y) {
    constexpr int CG = C / kGroups;
    constexpr int TPP = C / 8;
    constexpr int NG = 8 / CG > 1 ? 8 / CG : 1;   // groups touched by one 8-channel slice
    static_assert(kNT % TPP == 0, "threads stride whole pixels");
    const int hp = h + 2, wp = w + 2;
    const int row = blockIdx.x;                     // (b * (d + 2) + tp) * hp + ii
    const int ii = row % hp;
    const int bt2 = row / hp;
    const int tp = bt2 % (d + 2), b = bt2 / (d + 2);
    const int t = tp - 2;
    const int rowvec = wp * TPP;
    uint16_t* dst = y + (int64_t)row * rowvec * 8;
    if (t < 0) {   // causal zero frames
        for (int j = threadIdx.x; j < rowvec; j += kNT) *reinterpret_cast<u16x8*>(dst + (int64_t)j * 8) = u16x8{};
        return;
    }
    const int cv = threadIdx.x % TPP;
    float gm[8], btv[8];
    u16x8 pb{};
    load8(gamma + cv * 8, gm);
    load8(beta + cv * 8, btv);
    if constexpr (PRE_BIAS) pb = *reinterpret_cast<const u16x8*>(pre_bias + cv * 8);
    const int frame = b * d + t;
    const int g0 = cv * 8 / CG;
    float mean[NG], rstd[NG];
#pragma unroll
    for (int k = 0; k < NG; ++k) {
        mean[k] = stats[(frame * kGroups + g0 + k) * 2];
        rstd[k] = stats[(frame * kGroups + g0 + k) * 2 + 1];
    }
    const uint16_t* src = x + ((int64_t)frame * h + reflect(ii - 1, h)) * w * C + cv * 8;
    for (int j = threadIdx.x; j < rowvec; j += kNT) {
        u16x8 xv = load_nt(src + (int64_t)reflect(j / TPP - 1, w) * C);
        if constexpr (PRE_BIAS) xv = add_f16x8(xv, pb);   // fp16(x + b), one rounding
        u16x8 out;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float ve = h2f(xv[e]);
            const int k = (NG > 1) ? e / CG : 0;
            const float z = rt16(((ve - mean[k]) * rstd[k]) * gm[e] + btv[e]);
            out[e] = f2h(silu_fast(z));
        }
        *reinterpret_cast<u16x8*>(dst + (int64_t)j * 8) = out;
    }
}

template <int C, bool PB>
void launch_f16(const uint16_t* x, const uint16_t* pre_bias, const uint16_t* gamma, const uint16_t* beta, float eps,
                int batch, int d, int h, int w, uint16_t* y, float* stats, float* ws, hipStream_t stream) {
    const int hw = h * w, frames = batch * d;
    const int chunk = GnGeom<C>::CHUNK;
    const int nchunk = (hw + chunk - 1) / chunk;
    float* part_avg = ws;
    float* part_m2 = ws + (int64_t)frames * nchunk * kGroups;
    hipLaunchKernelGGL((gn_stats_partial<C, PB>), dim3(nchunk, frames), dim3(kNT), 0, stream, x, pre_bias, hw, nchunk,
                       part_avg, part_m2);
    hipLaunchKernelGGL(gn_stats_merge, dim3(kGroups, frames), dim3(64), 0, stream, part_avg, part_m2, hw, nchunk, chunk,
                       C, eps, stats);
    hipLaunchKernelGGL((norm_pack_f16<C, PB>), dim3(batch * (d + 2) * (h + 2)), dim3(kNT), 0, stream, x, pre_bias, gamma,
                       beta, stats, d, h, w, y);
}


// ---------------------------------------------------------------------------
// Checks and launch shared by h3v_gn_norm_pack_i8 and its no-allocation variant.
// own_stats: run the statistics pass (gn_partial, 256-pixel chunks); otherwise the workspace already holds
// the partials of `chunk`-pixel chunks, written by the conv that produced x.
int run_norm_pack_i8(const char* what, const uint16_t* x, const uint16_t* pre_bias, const uint16_t* gamma,
                     const uint16_t* beta, float eps, int c, int d, int h, int w, int chunk, bool own_stats, int8_t* q,
                     float* scale, float* stats, float* workspace, uint32_t* amax_scratch, hipStream_t stream) {
    H3V_REQUIRE(x && gamma && beta && q && scale && stats, "%s: null pointer argument", what);
    H3V_REQUIRE(c == 128 || c == 256, "%s: C must be 128 or 256 (got %d)", what, c);
    H3V_REQUIRE(d >= 1 && h >= 2 && w >= 2, "%s: requires D >= 1 and H, W >= 2", what);
    H3V_REQUIRE((int64_t)c * (d + 2) * (h + 2) * (w + 2) < ((int64_t)1 << 31), "%s: padded output exceeds int32 index range",
                what);
    H3V_REQUIRE(eps > 0.0f, "%s: eps must be positive", what);
    H3V_REQUIRE(aligned(x, 16) && aligned(gamma, 16) && aligned(beta, 16) && (!pre_bias || aligned(pre_bias, 16)) &&
                    aligned(q, 8),
                "%s: x, gamma, beta, pre_bias need 16-byte and q 8-byte alignment", what);
    if (c == 128) {
        if (pre_bias) launch_all<128, true>(x, pre_bias, gamma, beta, eps, d, h, w, chunk, own_stats, q, scale, stats, workspace, amax_scratch, stream);
        else launch_all<128, false>(x, pre_bias, gamma, beta, eps, d, h, w, chunk, own_stats, q, scale, stats, workspace, amax_scratch, stream);
    } else {
        if (pre_bias) launch_all<256, true>(x, pre_bias, gamma, beta, eps, d, h, w, chunk, own_stats, q, scale, stats, workspace, amax_scratch, stream);
        else launch_all<256, false>(x, pre_bias, gamma, beta, eps, d, h, w, chunk, own_stats, q, scale, stats, workspace, amax_scratch, stream);
    }
    return launch_status(what);
}

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
float* g_scratch_ptr[kMaxDevices] = {};

int scratch_for_current_device(const char* what, float** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail(H3V_ELAUNCH, "%s: hipGetDevice failed: %s", what, hipGetErrorString(e));
    H3V_REQUIRE(dev >= 0 && dev < kMaxDevices, "%s: device index %d out of range", what, dev);
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return fail(H3V_ELAUNCH, "%s: hipGetSymbolAddress(scratch) failed on device %d: %s", what, dev,
                        hipGetErrorString(e));
        g_scratch_ptr[dev] = static_cast<float*>(p);
    }
    *out = g_scratch_ptr[dev];
    return H3V_OK;
}

}  // namespace
}  // namespace h3v

using namespace h3v;

extern "C" {

int64_t h3v_gn_norm_pack_workspace_floats(int d, int h, int w) {
    if (d <= 0 || h <= 0 || w <= 0) return -1;
    return workspace_floats(d, h, w);
}

int h3v_gn_norm_pack_i8(const uint16_t* x, const uint16_t* pre_bias, const uint16_t* gamma, const uint16_t* beta,
                        float eps, int c, int d, int h, int w, int8_t* q, float* scale, float* stats,
                        float* workspace, uint32_t* amax_scratch, hipStream_t stream) {
    const char* what = "h3v_gn_norm_pack_i8";
    H3V_REQUIRE(workspace && amax_scratch, "%s: null pointer argument", what);
    H3V_REQUIRE(aligned(workspace, 16), "%s: workspace needs 16-byte alignment", what);
    return run_norm_pack_i8(what, x, pre_bias, gamma, beta, eps, c, d, h, w, kChunk, true, q, scale, stats, workspace,
                            amax_scratch, stream);
}

int h3v_gn_norm_pack_i8_partials(const uint16_t* x, const uint16_t* pre_bias, const uint16_t* gamma,
                                 const uint16_t* beta, float eps, int c, int d, int h, int w, int chunk, int8_t* q,
                                 float* scale, float* stats, float* workspace, uint32_t* amax_scratch,
                                 hipStream_t stream) {
    const char* what = "h3v_gn_norm_pack_i8_partials";
    H3V_REQUIRE(workspace && amax_scratch, "%s: null pointer argument", what);
    H3V_REQUIRE(aligned(workspace, 16), "%s: workspace needs 16-byte alignment", what);
    H3V_REQUIRE(chunk == kGnTileChunk || chunk == kChunk,
                "%s: chunk must be %d (window-conv tiles) or %d (pixel runs of h3v_conv3d_f16_gn) (got %d)", what,
                kGnTileChunk, kChunk, chunk);
    H3V_REQUIRE(chunk == kChunk || h >= 8, "%s: %d-pixel tiles need H at least 8 (got %d)", what, kGnTileChunk, h);
    H3V_REQUIRE(((int64_t)h * w) % chunk == 0,
                "%s: the partial statistics are those of %d-pixel chunks: H * W must be a multiple of %d (got %d x %d)",
                what, chunk, chunk, h, w);
    return run_norm_pack_i8(what, x, pre_bias, gamma, beta, eps, c, d, h, w, chunk, false, q, scale, stats, workspace,
                            amax_scratch, stream);
}

int h3v_gn_norm_pack_i8_noalloc(const uint16_t* x, const uint16_t* pre_bias, const uint16_t* gamma,
                                const uint16_t* beta, float eps, int c, int d, int h, int w, int8_t* q, float* scale,
                                float* stats, hipStream_t stream) {
    const char* what = "h3v_gn_norm_pack_i8_noalloc";
    H3V_REQUIRE(d >= 1 && h >= 2 && w >= 2, "%s: requires D >= 1 and H, W >= 2", what);
    const int64_t need = workspace_floats(d, h, w);
    H3V_REQUIRE(need <= kScratchWorkspaceFloats,
                "%s: [D=%d, H=%d, W=%d] needs %lld workspace floats; the static scratch holds %lld "
                "(use h3v_gn_norm_pack_i8 with a caller workspace)",
                what, d, h, w, (long long)need, (long long)kScratchWorkspaceFloats);
    float* base = nullptr;
    const int rc = scratch_for_current_device(what, &base);
    if (rc != H3V_OK) return rc;
    // word 0: the absmax key; the workspace starts 256 bytes in (16-byte alignment kept)
    return run_norm_pack_i8(what, x, pre_bias, gamma, beta, eps, c, d, h, w, kChunk, true, q, scale, stats,
                            base + kScratchHeadFloats, reinterpret_cast<uint32_t*>(base), stream);
}

int64_t h3v_gn_norm_pack_f16_workspace_floats(int batch, int c, int d, int h, int w) {
    if (batch <= 0 || d <= 0 || h <= 0 || w <= 0 || (c != 128 && c != 256 && c != 512 && c != 1024)) return -1;
    const int chunk = gn_chunk(c);
    return 2 * (int64_t)batch * d * kGroups * (((int64_t)h * w + chunk - 1) / chunk);
}

int h3v_gn_norm_pack_f16(const uint16_t* x, const uint16_t* pre_bias, const uint16_t* gamma, const uint16_t* beta,
                         float eps, int batch, int c, int d, int h, int w, uint16_t* y, float* stats, float* workspace,
                         hipStream_t stream) {
    const char* what = "h3v_gn_norm_pack_f16";
    H3V_REQUIRE(x && gamma && beta && y && stats && workspace, "%s: null pointer argument", what);
    H3V_REQUIRE(c == 128 || c == 256 || c == 512 || c == 1024, "%s: C must be 128, 256, 512 or 1024 (got %d)", what, c);
    H3V_REQUIRE(batch >= 1 && d >= 1 && h >= 2 && w >= 2, "%s: requires B, D >= 1 and H, W >= 2", what);
    H3V_REQUIRE((int64_t)batch * c * (d + 2) * (h + 2) * (w + 2) < ((int64_t)1 << 31) &&
                    (int64_t)batch * (d + 2) * (h + 2) < ((int64_t)1 << 31),
                "%s: padded output exceeds int32 index range", what);
    H3V_REQUIRE(eps > 0.0f, "%s: eps must be positive", what);
    H3V_REQUIRE(aligned(x, 16) && aligned(gamma, 16) && aligned(beta, 16) && (!pre_bias || aligned(pre_bias, 16)) &&
                    aligned(y, 16) && aligned(workspace, 16),
                "%s: x, gamma, beta, pre_bias, y and workspace need 16-byte alignment", what);
#define H3V_F16_CASE(CC)                                                                                            \
    if (c == CC) {                                                                                                  \
        if (pre_bias) launch_f16<CC, true>(x, pre_bias, gamma, beta, eps, batch, d, h, w, y, stats, workspace, stream); \
        else launch_f16<CC, false>(x, pre_bias, gamma, beta, eps, batch, d, h, w, y, stats, workspace, stream);       \
    }
    H3V_F16_CASE(128)
    H3V_F16_CASE(256)
    H3V_F16_CASE(512)
    H3V_F16_CASE(1024)
#undef H3V_F16_CASE
    return launch_status(what);
}

}  // extern "C"
