// INT8 MFMA GEMM / implicit-GEMM conv3d for gfx950 (CDNA4).
//
// One mainloop serves three reference operations:
//   * the CK CUTLASS dequant GEMM  (opt/int8_swiglu_fused.py:78-107, G1),
//   * the FFN-up GEMM with paired SwiGLU epilogue (opt/int8_ffn_up_fused.py:50-89, F2),
//   * the encoder's implicit-GEMM causal conv3d (opt/encoder_int8_pipeline.py:15-119, E4).
//
// C[m, n] = sum_k A[m, k] * W[n, k] with int8 operands and int32 accumulators.
// Both operands are K-contiguous.  For the conv, A is never materialised: row m
// is an output voxel (b, od, oh, ow) of an NDHWC int8 input and k = (kd, kh, kw, c)
// with c fastest, so A[m, k] = x[base(m) + tap_offset(k / C) + k % C], a sum of a
// per-row and a per-k term.  With C a multiple of the K tile every K tile is one
// tap and a contiguous channel slice.
//
// Tiling: BM x BN x BK workgroup tile of 8 waves (2 per SIMD), each owning a
// 128 x 64 block built from v_mfma_i32_32x32x32_i8.  Operands stream
// global -> LDS with LDS-DMA (global_load_lds_dwordx4) into an NSA-slot A ring
// and an NSB-slot B ring, issued NSA-1 / NSB-1 K steps ahead of the MFMAs by
// one wave per SIMD (the other keeps the matrix pipe busy); one barrier per K step.  The activation operand A misses L2 more often than the
// weights, so it gets the deeper ring when the LDS allows.  BK = 128 is
// the default: every row segment a K step fetches is then one whole 128-byte
// cache line (64-byte segments use half of each line fetched into L1 and
// halve the L2 -> LDS rate, measured 28 vs 63 B/clk/CU).  LDS rows are
// XOR-swizzled in 16-byte chunks so fragment reads are bank-conflict free.
// Workgroup ids are remapped so that each XCD (own L2) walks a contiguous,
// M-grouped range of tiles.
#include <type_traits>

#include "h3v_common.hpp"
#include "h3v_abi.hpp"

namespace h3v {
namespace {

enum class AMode { Gemm, Conv };
// Dequant: fp16(fma(fp32(acc) * sx, sw, bias)); SwiGLU: paired gate/up then SiLU(gate) * up;
// Int32: raw accumulators; F16Bias: fp16 operands with fp32 accumulators, fp16(acc + bias).
// F32Part: fp16 operands like F16Bias, the raw fp32 accumulators of one K split stored to
// out + split * M * ldo (split-K partials, summed by splitk_reduce_f16).
enum class Epi { Dequant, SwiGLU, Int32, F16Bias, F32Part };

template <Epi EP>
constexpr bool kF16Ops = EP == Epi::F16Bias || EP == Epi::F32Part;   // fp16 operands, fp32 accumulators

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 half8 __attribute__((ext_vector_type(8)));

struct GemmParams {
    const int8_t* a;
    const int8_t* b;
    int M, N, K;       // N = output columns (SwiGLU: output columns, weight has 2N rows)
    int64_t lda;       // Gemm: row stride of A in bytes
    // conv geometry (AMode::Conv): input NDHWC [B, Dp, Hp, Wp, C]
    int C, Dp, Hp, Wp, Do, Ho, Wo, KH, KW, SD, SH, SW;
    int causal_skip;
    // epilogue
    const float* sx;   // row scales (per row) or one tensor scale (sx_stride 0)
    int sx_stride;
    const float* sw;   // per weight row
    const uint16_t* bias;  // fp16 per weight row, nullable
    const uint16_t* res;   // fp16 residual in the output's layout, nullable: out = fp16(fp32(y) + fp32(res))
    const uint16_t* res_bias;  // fp16 per column, nullable (with res): out = fp16(fp32(res) + (fp32(y) + fp32(res_bias)))
    // conv3_halo_i8<..., PAD = true>: output [B, Do + pad_front, Ho + top + bottom, Wo + left + right, N],
    // a reflect border of 0 or 1 on each side (see write_tile)
    int pad_front, pad_top, pad_bottom, pad_left, pad_right;
    void* out;
    int64_t ldo;
    int tiles_m, tiles_n;
    int vec_epi;       // sw (and bias) aligned for 4-column vector loads and N % 4 == 0
    int vec_out;       // fp16 output 16-byte aligned with ldo % 8 == 0: 16-byte row stores
    int conv_tpf;      // conv: M tiles per output frame when they do not straddle frames, else 0
    uint32_t a_bytes;  // extents of A and W in bytes (buffer resource ranges, < 4 GiB)
    uint32_t b_bytes;
    int k_splits;      // tiled kernels: K blocks split evenly over gridDim.y = k_splits workgroups (0 or 1: none)
    // statistics epilogue of the window conv (h3v_conv3d_i8_gn; null gn_avg: off): the GroupNorm(32)
    // partial statistics of each 512-pixel output tile, in the producer workspace layout (GnWorkspace)
    float* gn_avg;
    float* gn_m2;
    uint32_t* gn_ext;
    const uint16_t* gn_bias;   // fp16 per output channel, nullable: statistics of fp16(out + gn_bias)
    int gn_nchunk;             // tiles per output frame
};

// Buffer resource word 3 for raw byte addressing (no swizzle, 32-bit format).
constexpr int kRsrcWord3 = 0x00020000;

constexpr int kXcds = 8;

// Workgroups are dispatched round-robin over the 8 XCDs (id % 8).  Remap so the
// ids that land on one XCD form one contiguous range of logical tiles.
__device__ __forceinline__ int xcd_remap(int bid, int nb) {
    int q = nb / kXcds, r = nb % kXcds;
    int x = bid % kXcds, l = bid / kXcds;
    return x * q + (x < r ? x : r) + l;
}

__device__ __forceinline__ void grouped_tile(int id, int tiles_m, int tiles_n, int group, int& tm, int& tn) {
    int width = group * tiles_n;
    int g = id / width;
    int first = g * group;
    int size = tiles_m - first < group ? tiles_m - first : group;
    tm = first + (id % width) % size;
    tn = (id % width) / size;
}

__device__ __forceinline__ int64_t conv_row_offset(const GemmParams& p, int m) {
    int ow = m % p.Wo;
    int r = m / p.Wo;
    int oh = r % p.Ho;
    r /= p.Ho;
    int od = r % p.Do;
    int b = r / p.Do;
    return ((((int64_t)b * p.Dp + (int64_t)od * p.SD) * p.Hp + (int64_t)oh * p.SH) * p.Wp + (int64_t)ow * p.SW) * p.C;
}

__device__ __forceinline__ int64_t conv_k_offset(const GemmParams& p, int k0) {
    int tap = k0 / p.C;
    int c0 = k0 - tap * p.C;
    int kd = tap / (p.KH * p.KW);
    int rem = tap - kd * p.KH * p.KW;
    int kh = rem / p.KW;
    int kw = rem - kh * p.KW;
    return (((int64_t)kd * p.Hp + kh) * p.Wp + kw) * p.C + c0;
}

// Output frame of GEMM row m (conv rows are ordered b, od, oh, ow).
__device__ __forceinline__ void conv_row_frame(const GemmParams& p, int m, int& b, int& od) {
    int r = m / (p.Wo * p.Ho);
    od = r % p.Do;
    b = r / p.Do;
}

// Causal-zero skip: the fused producer writes two zero frames in front of the
// input, so for output frame t the taps kd < 2 - t multiply zeros.  A tile may
// skip them only if every row in it allows it, i.e. for the largest frame.
__device__ __forceinline__ int conv_first_kblock(const GemmParams& p, int m0, int bm, int bk) {
    if (!p.causal_skip) return 0;
    int last = m0 + bm - 1 < p.M - 1 ? m0 + bm - 1 : p.M - 1;
    int b0, t0, b1, t1;
    conv_row_frame(p, m0, b0, t0);
    conv_row_frame(p, last, b1, t1);
    int tmax = (b0 != b1) ? p.Do - 1 : t1;
    int skip = 2 - tmax;
    if (skip <= 0) return 0;
    return skip * p.KH * p.KW * p.C / bk;
}

__device__ __forceinline__ float g1_value(int32_t acc, float sx, float sw, const uint16_t* bias, int col) {
    float v = (float)acc * sx;
    return bias ? __builtin_fmaf(v, sw, h2f(bias[col])) : v * sw;
}

// The same epilogue with the weight scale and bias already in registers; the
// bias presence is a compile-time choice so no per-element select is emitted.
template <bool HAS_BIAS>
__device__ __forceinline__ float g1_reg(int32_t acc, float sx, float sw, uint16_t b) {
    float v = (float)acc * sx;
    if constexpr (HAS_BIAS) return __builtin_fmaf(v, sw, h2f(b));
    else return v * sw;
}

typedef float f32x4 __attribute__((ext_vector_type(4)));

// Weight scales and fp16 bias of NQ column quads (4 consecutive weight rows
// c[q]..c[q]+3 each, c[q] a multiple of 4, below limit[q]), all issued before
// any is used.  With vec_epi (aligned, limits multiples of 4) a quad is one
// 16-byte and one 8-byte load, its start clamped to the last full quad;
// otherwise clamped scalar loads.  Quads past the end load valid neighbours
// and are never stored.
template <int NQ, bool HB>
__device__ __forceinline__ void load_cols(const GemmParams& p, const int (&c)[NQ], const int (&limit)[NQ],
                                          f32x4 (&sw)[NQ], u16x4 (&b)[NQ]) {
    if (p.vec_epi) {
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
            const int cc = c[q] < limit[q] - 4 ? c[q] : limit[q] - 4;
            sw[q] = *reinterpret_cast<const f32x4*>(p.sw + cc);
            if constexpr (HB) b[q] = *reinterpret_cast<const u16x4*>(p.bias + cc);
            else b[q] = u16x4{0, 0, 0, 0};
        }
    } else {
#pragma unroll
        for (int q = 0; q < NQ; ++q)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int ce = c[q] + e < limit[q] ? c[q] + e : limit[q] - 1;
                sw[q][e] = p.sw[ce];
                b[q][e] = HB ? p.bias[ce] : 0;
            }
    }
}

// LDS-DMA helpers.  global_load_lds_dwordx4 writes lane i's 16 bytes to
// M0 + 16*i, so one wave instruction fills 1 KB of LDS contiguously: 1024/BK
// tile rows of BK bytes.  Lane i loads row i/(BK/16) and puts its 16-byte chunk
// in slot i%(BK/16); the chunk it fetches is slot ^ swz(row), so slot s of row
// r holds k-chunk s ^ swz(r), with r the row's index in the tile (the same for
// the DMA lane and the fragment reader).  The swizzles make the 16-byte
// fragment reads (lane l: row l%32 of a 32-row block, chunk l/32 + 2*ks)
// conflict free both for 8-lane groups on 32 banks and for 16-lane groups on
// 64 banks:
//   BK = 64:  swz(r) = ((r >> 1) & 3) ^ ((r >> 3) & 1)
//   BK = 128: swz(r) = ((r >> 1) & 7) ^ ((r & 1) << 2)
typedef __attribute__((address_space(3))) void* lds_void_t;

template <int BK>
__device__ __forceinline__ int swz(int row) {
    if constexpr (BK == 64) return ((row >> 1) & 3) ^ ((row >> 3) & 1);
    else return ((row >> 1) & 7) ^ ((row & 1) << 2);
}

// 16 bytes per lane from a buffer (resource + per-lane 32-bit offset + uniform
// offset) straight into LDS.  The buffer form issues markedly cheaper than
// global_load_lds: in a barrier-free MFMA probe with eight 1 KB loads per wave
// per 32 MFMAs, MFMA throughput held 81% of peak against 62%.
__device__ __forceinline__ void lds_dma16(__amdgpu_buffer_rsrc_t rsrc, uint32_t voff, uint32_t soff, void* lds) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void_t)lds, 16, (int)voff, (int)soff, 0, 0);
}

// s_waitcnt with only the vector-memory counter constrained (gfx9 encoding:
// vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] << 14).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Workgroup barrier without the release/acquire fences of __syncthreads(): those
// would wait for every outstanding LDS-DMA load (vmcnt(0)) and drain the ring.
// LDS reads issued before the barrier are completed explicitly (lgkmcnt(0)).
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_s_waitcnt((15 << 4) | (0 << 8) | 0xC00F);  // lgkmcnt(0) only
    __builtin_amdgcn_s_barrier();
}

template <int LPS>
__device__ __forceinline__ void wait_stage(int ahead) {
    // wait until at most `ahead` later stages (LPS loads each) are still in flight
    if (ahead >= 3) wait_vmcnt<3 * LPS>();
    else if (ahead == 2) wait_vmcnt<2 * LPS>();
    else if (ahead == 1) wait_vmcnt<LPS>();
    else wait_vmcnt<0>();
}

// Epilogue of the tiled kernels: the wave's (BM/WGM) x (BN/WGN) block of
// int32 accumulators of the workgroup's BM x BN tile at (m0, n0), weight tile
// tn, is dequantized (or stored raw) to the output.  LDS_BYTES of LDS (the
// operand rings, idle by now) stage the fp16 tile.  SROWS: row r of the
// wave's accumulator block i is wave row r * FM + i (strided rows of the
// conv3_halo_i8 variant that reuses A fragments across kw taps) instead of
// i * 32 + r.  TILEW > 0: the tile is 512 / TILEW output rows of TILEW pixels each (a column block
// of output rows p.Wo wide) starting at row m0, so tile row r is output row
// m0 + (r / TILEW) * p.Wo + r % TILEW; 0: the tile's rows are consecutive from m0.
// LDS past the operand rings that the chunk-statistics epilogue of the FP16 implicit-GEMM conv uses: the
// lane sums [16][32], the group averages [32] and per wave of threads 0-255 the channel extremes [4][128][2].
constexpr int kGnChunkLdsBytes = (16 * 32 + 32 + 4 * 128 * 2) * 4;

template <int BM, int BN, int WGM, int WGN, int LDS_BYTES, Epi EP, int PADWO = 0, bool SROWS = false, int TILEW = 0,
          typename AccV>
__device__ __forceinline__ void write_tile(const GemmParams& p, AccV (&acc)[BM / WGM / 32][BN / WGN / 32],
                                           int8_t* smem, int m0, int n0, int tn) {
    static_assert(kF16Ops<EP> == std::is_same<AccV, f32x16>::value, "fp32 accumulators with fp16 operands only");
    constexpr int NW = WGM * WGN;
    constexpr int WM = BM / WGM, WN = BN / WGN;
    constexpr int FM = WM / 32, FN = WN / 32;
    constexpr int RING = LDS_BYTES;
    static_assert(!SROWS || ((EP == Epi::Dequant || EP == Epi::Int32 || EP == Epi::F16Bias) && FM == 4),
                  "strided rows: window-conv epilogues of 128-row wave blocks");
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform (scalar)
    const int wm = wave / WGN, wn = wave % WGN;
    // Epilogue.  The MFMAs compute W * A^T blocks, so in the v_mfma 32x32 result
    // layout lane l holds output row m = lane&31 of the block and, in register
    // r, output column n = (r/4)*8 + (l/32)*4 + r%4: four consecutive columns per
    // register quad.
    const int mrow = lane & 31;
    const int ncol = (lane >> 5) * 4;
    // tile row of this lane's rows in accumulator block i, and the output row of tile row r
    auto trow = [&](int i) { return wm * WM + (SROWS ? mrow * FM + i : i * 32 + mrow); };
    auto gidx = [&](int r) { return TILEW ? m0 + (r / TILEW) * p.Wo + r % TILEW : m0 + r; };
    if constexpr (EP == Epi::F32Part) {
        // this split's partial sums, straight from the MFMA layout: 16 bytes (4 columns) per store
        float* part = static_cast<float*>(p.out) + (int64_t)blockIdx.y * p.M * p.ldo;
#pragma unroll
        for (int j = 0; j < FN; ++j) {
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
                const int c0 = n0 + wn * WN + j * 32 + q4 * 8 + ncol;
                if (c0 >= p.N) continue;
                const bool full = c0 + 4 <= p.N && (p.ldo & 3) == 0;
#pragma unroll
                for (int i = 0; i < FM; ++i) {
                    const int row = m0 + wm * WM + i * 32 + mrow;
                    if (row >= p.M) continue;
                    float* dst = part + (int64_t)row * p.ldo + c0;
                    if (full) {
                        f32x4 v = {acc[i][j][q4 * 4], acc[i][j][q4 * 4 + 1], acc[i][j][q4 * 4 + 2], acc[i][j][q4 * 4 + 3]};
                        *reinterpret_cast<f32x4*>(dst) = v;
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            if (c0 + e < p.N) dst[e] = acc[i][j][q4 * 4 + e];
                    }
                }
            }
        }
    } else if constexpr (EP == Epi::Int32) {
#pragma unroll
        for (int j = 0; j < FN; ++j) {
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
                const int c0 = n0 + wn * WN + j * 32 + q4 * 8 + ncol;
                if (c0 >= p.N) continue;
                const bool full = c0 + 4 <= p.N && (p.ldo & 3) == 0;
#pragma unroll
                for (int i = 0; i < FM; ++i) {
                    const int row = gidx(trow(i));
                    if (row >= p.M) continue;
                    int32_t* dst = static_cast<int32_t*>(p.out) + (int64_t)row * p.ldo + c0;
                    if (full) {
                        v4i v = {acc[i][j][q4 * 4], acc[i][j][q4 * 4 + 1], acc[i][j][q4 * 4 + 2], acc[i][j][q4 * 4 + 3]};
                        *reinterpret_cast<v4i*>(dst) = v;
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            if (c0 + e < p.N) dst[e] = acc[i][j][q4 * 4 + e];
                    }
                }
            }
        }
    } else {
        // fp16 outputs go through LDS: each wave converts its block into the
        // (now idle) LDS ring, laid out as the workgroup's output tile
        // [BM][OUTW] with 16-byte chunks XOR-swizzled by row, and then every
        // thread stores 16-byte pieces of whole tile rows, so each store
        // instruction writes complete 128-byte lines (direct 8-byte stores from
        // the MFMA layout touch 32 partial lines per instruction and cost about
        // a third of the kernel).
        constexpr int OUTW = (EP == Epi::SwiGLU) ? BN / 2 : BN;
        constexpr int RCH = OUTW / 8;
        constexpr int SWM = (RCH < 32 ? RCH : 32) - 1;
        static_assert(RCH >= 8 && BM * OUTW * 2 <= RING, "output tile must fit the LDS ring");
        int8_t* ep = smem;
        // chunk swizzle key of tile row r: the rows one store instruction writes (32 consecutive
        // rows, or with SROWS rows FM apart) get distinct keys
        auto skey = [](int r) { return (SROWS ? r >> 2 : r) & SWM; };
        auto put = [&](int r, int c, const u16x4& v) {   // c: tile column, a multiple of 4
            const int ch = c >> 3;
            *reinterpret_cast<u16x4*>(ep + r * (OUTW * 2) + ((ch ^ skey(r)) << 4) + ((c & 4) << 1)) = v;
        };
        const bool has_bias = p.bias != nullptr;
        float sxr[FM];
#pragma unroll
        for (int i = 0; i < FM; ++i) {
            const int row = gidx(trow(i));
            sxr[i] = (EP != Epi::F16Bias && row < p.M) ? p.sx[(int64_t)row * p.sx_stride] : 0.0f;
        }
        // one instantiation per bias presence (uniform per launch)
        auto convert = [&](auto hb) {
        constexpr bool HB = decltype(hb)::value;
        // the wave's column parameters go out before the barrier, so their
        // latency overlaps it: FN * 4 quads (SwiGLU: FN / 2 * 4 gate/up pairs)
        constexpr int NQ = FN * 4;
        int qc[NQ], ql[NQ];
        f32x4 qsw[NQ] = {};
        u16x4 qb[NQ];
        if constexpr (EP == Epi::SwiGLU) {
#pragma unroll
            for (int j = 0; j < FN / 2; ++j)
#pragma unroll
                for (int q4 = 0; q4 < 4; ++q4) {
                    const int c0 = tn * (BN / 2) + (wn * WN) / 2 + j * 32 + q4 * 8 + ncol;
                    const int q = (j * 4 + q4) * 2;
                    qc[q] = c0;
                    ql[q] = p.N;
                    qc[q + 1] = p.N + c0;
                    ql[q + 1] = 2 * p.N;
                }
        } else {
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
                for (int q4 = 0; q4 < 4; ++q4) {
                    qc[j * 4 + q4] = n0 + wn * WN + j * 32 + q4 * 8 + ncol;
                    ql[j * 4 + q4] = p.N;
                }
        }
        if constexpr (EP == Epi::F16Bias) {
            // bias only: clamped columns, one 8-byte load per quad when aligned
#pragma unroll
            for (int q = 0; q < NQ; ++q) {
                if constexpr (HB) {
                    if (p.vec_epi) {
                        const int cc = qc[q] < ql[q] - 4 ? qc[q] : ql[q] - 4;
                        qb[q] = *reinterpret_cast<const u16x4*>(p.bias + cc);
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e) qb[q][e] = p.bias[qc[q] + e < ql[q] ? qc[q] + e : ql[q] - 1];
                    }
                } else {
                    qb[q] = u16x4{0, 0, 0, 0};
                }
            }
        } else {
            load_cols<NQ, HB>(p, qc, ql, qsw, qb);
        }
        lds_barrier();   // every wave has finished reading operand fragments
        if constexpr (EP == Epi::SwiGLU) {
#pragma unroll
            for (int j = 0; j < FN / 2; ++j) {
#pragma unroll
                for (int q4 = 0; q4 < 4; ++q4) {
                    const int tc = (wn * WN) / 2 + j * 32 + q4 * 8 + ncol;
                    const int q = (j * 4 + q4) * 2;
#pragma unroll
                    for (int i = 0; i < FM; ++i) {
                        u16x4 v;
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            float g = rt16(g1_reg<HB>(acc[i][2 * j][q4 * 4 + e], sxr[i], qsw[q][e], qb[q][e]));
                            float u = rt16(g1_reg<HB>(acc[i][2 * j + 1][q4 * 4 + e], sxr[i], qsw[q + 1][e], qb[q + 1][e]));
                            v[e] = f2h(silu(g) * u);
                        }
                        put(trow(i), tc, v);
                    }
                }
            }
        } else {
#pragma unroll
            for (int j = 0; j < FN; ++j) {
#pragma unroll
                for (int q4 = 0; q4 < 4; ++q4) {
                    const int tc = wn * WN + j * 32 + q4 * 8 + ncol;
                    const int q = j * 4 + q4;
#pragma unroll
                    for (int i = 0; i < FM; ++i) {
                        float y[4];
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            if constexpr (EP == Epi::F16Bias) {
                                const float a = acc[i][j][q4 * 4 + e];
                                y[e] = HB ? a + h2f(qb[q][e]) : a;
                            } else {
                                y[e] = g1_reg<HB>(acc[i][j][q4 * 4 + e], sxr[i], qsw[q][e], qb[q][e]);
                            }
                        }
                        put(trow(i), tc, f2h4(y[0], y[1], y[2], y[3]));
                    }
                }
            }
        }
        };
        if (has_bias) convert(std::true_type{});
        else convert(std::false_type{});
        const int gcol0 = (EP == Epi::SwiGLU) ? tn * (BN / 2) : n0;
        uint16_t* out = static_cast<uint16_t*>(p.out);
        // Padded output (PADWO = Wo, a tile of whole output rows of one frame): output pixel (t, i, j) of
        // batch item b goes to [b, t + pad_front, i + top, j + left] of [B, Do + pad_front, Ho + top +
        // bottom, Wo + left + right, N], and the reflect border of 0 or 1 per side is written with it: row
        // 1 again as row 0 (top), row Ho - 2 as row Ho + top (bottom), likewise columns.  That is the input
        // layout of the causal downsample conv that reads it.  Frames below pad_front are not written.
        int64_t pframe = 0;   // first padded pixel row of the tile's frame
        int oh0 = 0, ow0 = 0;
        uint16_t* tile_out = out;   // padded position of the tile's output pixel (0, 0), channel 0
        constexpr int TWP = TILEW ? TILEW : (PADWO > 0 ? PADWO : 1);   // pixels per tile row
        if constexpr (PADWO > 0) {
            const int fpix = p.Ho * PADWO;
            const int fr = m0 / fpix;
            oh0 = (m0 - fr * fpix) / PADWO;
            ow0 = (m0 - fr * fpix) - oh0 * PADWO;
            const int bi = fr / p.Do, od = fr - bi * p.Do;
            pframe = ((int64_t)bi * (p.Do + p.pad_front) + od + p.pad_front) * (p.Ho + p.pad_top + p.pad_bottom);
            tile_out = out + ((pframe + oh0 + p.pad_top) * (PADWO + p.pad_left + p.pad_right) + p.pad_left + ow0) * p.ldo;
        }
        // one 8-column chunk of tile row r (output row grow = gidx(r)); every caller has checked vec_out and N
        auto store_chunk = [&](int r, int grow, int gcol, const u16x8& v) {
            if constexpr (PADWO == 0) {
                *reinterpret_cast<u16x8*>(out + (int64_t)grow * p.ldo + gcol) = v;
            } else {
                const int ri = r / TWP, owr = r - ri * TWP, ow = ow0 + owr;
                const int wp = PADWO + p.pad_left + p.pad_right;
                // a tile spans 512 / TWP rows: the offset from tile_out stays below 2^31 elements
                *reinterpret_cast<u16x8*>(tile_out + (ri * wp + owr) * (int)p.ldo + gcol) = v;
                const int oh = oh0 + ri;
                const bool rt = p.pad_top && oh == 1, rb = p.pad_bottom && oh == p.Ho - 2;
                const bool cl = p.pad_left && ow == 1, cr = p.pad_right && ow == PADWO - 2;
                if (rt | rb | cl | cr) {   // border pixels: the reflected copies
                    // padded rows / columns that hold this pixel (-1: none)
                    const int r0 = oh + p.pad_top, r1 = rt ? 0 : -1, r2 = rb ? p.Ho + p.pad_top : -1;
                    const int c0 = ow + p.pad_left, c1 = cl ? 0 : -1, c2 = cr ? PADWO + p.pad_left : -1;
                    auto put = [&](int pr, int pc) {
                        if (pr >= 0 && pc >= 0)
                            *reinterpret_cast<u16x8*>(out + ((pframe + pr) * wp + pc) * p.ldo + gcol) = v;
                    };
                    put(r0, c1); put(r0, c2);
                    put(r1, c0); put(r1, c1); put(r1, c2);
                    put(r2, c0); put(r2, c1); put(r2, c2);
                }
            }
        };
        // Statistics epilogue (window conv, whole 512 x 128 tiles of one frame, batch one): the stores of
        // the plain path, then the GroupNorm(32) partial statistics of the tile as the encoder producer's
        // statistics pass would form them for a 512-pixel chunk, on the stored values (with the residual)
        // plus gn_bias (fp16 sum, one rounding).  Thread tid keeps tile columns 8 (tid % 16) .. + 7 of
        // tile pixels pl + 32 s (pl = tid / 16, s = 0 .. 15, tile pixel = tile row * TILEW + column):
        // per pixel a group's channels are summed left to right and added to the thread's running sum;
        // the 32 pixel lanes combine as the adjacent tree (pl, pl + 1), then pairs of pairs, ..., whose
        // first two levels are the shuffles to lanes ^ 16 and ^ 32 and the last three the sum over the
        // eight waves ((w0 + w1) + (w2 + w3)) + ((w4 + w5) + (w6 + w7)).  avg = sum / (512 cg); M2 is
        // the same sum of (v - avg)^2 per channel.  Max and min per channel are exact in any order.
        if constexpr (EP == Epi::Dequant && SROWS && TILEW > 0 && PADWO == 0) {
            if (p.gn_avg != nullptr) {
                static_assert(BM == 512 && RCH == 16 && NW == 8 && LDS_BYTES >= BM * OUTW * 2 + 9472,
                              "statistics epilogue: 512 x 128 tiles of 8 waves, 9.25 KB of LDS past the tile");
                constexpr int NT = NW * 64, PER = BM * RCH / NT;
                const int ch = tid & 15;
                const int gcol = gcol0 + ch * 8;
                float* const gred = reinterpret_cast<float*>(smem + BM * OUTW * 2);   // [wave][32]
                float* const gavg = gred + NW * 32;                                     // [32]
                // per wave and channel the (max, min) pair as two floats: the values are fp16, but kept as
                // fp32 here, since the compiler narrows a maximum of fp16 values to v_max3_f16 and then packs
                // two such results with a v_or_b32 that assumes the upper half of the register is zero,
                // which v_max3_f16 on gfx950 does not clear (the packed minima came out corrupted)
                float* const gext = gavg + 32;                                           // [wave][128][2]
                u16x8 v[PER];
                if (p.res != nullptr) {
#pragma unroll
                    for (int k = 0; k < PER; ++k)
                        v[k] = *reinterpret_cast<const u16x8*>(p.res + (int64_t)gidx((tid >> 4) + 32 * k) * p.ldo + gcol);
                }
                u16x8 gb{};
                if (p.gn_bias) gb = *reinterpret_cast<const u16x8*>(p.gn_bias + gcol);
                // tile row r is output row m0 + (r / TILEW) * Wo + r % TILEW: 32-bit element offsets from the
                // tile's first row (at most 8 * 256 rows of 256 channels)
                uint16_t* const tile_out = out + (int64_t)m0 * p.ldo + gcol;
                lds_barrier();   // the output tile is complete in LDS
                // all pieces from LDS first (with the residual added), then the stores
#pragma unroll
                for (int k = 0; k < PER; ++k) {
                    const int r = (tid >> 4) + 32 * k;
                    const u16x8 y = *reinterpret_cast<const u16x8*>(ep + r * (OUTW * 2) + ((ch ^ skey(r)) << 4));
                    v[k] = p.res != nullptr ? add_f16x8(v[k], y) : y;   // fp16(res + y), one rounding
                }
#pragma unroll
                for (int k = 0; k < PER; ++k) {
                    const int r = (tid >> 4) + 32 * k;
                    *reinterpret_cast<u16x8*>(tile_out + ((r / TILEW) * p.Wo + r % TILEW) * (int)p.ldo) = v[k];
                    if (p.gn_bias) v[k] = add_f16x8(v[k], gb);
                }
                const int fpix = p.Ho * p.Wo;
                const int fr = m0 / fpix, rem = m0 - fr * fpix;
                const int oh0 = rem / p.Wo, owb = rem - oh0 * p.Wo;
                const int chunk = (oh0 / (BM / TILEW)) * (p.Wo / TILEW) + owb / TILEW;
                const int64_t cbase = (int64_t)fr * kGnGroups * p.gn_nchunk + chunk;   // + group * nchunk
                auto stats = [&](auto cg_c) {
                    constexpr int CG = decltype(cg_c)::value;
                    constexpr int GPT = 8 / CG, NG = 128 / CG;
                    float ls[GPT], vmx[8], vmn[8];
#pragma unroll
                    for (int gi = 0; gi < GPT; ++gi) ls[gi] = 0.0f;
#pragma unroll
                    for (int e = 0; e < 8; ++e) { vmx[e] = -__builtin_inff(); vmn[e] = __builtin_inff(); }
#pragma unroll
                    for (int k = 0; k < PER; ++k) {
                        float f[8];
#pragma unroll
                        for (int e = 0; e < 8; ++e) {
                            f[e] = h2f(v[k][e]);
                            vmx[e] = __builtin_fmaxf(vmx[e], f[e]);
                            vmn[e] = __builtin_fminf(vmn[e], f[e]);
                        }
#pragma unroll
                        for (int gi = 0; gi < GPT; ++gi) {
                            float ps = f[gi * CG];
#pragma unroll
                            for (int i = 1; i < CG; ++i) ps = ps + f[gi * CG + i];
                            ls[gi] = ls[gi] + ps;
                        }
                    }
                    // the tree over the 32 pixel lanes; lanes 0-15 of each wave hold its part
                    auto lane_tree = [&](float (&x)[GPT]) {
#pragma unroll
                        for (int gi = 0; gi < GPT; ++gi) {
                            x[gi] = x[gi] + __shfl_xor(x[gi], 16, 64);
                            x[gi] = x[gi] + __shfl_xor(x[gi], 32, 64);
                        }
                        if (lane < 16) {
#pragma unroll
                            for (int gi = 0; gi < GPT; ++gi) gred[wave * 32 + ch * GPT + gi] = x[gi];
                        }
                    };
                    auto wave_tree = [&](int g) {
                        const float* r = gred + g;
                        return ((r[0] + r[32]) + (r[64] + r[96])) + ((r[128] + r[160]) + (r[192] + r[224]));
                    };
                    lane_tree(ls);
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        vmx[e] = __builtin_fmaxf(vmx[e], __shfl_xor(vmx[e], 16, 64));
                        vmx[e] = __builtin_fmaxf(vmx[e], __shfl_xor(vmx[e], 32, 64));
                        vmn[e] = __builtin_fminf(vmn[e], __shfl_xor(vmn[e], 16, 64));
                        vmn[e] = __builtin_fminf(vmn[e], __shfl_xor(vmn[e], 32, 64));
                    }
                    if (lane < 16) {
#pragma unroll
                        for (int e = 0; e < 8; ++e) {
                            gext[2 * (wave * 128 + ch * 8 + e)] = vmx[e];
                            gext[2 * (wave * 128 + ch * 8 + e) + 1] = vmn[e];
                        }
                    }
                    lds_barrier();
                    if (tid < NG) gavg[tid] = wave_tree(tid) / (float)(BM * CG);
                    if (tid >= 256 && tid < 384) {
                        const int c = tid - 256;
                        float mx = gext[2 * c], mn = gext[2 * c + 1];
#pragma unroll
                        for (int w = 1; w < NW; ++w) {
                            mx = __builtin_fmaxf(mx, gext[2 * (w * 128 + c)]);
                            mn = __builtin_fminf(mn, gext[2 * (w * 128 + c) + 1]);
                        }
                        // the extremes are stored values: exact as fp16
                        p.gn_ext[((int64_t)fr * p.gn_nchunk + chunk) * p.N + n0 + c] =
                            (uint32_t)f2h(mx) | ((uint32_t)f2h(mn) << 16);
                    }
                    lds_barrier();
                    float a[GPT], lm[GPT];
#pragma unroll
                    for (int gi = 0; gi < GPT; ++gi) { a[gi] = gavg[ch * GPT + gi]; lm[gi] = 0.0f; }
#pragma unroll
                    for (int k = 0; k < PER; ++k) {
#pragma unroll
                        for (int gi = 0; gi < GPT; ++gi) {
                            float dv = h2f(v[k][gi * CG]) - a[gi];
                            float pm = dv * dv;
#pragma unroll
                            for (int i = 1; i < CG; ++i) {
                                dv = h2f(v[k][gi * CG + i]) - a[gi];
                                pm = pm + dv * dv;
                            }
                            lm[gi] = lm[gi] + pm;
                        }
                    }
                    lane_tree(lm);
                    lds_barrier();
                    if (tid < NG) {
                        const int64_t dst = cbase + (int64_t)(n0 / CG + tid) * p.gn_nchunk;
                        p.gn_avg[dst] = gavg[tid];
                        p.gn_m2[dst] = wave_tree(tid);
                    }
                };
                if (p.N == 128) stats(std::integral_constant<int, 4>{});
                else stats(std::integral_constant<int, 8>{});
                return;
            }
        }
        if (p.res == nullptr) {
            lds_barrier();   // the output tile is complete in LDS
            constexpr int NT = NW * 64;
            if (PADWO == 0 && (BM * RCH) % NT == 0 && NT % RCH == 0 && p.vec_out && gcol0 + OUTW <= p.N &&
                p.ldo <= 65536) {
                // Every column of the tile lies inside N: a thread keeps one 8-column chunk for all its rows,
                // reads all its pieces from LDS first and stores them from the tile's first output row with
                // 32-bit element offsets (the tile spans at most 512 consecutive rows, or 8 rows of a frame at
                // most 256 wide); rows past M (the last tile of a GEMM) are skipped.
                constexpr int PER = BM * RCH / NT;
                const int ch = tid % RCH;
                uint16_t* const tile_out = out + (int64_t)m0 * p.ldo + gcol0 + ch * 8;
                u16x8 v[PER];
#pragma unroll
                for (int k = 0; k < PER; ++k) {
                    const int r = (tid + k * NT) / RCH;
                    v[k] = *reinterpret_cast<const u16x8*>(ep + r * (OUTW * 2) + ((ch ^ skey(r)) << 4));
                }
                const int rows = p.M - m0;
#pragma unroll
                for (int k = 0; k < PER; ++k) {
                    const int r = (tid + k * NT) / RCH;
                    const int orow = TILEW ? (r / (TILEW ? TILEW : 1)) * p.Wo + r % (TILEW ? TILEW : 1) : r;
                    if (TILEW || r < rows) *reinterpret_cast<u16x8*>(tile_out + orow * (int)p.ldo) = v[k];
                }
            } else {
#pragma unroll 4
                for (int idx = tid; idx < BM * RCH; idx += NW * 64) {
                    const int r = idx / RCH, ch = idx - r * RCH;
                    const int grow = gidx(r), gcol = gcol0 + ch * 8;
                    if (grow >= p.M || gcol >= p.N) continue;
                    const u16x8 v = *reinterpret_cast<const u16x8*>(ep + r * (OUTW * 2) + ((ch ^ skey(r)) << 4));
                    if (PADWO > 0 || (p.vec_out && gcol + 8 <= p.N)) {
                        store_chunk(r, grow, gcol, v);
                    } else {
                        uint16_t* dst = out + (int64_t)grow * p.ldo + gcol;
#pragma unroll
                        for (int e = 0; e < 8; ++e)
                            if (gcol + e < p.N) dst[e] = v[e];
                    }
                }
            }
            // Chunk statistics (h3v_conv3d_f16_gn: 256 x 128 tiles of 8 waves, 128 output channels, every tile
            // 256 consecutive pixels of one frame, batch one): the GroupNorm(32) partials of the tile exactly as
            // the INT8 producer's statistics pass (gn_partial, C = 128) forms them for a 256-pixel chunk, from
            // the staged tile instead of memory.  Threads 0-255: cv = tid % 16 owns channels 8 cv .. 8 cv + 7
            // (groups 2 cv, 2 cv + 1) and pl = tid / 16 the pixels pl + 16 s (s = 0 .. 15); per pixel a group's
            // four channels are summed left to right and added to the lane's running sum; the 16 pixel lanes
            // combine by the halving tree off = 8, 4, 2, 1 (lane i += lane i + off); avg = sum / 1024, and M2
            // the same sums of (v - avg)^2.  Channel maxima and minima are exact in any order.
            if constexpr (EP == Epi::F16Bias && BM == 256 && OUTW == 128 && NW == 8 && !SROWS && TILEW == 0 &&
                          PADWO == 0) {
                if (p.gn_avg != nullptr) {
                    constexpr int PL = 16, STEPS = 16, CG = 4;
                    float* const sred = reinterpret_cast<float*>(smem + RING);   // [PL][32]
                    float* const savg = sred + PL * 32;                         // [32]
                    float* const sext = savg + 32;                              // [wave][128][2], waves 0-3
                    const bool act = tid < 256;
                    const int cv = tid & 15, pl = (tid >> 4) & 15;
                    u16x8 xv[STEPS];
                    float ls[2] = {0.0f, 0.0f}, vmx[8], vmn[8];
#pragma unroll
                    for (int e = 0; e < 8; ++e) { vmx[e] = -__builtin_inff(); vmn[e] = __builtin_inff(); }
                    if (act) {
#pragma unroll
                        for (int st = 0; st < STEPS; ++st) {
                            const int r = pl + st * PL;
                            xv[st] = *reinterpret_cast<const u16x8*>(ep + r * (OUTW * 2) + ((cv ^ skey(r)) << 4));
                        }
#pragma unroll
                        for (int st = 0; st < STEPS; ++st) {
                            float f[8];
#pragma unroll
                            for (int e = 0; e < 8; ++e) {
                                f[e] = h2f(xv[st][e]);
                                vmx[e] = __builtin_fmaxf(vmx[e], f[e]);
                                vmn[e] = __builtin_fminf(vmn[e], f[e]);
                            }
#pragma unroll
                            for (int gi = 0; gi < 2; ++gi) {
                                float ps = f[gi * CG];
#pragma unroll
                                for (int i = 1; i < CG; ++i) ps = ps + f[gi * CG + i];
                                ls[gi] = ls[gi] + ps;
                            }
                        }
#pragma unroll
                        for (int gi = 0; gi < 2; ++gi) sred[pl * 32 + cv * 2 + gi] = ls[gi];
#pragma unroll
                        for (int e = 0; e < 8; ++e) {
                            vmx[e] = __builtin_fmaxf(vmx[e], __shfl_xor(vmx[e], 16, 64));
                            vmx[e] = __builtin_fmaxf(vmx[e], __shfl_xor(vmx[e], 32, 64));
                            vmn[e] = __builtin_fminf(vmn[e], __shfl_xor(vmn[e], 16, 64));
                            vmn[e] = __builtin_fminf(vmn[e], __shfl_xor(vmn[e], 32, 64));
                        }
                        if (lane < 16) {
#pragma unroll
                            for (int e = 0; e < 8; ++e) {
                                sext[2 * (wave * 128 + cv * 8 + e)] = vmx[e];
                                sext[2 * (wave * 128 + cv * 8 + e) + 1] = vmn[e];
                            }
                        }
                    }
                    const int hw = p.Ho * p.Wo;
                    const int fr = m0 / hw, chunk = (m0 - fr * hw) / 256;
                    // the halving tree of gn_partial over the lane sums of group g, in place
                    auto tree = [&](int g) {
                        for (int off = PL / 2; off >= 1; off >>= 1)
                            for (int i = 0; i < off; ++i) sred[i * 32 + g] = sred[i * 32 + g] + sred[(i + off) * 32 + g];
                        return sred[g];
                    };
                    lds_barrier();
                    if (tid < 32) savg[tid] = tree(tid) / (float)(256 * CG);
                    if (tid >= 256 && tid < 384) {
                        const int c = tid - 256;
                        float mx = sext[2 * c], mn = sext[2 * c + 1];
#pragma unroll
                        for (int w = 1; w < 4; ++w) {
                            mx = __builtin_fmaxf(mx, sext[2 * (w * 128 + c)]);
                            mn = __builtin_fminf(mn, sext[2 * (w * 128 + c) + 1]);
                        }
                        // the extremes are stored fp16 values: exact as fp16
                        p.gn_ext[((int64_t)fr * p.gn_nchunk + chunk) * 128 + c] =
                            (uint32_t)f2h(mx) | ((uint32_t)f2h(mn) << 16);
                    }
                    lds_barrier();
                    float lm[2] = {0.0f, 0.0f};
                    if (act) {
                        const float a0 = savg[cv * 2], a1 = savg[cv * 2 + 1];
#pragma unroll
                        for (int st = 0; st < STEPS; ++st) {
#pragma unroll
                            for (int gi = 0; gi < 2; ++gi) {
                                const float a = gi ? a1 : a0;
                                float dv = h2f(xv[st][gi * CG]) - a;
                                float pm = dv * dv;
#pragma unroll
                                for (int i = 1; i < CG; ++i) {
                                    dv = h2f(xv[st][gi * CG + i]) - a;
                                    pm = pm + dv * dv;
                                }
                                lm[gi] = lm[gi] + pm;
                            }
                        }
#pragma unroll
                        for (int gi = 0; gi < 2; ++gi) sred[pl * 32 + cv * 2 + gi] = lm[gi];
                    }
                    lds_barrier();
                    if (tid < 32) {
                        // group-major [frame][group][chunk], as gn_partial
                        const int64_t dst = ((int64_t)fr * 32 + tid) * p.gn_nchunk + chunk;
                        p.gn_m2[dst] = tree(tid);
                        p.gn_avg[dst] = savg[tid];
                    }
                }
            }
        } else {
            // The residual block's closing add, fused: out = fp16(fp32(res) + fp32(y)) with y the rounded
            // output.  Every residual piece this thread stores is loaded before the barrier (the
            // accumulators are dead by now), so the loads overlap the barrier and each other.
            constexpr int NT = NW * 64;
            constexpr int PER = (BM * RCH + NT - 1) / NT;
            u16x8 rv[PER] = {};
#pragma unroll
            for (int i = 0; i < PER; ++i) {
                const int idx = tid + i * NT;
                const int r = idx / RCH, ch = idx - r * RCH;
                const int grow = gidx(r), gcol = gcol0 + ch * 8;
                if (idx < BM * RCH && grow < p.M && p.vec_out && gcol + 8 <= p.N)
                    rv[i] = *reinterpret_cast<const u16x8*>(p.res + (int64_t)grow * p.ldo + gcol);
            }
            lds_barrier();   // the output tile is complete in LDS
            if (NT % RCH == 0 && (PADWO > 0 || (p.vec_out && gcol0 + OUTW <= p.N))) {
                // every piece is a whole 16-byte chunk and a thread keeps one chunk column: all pieces from
                // LDS with the residual added first, then the stores
                const int gcol = gcol0 + (tid % RCH) * 8;
                u16x8 rb{};
                if (p.res_bias) rb = *reinterpret_cast<const u16x8*>(p.res_bias + gcol);
#pragma unroll
                for (int i = 0; i < PER; ++i) {
                    const int idx = tid + i * NT;
                    if (idx >= BM * RCH) continue;
                    const int r = idx / RCH, ch = idx - r * RCH;
                    const u16x8 v = *reinterpret_cast<const u16x8*>(ep + r * (OUTW * 2) + ((ch ^ skey(r)) << 4));
                    if (p.res_bias) {   // fp16(res + (y + b)): both adds in fp32, one rounding
#pragma unroll
                        for (int e = 0; e < 8; ++e) rv[i][e] = f2h(h2f(rv[i][e]) + (h2f(v[e]) + h2f(rb[e])));
                    } else {
                        rv[i] = add_f16x8(rv[i], v);   // fp16(res + y), one rounding
                    }
                }
#pragma unroll
                for (int i = 0; i < PER; ++i) {
                    const int idx = tid + i * NT;
                    const int r = idx / RCH;
                    const int grow = gidx(r);
                    if (idx >= BM * RCH || grow >= p.M) continue;
                    store_chunk(r, grow, gcol, rv[i]);
                }
                return;
            }
#pragma unroll
            for (int i = 0; i < PER; ++i) {
                const int idx = tid + i * NT;
                const int r = idx / RCH, ch = idx - r * RCH;
                const int grow = gidx(r), gcol = gcol0 + ch * 8;
                if (idx >= BM * RCH || grow >= p.M || gcol >= p.N) continue;
                u16x8 v = *reinterpret_cast<const u16x8*>(ep + r * (OUTW * 2) + ((ch ^ skey(r)) << 4));
                if (PADWO > 0 || (p.vec_out && gcol + 8 <= p.N)) {
                    if (p.res_bias) {   // fp16(res + (y + b)): both adds in fp32, one rounding
                        const u16x8 rb = *reinterpret_cast<const u16x8*>(p.res_bias + gcol);
#pragma unroll
                        for (int e = 0; e < 8; ++e) v[e] = f2h(h2f(rv[i][e]) + (h2f(v[e]) + h2f(rb[e])));
                    } else {
                        v = add_f16x8(rv[i], v);   // fp16(res + y), one rounding
                    }
                    store_chunk(r, grow, gcol, v);
                } else {
                    uint16_t* dst = out + (int64_t)grow * p.ldo + gcol;
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        if (gcol + e < p.N) {
                            const int64_t o = (int64_t)grow * p.ldo + gcol + e;
                            const float y = p.res_bias ? h2f(v[e]) + h2f(p.res_bias[gcol + e]) : h2f(v[e]);
                            dst[e] = f2h(h2f(p.res[o]) + y);
                        }
                }
            }
        }
    }
}

// BM x BN x BK workgroup tile, WGM x WGN waves of (BM/WGM) x (BN/WGN).  A and B
// stream through separate LDS rings of NSA and NSB slots.  Loads are issued B
// before A for each stage, so with NSB = 2 < NSA the barrier that publishes
// stage it+1 can leave the newest A batch (stage it+NSA-1) in flight: vmcnt
// counts loads in issue order.
template <int BM, int BN, int BK, int WGM, int WGN, int NSA, int NSB, AMode AM, Epi EP>
__global__ __launch_bounds__(WGM * WGN * 64) void gemm_i8_mfma(GemmParams p) {
    static_assert(BK == 64 || BK == 128, "K step");
    constexpr int NW = WGM * WGN;
    constexpr int WM = BM / WGM, WN = BN / WGN;
    constexpr int FM = WM / 32, FN = WN / 32;
    constexpr int KS = BK / 32;                               // MFMA K sub-steps per K step
    constexpr int RPI = 1024 / BK;                            // tile rows per DMA instruction
    constexpr int LPR = BK / 16;                              // DMA lanes per tile row
    constexpr int A_BYTES = BM * BK, B_BYTES = BN * BK;
    constexpr int B_RING = NSA * A_BYTES, RING = NSA * A_BYTES + NSB * B_BYTES;
    // Only the first half of the waves (one per SIMD: wave w runs on SIMD w % 4) issue the DMA.
    // A global_load_lds instruction holds up its wave's MFMA issue for about as long as the
    // transfer takes; with every wave issuing, both waves of a SIMD stall together and its matrix
    // pipe idles (measured: 62% of peak for MFMA + DMA on all waves, 72% with one issuing wave per
    // SIMD, in a barrier-free probe).  The other wave keeps the pipe busy meanwhile.
    constexpr int NWD = NW / 2;                               // DMA-issuing waves
    constexpr int A_PW = BM / RPI / NWD, B_PW = BN / RPI / NWD; // row groups per issuing wave
    constexpr int LPS = A_PW + B_PW;                          // DMA instructions per stage per issuing wave
    static_assert(A_PW * RPI * NWD == BM && B_PW * RPI * NWD == BN, "tile rows must split into row groups per wave");
    static_assert(EP != Epi::SwiGLU || (WN % 64) == 0, "SwiGLU pairs need 64-column wave tiles");
    static_assert(NSA >= 2 && NSA <= 4 && NSB >= 2 && NSB <= NSA && (NSA == NSB || NSB == 2), "LDS ring depths");
    static_assert((NSA - 1) * A_PW + (NSB - 1) * B_PW < 64, "outstanding DMA must fit vmcnt");

    extern __shared__ __attribute__((aligned(1024))) int8_t smem[];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform (scalar)
    const int wm = wave / WGN, wn = wave % WGN;

    int tm, tn;
    grouped_tile(xcd_remap(blockIdx.x, gridDim.x), p.tiles_m, p.tiles_n, 8, tm, tn);
    if constexpr (AM == AMode::Conv) {
        // Visit the tiles of one row block for every frame consecutively: the
        // output frames t, t-1, t-2 that read input frame t through kd = 0, 1, 2
        // then run together and share its rows in L2 (frame-major order fetched
        // the input about 2.8 times from HBM).
        if (p.conv_tpf > 0) {
            const int nf = p.tiles_m / p.conv_tpf;
            tm = (tm % nf) * p.conv_tpf + tm / nf;
        }
    }
    const int m0 = tm * BM, n0 = tn * BN;

    const int lrow = lane / LPR;
    const int lslot = lane % LPR;
    const bool dma_wave = wave < NWD;
    const int dw = dma_wave ? wave : 0;                       // index among the issuing waves

    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc((void*)p.a, 0, (int)p.a_bytes, kRsrcWord3);
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc((void*)p.b, 0, (int)p.b_bytes, kRsrcWord3);
    uint32_t aoff[A_PW];
#pragma unroll
    for (int j = 0; j < A_PW; ++j) {
        const int r = (dw * A_PW + j) * RPI + lrow;
        int m = m0 + r;
        m = m < p.M ? m : p.M - 1;
        aoff[j] = (uint32_t)((AM == AMode::Gemm ? (int64_t)m * p.lda : conv_row_offset(p, m)) + ((lslot ^ swz<BK>(r)) << 4));
    }
    uint32_t boff[B_PW];
#pragma unroll
    for (int j = 0; j < B_PW; ++j) {
        int r = (dw * B_PW + j) * RPI + lrow;
        int wrow;
        if constexpr (EP == Epi::SwiGLU) {
            // tile row r -> pair r/64, half (r/32)&1 (0 gate, 1 up), column r&31
            int c = tn * (BN / 2) + (r >> 6) * 32 + (r & 31);
            c = c < p.N ? c : p.N - 1;
            wrow = ((r >> 5) & 1) ? p.N + c : c;
        } else {
            int n = n0 + r;
            wrow = n < p.N ? n : p.N - 1;
        }
        boff[j] = (uint32_t)((int64_t)wrow * p.K + ((lslot ^ swz<BK>(r)) << 4));
    }

    // K blocks of this workgroup: split blockIdx.y of k_splits (the whole K without a split), minus the
    // causal-zero taps of a conv tile's first frames
    const int nsplit = p.k_splits > 1 ? p.k_splits : 1;
    const int kper = p.K / BK / nsplit;
    const int kend = (int)blockIdx.y * kper + kper;
    int kb0 = (int)blockIdx.y * kper;
    if constexpr (AM == AMode::Conv) {
        const int skip = conv_first_kblock(p, m0, BM, BK);
        kb0 = skip > kb0 ? skip : kb0;
    }
    const int nk = kend > kb0 ? kend - kb0 : 0;

    // A stages are issued strictly in order, so the conv's k offset is kept as a
    // running (kd, kh, kw, c0) position advanced by BK per issue: no integer
    // division in the loop.
    int ck_kd = 0, ck_kh = 0, ck_kw = 0, ck_c0 = 0;
    if constexpr (AM == AMode::Conv) {
        const int k0 = kb0 * BK;
        const int tap = k0 / p.C;
        ck_c0 = k0 - tap * p.C;
        ck_kd = tap / (p.KH * p.KW);
        const int rem = tap - ck_kd * p.KH * p.KW;
        ck_kh = rem / p.KW;
        ck_kw = rem - ck_kh * p.KW;
    }
    auto issue_a = [&](int it) {
        int8_t* sa = smem + (it % NSA) * A_BYTES;
        int64_t koff;
        if constexpr (AM == AMode::Gemm) {
            koff = (int64_t)(kb0 + it) * BK;
        } else {
            koff = (((int64_t)ck_kd * p.Hp + ck_kh) * p.Wp + ck_kw) * p.C + ck_c0;
            ck_c0 += BK;
            if (ck_c0 == p.C) {
                ck_c0 = 0;
                if (++ck_kw == p.KW) {
                    ck_kw = 0;
                    if (++ck_kh == p.KH) {
                        ck_kh = 0;
                        ++ck_kd;
                    }
                }
            }
        }
        if (!dma_wave) return;
#pragma unroll
        for (int j = 0; j < A_PW; ++j) lds_dma16(ra, aoff[j], (uint32_t)koff, sa + (dw * A_PW + j) * 1024);
    };
    auto issue_b = [&](int it) {
        const int kb = kb0 + it;
        int8_t* sb = smem + B_RING + (it % NSB) * B_BYTES;
        if (!dma_wave) return;
#pragma unroll
        for (int j = 0; j < B_PW; ++j) lds_dma16(rb, boff[j], (uint32_t)kb * BK, sb + (dw * B_PW + j) * 1024);
    };

    // F16Bias: fp16 operands with p.C and p.K given in bytes (2 per element), so every k
    // offset above stays a byte offset; v_mfma_f32_32x32x16_f16 reads the same 16 bytes per
    // lane as the int8 instruction and accumulates in fp32.
    using Acc = std::conditional_t<kF16Ops<EP>, f32x16, v16i>;
    Acc acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = Acc{};

    // fragment addressing: lane reads row (lane & 31) of a 32-row block, 16-byte
    // k-chunk (lane >> 5) + 2*ks of the K step
    const int frow = lane & 31;
    const int fhi = lane >> 5;
    auto load_frags = [&](int it, int ks, v4i (&af)[FM], v4i (&bf)[FN]) {
        const int8_t* sa = smem + (it % NSA) * A_BYTES;
        const int8_t* sb = smem + B_RING + (it % NSB) * B_BYTES;
        const int kc = fhi + 2 * ks;
#pragma unroll
        for (int i = 0; i < FM; ++i) {
            const int r = wm * WM + i * 32 + frow;
            af[i] = *reinterpret_cast<const v4i*>(sa + r * BK + ((kc ^ swz<BK>(r)) << 4));
        }
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int r = wn * WN + j * 32 + frow;
            bf[j] = *reinterpret_cast<const v4i*>(sb + r * BK + ((kc ^ swz<BK>(r)) << 4));
        }
    };
    auto mfma_all = [&](const v4i (&af)[FM], const v4i (&bf)[FN]) {
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                if constexpr (kF16Ops<EP>)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, bf[j]),
                                                                       __builtin_bit_cast(half8, af[i]), acc[i][j], 0, 0, 0);
                else
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(bf[j], af[i], acc[i][j], 0, 0, 0);
            }
    };

    // Prologue: fill both rings (B before A per stage), then wait for stage 0.
    v4i fa[2][FM], fb[2][FN];
#pragma unroll
    for (int s = 0; s < NSA; ++s) {
        if (s < NSB && s < nk) issue_b(s);
        if (s < nk) issue_a(s);
    }
    if (nk > 0) {
        if (nk >= NSA) wait_vmcnt<(NSA - 1) * A_PW + (NSB - 1) * B_PW>();
        else wait_vmcnt<0>();
        lds_barrier();
        load_frags(0, 0, fa[0], fb[0]);
    }
    // Per K step, KS sub-steps of 32: MFMA sub-step ks while reading the
    // fragments of ks+1 into the other register buffer.  Before the last
    // sub-step the barrier publishes the next stage and the freed ring slot is
    // refilled; the last sub-step's MFMAs then hide the reads of the next K
    // step's first fragments.  sched_group_barrier interleaves the MFMAs with
    // the LDS reads so the reads hide under the matrix pipeline.
    constexpr int NFRAG = FM + FN;
    constexpr int NMFMA = FM * FN;
    static_assert(KS % 2 == 0, "fragment double buffer parity");
    for (int it = 0; it < nk; ++it) {
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const int cur = ks & 1;
            if (ks == KS - 1) {
                const bool more = it + 1 < nk;
                if (more) {
                    // stage it+1 must have landed; later loads may stay in flight
                    if constexpr (NSA == NSB) {
                        wait_stage<LPS>(nk - 2 - it < NSA - 2 ? nk - 2 - it : NSA - 2);
                    } else {
                        // the only load issued after B(it+1) is A(it+NSA-1)
                        if (it + NSA - 1 < nk) wait_vmcnt<A_PW>();
                        else wait_vmcnt<0>();
                    }
                    lds_barrier();
                    if (it + NSB < nk) issue_b(it + NSB);
                    if (it + NSA < nk) issue_a(it + NSA);
                }
                __builtin_amdgcn_sched_barrier(0);
                mfma_all(fa[cur], fb[cur]);
                // on the last step this re-reads a stale slot; the values are never used
                load_frags(more ? it + 1 : it, 0, fa[cur ^ 1], fb[cur ^ 1]);
            } else {
                mfma_all(fa[cur], fb[cur]);
                load_frags(it, ks + 1, fa[cur ^ 1], fb[cur ^ 1]);
            }
#pragma unroll
            for (int g = 0; g < NFRAG; ++g) {
                __builtin_amdgcn_sched_group_barrier(0x008, NMFMA / NFRAG, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }

    write_tile<BM, BN, WGM, WGN, RING, EP>(p, acc, smem, m0, n0, tn);
}

// Ping-pong INT8 GEMM (AMode::Gemm, Dequant or Int32 epilogue): 256 x 256 x 128 tiles, 8 waves in two
// groups of four (one wave of each group per SIMD: wave w runs on SIMD w % 4).  Group g owns output rows
// 128 g .. 128 g + 127 of the tile, and wave s of a group the 64 columns 64 s .. 64 s + 63: a 128 x 64 block
// of v_mfma_i32_32x32x32_i8 accumulators, as in gemm_i8_mfma.  Instead of interleaving fragment reads with
// MFMAs inside every wave, the two waves of a SIMD alternate whole phases, one workgroup barrier apart:
//
//   phase 2k     group 0 reads all fragments of K step k from LDS (24 x 16 bytes per lane) and issues
//                the weight DMA of step k + 1; group 1 runs its 32 MFMAs of step k - 1;
//   phase 2k + 1 group 0 runs its 32 MFMAs of step k; group 1 reads its fragments of step k and issues
//                the activation DMA of step k + 2.
//
// So on every SIMD one wave issues nothing but MFMAs for a whole phase while its partner does the LDS reads,
// the LDS-DMA issue and the waits, and the matrix pipe never waits on a fragment read of its own wave.
// Ring: three activation slots and two weight slots of 32 KB (160 KB).  Stage k is read in phases 2k and
// 2k + 1; its slots are refilled (A k + 3, B k + 2) from phase 2k + 2 on, and every issuing wave waits for
// its own loads of stage k + 1 before the barrier that ends phase 2k + 1.  Group 1 starts one phase late
// (an extra barrier up front) and skips the barrier after its last MFMA phase, so both groups pass the same
// number of barriers.  Epilogue: each wave converts its own block into a private 16 KB LDS region and stores
// it as whole 128-byte row segments (no workgroup barrier), so group 0's epilogue runs while group 1 still
// issues its last MFMAs.
template <Epi EP>
__global__ __launch_bounds__(512) void gemm_i8_pingpong(GemmParams p) {
    static_assert(EP == Epi::Dequant || EP == Epi::Int32, "ping-pong GEMM epilogues");
    constexpr int BM = 256, BN = 256, BK = 128;
    constexpr int SLOT = 256 * BK;                        // 32 KB per operand slot
    constexpr int NSA = 3;                                // activation slots; weights have 2
    constexpr int PW = 8;                                 // DMA instructions per issuing wave and stage
    extern __shared__ __attribute__((aligned(1024))) int8_t smem[];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int grp = wave >> 2, sw4 = wave & 3;

    // Tiles of the partial last row block (when M % 256 != 0) take the first workgroup ids.  They skip the
    // MFMAs of their empty rows and finish early, so the CUs that ran them start their full tiles out of
    // step with the rest and the tiles' ends (128 KB of stores each) spread out instead of all falling
    // together: H3 FFN-up (64 tail tiles, then 7 rounds of full ones) 243.5 -> 235.5 us against the tail
    // tiles last.  The full tiles are mapped as in the other GEMMs: per-XCD contiguous ranges, grouped by
    // row blocks (the tail count is a multiple of 8 for the decoder widths, so each full tile keeps its
    // XCD).  Groups of 4 row blocks for outputs of 16 or more column tiles, else 8: H3 QKV 98.4 -> 96.6 us
    // and FFN-up 231.6 -> 228.5 us with 4, attention-out 33.7 -> 34.4 us (mean of four same-box A/B runs,
    // bit-identical); 16 was slower on every shape.
    int tm, tn;
    const int ntail = p.M % BM ? p.tiles_n : 0;
    const int nfull = p.tiles_m * p.tiles_n - ntail;
    if ((int)blockIdx.x < ntail) {
        tm = p.tiles_m - 1;
        tn = blockIdx.x;
    } else {
        grouped_tile(xcd_remap(blockIdx.x - ntail, nfull), p.tiles_m - (ntail ? 1 : 0), p.tiles_n,
                     p.tiles_n >= 16 ? 4 : 8, tm, tn);
    }
    const int m0 = tm * BM, n0 = tn * BN;
    const int nk = p.K / BK;

    // DMA: group 1 moves the activation rows, group 0 the weight rows; wave s of a group the 64 tile rows
    // 64 s .. 64 s + 63, eight rows of 128 bytes per instruction (lane: row lane / 8, chunk lane % 8 of it,
    // fetched from k-chunk (lane % 8) ^ swz(row))
    const int lrow = lane >> 3, lslot = lane & 7;
    const __amdgpu_buffer_rsrc_t rsrc =
        grp ? __builtin_amdgcn_make_buffer_rsrc((void*)p.a, 0, (int)p.a_bytes, kRsrcWord3)
            : __builtin_amdgcn_make_buffer_rsrc((void*)p.b, 0, (int)p.b_bytes, kRsrcWord3);
    uint32_t doff[PW];
#pragma unroll
    for (int j = 0; j < PW; ++j) {
        const int r = (sw4 * PW + j) * 8 + lrow;
        int64_t base;
        if (grp) {
            const int m = m0 + r < p.M ? m0 + r : p.M - 1;
            base = (int64_t)m * p.lda;
        } else {
            const int n = n0 + r < p.N ? n0 + r : p.N - 1;
            base = (int64_t)n * p.K;
        }
        doff[j] = (uint32_t)(base + ((lslot ^ swz<BK>(r)) << 4));
    }
    int8_t* const ring = grp ? smem : smem + NSA * SLOT;
    auto issue = [&](int k) {
        int8_t* dst = ring + (grp ? k % NSA : k & 1) * SLOT + sw4 * PW * 1024;
#pragma unroll
        for (int j = 0; j < PW; ++j) lds_dma16(rsrc, doff[j], (uint32_t)(k * BK), dst + j * 1024);
    };

    v16i acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = v16i{};

    // 32-row accumulator blocks of this wave that hold rows below M (4 except in the last row of tiles: the
    // H3 decoder's M = 7188 leaves 20 rows in it); the MFMAs of the others are skipped, so a tail tile costs a
    // fraction of a full one
    const int vrows = p.M - m0 - grp * 128;
    const int vblk = __builtin_amdgcn_readfirstlane(vrows >= 128 ? 4 : (vrows <= 0 ? 0 : (vrows + 31) / 32));

    // fragments of one K step: lane reads row (lane & 31) of a 32-row block, k-chunk (lane >> 5) + 2 ks
    const int frow = lane & 31, fhi = lane >> 5;
    v4i fa[4][4], fb[4][2];   // [ks][block]
    auto load_frags = [&](int k) {
        const int8_t* sa = smem + (k % NSA) * SLOT;
        const int8_t* sb = smem + NSA * SLOT + (k & 1) * SLOT;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const int kc = fhi + 2 * ks;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r = grp * 128 + i * 32 + frow;
                fa[ks][i] = *reinterpret_cast<const v4i*>(sa + r * BK + ((kc ^ swz<BK>(r)) << 4));
            }
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int r = sw4 * 64 + j * 32 + frow;
                fb[ks][j] = *reinterpret_cast<const v4i*>(sb + r * BK + ((kc ^ swz<BK>(r)) << 4));
            }
        }
    };
    auto mfma_blocks = [&](auto nb) {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
#pragma unroll
            for (int i = 0; i < decltype(nb)::value; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fb[ks][j], fa[ks][i], acc[i][j], 0, 0, 0);
    };

    // the K loop for NB valid accumulator blocks (one instantiation per count, so no branch sits between the
    // MFMAs of a phase)
    auto kloop = [&](auto nb) {
    // prologue: weights 0, 1 by group 0; activations 0, 1, 2 by group 1; stage 0 lands before the first barrier
    if (grp == 0) {
        issue(0);
        if (nk > 1) { issue(1); wait_vmcnt<PW>(); } else { wait_vmcnt<0>(); }
    } else {
        issue(0);
        if (nk > 1) issue(1);
        if (nk > 2) { issue(2); wait_vmcnt<2 * PW>(); }
        else if (nk > 1) wait_vmcnt<PW>();
        else wait_vmcnt<0>();
    }
    lds_barrier();
    if (grp == 1) lds_barrier();                      // group 1 runs one phase behind
    __builtin_amdgcn_sched_barrier(0);
    for (int k = 0; k < nk; ++k) {
        // load phase of step k
        load_frags(k);
        if (k >= 1) {
            if (grp == 0) { if (k + 1 < nk) issue(k + 1); }
            else { if (k + 2 < nk) issue(k + 2); }
        }
        if (grp == 1 && k + 1 < nk) {                 // activations of step k + 1 land before group 0 reads them
            if (k + 2 < nk) wait_vmcnt<PW>();
            else wait_vmcnt<0>();
        }
        lds_barrier();
        __builtin_amdgcn_sched_barrier(0);
        // MFMA phase of step k
        mfma_blocks(nb);
        __builtin_amdgcn_sched_barrier(0);
        if (grp == 0) {
            if (k + 1 < nk) wait_vmcnt<0>();          // weights of step k + 1
            lds_barrier();
        } else if (k + 1 < nk) {
            lds_barrier();
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    };
    if (vblk == 4) kloop(std::integral_constant<int, 4>{});
    else if (vblk == 3) kloop(std::integral_constant<int, 3>{});
    else if (vblk == 2) kloop(std::integral_constant<int, 2>{});
    else if (vblk == 1) kloop(std::integral_constant<int, 1>{});
    else kloop(std::integral_constant<int, 0>{});

    // epilogue: lane holds rows m0 + 128 grp + 32 i + (lane & 31) and, in register r of block j, column
    // n0 + 64 s + 32 j + (r / 4) * 8 + (lane >> 5) * 4 + r % 4
    const int rbase = m0 + grp * 128;
    const int cbase = n0 + sw4 * 64;
    if constexpr (EP == Epi::Int32) {
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
                const int c0 = cbase + j * 32 + q4 * 8 + fhi * 4;
                if (c0 >= p.N) continue;
                const bool full = c0 + 4 <= p.N && (p.ldo & 3) == 0;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int row = rbase + i * 32 + frow;
                    if (row >= p.M) continue;
                    int32_t* dst = static_cast<int32_t*>(p.out) + (int64_t)row * p.ldo + c0;
                    if (full) {
                        *reinterpret_cast<v4i*>(dst) =
                            v4i{acc[i][j][q4 * 4], acc[i][j][q4 * 4 + 1], acc[i][j][q4 * 4 + 2], acc[i][j][q4 * 4 + 3]};
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            if (c0 + e < p.N) dst[e] = acc[i][j][q4 * 4 + e];
                    }
                }
            }
    } else {
        // the wave's 128 x 64 fp16 block in its own 16 KB of LDS: row r at 128 r, 16-byte chunk c (8 columns)
        // at slot c ^ ((r >> 1) & 7), so the 8-byte writes of 32 rows and the 16-byte row reads stay at the
        // minimum of two passes per 256 bytes
        int8_t* stage = smem + wave * (128 * 128);
        float sx[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = rbase + i * 32 + frow;
            sx[i] = row < p.M ? p.sx[(int64_t)row * p.sx_stride] : 0.0f;
        }
        int qc[8], ql[8];
        f32x4 qsw[8] = {};
        u16x4 qb[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            qc[q] = cbase + (q >> 2) * 32 + (q & 3) * 8 + fhi * 4;
            ql[q] = p.N;
        }
        auto convert = [&](auto hb) {
            constexpr bool HB = decltype(hb)::value;
            load_cols<8, HB>(p, qc, ql, qsw, qb);
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int q4 = 0; q4 < 4; ++q4) {
                    const int q = j * 4 + q4;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        float y[4];
#pragma unroll
                        for (int e = 0; e < 4; ++e) y[e] = g1_reg<HB>(acc[i][j][q4 * 4 + e], sx[i], qsw[q][e], qb[q][e]);
                        const int r = i * 32 + frow;
                        *reinterpret_cast<u16x4*>(stage + r * 128 + ((q ^ ((r >> 1) & 7)) << 4) + fhi * 8) =
                            f2h4(y[0], y[1], y[2], y[3]);
                    }
                }
        };
        if (p.bias) convert(std::true_type{});
        else convert(std::false_type{});
        __builtin_amdgcn_s_waitcnt((15 << 4) | (0 << 8) | 0xC00F);   // this wave's LDS writes are done
        uint16_t* out = static_cast<uint16_t*>(p.out);
        const int c8 = lane & 7;
        const int gcol = cbase + c8 * 8;
        if (p.vec_out && cbase + 64 <= p.N && p.ldo <= (1 << 20)) {
            // The wave's 64 columns lie inside N (every decoder GEMM): all 16 row pieces are read from LDS
            // first, then stored from one wave-uniform base with 32-bit offsets, so no store waits for its
            // own LDS read and no per-row 64-bit address is formed.  Rows past M (the last row of tiles)
            // are skipped.
            u16x8 v[16];
#pragma unroll
            for (int t = 0; t < 16; ++t) {
                const int r = t * 8 + (lane >> 3);
                v[t] = *reinterpret_cast<const u16x8*>(stage + r * 128 + ((c8 ^ ((r >> 1) & 7)) << 4));
            }
            uint16_t* const base = out + (int64_t)rbase * p.ldo + cbase;   // wave-uniform
            const int rows = p.M - rbase;   // wave-uniform; 128 or fewer in the last row of tiles (even <= 0)
            const int off = (lane >> 3) * (int)p.ldo + c8 * 8;
            if (rows >= 128) {
#pragma unroll
                for (int t = 0; t < 16; ++t) *reinterpret_cast<u16x8*>(base + off + t * 8 * (int)p.ldo) = v[t];
            } else {
#pragma unroll
                for (int t = 0; t < 16; ++t)
                    if (t * 8 + (lane >> 3) < rows) *reinterpret_cast<u16x8*>(base + off + t * 8 * (int)p.ldo) = v[t];
            }
            return;
        }
#pragma unroll 4
        for (int t = 0; t < 16; ++t) {
            const int r = t * 8 + (lane >> 3);
            const int grow = rbase + r;
            const u16x8 v = *reinterpret_cast<const u16x8*>(stage + r * 128 + ((c8 ^ ((r >> 1) & 7)) << 4));
            if (grow >= p.M || gcol >= p.N) continue;
            uint16_t* dst = out + (int64_t)grow * p.ldo + gcol;
            if (p.vec_out && gcol + 8 <= p.N) {
                *reinterpret_cast<u16x8*>(dst) = v;
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    if (gcol + e < p.N) dst[e] = v[e];
            }
        }
    }
}

// Window row pitch in pixels of conv3_halo_i8 for tiles TW pixels wide: TW + 2 rounded up to 16 (the
// plain swizzle works on 16-pixel groups) or, in the strided-pixel variant, to 8 (whole 256-byte lines).
constexpr int halo_hpl(int tw, bool sp) { return sp ? (tw + 2 + 7) / 8 * 8 : (tw + 2 + 15) / 16 * 16; }

// LDS of conv3_halo_i8 with TW-pixel tile rows: two stages of window + weights, or the fp16 output
// tile if larger; the strided-pixel variant adds the statistics epilogue's reduction space.
constexpr int kGnLdsBytes = 12288;
constexpr int halo_lds_bytes(int tw, bool sp) {
    const int hb = ((512 / tw + 2) * halo_hpl(tw, sp) * 32 + 4095) / 4096 * 4096;
    const int ring = 2 * (hb + 9 * 128 * 32);
    return (ring > 512 * 128 * 2 ? ring : 512 * 128 * 2) + (sp ? kGnLdsBytes : 0);
}

// Compile-time loop: f(std::integral_constant<int, 0>{}) ... f(std::integral_constant<int, N - 1>{}).
template <typename F, int... I>
__device__ __forceinline__ void static_for_seq(F& f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_seq(f, std::make_integer_sequence<int, N>{});
}

// 16-byte slot (0..15) of half h of window pixel px inside its 256-byte line of 8 pixels, in the
// strided-pixel variant of conv3_halo_i8.  Its fragment reads take pixels px0 + 4r (r = 0..15 in one
// 16-lane group) and one half: two pixels of each of 8 consecutive lines, at line offsets a and
// a + 4 (a = px0 & 3).  With L the line, b = (px >> 2) & 1 and a = px & 3, the slot is
// ((b ^ (L >> 2)) & 1) << 3 | ((2a + h) ^ (b << 2) ^ (L & 3)): its low three bits are distinct over
// the eight (L & 3, b) pairs of any 8 consecutive lanes (8-lane groups on 32 banks), and bit 3
// separates lines L and L + 4, so 16 lanes hit 16 distinct slots (16-lane groups on 64 banks).  It
// is a bijection of (px & 7, h) onto the line's 16 slots and depends on the column only, so the kh
// shift (whole window rows, each a whole number of lines) keeps it.
__device__ __forceinline__ int sp_slot(int px, int h) {
    const int L = px >> 3, b = (px >> 2) & 1;
    return (((b ^ (L >> 2)) & 1) << 3) | ((2 * (px & 3) + h) ^ (b << 2) ^ (L & 3));
}

// Stride-1 3x3x3 convolution with the input window of a tile held in LDS.
//
// A tile is BM = 512 output voxels of one frame, RO = 512 / TW output rows of a
// TW-pixel column block (TW = WO: whole rows), times BN = 128 output channels.
// For one depth tap kd and one 32-byte channel slice the nine (kh, kw) taps of
// every voxel in the tile read the same RO + 2 input rows of TW + 2 pixels, so a
// stage stages that window once (32 bytes per pixel) together with the nine
// taps' weights ([9][128][32]) and runs 9 MFMA K steps on it; the implicit-GEMM
// kernel above fetches every input row up to nine times per depth tap instead.
// LDS-DMA instructions, whose issue is what holds the matrix pipe back, drop
// 2.6x.  Stages run kd-major (kd0..2) then channel slice, double-buffered: one
// barrier per 9 taps.  Causal-zero depth taps (output frames 0 and 1 of the
// fused producer's input) are skipped per tile; the tile is one frame.
//
// Window layout: pixel (row hr, column px) at LDS pixel hr * HPL + px with
// HPL = TW + 2 rounded up (halo_hpl), so a (kh, kw) shift of the window is a
// uniform offset for kh and a per-lane one for kw.  Plain kernel: each pixel's
// two 16-byte halves are swapped when (px >> 3) & 1, which keeps the 16-lane
// fragment reads (16 consecutive pixels, one half) on 16 distinct 16-byte bank
// groups.  Weight rows (tap, n) are swizzled the same way by (n >> 3) & 1.
// ES = 1: int8 operands, v_mfma_i32_32x32x32_i8, int32 accumulators (32 channels per 32-byte slice);
// ES = 2: fp16 operands, v_mfma_f32_32x32x16_f16, fp32 accumulators (16 channels per slice).  Both
// MFMAs read 16 bytes per lane in the same row / k-half layout, so staging and fragments are shared.
//
// SP (strided pixels; int8 dequant or int32 output at WO >= 128, fp16 at WO 64; channel bytes a
// multiple of 128): row r of a wave's accumulator block i is the wave's tile pixel 4r + i, and each
// group of four (4r .. 4r + 3) lies in one output row.  Tap (kh, kw) reads window pixels
// px0 + i + kw (px0 the group's first column): block i of tap kw is "virtual block" V[i + kw] of
// the six V[v] = pixels px0 + v (v = 0..5) of window row kh.  One kh's three taps read six A
// fragments instead of twelve (4 fragment reads per 8 MFMAs instead of 6); the window lines are
// swizzled by sp_slot for the stride-4 reads.  The blocks rotate through eight register slots, V[v]
// of the g-th kh in slot (6g + v) % 8: a kh's last tap reads slots base + 2 .. base + 5, so the next
// kh's first four blocks load into base + 6 .. base + 9 while it runs, as many registers as the
// plain double buffer.
//
// TW < WO (with SP: column blocks of 64 pixels): the window of a tile is RO + 2 = 10 rows of 66
// pixels instead of 4 rows of 258 at Wo 256: 6 window DMA instructions per issuing wave and stage
// instead of 9.  A wave's 128 pixels are two rows of the block.
template <int WO, Epi EP, int ES = 1, bool PAD = false, bool SP = false, int TW = WO>
__global__ __launch_bounds__(512) void conv3_halo_i8(GemmParams p) {
    static_assert((ES == 2) == (EP == Epi::F16Bias), "fp16 operands use the F16Bias epilogue");
    static_assert(!SP || (((ES == 1 && (EP == Epi::Dequant || EP == Epi::Int32)) || (ES == 2 && EP == Epi::F16Bias)) &&
                          (TW % 128 == 0 || 128 % TW == 0)),
                  "strided pixels: waves of whole tile rows");
    static_assert(TW == WO || (SP && WO % TW == 0), "column blocks: strided-pixel kernel only");
    using Acc = std::conditional_t<ES == 1, v16i, f32x16>;
    constexpr int BM = 512, BN = 128, WGM = 4, WGN = 2, NWD = 4;
    constexpr int WM = BM / WGM, WN = BN / WGN;
    constexpr int FM = WM / 32, FN = WN / 32;
    constexpr int RO = BM / TW;                               // output rows per tile
    constexpr int HR = RO + 2;                                // window rows
    constexpr int HPL = halo_hpl(TW, SP);                     // LDS pixels per window row
    constexpr int ROWB = HPL * 32;                            // LDS bytes per window row
    constexpr int HB = (HR * ROWB + 4095) / 4096 * 4096;      // window bytes (whole instructions per issuing wave)
    constexpr int WB = 9 * BN * 32;                           // weight bytes of a stage
    constexpr int STAGE = HB + WB;
    constexpr int NH = HB / 1024 / NWD, NWT = WB / 1024 / NWD; // DMA instructions per issuing wave and stage
    constexpr int LDS = (2 * STAGE > BM * BN * 2 ? 2 * STAGE : BM * BN * 2) + (SP ? kGnLdsBytes : 0);
    static_assert(WO == 32 || WO == 64 || WO == 128 || WO == 256, "output width");
    static_assert(LDS <= 163840, "LDS");
    static_assert(LDS == halo_lds_bytes(TW, SP), "host and kernel LDS sizes");
    static_assert(NH + NWT < 64, "outstanding DMA must fit vmcnt");

    extern __shared__ __attribute__((aligned(1024))) int8_t smem[];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform (scalar)
    const int wm = wave / WGN, wn = wave % WGN;

    // tile -> (weight tile, row block, frame, column block): the weight tiles of one window are adjacent,
    // then a group of RBG row blocks, then the frames, then the column blocks, then the next row group.
    // RBG = 8 / weight tiles, so the 32 workgroups an XCD runs at once cover 8 / RBG weight tiles x RBG
    // row blocks x 4 frames of one column block: the rows of neighbouring row blocks and the frames of
    // neighbouring output frames they share are read while that XCD's L2 still holds them.  Stage-0
    // conv (one weight tile), against frames, then column blocks, then row blocks: input fetched from
    // beyond L2 1.53x -> 0.98x the int8 bytes, 430.2 -> 410.6 us (same box); 4 frames per 32 tiles beat 2
    // and 8 on every window conv measured.
    int id = xcd_remap(blockIdx.x, gridDim.x);
    const int tn = id % p.tiles_n;
    id /= p.tiles_n;
    const int nfr = p.M / (p.Ho * WO);                        // batch * Do
    constexpr int NCB = WO / TW;                              // column blocks per output row
    const int rbg = p.tiles_n >= 8 ? 1 : 8 / p.tiles_n;       // row blocks per group
    const int nrb = p.Ho / RO;
    const int gsz = rbg * nfr * NCB;
    const int rg = id / gsz;
    int rem = id - rg * gsz;
    const int rbn = nrb - rg * rbg < rbg ? nrb - rg * rbg : rbg;
    const int rb = rg * rbg + rem % rbn;
    rem /= rbn;
    const int fr = rem % nfr;
    const int cb = rem / nfr;
    const int od = fr % p.Do;
    const int bi = fr / p.Do;
    const int oh0 = rb * RO;
    const int owb = cb * TW;                                  // first output column of the tile
    const int m0 = (fr * p.Ho + oh0) * WO + owb;
    const int n0 = tn * BN;
    const int CB = p.C * ES;                                  // bytes per pixel
    const int CQ = CB / 32;                                   // 32-byte channel slices
    const int kd0 = (p.causal_skip && od < 2) ? 2 - od : 0;
    const int nst = (3 - kd0) * CQ;                           // even: C * ES % 64 == 0
    const uint32_t frame_bytes = (uint32_t)p.Hp * p.Wp * CB;

    const bool dma_wave = wave < NWD;
    const int dw = dma_wave ? wave : 0;
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc((void*)p.a, 0, (int)p.a_bytes, kRsrcWord3);
    const __amdgpu_buffer_rsrc_t rb_ = __builtin_amdgcn_make_buffer_rsrc((void*)p.b, 0, (int)p.b_bytes, kRsrcWord3);
    // per-lane DMA source offsets; the stage adds kd and the channel slice as the uniform offset
    uint32_t hoff[NH], woff[NWT];
    {
        const uint32_t tile_base = (uint32_t)((((int64_t)(bi * p.Dp + od) * p.Hp + oh0) * p.Wp + owb) * CB);
#pragma unroll
        for (int j = 0; j < NH; ++j) {
            const int s16 = (dw + NWD * j) * 64 + lane;       // 16-byte slot of the window buffer
            int hr, px, half;
            if constexpr (SP) {   // inverse of sp_slot inside the slot's 256-byte line
                hr = s16 / (2 * HPL);
                const int w = s16 - hr * (2 * HPL);
                const int L = w >> 4, sl = w & 15;
                const int b = ((sl >> 3) ^ (L >> 2)) & 1;
                const int t = (sl & 7) ^ (b << 2) ^ (L & 3);
                px = 8 * L + 4 * b + (t >> 1);
                half = t & 1;
            } else {
                const int pix = s16 >> 1;
                hr = pix / HPL;
                px = pix - hr * HPL;
                half = (s16 & 1) ^ ((px >> 3) & 1);
            }
            // padding slots load a valid in-window pixel; they are never read
            if (hr >= HR) hr = HR - 1;
            if (px > TW + 1) px = TW + 1;
            hoff[j] = tile_base + (uint32_t)((hr * p.Wp + px) * CB + half * 16);
        }
#pragma unroll
        for (int j = 0; j < NWT; ++j) {
            const int s16 = (dw + NWD * j) * 64 + lane;
            const int row = s16 >> 1;                         // tap * 128 + n
            const int t9 = row >> 7, n = row & 127;
            const int half = (s16 & 1) ^ ((n >> 3) & 1);
            woff[j] = (uint32_t)(n0 + n) * (uint32_t)(p.K * ES) + (uint32_t)(t9 * CB + half * 16);
        }
    }
    auto issue = [&](int kd, int cq, int slot) {
        if (!dma_wave) return;
        int8_t* base = smem + slot * STAGE;
        const uint32_t sh = (uint32_t)kd * frame_bytes + (uint32_t)cq * 32;
        const uint32_t sw = (uint32_t)(kd * 9 * CB + cq * 32);
#pragma unroll
        for (int j = 0; j < NH; ++j) lds_dma16(ra, hoff[j], sh, base + (dw + NWD * j) * 1024);
#pragma unroll
        for (int j = 0; j < NWT; ++j) lds_dma16(rb_, woff[j], sw, base + HB + (dw + NWD * j) * 1024);
    };

    // fragment addresses: lane reads output row (lane & 31) of a 32-row block and
    // the 16-byte half (lane >> 5) of its pixel / weight row
    const int frow = lane & 31;
    const int fhi = lane >> 5;
    int baddr[FN];
#pragma unroll
    for (int j = 0; j < FN; ++j) {
        const int n = wn * WN + j * 32 + frow;
        baddr[j] = HB + n * 32 + ((fhi ^ ((n >> 3) & 1)) << 4);
    }

    Acc acc[FM][FN];
    // zero accumulators; the empty asm pins the moves where this is called (otherwise they sink to just
    // before the first MFMA, after the first wait and barrier)
    auto zero_acc = [&]() {
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                Acc z = {};
                asm volatile("" : "+v"(z));
                acc[i][j] = z;
            }
    };

    // stage s covers depth tap kd0 + s / CQ and channel slice s % CQ; the issue
    // position is kept as a running (kd, cq) pair
    int ikd = kd0, icq = 0;
    auto issue_next = [&](int slot) {
        issue(ikd, icq, slot);
        if (++icq == CQ) {
            icq = 0;
            ++ikd;
        }
    };
    constexpr int NMFMA = FM * FN;

    if constexpr (SP) {
        static_assert(FM == 4 && WM == 128 && TW % 4 == 0, "strided pixels: 4 blocks of 32 rows per wave");
        const int t0 = wm * WM + 4 * frow;                    // tile pixel of this lane's group of four
        const int orow = t0 / TW, ow0 = t0 % TW;
        int vaddr[6];   // LDS offset of virtual block V[v] in window row kh = 0
#pragma unroll
        for (int v = 0; v < 6; ++v) {
            const int px = ow0 + v;              // at most TW + 1: the group's row, never the next one
            vaddr[v] = orow * ROWB + (px >> 3) * 256 + (sp_slot(px, fhi) << 4);
        }
        v4i av[8], bq[2][FN];
        auto ld_a = [&](int slot, int kh, int v, v4i& dst) {
            dst = *reinterpret_cast<const v4i*>(smem + slot * STAGE + vaddr[v] + kh * ROWB);
        };
        auto ld_b = [&](int slot, int t9, v4i (&bf)[FN]) {
            const int8_t* sb = smem + slot * STAGE + t9 * (BN * 32);
#pragma unroll
            for (int j = 0; j < FN; ++j) bf[j] = *reinterpret_cast<const v4i*>(sb + baddr[j]);
        };
        issue_next(0);
        issue_next(1);
        zero_acc();                                           // while the first two stages are in flight
        wait_vmcnt<NH + NWT>();                               // stage 0 landed, stage 1 may be in flight
        lds_barrier();
#pragma unroll
        for (int v = 0; v < 4; ++v) ld_a(0, 0, v, av[v]);
        ld_b(0, 0, bq[0]);
        // Stage Q of a group of four (LDS slot Q & 1; the register slots rotate with period four
        // stages): tap (kh, kw) multiplies V[kw .. kw + 3] of its kh, then loads what the next tap
        // adds: V[4] after kw = 0, V[5] after kw = 1, the next kh's V[0 .. 3] after kw = 2 (from the
        // next stage's LDS slot after the stage's last tap), each with the next tap's weights.
        auto run_stage = [&](auto q_c, int s) {
            constexpr int Q = decltype(q_c)::value;
            constexpr int SL = Q & 1;
            static_for<9>([&](auto t_c) {
                constexpr int T9 = decltype(t_c)::value;
                constexpr int KH = T9 / 3, KW = T9 % 3;
                constexpr int BASE = (2 * Q + 6 * KH) & 7;    // register slot of V[0] of this kh
                constexpr int NB = (BASE + 6) & 7;            // register slot of V[0] of the next kh
                constexpr int CUR = (Q + T9) & 1;
                constexpr int NR = FN + (KW == 2 ? 4 : 1);    // fragment reads issued under this tap
                auto mfma_tap = [&]() {
#pragma unroll
                    for (int i = 0; i < FM; ++i)
#pragma unroll
                        for (int j = 0; j < FN; ++j) {
                            if constexpr (ES == 1)
                                acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(bq[CUR][j], av[(BASE + KW + i) & 7],
                                                                                  acc[i][j], 0, 0, 0);
                            else
                                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                                    __builtin_bit_cast(half8, bq[CUR][j]), __builtin_bit_cast(half8, av[(BASE + KW + i) & 7]),
                                    acc[i][j], 0, 0, 0);
                        }
                };
                if constexpr (T9 == 8) {
                    const bool more = s + 1 < nst;
                    if (more) {
                        wait_vmcnt<0>();                      // stage s+1 landed
                        lds_barrier();                        // and every wave is done with slot SL
                        if (s + 2 < nst) issue_next(SL);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                    mfma_tap();
                    if (more) {
#pragma unroll
                        for (int v = 0; v < 4; ++v) ld_a(SL ^ 1, 0, v, av[(NB + v) & 7]);
                        ld_b(SL ^ 1, 0, bq[CUR ^ 1]);
                    }
                } else {
                    mfma_tap();
                    if constexpr (KW < 2) {
                        ld_a(SL, KH, 4 + KW, av[(BASE + 4 + KW) & 7]);
                    } else {
#pragma unroll
                        for (int v = 0; v < 4; ++v) ld_a(SL, KH + 1, v, av[(NB + v) & 7]);
                    }
                    ld_b(SL, T9 + 1, bq[CUR ^ 1]);
                }
#pragma unroll
                for (int g = 0; g < NR; ++g) {
                    __builtin_amdgcn_sched_group_barrier(0x008, NMFMA / NR, 0);
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                }
                __builtin_amdgcn_sched_barrier(0);
            });
        };
        for (int s = 0; s < nst; s += 4) {   // nst % 4 == 0: launch_halo takes SP only for C % 128 == 0
            run_stage(std::integral_constant<int, 0>{}, s);
            run_stage(std::integral_constant<int, 1>{}, s + 1);
            run_stage(std::integral_constant<int, 2>{}, s + 2);
            run_stage(std::integral_constant<int, 3>{}, s + 3);
        }
        write_tile<BM, BN, WGM, WGN, LDS, EP, (PAD ? WO : 0), true, (TW < WO ? TW : 0)>(p, acc, smem, m0, n0, tn);
        return;
    }

    int aaddr[FM][3];
#pragma unroll
    for (int i = 0; i < FM; ++i) {
        const int r = wm * WM + i * 32 + frow;
        const int orow = r / WO, ow = r % WO;
#pragma unroll
        for (int kw = 0; kw < 3; ++kw) {
            const int px = ow + kw;
            aaddr[i][kw] = (orow * HPL + px) * 32 + ((fhi ^ ((px >> 3) & 1)) << 4);
        }
    }

    auto load_frags = [&](int slot, int t9, v4i (&af)[FM], v4i (&bf)[FN]) {
        const int8_t* s = smem + slot * STAGE;
        const int kh = t9 / 3, kw = t9 % 3;
#pragma unroll
        for (int i = 0; i < FM; ++i) af[i] = *reinterpret_cast<const v4i*>(s + aaddr[i][kw] + kh * ROWB);
#pragma unroll
        for (int j = 0; j < FN; ++j) bf[j] = *reinterpret_cast<const v4i*>(s + baddr[j] + t9 * (BN * 32));
    };
    auto mfma_all = [&](const v4i (&af)[FM], const v4i (&bf)[FN]) {
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                if constexpr (ES == 1)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(bf[j], af[i], acc[i][j], 0, 0, 0);
                else
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, bf[j]),
                                                                      __builtin_bit_cast(half8, af[i]), acc[i][j], 0, 0, 0);
            }
    };

    v4i fa[2][FM], fb[2][FN];
    issue_next(0);
    issue_next(1);
    zero_acc();                                               // while the first two stages are in flight
    wait_vmcnt<NH + NWT>();                                   // stage 0 landed, stage 1 may be in flight
    lds_barrier();
    load_frags(0, 0, fa[0], fb[0]);

    constexpr int NFRAG = FM + FN;
    // One stage: 9 taps, fragments double-buffered in registers across taps
    // (and across the stage boundary: the last tap's MFMAs hide the reads of the
    // next stage's first fragments).  With 9 taps the register buffer parity
    // flips every stage, so stages are processed in (slot 0, slot 1) pairs.
    auto run_stage = [&](auto slot_c, int s) {
        constexpr int SL = decltype(slot_c)::value;
#pragma unroll
        for (int t9 = 0; t9 < 9; ++t9) {
            const int cur = (SL + t9) & 1;
            if (t9 == 8) {
                const bool more = s + 1 < nst;
                if (more) {
                    wait_vmcnt<0>();                          // stage s+1 landed
                    lds_barrier();                            // and every wave is done with slot SL
                    if (s + 2 < nst) issue_next(SL);
                }
                __builtin_amdgcn_sched_barrier(0);
                mfma_all(fa[cur], fb[cur]);
                if (more) load_frags(SL ^ 1, 0, fa[cur ^ 1], fb[cur ^ 1]);
            } else {
                mfma_all(fa[cur], fb[cur]);
                load_frags(SL, t9 + 1, fa[cur ^ 1], fb[cur ^ 1]);
            }
#pragma unroll
            for (int g = 0; g < NFRAG; ++g) {
                __builtin_amdgcn_sched_group_barrier(0x008, NMFMA / NFRAG, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    for (int s = 0; s < nst; s += 2) {
        run_stage(std::integral_constant<int, 0>{}, s);
        run_stage(std::integral_constant<int, 1>{}, s + 1);
    }

    write_tile<BM, BN, WGM, WGN, LDS, EP, (PAD ? WO : 0)>(p, acc, smem, m0, n0, tn);
}

// Shape-general path (any K, any channel count, unaligned pointers): one thread
// per output, scalar integer dot product.  Used only where the tiled kernel's
// divisibility or alignment preconditions fail; results are identical because
// the integer sum is exact and the epilogue is shared.
template <AMode AM, Epi EP>
__global__ __launch_bounds__(256) void gemm_i8_generic(GemmParams p) {
    int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (int64_t)p.M * p.N) return;
    int row = (int)(idx / p.N), col = (int)(idx % p.N);
    auto dot = [&](int wrow) {
        const int8_t* w = p.b + (int64_t)wrow * p.K;
        int32_t s = 0;
        if constexpr (AM == AMode::Gemm) {
            const int8_t* a = p.a + (int64_t)row * p.lda;
            for (int k = 0; k < p.K; ++k) s += (int32_t)a[k] * (int32_t)w[k];
        } else {
            int64_t base = conv_row_offset(p, row);
            for (int k = 0; k < p.K; ++k) {
                int tap = k / p.C, c = k - tap * p.C;
                int kd = tap / (p.KH * p.KW), rem = tap - kd * p.KH * p.KW;
                int kh = rem / p.KW, kw = rem - kh * p.KW;
                int64_t off = (((int64_t)kd * p.Hp + kh) * p.Wp + kw) * p.C + c;
                s += (int32_t)p.a[base + off] * (int32_t)w[k];
            }
        }
        return s;
    };
    float sx = (EP == Epi::Int32) ? 0.0f : p.sx[(int64_t)row * p.sx_stride];
    if constexpr (EP == Epi::SwiGLU) {
        float g = rt16(g1_value(dot(col), sx, p.sw[col], p.bias, col));
        float u = rt16(g1_value(dot(p.N + col), sx, p.sw[p.N + col], p.bias, p.N + col));
        static_cast<uint16_t*>(p.out)[(int64_t)row * p.ldo + col] = f2h(silu(g) * u);
    } else if constexpr (EP == Epi::Int32) {
        static_cast<int32_t*>(p.out)[(int64_t)row * p.ldo + col] = dot(col);
    } else {
        const int64_t o = (int64_t)row * p.ldo + col;
        const uint16_t y = f2h(g1_value(dot(col), sx, p.sw[col], p.bias, col));
        static_cast<uint16_t*>(p.out)[o] = p.res ? f2h(h2f(p.res[o]) + h2f(y)) : y;
    }
}

template <int BM, int BN, int BK, int WGM, int WGN, int NSA, int NSB, AMode AM, Epi EP>
int launch_tiled(GemmParams p, hipStream_t stream, const char* what) {
    int ncols = (EP == Epi::SwiGLU) ? 2 * p.N : p.N;
    p.tiles_m = (p.M + BM - 1) / BM;
    p.tiles_n = (ncols + BN - 1) / BN;
    p.vec_epi = (p.sw == nullptr || aligned(p.sw, 16)) && (p.bias == nullptr || aligned(p.bias, 8)) && p.N % 4 == 0;
    p.vec_out = aligned(p.out, 16) && (p.res == nullptr || aligned(p.res, 16)) && p.ldo % 8 == 0;
    p.conv_tpf = 0;
    if (AM == AMode::Conv && ((int64_t)p.Ho * p.Wo) % BM == 0) p.conv_tpf = (int)((int64_t)p.Ho * p.Wo / BM);
    int64_t grid = (int64_t)p.tiles_m * p.tiles_n;
    if (grid > 0x7fffffff) return fail(H3V_EINVAL, "%s: too many tiles", what);
    {
        const int64_t a_bytes = AM == AMode::Gemm ? (int64_t)p.M * p.lda
                                                  : (int64_t)(p.M / ((int64_t)p.Do * p.Ho * p.Wo)) * p.Dp * p.Hp * p.Wp * p.C;
        const int64_t b_bytes = (int64_t)((EP == Epi::SwiGLU) ? 2 * p.N : p.N) * p.K;
        if (a_bytes >= ((int64_t)1 << 32) || b_bytes >= ((int64_t)1 << 32))
            return fail(H3V_EINVAL, "%s: an operand exceeds 4 GiB (%lld, %lld bytes)", what, (long long)a_bytes,
                        (long long)b_bytes);
        p.a_bytes = (uint32_t)a_bytes;
        p.b_bytes = (uint32_t)b_bytes;
    }
    constexpr size_t kLds = (size_t)(NSA * BM + NSB * BN) * BK;   // LDS rings (at most 160 KB on gfx950)
    static_assert(kLds <= 163840, "LDS rings exceed 160 KB");
    // the chunk-statistics epilogue (h3v_conv3d_f16_gn) needs its reduction space past the rings
    constexpr bool kChunkStats = EP == Epi::F16Bias && BM == 256 && BN == 128 && WGM * WGN == 8;
    constexpr size_t kLdsMax = kLds + (kChunkStats ? kGnChunkLdsBytes : 0);
    static_assert(kLdsMax <= 163840, "LDS exceeds 160 KB");
    if (p.gn_avg != nullptr && !kChunkStats) return fail(H3V_EINVAL, "%s: no statistics epilogue for this tile", what);
    const size_t lds = p.gn_avg != nullptr ? kLdsMax : kLds;
    auto kernel = &gemm_i8_mfma<BM, BN, BK, WGM, WGN, NSA, NSB, AM, EP>;
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)kLdsMax);
    if (attr != hipSuccess) return fail(H3V_ELAUNCH, "%s: cannot reserve %zu bytes of LDS: %s", what, kLdsMax,
                                        hipGetErrorString(attr));
    const int splits = p.k_splits > 1 ? p.k_splits : 1;
    if ((p.K / BK) % splits != 0 || (splits > 1 && EP != Epi::F32Part))
        return fail(H3V_EINVAL, "%s: %d K splits do not divide %d K blocks", what, splits, p.K / BK);
    hipLaunchKernelGGL(kernel, dim3((unsigned)grid, (unsigned)splits), dim3(WGM * WGN * 64), lds, stream, p);
    return launch_status(what);
}

// Fraction of the CU slots busy over the rounds a launch of `tiles` one-per-CU workgroups takes.
double round_fill(int64_t tiles) {
    constexpr int64_t kCUs = 256;
    const int64_t rounds = (tiles + kCUs - 1) / kCUs;
    return rounds ? (double)tiles / (double)(rounds * kCUs) : 1.0;
}

// Sum of the K-split partials [S][M][N] (fp32, split-major) in split order, then the F16Bias epilogue:
// y = fp16(sum + bias), with a residual fp16(fp32(res) + fp32(y)).  M * N and N are multiples of 4.
__global__ __launch_bounds__(256) void splitk_reduce_f16(const float* __restrict__ part, int splits, int64_t mn, int n,
                                                         const uint16_t* __restrict__ bias,
                                                         const uint16_t* __restrict__ res, uint16_t* __restrict__ out) {
    const int64_t i4 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (i4 >= mn) return;
    f32x4 v = *reinterpret_cast<const f32x4*>(part + i4);
    for (int sp = 1; sp < splits; ++sp) {
        const f32x4 w = *reinterpret_cast<const f32x4*>(part + sp * mn + i4);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = v[e] + w[e];
    }
    const int c = (int)(i4 % n);
    u16x4 y;
#pragma unroll
    for (int e = 0; e < 4; ++e) y[e] = f2h(bias ? v[e] + h2f(bias[c + e]) : v[e]);
    if (res) {
        const u16x4 r = *reinterpret_cast<const u16x4*>(res + i4);
#pragma unroll
        for (int e = 0; e < 4; ++e) y[e] = f2h(h2f(r[e]) + h2f(y[e]));
    }
    *reinterpret_cast<u16x4*>(out + i4) = y;
}

// Stride-1 3x3x3 convolution through conv3_halo_i8 with ES-byte elements: requires
// C * ES % 64 == 0, N % 128 == 0, Wo in {32, 64, 128, 256} and Ho a multiple of 512 / Wo.
bool halo_conv_fits(const GemmParams& p, int es = 1) {
    const bool shape = p.KH == 3 && p.KW == 3 && p.K == 27 * p.C && p.SD == 1 && p.SH == 1 && p.SW == 1 &&
                       (p.C * es) % 64 == 0 && p.N % 128 == 0 &&
                       (p.Wo == 32 || p.Wo == 64 || p.Wo == 128 || p.Wo == 256) && p.Ho % (512 / p.Wo) == 0;
    return shape && aligned(p.a, 16) && aligned(p.b, 16) && (int64_t)p.Hp * p.Wp * p.C * es * 3 < ((int64_t)1 << 31);
}

enum class F16Kind { Halo256, Halo128, Halo64, Halo32, Tiled512x128, Tiled256x128, Tiled256x256, Tiled256x128k64,
                     Tiled256x256k64, Tiled256x128k64r3 };
struct F16Plan {
    F16Kind kind;
    int splits;
};

// K splits for a launch of `tiles` workgroups over `kblocks` K blocks: none at half a round or more;
// otherwise the largest S <= 16 that keeps tiles * S within one round of the 256 CUs, divides the K
// blocks and leaves each split at least 8 of them.
int f16_splits(int64_t tiles, int kblocks) {
    if (2 * tiles > 256) return 1;
    int best = 1;
    for (int sp = 2; sp <= 16; ++sp)
        if (tiles * sp <= 256 && kblocks % sp == 0 && kblocks / sp >= 8) best = sp;
    return best;
}

// Kernel, tile and K split of h3v_conv3d_f16 for the geometry in p (C and K in elements; the implicit
// GEMM counts them in bytes).  Splits only when the caller supplies a workspace (may_split).
F16Plan plan_conv_f16(const GemmParams& p, bool may_split) {
    if (halo_conv_fits(p, 2)) {
        if (p.Wo == 256) return {F16Kind::Halo256, 1};
        if (p.Wo == 128) return {F16Kind::Halo128, 1};
        if (p.Wo == 64) return {F16Kind::Halo64, 1};
        return {F16Kind::Halo32, 1};
    }
    const int cb = p.C * 2;
    const int64_t kb = (int64_t)p.K * 2;
    const int64_t m256 = (p.M + 255) / 256;
    if (cb % 128 == 0) {
        const int kblocks = (int)(kb / 128);
        if (p.N <= 128) {
            // A K split when even 256-row tiles leave most CUs idle (conv_out: 1024 -> 48 at 5 x 16 x 16)
            if (may_split && p.N % 4 == 0) {
                const int sp = f16_splits(m256, kblocks);
                if (sp > 1) return {F16Kind::Tiled256x128, sp};
            }
            // 512 x 128 tiles unless their last round leaves many CUs idle where 256 x 128 tiles (eight
            // 64 x 64 wave blocks, about 10% slower per tile) fill the chip better: the stage-0
            // downsample (544 tiles = 2.1 rounds) 353.5 -> 312.6 us, conv_out (10 tiles) 461.5 -> 285.3 us
            if (round_fill((p.M + 511) / 512) < 0.9 * round_fill(m256)) return {F16Kind::Tiled256x128, 1};
            return {F16Kind::Tiled512x128, 1};
        }
        const int64_t t256 = m256 * ((p.N + 255) / 256);
        if (may_split && p.N % 4 == 0) {
            const int sp = f16_splits(t256, kblocks);
            if (sp > 1) return {F16Kind::Tiled256x256, sp};
        }
        // Cout > 128 with so few 256 x 256 tiles that even twice as many fit one round on the 256 CUs
        // (the 16^2 suffix stage: 80 tiles): 256 x 128 tiles of eight 64 x 64 wave blocks.  At 144 tiles
        // (the stride-2 downsample) the 288 smaller tiles need a second round and ran 35% slower.
        if (2 * t256 <= 256) return {F16Kind::Tiled256x128, 1};
        return {F16Kind::Tiled256x256, 1};
    }
    const bool few = p.N > 128 && 2 * m256 * ((p.N + 255) / 256) <= 256;
    // Cout <= 128 with K steps of 64 bytes (conv_in: 32 tap-folded channels x 3 taps): 256 x 128 tiles over
    // a 3-deep A ring and a 2-deep B ring take 64 KB of LDS, so two workgroups share a CU and one's
    // operand waits hide under the other's MFMAs (512 x 128 tiles with 4-deep rings: 99.3 -> 94.3 us;
    // 128 x 128 tiles with 2-deep rings: 110.9 us)
    if (p.N <= 128) return {F16Kind::Tiled256x128k64r3, 1};
    if (few) return {F16Kind::Tiled256x128k64, 1};
    return {F16Kind::Tiled256x256k64, 1};
}

template <int WO, Epi EP, int ES = 1, bool PAD = false>
int launch_halo(GemmParams p, hipStream_t stream, const char* what) {
    p.tiles_m = p.M / 512;
    p.tiles_n = p.N / 128;
    p.vec_epi = (p.sw == nullptr || aligned(p.sw, 16)) && (p.bias == nullptr || aligned(p.bias, 8)) && p.N % 4 == 0;
    p.vec_out = aligned(p.out, 16) && (p.res == nullptr || aligned(p.res, 16)) && p.ldo % 8 == 0;
    p.conv_tpf = 0;
    const int64_t grid = (int64_t)p.tiles_m * p.tiles_n;
    const int64_t a_bytes = (int64_t)(p.M / ((int64_t)p.Do * p.Ho * p.Wo)) * p.Dp * p.Hp * p.Wp * p.C * ES;
    const int64_t b_bytes = (int64_t)p.N * p.K * ES;
    if (a_bytes >= ((int64_t)1 << 32) || b_bytes >= ((int64_t)1 << 31))
        return fail(H3V_EINVAL, "%s: an operand exceeds the 32-bit offset range (%lld, %lld bytes)", what,
                    (long long)a_bytes, (long long)b_bytes);
    p.a_bytes = (uint32_t)a_bytes;
    p.b_bytes = (uint32_t)b_bytes;
    if (PAD && !p.vec_out) return fail(H3V_EINVAL, "%s: the padded output needs 16-byte aligned out and residual", what);
    // the strided-pixel variant where it applies (int8 dequant or int32 at Wo 128 or 256, fp16 at Wo 64;
    // stages in groups of four), on column blocks of 64 pixels
    constexpr bool kSp = (ES == 1 && (EP == Epi::Dequant || EP == Epi::Int32) && WO >= 128) ||
                         (ES == 2 && EP == Epi::F16Bias && WO == 64);
    constexpr int kTw = kSp ? 64 : WO;
    constexpr int lds = halo_lds_bytes(WO, false), lds_sp = halo_lds_bytes(kTw, true);
    static_assert(lds <= 163840 && lds_sp <= 163840, "LDS exceeds 160 KB");
    const bool sp = kSp && (p.C * ES) % 128 == 0 && p.Ho % (512 / kTw) == 0;   // whole 8-row tiles of the column blocks
    if (p.gn_avg && !sp) return fail(H3V_EINVAL, "%s: the statistics epilogue needs the strided-pixel kernel", what);
    auto kernel = sp ? &conv3_halo_i8<WO, EP, ES, PAD, kSp, kTw> : &conv3_halo_i8<WO, EP, ES, PAD, false>;
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(&conv3_halo_i8<WO, EP, ES, PAD, false>),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    static const hipError_t attr_sp =
        kSp ? hipFuncSetAttribute(reinterpret_cast<const void*>(&conv3_halo_i8<WO, EP, ES, PAD, kSp, kTw>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, lds_sp)
            : hipSuccess;
    const hipError_t ae = attr != hipSuccess ? attr : attr_sp;
    if (ae != hipSuccess) return fail(H3V_ELAUNCH, "%s: cannot reserve %d bytes of LDS: %s", what, sp ? lds_sp : lds,
                                      hipGetErrorString(ae));
    hipLaunchKernelGGL(kernel, dim3((unsigned)grid), dim3(512), sp ? lds_sp : lds, stream, p);
    return launch_status(what);
}

template <Epi EP>
int launch_pingpong(GemmParams p, hipStream_t stream, const char* what) {
    p.tiles_m = (p.M + 255) / 256;
    p.tiles_n = (p.N + 255) / 256;
    p.vec_epi = (p.sw == nullptr || aligned(p.sw, 16)) && (p.bias == nullptr || aligned(p.bias, 8)) && p.N % 4 == 0;
    p.vec_out = aligned(p.out, 16) && p.ldo % 8 == 0;
    const int64_t tiles = (int64_t)p.tiles_m * p.tiles_n;
    if (tiles > 0x7fffffff) return fail(H3V_EINVAL, "%s: too many tiles", what);
    const int64_t a_bytes = (int64_t)p.M * p.lda, b_bytes = (int64_t)p.N * p.K;
    if (a_bytes >= ((int64_t)1 << 32) || b_bytes >= ((int64_t)1 << 32))
        return fail(H3V_EINVAL, "%s: an operand exceeds 4 GiB (%lld, %lld bytes)", what, (long long)a_bytes,
                    (long long)b_bytes);
    p.a_bytes = (uint32_t)a_bytes;
    p.b_bytes = (uint32_t)b_bytes;
    constexpr size_t lds = 5 * 256 * 128;   // three activation and two weight slots: 160 KB
    auto kernel = &gemm_i8_pingpong<EP>;
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (attr != hipSuccess) return fail(H3V_ELAUNCH, "%s: cannot reserve %zu bytes of LDS: %s", what, lds,
                                        hipGetErrorString(attr));
    hipLaunchKernelGGL(kernel, dim3((unsigned)tiles), dim3(512), lds, stream, p);
    return launch_status(what);
}

template <AMode AM, Epi EP>
int launch_generic(GemmParams p, hipStream_t stream, const char* what) {
    int64_t total = (int64_t)p.M * p.N;
    int64_t blocks = (total + 255) / 256;
    if (blocks > 0x7fffffff) return fail(H3V_EINVAL, "%s: problem too large for the generic path", what);
    hipLaunchKernelGGL((gemm_i8_generic<AM, EP>), dim3((unsigned)blocks), dim3(256), 0, stream, p);
    return launch_status(what);
}

template <Epi EP>
int run_gemm(GemmParams p, hipStream_t stream, const char* what) {
    const bool al = p.lda % 16 == 0 && aligned(p.a, 16) && aligned(p.b, 16);
    // K <= 4096: the two-stage ring (one barrier-to-use step of prefetch) measured faster
    // than three A stages (FFN-up 7188 x 16384 x 2048: 285 vs 305 us); long K keeps the
    // deeper A ring (FFN-down 7188 x 2048 x 8192: 116 vs 132 us).
    if constexpr (EP == Epi::Dequant || EP == Epi::Int32)
        if (al && p.K % 128 == 0) return launch_pingpong<EP>(p, stream, what);
    if (al && p.K % 128 == 0 && p.K <= 4096) return launch_tiled<256, 256, 128, 2, 4, 2, 2, AMode::Gemm, EP>(p, stream, what);
    if (al && p.K % 128 == 0) return launch_tiled<256, 256, 128, 2, 4, 3, 2, AMode::Gemm, EP>(p, stream, what);
    if (al && p.K % 64 == 0) return launch_tiled<256, 256, 64, 2, 4, 4, 4, AMode::Gemm, EP>(p, stream, what);
    return launch_generic<AMode::Gemm, EP>(p, stream, what);
}

template <Epi EP>
int run_conv(GemmParams p, hipStream_t stream, const char* what) {
    const bool al = aligned(p.a, 16) && aligned(p.b, 16);
    // A small conv whose 512 x 128 window tiles would occupy under half of the 256 CUs (a single
    // 9 x 64 x 64 clip at 128 -> 128 channels: 36864 voxels = 72 tiles) runs as the implicit GEMM on
    // 256 x 128 tiles of eight 64 x 64 wave blocks instead: twice the workgroups, 28.3 vs 36.7 us there.
    const int64_t halo_tiles = ((int64_t)p.M / 512) * (p.N / 128);
    if (al && p.C % 128 == 0 && halo_tiles < 128 && halo_conv_fits(p))
        return launch_tiled<256, 128, 128, 4, 2, 2, 2, AMode::Conv, EP>(p, stream, what);
    if (halo_conv_fits(p)) {
        if (p.Wo == 256) return launch_halo<256, EP>(p, stream, what);
        if (p.Wo == 128) return launch_halo<128, EP>(p, stream, what);
        if (p.Wo == 64) return launch_halo<64, EP>(p, stream, what);
        return launch_halo<32, EP>(p, stream, what);
    }
    if (al && p.C % 128 == 0) {
        if (p.N <= 128) return launch_tiled<512, 128, 128, 4, 2, 2, 2, AMode::Conv, EP>(p, stream, what);
        return launch_tiled<256, 256, 128, 2, 4, 3, 2, AMode::Conv, EP>(p, stream, what);
    }
    if (al && p.C % 64 == 0) {
        if (p.N <= 128) return launch_tiled<512, 128, 64, 4, 2, 4, 4, AMode::Conv, EP>(p, stream, what);
        return launch_tiled<256, 256, 64, 2, 4, 4, 4, AMode::Conv, EP>(p, stream, what);
    }
    p.causal_skip = 0;  // the generic path always runs the full reduction
    return launch_generic<AMode::Conv, EP>(p, stream, what);
}

int check_gemm_dims(const char* what, int64_t m, int64_t n, int64_t k) {
    if (m <= 0 || n <= 0 || k <= 0) return fail(H3V_EINVAL, "%s: M, N, K must be positive (got %lld, %lld, %lld)", what, (long long)m, (long long)n, (long long)k);
    if (m > 0x7fffffff || n > 0x3fffffff || k > 0x7fffffff) return fail(H3V_EINVAL, "%s: dimensions exceed 32-bit index range", what);
    if (k * 128 * 128 >= (int64_t)1 << 31) return fail(H3V_EINVAL, "%s: K=%lld overflows the int32 accumulator bound", what, (long long)k);
    return H3V_OK;
}

int fill_conv(GemmParams& p, const char* what, int batch, int cin, int d, int h, int w, int cout,
              int kd, int kh, int kw, int sd, int sh, int sw) {
    if (batch <= 0 || cin <= 0 || cout <= 0 || d <= 0 || h <= 0 || w <= 0)
        return fail(H3V_EINVAL, "%s: dimensions must be positive", what);
    if (kd <= 0 || kh <= 0 || kw <= 0 || sd <= 0 || sh <= 0 || sw <= 0)
        return fail(H3V_EINVAL, "%s: kernel and stride must be positive", what);
    if (d < kd || h < kh || w < kw) return fail(H3V_EINVAL, "%s: input is too small for a valid convolution", what);
    int64_t taps = (int64_t)kd * kh * kw;
    int64_t k = taps * cin;
    int64_t dout = (d - kd) / sd + 1, hout = (h - kh) / sh + 1, wout = (w - kw) / sw + 1;
    int64_t m = (int64_t)batch * dout * hout * wout;
    if ((int64_t)batch * d * h * w * cin >= ((int64_t)1 << 31) * 64)
        return fail(H3V_EINVAL, "%s: input too large", what);
    int rc = check_gemm_dims(what, m, cout, k);
    if (rc) return rc;
    if (k * 127 * 127 >= (int64_t)1 << 31) return fail(H3V_EINVAL, "%s: INT32 accumulator bound exceeded", what);
    p.M = (int)m;
    p.N = cout;
    p.K = (int)k;
    p.lda = 0;
    p.C = cin;
    p.Dp = d; p.Hp = h; p.Wp = w;
    p.Do = (int)dout; p.Ho = (int)hout; p.Wo = (int)wout;
    p.KH = kh; p.KW = kw;
    p.SD = sd; p.SH = sh; p.SW = sw;
    p.ldo = cout;
    return H3V_OK;
}

}  // namespace
}  // namespace h3v

using namespace h3v;

extern "C" {

int h3v_gemm_i8_dequant(const int8_t* a, const float* a_scale, const int8_t* w, const float* w_scale,
                        const uint16_t* bias, uint16_t* out, int64_t m, int64_t n, int64_t k,
                        hipStream_t stream) {
    const char* what = "h3v_gemm_i8_dequant";
    H3V_REQUIRE(a && a_scale && w && w_scale && out, "%s: null pointer argument", what);
    int rc = check_gemm_dims(what, m, n, k);
    if (rc) return rc;
    GemmParams p{};
    p.a = a; p.b = w; p.M = (int)m; p.N = (int)n; p.K = (int)k; p.lda = k;
    p.sx = a_scale; p.sx_stride = 1; p.sw = w_scale; p.bias = bias; p.out = out; p.ldo = n;
    return run_gemm<Epi::Dequant>(p, stream, what);
}

int h3v_gemm_i8_swiglu(const int8_t* a, const float* a_scale, const int8_t* w, const float* w_scale,
                       const uint16_t* bias, uint16_t* act, int64_t m, int64_t n, int64_t k,
                       hipStream_t stream) {
    const char* what = "h3v_gemm_i8_swiglu";
    H3V_REQUIRE(a && a_scale && w && w_scale && act, "%s: null pointer argument", what);
    int rc = check_gemm_dims(what, m, 2 * n, k);
    if (rc) return rc;
    GemmParams p{};
    p.a = a; p.b = w; p.M = (int)m; p.N = (int)n; p.K = (int)k; p.lda = k;
    p.sx = a_scale; p.sx_stride = 1; p.sw = w_scale; p.bias = bias; p.out = act; p.ldo = n;
    return run_gemm<Epi::SwiGLU>(p, stream, what);
}

int h3v_gemm_i8_i32(const int8_t* a, const int8_t* w, int32_t* acc, int64_t m, int64_t n, int64_t k,
                    hipStream_t stream) {
    const char* what = "h3v_gemm_i8_i32";
    H3V_REQUIRE(a && w && acc, "%s: null pointer argument", what);
    int rc = check_gemm_dims(what, m, n, k);
    if (rc) return rc;
    GemmParams p{};
    p.a = a; p.b = w; p.M = (int)m; p.N = (int)n; p.K = (int)k; p.lda = k; p.out = acc; p.ldo = n;
    return run_gemm<Epi::Int32>(p, stream, what);
}

int h3v_conv3d_i8(const int8_t* qx, const float* x_scale, const int8_t* qw, const float* w_scale,
                  const uint16_t* bias, uint16_t* out, int batch, int cin, int d, int h, int w, int cout,
                  int kd, int kh, int kw, int sd, int sh, int sw, int causal_skip, hipStream_t stream) {
    const char* what = "h3v_conv3d_i8";
    H3V_REQUIRE(qx && x_scale && qw && w_scale && out, "%s: null pointer argument", what);
    GemmParams p{};
    int rc = fill_conv(p, what, batch, cin, d, h, w, cout, kd, kh, kw, sd, sh, sw);
    if (rc) return rc;
    p.a = qx; p.b = qw; p.sx = x_scale; p.sx_stride = 0; p.sw = w_scale; p.bias = bias; p.out = out;
    p.causal_skip = (causal_skip && kd == 3 && sd == 1) ? 1 : 0;
    return run_conv<Epi::Dequant>(p, stream, what);
}

int h3v_conv3d_i8_residual(const int8_t* qx, const float* x_scale, const int8_t* qw, const float* w_scale,
                           const uint16_t* bias, const uint16_t* residual, uint16_t* out, int batch, int cin, int d,
                           int h, int w, int cout, int kd, int kh, int kw, int sd, int sh, int sw, int causal_skip,
                           hipStream_t stream) {
    const char* what = "h3v_conv3d_i8_residual";
    H3V_REQUIRE(qx && x_scale && qw && w_scale && residual && out, "%s: null pointer argument", what);
    H3V_REQUIRE(residual != out, "%s: the residual must not alias the output", what);
    GemmParams p{};
    int rc = fill_conv(p, what, batch, cin, d, h, w, cout, kd, kh, kw, sd, sh, sw);
    if (rc) return rc;
    p.a = qx; p.b = qw; p.sx = x_scale; p.sx_stride = 0; p.sw = w_scale; p.bias = bias; p.out = out;
    p.res = residual;
    p.causal_skip = (causal_skip && kd == 3 && sd == 1) ? 1 : 0;
    return run_conv<Epi::Dequant>(p, stream, what);
}

int h3v_conv3d_i8_gn(const int8_t* qx, const float* x_scale, const int8_t* qw, const float* w_scale,
                     const uint16_t* bias, const uint16_t* residual, uint16_t* out, int cin, int d, int h, int w,
                     int cout, int causal_skip, const uint16_t* gn_bias, float* workspace, hipStream_t stream) {
    const char* what = "h3v_conv3d_i8_gn";
    H3V_REQUIRE(qx && x_scale && qw && w_scale && out && workspace, "%s: null pointer argument", what);
    H3V_REQUIRE(residual != out, "%s: the residual must not alias the output", what);
    GemmParams p{};
    int rc = fill_conv(p, what, 1, cin, d, h, w, cout, 3, 3, 3, 1, 1, 1);
    if (rc) return rc;
    p.a = qx; p.b = qw; p.sx = x_scale; p.sx_stride = 0; p.sw = w_scale; p.bias = bias; p.out = out;
    p.res = residual;
    p.causal_skip = causal_skip ? 1 : 0;
    H3V_REQUIRE(halo_conv_fits(p) && cin % 128 == 0 && (cout == 128 || cout == 256) && (p.Wo == 128 || p.Wo == 256) &&
                    p.Ho % 8 == 0,
                "%s: needs Cin %% 128 == 0, Cout 128 or 256, output width 128 or 256 and output height a multiple of 8 "
                "(got Cin %d, Cout %d, output %d x %d)", what, cin, cout, p.Ho, p.Wo);
    H3V_REQUIRE(aligned(out, 16) && (!residual || aligned(residual, 16)) && (!gn_bias || aligned(gn_bias, 16)) &&
                    aligned(workspace, 16),
                "%s: out, residual, gn_bias and workspace need 16-byte alignment", what);
    const GnWorkspace g = gn_workspace(workspace, p.Do, p.Ho * p.Wo, kGnTileChunk);
    p.gn_avg = g.avg;
    p.gn_m2 = g.m2;
    p.gn_ext = g.ext;
    p.gn_bias = gn_bias;
    p.gn_nchunk = g.nchunk;
    return p.Wo == 256 ? launch_halo<256, Epi::Dequant>(p, stream, what) : launch_halo<128, Epi::Dequant>(p, stream, what);
}

int h3v_conv3d_i8_residual_padded(const int8_t* qx, const float* x_scale, const int8_t* qw, const float* w_scale,
                                  const uint16_t* bias, const uint16_t* residual, const uint16_t* residual_bias,
                                  uint16_t* out, int batch, int cin, int d, int h, int w, int cout, int causal_skip,
                                  int front, int top, int bottom, int left, int right, hipStream_t stream) {
    const char* what = "h3v_conv3d_i8_residual_padded";
    H3V_REQUIRE(qx && x_scale && qw && w_scale && out, "%s: null pointer argument", what);
    H3V_REQUIRE(residual || !residual_bias, "%s: residual_bias needs a residual", what);
    H3V_REQUIRE(residual != out, "%s: the residual must not alias the output", what);
    H3V_REQUIRE(front >= 0 && front <= 16, "%s: front must be in [0, 16] (got %d)", what, front);
    H3V_REQUIRE(cout <= 65536, "%s: at most 65536 output channels (got %d)", what, cout);
    H3V_REQUIRE((top | bottom | left | right) >= 0 && (top | bottom | left | right) <= 1,
                "%s: the reflect border is 0 or 1 on each side (got %d, %d, %d, %d)", what, top, bottom, left, right);
    GemmParams p{};
    int rc = fill_conv(p, what, batch, cin, d, h, w, cout, 3, 3, 3, 1, 1, 1);
    if (rc) return rc;
    p.a = qx; p.b = qw; p.sx = x_scale; p.sx_stride = 0; p.sw = w_scale; p.bias = bias; p.out = out;
    p.res = residual;
    p.res_bias = residual_bias;
    p.pad_front = front;
    p.pad_top = top; p.pad_bottom = bottom; p.pad_left = left; p.pad_right = right;
    p.causal_skip = causal_skip ? 1 : 0;
    H3V_REQUIRE(halo_conv_fits(p) && p.Ho >= 2 && p.Wo >= 2,
                "%s: needs Cin %% 64 == 0, Cout %% 128 == 0, output width 32, 64, 128 or 256 and output height a "
                "multiple of 512 / width, at least 2 (got Cin %d, Cout %d, output %d x %d)", what, cin, cout, p.Ho,
                p.Wo);
    H3V_REQUIRE(aligned(out, 16) && (!residual || aligned(residual, 16)) &&
                    (!residual_bias || aligned(residual_bias, 16)),
                "%s: out, residual and residual_bias need 16-byte alignment", what);
    switch (p.Wo) {
        case 256: return launch_halo<256, Epi::Dequant, 1, true>(p, stream, what);
        case 128: return launch_halo<128, Epi::Dequant, 1, true>(p, stream, what);
        case 64: return launch_halo<64, Epi::Dequant, 1, true>(p, stream, what);
        default: return launch_halo<32, Epi::Dequant, 1, true>(p, stream, what);
    }
}

static int conv3d_f16_common(const uint16_t* x, const uint16_t* w, const uint16_t* bias, const uint16_t* residual,
                             uint16_t* out, int batch, int cin, int d, int h, int wd, int cout, int kd, int kh, int kw,
                             int sd, int sh, int sw, int causal_skip, float* workspace, int64_t workspace_floats,
                             bool may_split, hipStream_t stream, const char* what) {
    H3V_REQUIRE(x && w && out, "%s: null pointer argument", what);
    H3V_REQUIRE(residual != out, "%s: the residual must not alias the output", what);
    GemmParams p{};
    int rc = fill_conv(p, what, batch, cin, d, h, wd, cout, kd, kh, kw, sd, sh, sw);
    if (rc) return rc;
    p.a = reinterpret_cast<const int8_t*>(x);
    p.b = reinterpret_cast<const int8_t*>(w);
    p.bias = bias;
    p.res = residual;
    p.out = out;
    p.causal_skip = (causal_skip && kd == 3 && sd == 1) ? 1 : 0;
    H3V_REQUIRE(cin % 32 == 0 && aligned(x, 16) && aligned(w, 16),
                "%s: requires Cin %% 32 == 0 and 16-byte aligned x and w (got Cin %d)", what, cin);
    const F16Plan plan = plan_conv_f16(p, may_split);
    switch (plan.kind) {
        case F16Kind::Halo256: return launch_halo<256, Epi::F16Bias, 2>(p, stream, what);
        case F16Kind::Halo128: return launch_halo<128, Epi::F16Bias, 2>(p, stream, what);
        case F16Kind::Halo64: return launch_halo<64, Epi::F16Bias, 2>(p, stream, what);
        case F16Kind::Halo32: return launch_halo<32, Epi::F16Bias, 2>(p, stream, what);
        default: break;
    }
    // implicit GEMM with channels and reduction counted in bytes
    p.C = cin * 2;
    p.K = p.K * 2;
    if (plan.splits > 1) {
        const int64_t need = (int64_t)plan.splits * p.M * p.N;
        H3V_REQUIRE(workspace != nullptr && workspace_floats >= need && aligned(workspace, 16),
                    "%s: this shape splits K %d ways and needs a 16-byte aligned workspace of %lld floats (got %lld)",
                    what, plan.splits, (long long)need, (long long)workspace_floats);
        H3V_REQUIRE(p.N % 4 == 0 && aligned(out, 8) && (residual == nullptr || aligned(residual, 8)),
                    "%s: a split reduction needs Cout %% 4 == 0 and 8-byte aligned output and residual", what);
        GemmParams q = p;
        q.out = workspace;
        q.bias = nullptr;
        q.res = nullptr;
        q.k_splits = plan.splits;
        rc = plan.kind == F16Kind::Tiled256x256
                 ? launch_tiled<256, 256, 128, 2, 4, 3, 2, AMode::Conv, Epi::F32Part>(q, stream, what)
                 : launch_tiled<256, 128, 128, 4, 2, 2, 2, AMode::Conv, Epi::F32Part>(q, stream, what);
        if (rc) return rc;
        const int64_t mn = (int64_t)p.M * p.N;
        hipLaunchKernelGGL(splitk_reduce_f16, dim3((unsigned)((mn / 4 + 255) / 256)), dim3(256), 0, stream,
                           (const float*)workspace, plan.splits, mn, p.N, bias, residual, out);
        return launch_status(what);
    }
    switch (plan.kind) {
        case F16Kind::Tiled512x128: return launch_tiled<512, 128, 128, 4, 2, 2, 2, AMode::Conv, Epi::F16Bias>(p, stream, what);
        case F16Kind::Tiled256x128: return launch_tiled<256, 128, 128, 4, 2, 2, 2, AMode::Conv, Epi::F16Bias>(p, stream, what);
        case F16Kind::Tiled256x256: return launch_tiled<256, 256, 128, 2, 4, 3, 2, AMode::Conv, Epi::F16Bias>(p, stream, what);
        case F16Kind::Tiled256x128k64: return launch_tiled<256, 128, 64, 4, 2, 4, 4, AMode::Conv, Epi::F16Bias>(p, stream, what);
        case F16Kind::Tiled256x128k64r3: return launch_tiled<256, 128, 64, 4, 2, 3, 2, AMode::Conv, Epi::F16Bias>(p, stream, what);
        default: return launch_tiled<256, 256, 64, 2, 4, 4, 4, AMode::Conv, Epi::F16Bias>(p, stream, what);
    }
}

int h3v_conv3d_f16(const uint16_t* x, const uint16_t* w, const uint16_t* bias, const uint16_t* residual,
                   uint16_t* out, int batch, int cin, int d, int h, int wd, int cout, int kd, int kh, int kw, int sd,
                   int sh, int sw, int causal_skip, hipStream_t stream) {
    return conv3d_f16_common(x, w, bias, residual, out, batch, cin, d, h, wd, cout, kd, kh, kw, sd, sh, sw,
                             causal_skip, nullptr, 0, false, stream, "h3v_conv3d_f16");
}

int h3v_conv3d_f16_ws(const uint16_t* x, const uint16_t* w, const uint16_t* bias, const uint16_t* residual,
                      uint16_t* out, int batch, int cin, int d, int h, int wd, int cout, int kd, int kh, int kw,
                      int sd, int sh, int sw, int causal_skip, float* workspace, int64_t workspace_floats,
                      hipStream_t stream) {
    return conv3d_f16_common(x, w, bias, residual, out, batch, cin, d, h, wd, cout, kd, kh, kw, sd, sh, sw,
                             causal_skip, workspace, workspace_floats, true, stream, "h3v_conv3d_f16_ws");
}

int h3v_conv3d_f16_gn(const uint16_t* x, const uint16_t* w, const uint16_t* bias, uint16_t* out, int cin, int d,
                      int h, int wd, int cout, int kd, int kh, int kw, int sd, int sh, int sw, int causal_skip,
                      float* workspace, hipStream_t stream) {
    const char* what = "h3v_conv3d_f16_gn";
    H3V_REQUIRE(x && w && out && workspace, "%s: null pointer argument", what);
    GemmParams p{};
    int rc = fill_conv(p, what, 1, cin, d, h, wd, cout, kd, kh, kw, sd, sh, sw);
    if (rc) return rc;
    const int64_t hw = (int64_t)p.Ho * p.Wo;
    H3V_REQUIRE(cout == 128 && hw % 256 == 0,
                "%s: the chunk statistics need 128 output channels and an output frame of a multiple of 256 pixels "
                "(got Cout %d, %d x %d)", what, cout, p.Ho, p.Wo);
    H3V_REQUIRE(cin % 32 == 0 && aligned(x, 16) && aligned(w, 16) && aligned(out, 16) && aligned(workspace, 16),
                "%s: requires Cin %% 32 == 0 and 16-byte aligned x, w, out and workspace (got Cin %d)", what, cin);
    p.a = reinterpret_cast<const int8_t*>(x);
    p.b = reinterpret_cast<const int8_t*>(w);
    p.bias = bias;
    p.out = out;
    p.causal_skip = (causal_skip && kd == 3 && sd == 1) ? 1 : 0;
    const GnWorkspace g = gn_workspace(workspace, p.Do, (int)hw, kGnSizingChunk);
    p.gn_avg = g.avg;
    p.gn_m2 = g.m2;
    p.gn_ext = g.ext;
    p.gn_nchunk = g.nchunk;
    // the implicit GEMM on 256 x 128 tiles (one tile = one statistics chunk); these are the kernels
    // h3v_conv3d_f16 itself runs for conv_in (64-byte K steps) and the stage-0 downsample
    const bool k64 = (cin * 2) % 128 != 0;
    p.C = cin * 2;
    p.K = p.K * 2;
    return k64 ? launch_tiled<256, 128, 64, 4, 2, 3, 2, AMode::Conv, Epi::F16Bias>(p, stream, what)
               : launch_tiled<256, 128, 128, 4, 2, 2, 2, AMode::Conv, Epi::F16Bias>(p, stream, what);
}

int64_t h3v_conv3d_f16_workspace_floats(int batch, int cin, int d, int h, int wd, int cout, int kd, int kh, int kw,
                                        int sd, int sh, int sw) {
    GemmParams p{};
    if (fill_conv(p, "h3v_conv3d_f16_workspace_floats", batch, cin, d, h, wd, cout, kd, kh, kw, sd, sh, sw))
        return -1;
    p.a = p.b = reinterpret_cast<const int8_t*>(16);   // alignment only; plan_conv_f16 reads no memory
    const F16Plan plan = plan_conv_f16(p, true);
    return plan.splits > 1 ? (int64_t)plan.splits * p.M * p.N : 0;
}

int h3v_conv3d_i8_i32(const int8_t* qx, const int8_t* qw, int32_t* acc, int batch, int cin, int d, int h,
                      int w, int cout, int kd, int kh, int kw, int sd, int sh, int sw, int causal_skip,
                      hipStream_t stream) {
    const char* what = "h3v_conv3d_i8_i32";
    H3V_REQUIRE(qx && qw && acc, "%s: null pointer argument", what);
    GemmParams p{};
    int rc = fill_conv(p, what, batch, cin, d, h, w, cout, kd, kh, kw, sd, sh, sw);
    if (rc) return rc;
    p.a = qx; p.b = qw; p.out = acc;
    p.causal_skip = (causal_skip && kd == 3 && sd == 1) ? 1 : 0;
    return run_conv<Epi::Int32>(p, stream, what);
}

}  // extern "C"
