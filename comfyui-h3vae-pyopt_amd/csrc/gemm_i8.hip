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
// Tiling: BM x BN x 64 workgroup tile, 2 x 2 waves, each wave owning a
// (BM/2) x (BN/2) block built from v_mfma_i32_32x32x32_i8.  Global -> register ->
// LDS double buffering with one barrier per K step; LDS rows are padded to
// 80 bytes so the 16-byte fragment reads of 8 consecutive lanes hit distinct
// banks.  Workgroup ids are remapped so that each XCD (own L2) walks a
// contiguous, M-grouped range of tiles.
#include "h3v_common.hpp"
#include "h3v_abi.hpp"

namespace h3v {
namespace {

enum class AMode { Gemm, Conv };
enum class Epi { Dequant, SwiGLU, Int32 };

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
    void* out;
    int64_t ldo;
    int tiles_m, tiles_n;
};

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

template <int BM, int BN, int BK, AMode AM, Epi EP>
__global__ __launch_bounds__(256, 1) void gemm_i8_mfma(GemmParams p) {
    constexpr int NT = 256;
    constexpr int WGN = 2;
    constexpr int WM = BM / 2, WN = BN / 2;
    constexpr int FM = WM / 32, FN = WN / 32;
    constexpr int LDS = BK + 16;        // padded row stride (bytes)
    constexpr int CPR = BK / 16;        // 16-byte chunks per row
    constexpr int RPP = NT / CPR;       // rows covered per pass of the block
    constexpr int A_CH = BM / RPP, B_CH = BN / RPP;
    static_assert(BM % RPP == 0 && BN % RPP == 0, "tile rows must be a multiple of rows per pass");
    static_assert(EP != Epi::SwiGLU || (WN % 64) == 0, "SwiGLU pairs need 64-column wave tiles");

    extern __shared__ __attribute__((aligned(16))) int8_t smem[];
    int8_t* sA = smem;
    int8_t* sB = smem + 2 * BM * LDS;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / WGN, wn = wave % WGN;

    int tm, tn;
    grouped_tile(xcd_remap(blockIdx.x, gridDim.x), p.tiles_m, p.tiles_n, 8, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;

    const int crow = tid / CPR;
    const int ccol = (tid % CPR) * 16;

    int64_t abase[A_CH];
#pragma unroll
    for (int i = 0; i < A_CH; ++i) {
        int m = m0 + crow + i * RPP;
        m = m < p.M ? m : p.M - 1;
        abase[i] = (AM == AMode::Gemm ? (int64_t)m * p.lda : conv_row_offset(p, m)) + ccol;
    }
    const int8_t* bptr[B_CH];
#pragma unroll
    for (int i = 0; i < B_CH; ++i) {
        int r = crow + i * RPP;
        int wrow;
        if constexpr (EP == Epi::SwiGLU) {
            // tile row r -> pair r/64, half (r/32)&1 (0 gate, 1 up), lane r&31
            int c = tn * (BN / 2) + (r >> 6) * 32 + (r & 31);
            c = c < p.N ? c : p.N - 1;
            wrow = ((r >> 5) & 1) ? p.N + c : c;
        } else {
            int n = n0 + r;
            wrow = n < p.N ? n : p.N - 1;
        }
        bptr[i] = p.b + (int64_t)wrow * p.K + ccol;
    }

    const int nkb = p.K / BK;
    const int kb0 = (AM == AMode::Conv) ? conv_first_kblock(p, m0, BM, BK) : 0;

    v16i acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = v16i{};

    v4i ra[A_CH], rb[B_CH];
    auto gload = [&](int kb) {
        int64_t koff = (AM == AMode::Gemm) ? (int64_t)kb * BK : conv_k_offset(p, kb * BK);
#pragma unroll
        for (int i = 0; i < A_CH; ++i) ra[i] = *reinterpret_cast<const v4i*>(p.a + abase[i] + koff);
#pragma unroll
        for (int i = 0; i < B_CH; ++i) rb[i] = *reinterpret_cast<const v4i*>(bptr[i] + (int64_t)kb * BK);
    };
    auto sstore = [&](int buf) {
        int8_t* a = sA + buf * BM * LDS + crow * LDS + ccol;
        int8_t* b = sB + buf * BN * LDS + crow * LDS + ccol;
#pragma unroll
        for (int i = 0; i < A_CH; ++i) *reinterpret_cast<v4i*>(a + i * RPP * LDS) = ra[i];
#pragma unroll
        for (int i = 0; i < B_CH; ++i) *reinterpret_cast<v4i*>(b + i * RPP * LDS) = rb[i];
    };

    if (kb0 < nkb) {
        gload(kb0);
        sstore(0);
    }
    __syncthreads();

    const int frow = lane & 31;
    const int fk = (lane >> 5) * 16;
    for (int kb = kb0; kb < nkb; ++kb) {
        const int buf = (kb - kb0) & 1;
        if (kb + 1 < nkb) gload(kb + 1);
        const int8_t* a_base = sA + buf * BM * LDS + (wm * WM + frow) * LDS + fk;
        const int8_t* b_base = sB + buf * BN * LDS + (wn * WN + frow) * LDS + fk;
#pragma unroll
        for (int ks = 0; ks < BK / 32; ++ks) {
            v4i af[FM], bf[FN];
#pragma unroll
            for (int i = 0; i < FM; ++i) af[i] = *reinterpret_cast<const v4i*>(a_base + i * 32 * LDS + ks * 32);
#pragma unroll
            for (int j = 0; j < FN; ++j) bf[j] = *reinterpret_cast<const v4i*>(b_base + j * 32 * LDS + ks * 32);
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        if (kb + 1 < nkb) sstore(buf ^ 1);
        __syncthreads();
    }

    // Epilogue.  v_mfma 32x32 result layout: lane holds column lane&31 and rows
    // (r/4)*8 + (lane/32)*4 + r%4 for register r.
    const int col_l = lane & 31;
    const int row_l = (lane >> 5) * 4;
    if constexpr (EP == Epi::SwiGLU) {
        uint16_t* out = static_cast<uint16_t*>(p.out);
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN / 2; ++j) {
                int c = tn * (BN / 2) + (wn * WN) / 2 + j * 32 + col_l;
                if (c >= p.N) continue;
                float swg = p.sw[c], swu = p.sw[p.N + c];
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    int row = m0 + wm * WM + i * 32 + (r >> 2) * 8 + row_l + (r & 3);
                    if (row >= p.M) continue;
                    float sx = p.sx[(int64_t)row * p.sx_stride];
                    float g = rt16(g1_value(acc[i][2 * j][r], sx, swg, p.bias, c));
                    float u = rt16(g1_value(acc[i][2 * j + 1][r], sx, swu, p.bias, p.N + c));
                    out[(int64_t)row * p.ldo + c] = f2h(silu(g) * u);
                }
            }
    } else {
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                int col = n0 + wn * WN + j * 32 + col_l;
                if (col >= p.N) continue;
                float sw = 0.0f;
                if constexpr (EP == Epi::Dequant) sw = p.sw[col];
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    int row = m0 + wm * WM + i * 32 + (r >> 2) * 8 + row_l + (r & 3);
                    if (row >= p.M) continue;
                    if constexpr (EP == Epi::Int32) {
                        static_cast<int32_t*>(p.out)[(int64_t)row * p.ldo + col] = acc[i][j][r];
                    } else {
                        float sx = p.sx[(int64_t)row * p.sx_stride];
                        static_cast<uint16_t*>(p.out)[(int64_t)row * p.ldo + col] =
                            f2h(g1_value(acc[i][j][r], sx, sw, p.bias, col));
                    }
                }
            }
    }
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
        static_cast<uint16_t*>(p.out)[(int64_t)row * p.ldo + col] = f2h(g1_value(dot(col), sx, p.sw[col], p.bias, col));
    }
}

constexpr int kBK = 64;

template <int BM, int BN, AMode AM, Epi EP>
int launch_tiled(GemmParams p, hipStream_t stream, const char* what) {
    int ncols = (EP == Epi::SwiGLU) ? 2 * p.N : p.N;
    p.tiles_m = (p.M + BM - 1) / BM;
    p.tiles_n = (ncols + BN - 1) / BN;
    int64_t grid = (int64_t)p.tiles_m * p.tiles_n;
    if (grid > 0x7fffffff) return fail(H3V_EINVAL, "%s: too many tiles", what);
    size_t lds = (size_t)2 * (BM + BN) * (kBK + 16);
    hipLaunchKernelGGL((gemm_i8_mfma<BM, BN, kBK, AM, EP>), dim3((unsigned)grid), dim3(256), lds, stream, p);
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
    bool tiled = p.K % kBK == 0 && p.lda % 16 == 0 && aligned(p.a, 16) && aligned(p.b, 16);
    if (!tiled) return launch_generic<AMode::Gemm, EP>(p, stream, what);
    return launch_tiled<256, 256, AMode::Gemm, EP>(p, stream, what);
}

template <Epi EP>
int run_conv(GemmParams p, hipStream_t stream, const char* what) {
    bool tiled = p.C % kBK == 0 && aligned(p.a, 16) && aligned(p.b, 16);
    if (!tiled) {
        p.causal_skip = 0;  // the generic path always runs the full reduction
        return launch_generic<AMode::Conv, EP>(p, stream, what);
    }
    if (p.N <= 128) return launch_tiled<256, 128, AMode::Conv, EP>(p, stream, what);
    return launch_tiled<256, 256, AMode::Conv, EP>(p, stream, what);
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
