/*
 * h3v_oracle.c -- CPU restatement of the H3 VAE INT8 hot-path arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * (or as the timed CPU baseline).  The product path never calls it.
 *
 * Every routine is written as plain scalar C with IEEE-754 binary32
 * arithmetic, no FMA contraction (built with -ffp-contract=off) and explicit
 * fmaf() only where the reference contract names a fused multiply-add.  FP16
 * values travel as raw uint16_t bit patterns and are converted by the
 * round-to-nearest-even routines below.
 *
 * Reduction orders that the reference leaves to its compiler are fixed here
 * and documented per function; the HIP kernels use the same orders, so the
 * oracle and the kernels agree bit for bit.  Where the reference order is
 * published (the norm1 W16 sum of squares) that order is used.
 *
 * References are file:line in fishelegs/ComfyUI-H3VAE-PyOpt.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define API __attribute__((visibility("default")))

/* ------------------------------------------------------------------------ */
/* binary16 <-> binary32, round to nearest even                              */
/* ------------------------------------------------------------------------ */

static inline uint32_t f_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float bits_f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

API float ora_h2f(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exp = (h >> 10) & 0x1f;
    uint32_t man = h & 0x3ff;
    if (exp == 0x1f) return bits_f(sign | 0x7f800000u | (man << 13));  /* inf / nan */
    if (exp == 0) {
        /* zero or subnormal: value = man * 2^-24, exact in binary32 */
        float v = (float)man * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    return bits_f(sign | ((exp + 112) << 23) | (man << 13));
}

API uint16_t ora_f2h(float f) {
    uint32_t u = f_bits(f);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t a = u & 0x7fffffffu;
    if (a >= 0x7f800000u) {                       /* inf or nan */
        if (a == 0x7f800000u) return sign | 0x7c00u;
        return sign | 0x7e00u | (uint16_t)((a >> 13) & 0x3ffu);
    }
    if (a >= 0x477ff000u) return sign | 0x7c00u;  /* >= 65520 rounds to inf */
    if (a >= 0x38800000u) {                       /* normal binary16 range */
        uint32_t e = (a >> 23) - 112;             /* rebias 127 -> 15 */
        uint32_t m = a & 0x7fffffu;
        uint32_t r = m & 0x1fffu;                 /* 13 dropped bits */
        uint32_t h = (e << 10) | (m >> 13);
        if (r > 0x1000u || (r == 0x1000u && (h & 1u))) h += 1;  /* carries into exponent correctly */
        return sign | (uint16_t)h;
    }
    /* subnormal binary16 (or zero): value / 2^-24, round to nearest even */
    {
        float v = bits_f(a);
        float scaled = v * 16777216.0f;           /* exact: power-of-two scale */
        float r = rintf(scaled);                  /* nearest even */
        return sign | (uint16_t)(int)r;           /* r <= 1024 -> 0x400 is the smallest normal */
    }
}

static inline float hf(uint16_t h) { return ora_h2f(h); }
static inline float rt16(float f) { return ora_h2f(ora_f2h(f)); }

/* ------------------------------------------------------------------------ */
/* exp: Cody-Waite reduction + degree-7 Taylor polynomial (own method)       */
/* ------------------------------------------------------------------------ */
/*
 * exp(x) = 2^n * exp(r),  n = rint(x * log2(e)),  r = (x - n*LN2_HI) - n*LN2_LO.
 * LN2_HI carries the leading 15 bits of ln 2, so n*LN2_HI is exact for |n| < 2^9.
 * exp(r) for |r| <= 0.35 by Horner on the Taylor series to r^7 (truncation
 * error < 6e-9 relative).  2^n applied with ldexpf (single rounding).
 * Same operation order in the HIP kernels (h3v_expf in csrc/h3v_math.hpp).
 */
API float ora_expf(float x) {
    if (x != x) return x;
    if (x > 88.72283935546875f) return INFINITY;
    if (x < -103.972084045410156f) return 0.0f;
    const float LOG2E = 0x1.715476p+0f;
    const float LN2_HI = 0x1.62e4p-1f;     /* 15 significant bits of ln 2 */
    const float LN2_LO = 0x1.7f7d1cp-20f;  /* ln 2 - LN2_HI */
    float n = rintf(x * LOG2E);
    float r = fmaf(-n, LN2_HI, x);          /* n * LN2_HI is exact: one rounding either way */
    r = fmaf(-n, LN2_LO, r);
    float p = 0x1.a01a02p-13f;             /* 1/5040 */
    p = fmaf(p, r, 0x1.6c16c2p-10f);       /* 1/720  */
    p = fmaf(p, r, 0x1.111112p-7f);        /* 1/120  */
    p = fmaf(p, r, 0x1.555556p-5f);        /* 1/24   */
    p = fmaf(p, r, 0x1.555556p-3f);        /* 1/6    */
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    return ldexpf(p, (int)n);
}

/* SiLU as the reference writes it: z / (1 + exp(-z)) in binary32. */
static inline float silu32(float z) { return z / (1.0f + ora_expf(-z)); }

/* 1/sqrt(x) as two correctly rounded operations. */
static inline float rsqrt_rn(float x) { return 1.0f / sqrtf(x); }

/* ------------------------------------------------------------------------ */
/* Fixed reduction trees                                                     */
/* ------------------------------------------------------------------------ */
/*
 * Butterfly over an array of partials: level 1 pairs i with i^16, i^8 ... i^1
 * inside groups of 32 ("warps"), level 2 pairs warp partials w with w^(nw/2)
 * ... w^1.  Because a+b == b+a exactly, the butterfly equals the halving tree
 * T[i] = T[i] + T[i+off] on the lower half.
 */
static float butterfly(float* p, int n) {
    int warp = n < 32 ? n : 32;
    int nw = n / warp;
    for (int w = 0; w < nw; ++w) {
        float* t = p + w * warp;
        for (int off = warp / 2; off >= 1; off >>= 1)
            for (int i = 0; i < off; ++i) t[i] = t[i] + t[i + off];
    }
    /* gather the warp partials */
    for (int w = 1; w < nw; ++w) p[w] = p[w * warp];
    for (int off = nw / 2; off >= 1; off >>= 1)
        for (int i = 0; i < off; ++i) p[i] = p[i] + p[i + off];
    return p[0];
}

/*
 * Published norm1 W16 sum of squares (docs/decoder_norm1_contract_2026-10-03.md:57-70):
 * per virtual thread four consecutive values x0..x3,
 *   s1 = x1*x1; a = fma(x0,x0,s1); b = fma(x2,x2,a); s3 = x3*x3; p = s3 + b,
 * then the 32-lane butterfly and the warp-partial butterfly.
 */
static float sumsq_w16(const float* x, int k, float* scratch) {
    int n = k / 4;
    for (int t = 0; t < n; ++t) {
        const float* v = x + 4 * t;
        float s1 = v[1] * v[1];
        float a = fmaf(v[0], v[0], s1);
        float b = fmaf(v[2], v[2], a);
        float s3 = v[3] * v[3];
        scratch[t] = s3 + b;
    }
    return butterfly(scratch, n);
}

/* Plain tree: per virtual thread ((t0+t1)+t2)+t3 of already rounded terms, then the butterfly. */
static float sum_plain(const float* terms, int k, float* scratch) {
    int n = k / 4;
    for (int t = 0; t < n; ++t) {
        const float* v = terms + 4 * t;
        scratch[t] = ((v[0] + v[1]) + v[2]) + v[3];
    }
    return butterfly(scratch, n);
}

/* Exposed for pinning the fixed trees in tests. */
API float ora_tree_sumsq_w16(const float* x, int k) {
    float* tmp = (float*)malloc(sizeof(float) * (size_t)k);
    float r = sumsq_w16(x, k, tmp);
    free(tmp);
    return r;
}

API float ora_tree_sum_plain(const float* terms, int k) {
    float* tmp = (float*)malloc(sizeof(float) * (size_t)k);
    float r = sum_plain(terms, k, tmp);
    free(tmp);
    return r;
}

/* ------------------------------------------------------------------------ */
/* Q1: comfy-kitchen 0.2.34 row quantization as restated by the reference    */
/* opt/int8_swiglu_fused.py:29-37, opt/int8_ffn_up_fused.py:96-103           */
/* ------------------------------------------------------------------------ */
static void q1_row(const float* a, int64_t k, int8_t* q, float* s_out) {
    float amax = 0.0f;
    for (int64_t i = 0; i < k; ++i) { float v = fabsf(a[i]); if (v > amax) amax = v; }
    float s = amax * (1.0f / 127.0f);
    if (!(s >= 1.0e-30f)) s = 1.0e-30f;           /* max(s, 1e-30) */
    float d = rt16(s);                            /* divide in the source dtype */
    for (int64_t i = 0; i < k; ++i) {
        float v = rt16(a[i] / d);
        v = rintf(v);                             /* ties to even */
        if (v != v) v = -128.0f;
        if (v > 127.0f) v = 127.0f;
        if (v < -128.0f) v = -128.0f;
        q[i] = (int8_t)(int)v;
    }
    *s_out = s;
}

API void ora_row_quant(const uint16_t* x, int64_t m, int64_t k, int8_t* q, float* s) {
    #pragma omp parallel
    {
        float* row = (float*)malloc(sizeof(float) * (size_t)k);
        #pragma omp for schedule(static)
        for (int64_t r = 0; r < m; ++r) {
            for (int64_t i = 0; i < k; ++i) row[i] = hf(x[r * k + i]);
            q1_row(row, k, q + r * k, s + r);
        }
        free(row);
    }
}

/* F6: SwiGLU of an fp16 [gate | up] row then Q1 (opt/int8_swiglu_fused.py:22-38). */
API void ora_swiglu_row_quant(const uint16_t* x, int64_t m, int64_t k, int8_t* q, float* s) {
    #pragma omp parallel
    {
        float* row = (float*)malloc(sizeof(float) * (size_t)k);
        #pragma omp for schedule(static)
        for (int64_t r = 0; r < m; ++r) {
            for (int64_t i = 0; i < k; ++i) {
                float g = hf(x[r * 2 * k + i]);
                float u = hf(x[r * 2 * k + k + i]);
                row[i] = rt16(silu32(g) * u);
            }
            q1_row(row, k, q + r * k, s + r);
        }
        free(row);
    }
}

/* ------------------------------------------------------------------------ */
/* INT8 GEMM: int32 accumulators of A[M,K] . W[N,K]^T                         */
/* ------------------------------------------------------------------------ */
API void ora_gemm_i8_acc(const int8_t* a, const int8_t* w, int32_t* acc,
                         int64_t m, int64_t n, int64_t k) {
    #pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < m; ++r) {
        const int8_t* ar = a + r * k;
        for (int64_t c = 0; c < n; ++c) {
            const int8_t* wc = w + c * k;
            int32_t s = 0;
            for (int64_t i = 0; i < k; ++i) s += (int32_t)ar[i] * (int32_t)wc[i];
            acc[r * n + c] = s;
        }
    }
}

/*
 * G1 epilogue (opt/int8_ffn_up_fused.py:76-84; CK visitor tree in
 * docs/benchmarks/decoder_int8_ffn_2026-10-03.json:5370):
 *   v = fp32(acc) * sx[m];  v = bias ? fma(v, sw[n], fp32(b[n])) : v * sw[n];  out = fp16(v)
 * sx_stride 0 broadcasts one scale (the encoder conv's per-tensor scale).
 */
static inline float g1_value(int32_t acc, float sx, float sw, const uint16_t* bias, int64_t c) {
    float v = (float)acc * sx;
    return bias ? fmaf(v, sw, hf(bias[c])) : v * sw;
}

API void ora_gemm_dequant(const int32_t* acc, const float* sx, int64_t sx_stride,
                          const float* sw, const uint16_t* bias, uint16_t* out,
                          int64_t m, int64_t n) {
    #pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < m; ++r)
        for (int64_t c = 0; c < n; ++c)
            out[r * n + c] = ora_f2h(g1_value(acc[r * n + c], sx[r * sx_stride], sw[c], bias, c));
}

/*
 * F2 epilogue (opt/int8_ffn_up_fused.py:63-88): output column c pairs weight
 * row c (gate) with row nh + c (up).  acc is [M, 2*nh] in weight-row order.
 */
API void ora_gemm_swiglu(const int32_t* acc, const float* sx, const float* sw,
                         const uint16_t* bias, uint16_t* act, int64_t m, int64_t nh) {
    #pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < m; ++r)
        for (int64_t c = 0; c < nh; ++c) {
            float g = rt16(g1_value(acc[r * 2 * nh + c], sx[r], sw[c], bias, c));
            float u = rt16(g1_value(acc[r * 2 * nh + nh + c], sx[r], sw[nh + c], bias, nh + c));
            act[r * nh + c] = ora_f2h(silu32(g) * u);
        }
}

/* ------------------------------------------------------------------------ */
/* E1: static per-output-channel conv weight quant (opt/encoder_int8.py:303-327) */
/* ------------------------------------------------------------------------ */
/*
 * w: float32 [O, C, kd, kh, kw] (any source dtype widened to fp32).  Packs to
 * [O, (kd,kh,kw,c)] with c fastest.  scale = amax * fp32(1/127) (the GPU
 * install path multiplies by the rounded reciprocal; the reference's CPU
 * test path divides, which can differ by one ulp), 0 -> 1;
 * q = clamp(round_half_even(w / scale), +-127).
 */
API void ora_prepare_conv_weight(const float* w, int o, int c, int kd, int kh, int kw,
                                 int8_t* q, float* scale) {
    int64_t taps = (int64_t)kd * kh * kw, k = taps * c;
    for (int oc = 0; oc < o; ++oc) {
        float amax = 0.0f;
        for (int64_t i = 0; i < k; ++i) { float v = fabsf(w[oc * k + i]); if (v > amax) amax = v; }
        float s = amax * (1.0f / 127.0f);
        if (!(s > 0.0f)) s = 1.0f;
        scale[oc] = s;
        for (int ic = 0; ic < c; ++ic)
            for (int64_t t = 0; t < taps; ++t) {
                float v = rintf(w[(oc * c + ic) * taps + t] / s);
                if (v > 127.0f) v = 127.0f;
                if (v < -127.0f) v = -127.0f;
                q[oc * k + t * c + ic] = (int8_t)(int)v;
            }
    }
}

/* ------------------------------------------------------------------------ */
/* E3: per-tensor dynamic activation quant (opt/encoder_int8.py:343-378)     */
/* ------------------------------------------------------------------------ */
/* scale = amax *rn fp32(1/127), 0 -> 1 (merge_scale, :356-364). */
API float ora_tensor_scale_from_amax(float amax) {
    float s = amax * (1.0f / 127.0f);
    return s > 0.0f ? s : 1.0f;
}

API float ora_tensor_amax(const uint16_t* x, int64_t n) {
    float amax = 0.0f;
    for (int64_t i = 0; i < n; ++i) { float v = fabsf(hf(x[i])); if (v > amax) amax = v; }
    return amax;
}

/* round half away from zero as floor(v+0.5) (:372-377), clamp to +-127. */
static inline int8_t e3_quant(float v, float s) {
    float t = v / s;
    float r = t >= 0.0f ? floorf(t + 0.5f) : -floorf(-t + 0.5f);
    if (r > 127.0f) r = 127.0f;
    if (r < -127.0f) r = -127.0f;
    return (int8_t)(int)r;
}

API void ora_tensor_quant(const uint16_t* x, int64_t n, float s, int8_t* q) {
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) q[i] = e3_quant(hf(x[i]), s);
}

/* ------------------------------------------------------------------------ */
/* E4: valid conv3d as implicit GEMM over NDHWC int8 (opt/encoder_int8_pipeline.py:73-119) */
/* ------------------------------------------------------------------------ */
/*
 * qx: int8 [B, Dp, Hp, Wp, C]; qw: int8 [O, kd*kh*kw*C] (k = (kd,kh,kw,c), c fastest);
 * acc: int32 [B, Do, Ho, Wo, O].  Plain loops; integer sums are order free.
 */
API void ora_conv3d_acc(const int8_t* qx, const int8_t* qw, int32_t* acc,
                        int b, int c, int dp, int hp, int wp, int o,
                        int kd, int kh, int kw, int sd, int sh, int sw) {
    int dout = (dp - kd) / sd + 1, hout = (hp - kh) / sh + 1, wout = (wp - kw) / sw + 1;
    int64_t kk = (int64_t)kd * kh * kw * c;
    int64_t mtot = (int64_t)b * dout * hout * wout;
    #pragma omp parallel for schedule(static)
    for (int64_t m = 0; m < mtot; ++m) {
        int64_t r = m;
        int ow = (int)(r % wout); r /= wout;
        int oh = (int)(r % hout); r /= hout;
        int od = (int)(r % dout); int ob = (int)(r / dout);
        for (int oc = 0; oc < o; ++oc) {
            const int8_t* wr = qw + oc * kk;
            int32_t s = 0;
            for (int a = 0; a < kd; ++a)
                for (int bb = 0; bb < kh; ++bb)
                    for (int e = 0; e < kw; ++e) {
                        const int8_t* xp = qx + ((((int64_t)ob * dp + od * sd + a) * hp + oh * sh + bb) * wp + ow * sw + e) * c;
                        const int8_t* wp_ = wr + (int64_t)((a * kh + bb) * kw + e) * c;
                        for (int ic = 0; ic < c; ++ic) s += (int32_t)xp[ic] * (int32_t)wp_[ic];
                    }
            acc[m * o + oc] = s;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* E6: per-frame GroupNorm(32) statistics                                    */
/* opt/encoder_fused_temporal_norm.py:12-51, opt/encoder_fused_norm_bias.py:14-39 */
/* ------------------------------------------------------------------------ */
/*
 * x: fp16 NDHWC [D, H, W, C] (batch one).  Optional pre_bias: v = fp16(v + b[c]).
 * Fixed order (shared with csrc/gn_pack.hip):
 *   chunks of 256 pixels (65536 / C for C > 256); inside a chunk, "pixel lane"
 *   pl = 0..PL-1 with PL = 256 / TPP (TPP = C/8 threads per pixel for C <= 256,
 *   32 above: one per group) owns pixels pl, pl+PL, ...; for each group (cg = C/32
 *   channels) the lane sums channel values left to right per pixel, then adds
 *   that pixel sum to its running sum; lanes combine by the halving tree
 *   (off = PL/2 .. 1).  avg = S / n.  Second pass the same with
 *   (v-avg)^2 terms.  Chunks merge sequentially as in _merge:
 *   mean = (sum_j avg_j*n_j) / N, var = (sum_j (m2_j + (n_j*d_j)*d_j)) / N,
 *   rstd = 1/sqrt(max(var,0) + eps).
 * stats: [D, 32, 2] = (mean, rstd).
 */
#define GN_CHUNK 256
#define GN_GROUPS 32

static inline float gn_load(const uint16_t* x, const uint16_t* pre_bias, int64_t idx, int ch) {
    float v = hf(x[idx]);
    if (pre_bias) v = rt16(v + hf(pre_bias[ch]));
    return v;
}

API void ora_gn_stats(const uint16_t* x, const uint16_t* pre_bias, int d, int h, int w, int c,
                      float eps, float* stats) {
    int hw = h * w;
    int cg = c / GN_GROUPS;
    int tpp = c <= 256 ? c / 8 : 32;
    int chunk = c <= 256 ? GN_CHUNK : 65536 / c;
    int pl_n = 256 / tpp;
    int steps = chunk / pl_n;
    int nchunk = (hw + chunk - 1) / chunk;
    #pragma omp parallel for schedule(static)
    for (int t = 0; t < d; ++t) {
        float* avg = (float*)malloc(sizeof(float) * (size_t)nchunk * GN_GROUPS);
        float* m2 = (float*)malloc(sizeof(float) * (size_t)nchunk * GN_GROUPS);
        int* cnt = (int*)malloc(sizeof(int) * (size_t)nchunk);
        float lanes[256];
        for (int j = 0; j < nchunk; ++j) {
            int p0 = j * chunk;
            int npix = hw - p0 < chunk ? hw - p0 : chunk;
            cnt[j] = npix;
            for (int g = 0; g < GN_GROUPS; ++g) {
                float n = (float)(npix * cg);
                for (int pl = 0; pl < pl_n; ++pl) {
                    float ls = 0.0f;
                    for (int s = 0; s < steps; ++s) {
                        int p = pl + s * pl_n;
                        if (p >= npix) continue;
                        int64_t base = ((int64_t)t * hw + p0 + p) * c + g * cg;
                        float ps = gn_load(x, pre_bias, base, g * cg);
                        for (int i = 1; i < cg; ++i) ps = ps + gn_load(x, pre_bias, base + i, g * cg + i);
                        ls = ls + ps;
                    }
                    lanes[pl] = ls;
                }
                for (int off = pl_n / 2; off >= 1; off >>= 1)
                    for (int i = 0; i < off; ++i) lanes[i] = lanes[i] + lanes[i + off];
                float a = lanes[0] / n;
                for (int pl = 0; pl < pl_n; ++pl) {
                    float lm = 0.0f;
                    for (int s = 0; s < steps; ++s) {
                        int p = pl + s * pl_n;
                        if (p >= npix) continue;
                        int64_t base = ((int64_t)t * hw + p0 + p) * c + g * cg;
                        float dv = gn_load(x, pre_bias, base, g * cg) - a;
                        float pm = dv * dv;
                        for (int i = 1; i < cg; ++i) {
                            dv = gn_load(x, pre_bias, base + i, g * cg + i) - a;
                            pm = pm + dv * dv;
                        }
                        lm = lm + pm;
                    }
                    lanes[pl] = lm;
                }
                for (int off = pl_n / 2; off >= 1; off >>= 1)
                    for (int i = 0; i < off; ++i) lanes[i] = lanes[i] + lanes[i + off];
                avg[j * GN_GROUPS + g] = a;
                m2[j * GN_GROUPS + g] = lanes[0];
            }
        }
        float total = (float)(hw * cg);
        for (int g = 0; g < GN_GROUPS; ++g) {
            float san = 0.0f;
            for (int j = 0; j < nchunk; ++j) san = san + avg[j * GN_GROUPS + g] * (float)(cnt[j] * cg);
            float mean = san / total;
            float sv = 0.0f;
            for (int j = 0; j < nchunk; ++j) {
                float dl = avg[j * GN_GROUPS + g] - mean;
                float nj = (float)(cnt[j] * cg);
                sv = sv + (m2[j * GN_GROUPS + g] + (nj * dl) * dl);
            }
            float var = sv / total;
            if (var < 0.0f) var = 0.0f;
            stats[(t * GN_GROUPS + g) * 2] = mean;
            stats[(t * GN_GROUPS + g) * 2 + 1] = rsqrt_rn(var + eps);
        }
        free(avg); free(m2); free(cnt);
    }
}

/*
 * E6b: the same statistics over 512-pixel conv tiles (the window conv's statistics epilogue in
 * csrc/gemm_i8.hip `write_tile`, read back by h3v_gn_norm_pack_i8_partials).  Chunk j of a frame
 * is the tile of rows 8 rb .. 8 rb + 7 and columns 64 cb .. 64 cb + 63, j = rb * (W / 64) + cb;
 * tile pixel r = (row - 8 rb) * 64 + (column - 64 cb).  Per group (cg channels), pixel lane
 * pl = 0..31 takes tile pixels pl + 32 s, s = 0..15: the group's channels of a pixel summed left
 * to right, added to the lane's running sum.  The lanes combine as the adjacent tree: for
 * off = 1, 2, 4, 8, 16, lane i (a multiple of 2 off) adds lane i + off.  avg = S / (512 cg); M2
 * the same with (v - avg)^2 terms.  Outputs in the producer workspace layout:
 * avg, m2 [D][32][nchunk]; ext [D][nchunk][C] = fp16 max | fp16 min << 16 per channel.
 * Requires H % 8 == 0 and W % 64 == 0.
 */
#define GN_TILE_ROWS 8
#define GN_TILE_COLS 64
#define GN_TILE_LANES 32

API void ora_gn_partials_tiled(const uint16_t* x, const uint16_t* pre_bias, int d, int h, int w, int c,
                               float* avg, float* m2, uint32_t* ext) {
    int cg = c / GN_GROUPS;
    int ncb = w / GN_TILE_COLS;
    int nchunk = (h / GN_TILE_ROWS) * ncb;
    int tpix = GN_TILE_ROWS * GN_TILE_COLS;
    int steps = tpix / GN_TILE_LANES;
    #pragma omp parallel for schedule(static)
    for (int tj = 0; tj < d * nchunk; ++tj) {
        int t = tj / nchunk, j = tj % nchunk;
        int rb = j / ncb, cb = j % ncb;
        float lanes[GN_TILE_LANES];
        /* image index of tile pixel r */
        #define TILE_PIX(r) (((int64_t)t * h + rb * GN_TILE_ROWS + (r) / GN_TILE_COLS) * w + \
                             cb * GN_TILE_COLS + (r) % GN_TILE_COLS)
        for (int g = 0; g < GN_GROUPS; ++g) {
            for (int pl = 0; pl < GN_TILE_LANES; ++pl) {
                float ls = 0.0f;
                for (int st = 0; st < steps; ++st) {
                    int64_t base = TILE_PIX(pl + GN_TILE_LANES * st) * c + g * cg;
                    float ps = gn_load(x, pre_bias, base, g * cg);
                    for (int i = 1; i < cg; ++i) ps = ps + gn_load(x, pre_bias, base + i, g * cg + i);
                    ls = ls + ps;
                }
                lanes[pl] = ls;
            }
            for (int off = 1; off < GN_TILE_LANES; off <<= 1)
                for (int i = 0; i < GN_TILE_LANES; i += 2 * off) lanes[i] = lanes[i] + lanes[i + off];
            float a = lanes[0] / (float)(tpix * cg);
            for (int pl = 0; pl < GN_TILE_LANES; ++pl) {
                float lm = 0.0f;
                for (int st = 0; st < steps; ++st) {
                    int64_t base = TILE_PIX(pl + GN_TILE_LANES * st) * c + g * cg;
                    float dv = gn_load(x, pre_bias, base, g * cg) - a;
                    float pm = dv * dv;
                    for (int i = 1; i < cg; ++i) {
                        dv = gn_load(x, pre_bias, base + i, g * cg + i) - a;
                        pm = pm + dv * dv;
                    }
                    lm = lm + pm;
                }
                lanes[pl] = lm;
            }
            for (int off = 1; off < GN_TILE_LANES; off <<= 1)
                for (int i = 0; i < GN_TILE_LANES; i += 2 * off) lanes[i] = lanes[i] + lanes[i + off];
            avg[((int64_t)t * GN_GROUPS + g) * nchunk + j] = a;
            m2[((int64_t)t * GN_GROUPS + g) * nchunk + j] = lanes[0];
        }
        for (int ch = 0; ch < c; ++ch) {
            float mx = -INFINITY, mn = INFINITY;
            for (int r = 0; r < tpix; ++r) {
                float v = gn_load(x, pre_bias, TILE_PIX(r) * c + ch, ch);
                mx = fmaxf(mx, v);
                mn = fminf(mn, v);
            }
            ext[((int64_t)t * nchunk + j) * c + ch] = (uint32_t)ora_f2h(mx) | ((uint32_t)ora_f2h(mn) << 16);
        }
        #undef TILE_PIX
    }
}

/* Chan merge of equal chunks (as in ora_gn_stats) -> stats [D, 32, 2] = (mean, rstd). */
API void ora_gn_merge_equal(const float* avg, const float* m2, int d, int nchunk, int chunk_pixels, int c,
                            float eps, float* stats) {
    int cg = c / GN_GROUPS;
    for (int t = 0; t < d; ++t)
        for (int g = 0; g < GN_GROUPS; ++g) {
            const float* a = avg + ((int64_t)t * GN_GROUPS + g) * nchunk;
            const float* m = m2 + ((int64_t)t * GN_GROUPS + g) * nchunk;
            float nj = (float)(chunk_pixels * cg);
            float total = (float)(nchunk * chunk_pixels * cg);
            float san = 0.0f;
            for (int j = 0; j < nchunk; ++j) san = san + a[j] * nj;
            float mean = san / total;
            float sv = 0.0f;
            for (int j = 0; j < nchunk; ++j) {
                float dl = a[j] - mean;
                sv = sv + (m[j] + (nj * dl) * dl);
            }
            float var = sv / total;
            if (var < 0.0f) var = 0.0f;
            stats[(t * GN_GROUPS + g) * 2] = mean;
            stats[(t * GN_GROUPS + g) * 2 + 1] = rsqrt_rn(var + eps);
        }
}

/*
 * Norm / SiLU / causal + reflect pad producer
 * (opt/encoder_int8_norm_recompute.py:18-48):
 *   z = fp16(((v - mean) * rstd) * gamma + beta); z = fp16(z / (1 + exp(-z)))
 * output NDHWC [D+2, H+2, W+2, C]; frames 0,1 are zeros; spatial reflect 1.
 * Writes the fp16 values (y, nullable), returns absmax; writes int8 (q,
 * nullable) with the E3 rounding against `scale`.
 */
static inline int reflect(int i, int n) { return i < 0 ? -i : (i >= n ? 2 * n - 2 - i : i); }

API float ora_norm_pack(const uint16_t* x, const uint16_t* pre_bias, const uint16_t* gamma,
                        const uint16_t* beta, const float* stats, int d, int h, int w, int c,
                        uint16_t* y, int8_t* q, float scale) {
    int hp = h + 2, wp = w + 2;
    int cg = c / GN_GROUPS;
    float amax = 0.0f;
    #pragma omp parallel for schedule(static) reduction(max:amax)
    for (int tp = 0; tp < d + 2; ++tp) {
        for (int i = 0; i < hp; ++i)
            for (int j = 0; j < wp; ++j)
                for (int ch = 0; ch < c; ++ch) {
                    int64_t oidx = (((int64_t)tp * hp + i) * wp + j) * c + ch;
                    float z = 0.0f;
                    int t = tp - 2;
                    if (t >= 0) {
                        int si = reflect(i - 1, h), sj = reflect(j - 1, w);
                        float v = gn_load(x, pre_bias, (((int64_t)t * h + si) * w + sj) * c + ch, ch);
                        int g = ch / cg;
                        float mean = stats[(t * GN_GROUPS + g) * 2];
                        float rstd = stats[(t * GN_GROUPS + g) * 2 + 1];
                        float zz = rt16(((v - mean) * rstd) * hf(gamma[ch]) + hf(beta[ch]));
                        z = rt16(silu32(zz));
                    }
                    if (y) y[oidx] = ora_f2h(z);
                    if (q) q[oidx] = e3_quant(z, scale);
                    float az = fabsf(z);
                    if (az > amax) amax = az;
                }
    }
    return amax;
}

/* ------------------------------------------------------------------------ */
/* Decoder producers                                                         */
/* ------------------------------------------------------------------------ */
/*
 * N1 norm1 producer (opt/int8_norm1_quant.py:113-123, recipe
 * docs/decoder_norm1_contract_2026-10-03.md:57-70):
 *   raw = fma(o, g, h); h_out = fp16(raw); ss = W16 tree of raw^2;
 *   inv = 1/sqrt(ss/K + eps); n = fp16((fp32(h_out) * inv) * w); Q1(n).
 * recipe 0: W16 fma-chain sum of squares (norm1).
 * recipe 1: plain tree of rounded squares (norm2, opt/int8_norm_quant.py:22-43).
 */
API void ora_residual_rms_quant(const uint16_t* h, const uint16_t* o, const uint16_t* g,
                                const uint16_t* w, float eps, int64_t m, int k, int recipe,
                                uint16_t* h_out, int8_t* q, float* s) {
    #pragma omp parallel
    {
        float* raw = (float*)malloc(sizeof(float) * (size_t)k);
        float* tmp = (float*)malloc(sizeof(float) * (size_t)k);
        float* nrm = (float*)malloc(sizeof(float) * (size_t)k);
        #pragma omp for schedule(static)
        for (int64_t r = 0; r < m; ++r) {
            for (int i = 0; i < k; ++i)
                raw[i] = fmaf(hf(o[r * k + i]), hf(g[i]), hf(h[r * k + i]));
            float ss;
            if (recipe == 0) {
                ss = sumsq_w16(raw, k, tmp);
            } else {
                for (int i = 0; i < k; ++i) nrm[i] = raw[i] * raw[i];
                ss = sum_plain(nrm, k, tmp);
            }
            float inv = rsqrt_rn(ss / (float)k + eps);
            for (int i = 0; i < k; ++i) {
                uint16_t hb = ora_f2h(raw[i]);
                h_out[r * k + i] = hb;
                nrm[i] = rt16((hf(hb) * inv) * hf(w[i]));
            }
            q1_row(nrm, k, q + r * k, s + r);
        }
        free(raw); free(tmp); free(nrm);
    }
}

/* N3 block-0 RMSNorm (opt/decoder_block0_norm.py:39-59): W16 tree of x^2. */
API void ora_rms_fp16(const uint16_t* x, const uint16_t* gamma, float eps, int64_t m, int k,
                      uint16_t* out) {
    #pragma omp parallel
    {
        float* xv = (float*)malloc(sizeof(float) * (size_t)k);
        float* tmp = (float*)malloc(sizeof(float) * (size_t)k);
        #pragma omp for schedule(static)
        for (int64_t r = 0; r < m; ++r) {
            for (int i = 0; i < k; ++i) xv[i] = hf(x[r * k + i]);
            float inv = rsqrt_rn(sumsq_w16(xv, k, tmp) / (float)k + eps);
            for (int i = 0; i < k; ++i) out[r * k + i] = ora_f2h((xv[i] * inv) * hf(gamma[i]));
        }
        free(xv); free(tmp);
    }
}

/*
 * N4 final residual + LayerNorm (opt/decoder_final_norm.py:35-56):
 *   raw = fma(o, gate, h); mean = tree(raw)/K; m2 = tree((raw-mean)^2);
 *   inv = 1/sqrt(m2/K + eps); y = fp16(fma((raw - mean) * inv, gamma, beta)).
 * The reference's Welford order is compiler-owned; this fixes a two-pass order.
 */
API void ora_residual_layernorm(const uint16_t* h, const uint16_t* o, const uint16_t* gate,
                                const uint16_t* gamma, const uint16_t* beta, float eps,
                                int64_t m, int k, uint16_t* out) {
    #pragma omp parallel
    {
        float* raw = (float*)malloc(sizeof(float) * (size_t)k);
        float* tmp = (float*)malloc(sizeof(float) * (size_t)k);
        float* sq = (float*)malloc(sizeof(float) * (size_t)k);
        #pragma omp for schedule(static)
        for (int64_t r = 0; r < m; ++r) {
            for (int i = 0; i < k; ++i)
                raw[i] = fmaf(hf(o[r * k + i]), hf(gate[i]), hf(h[r * k + i]));
            float mean = sum_plain(raw, k, tmp) / (float)k;
            for (int i = 0; i < k; ++i) { float dv = raw[i] - mean; sq[i] = dv * dv; }
            float var = sum_plain(sq, k, tmp) / (float)k;
            float inv = rsqrt_rn(var + eps);
            for (int i = 0; i < k; ++i)
                out[r * k + i] = ora_f2h(fmaf((raw[i] - mean) * inv, hf(gamma[i]), hf(beta[i])));
        }
        free(raw); free(tmp); free(sq);
    }
}

/*
 * R1 QK RMSNorm + partial rotate-half RoPE (opt/decoder_fused_qk_rope.py:12-35):
 * x: fp16 [tokens, heads, 3*dh] with per-head [q | k | v]; cos/sin fp16 [tokens, rot].
 *   q = fp16(q * (1/sqrt(tree(q*q)/dh + eps)))  (same for k)
 *   d < rot: qo = fp32(fp16(q[d]*c[d])) + fp32(fp16(qr[d]*s[d])), qr[d] = -q[d+rot/2] (d < rot/2)
 *            or q[d-rot/2]; stored fp16.  d >= rot: q passes through.
 */
API void ora_qk_rope(const uint16_t* x, const uint16_t* cosv, const uint16_t* sinv,
                     int64_t tokens, int heads, int dh, int rot, float eps,
                     uint16_t* qo, uint16_t* ko) {
    #pragma omp parallel
    {
        float* v = (float*)malloc(sizeof(float) * (size_t)dh);
        float* sq = (float*)malloc(sizeof(float) * (size_t)dh);
        float* tmp = (float*)malloc(sizeof(float) * (size_t)dh);
        #pragma omp for schedule(static)
        for (int64_t tk = 0; tk < tokens; ++tk)
            for (int hd = 0; hd < heads; ++hd)
                for (int which = 0; which < 2; ++which) {
                    const uint16_t* src = x + (tk * heads + hd) * (int64_t)(3 * dh) + which * dh;
                    uint16_t* dst = (which ? ko : qo) + (tk * heads + hd) * (int64_t)dh;
                    for (int i = 0; i < dh; ++i) { v[i] = hf(src[i]); sq[i] = v[i] * v[i]; }
                    float inv = rsqrt_rn(sum_plain(sq, dh, tmp) / (float)dh + eps);
                    for (int i = 0; i < dh; ++i) v[i] = rt16(v[i] * inv);
                    int half = rot / 2;
                    for (int i = 0; i < dh; ++i) {
                        float outv;
                        if (i < rot) {
                            float rv = i < half ? -v[i + half] : v[i - half];
                            float cc = hf(cosv[tk * rot + i]), ss = hf(sinv[tk * rot + i]);
                            outv = rt16(v[i] * cc) + rt16(rv * ss);
                        } else {
                            outv = v[i];
                        }
                        dst[i] = ora_f2h(outv);
                    }
                }
        free(v); free(sq); free(tmp);
    }
}

/* ------------------------------------------------------------------------ */
/* E9 residual + bias pack before the stage-1 downsample conv                */
/* (opt/encoder_fused_residual_pack.py:12-55, _residual_pack :12-33)         */
/* ------------------------------------------------------------------------ */

/* x, r: fp16 NDHWC [d, h, w, c]; bias fp16 [c]; out fp16 [d+2, h+1, w+1, c].
 * Two leading zero frames; the extra bottom row / right column reflect
 * (index h -> h-2, w -> w-2, :25-26); y = fp32 r + (fp32 x + fp32 b), one
 * fp16 rounding at the store (:31-32). */
API void ora_residual_downsample_pack(const uint16_t* x, const uint16_t* r, const uint16_t* bias, uint16_t* out,
                                      int c, int d, int h, int w) {
    const int64_t ho = h + 1, wo = w + 1;
    for (int64_t t2 = 0; t2 < d + 2; ++t2)
        for (int64_t y = 0; y < ho; ++y)
            for (int64_t xw = 0; xw < wo; ++xw) {
                uint16_t* dst = out + ((t2 * ho + y) * wo + xw) * c;
                if (t2 < 2) {
                    memset(dst, 0, sizeof(uint16_t) * (size_t)c);
                    continue;
                }
                const int64_t t = t2 - 2;
                const int64_t hs = y == h ? h - 2 : y;
                const int64_t ws = xw == w ? w - 2 : xw;
                const int64_t src = ((t * h + hs) * w + ws) * c;
                for (int ch = 0; ch < c; ++ch)
                    dst[ch] = ora_f2h(hf(r[src + ch]) + (hf(x[src + ch]) + hf(bias[ch])));
            }
}

/* Pixel finalisation (reference opt/fp16_finalize.py:24-54, FMA disabled at
 * launch): contiguous [B, 3, T, H, W] of fp16 (is_f16) or fp32 decoded pixels ->
 * fp32 v = fp32(x) * std[c] + mean[c] (two roundings), then v < 0 -> 0,
 * v > 1 -> 1; NaN and an in-range -0 pass through unchanged. */
API void ora_finalize_pixels(const void* x, int is_f16, int64_t b, int64_t thw, const float* std, const float* mean,
                             float* out) {
    for (int64_t i = 0; i < b * 3 * thw; ++i) {
        const int c = (int)((i / thw) % 3);
        const float xv = is_f16 ? hf(((const uint16_t*)x)[i]) : ((const float*)x)[i];
        const float m = xv * std[c];
        const float v = m + mean[c];
        out[i] = v < 0.0f ? 0.0f : (v > 1.0f ? 1.0f : v);
    }
}

API int ora_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

API void ora_set_num_threads(int n) {
#ifdef _OPENMP
    omp_set_num_threads(n);
#else
    (void)n;
#endif
}
