/*
 * oracle.c -- CPU restatement of the SigLIP2 Q8_0 matmul hot path.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h): the tests' parity reference and the timed CPU
 * baseline, never part of the product.  Built with -ffp-contract=off so every
 * float operation rounds where the restated code rounds; fused multiply-adds
 * appear only as explicit fmaf() calls.
 */
#include "oracle.h"
#include "cpu_q8.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define ORC_BLOCK_BYTES 34 /* fp16 d + 32 int8 */

static int orc_threads(int n) {
#ifdef _OPENMP
    return n > 0 ? n : omp_get_max_threads();
#else
    (void)n;
    return 1;
#endif
}

/* ------------------------------------------------------------------------ */
/* fp16                                                                      */
/* ------------------------------------------------------------------------ */

uint16_t orc_fp32_to_fp16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t exp = (x >> 23) & 0xffu;
    uint32_t man = x & 0x7fffffu;
    if (exp == 0xffu) { /* inf / nan (nan stays quiet) */
        return (uint16_t)(sign | 0x7c00u | (man ? (0x200u | (man >> 13)) : 0u));
    }
    const int32_t e = (int32_t)exp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign; /* below half the smallest subnormal */
        man |= 0x800000u;
        const int shift = 14 - e;           /* 14..24 */
        uint32_t h = man >> shift;
        const uint32_t rem = man & ((1u << shift) - 1u);
        const uint32_t mid = 1u << (shift - 1);
        if (rem > mid || (rem == mid && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
    uint32_t h = ((uint32_t)e << 10) | (man >> 13);
    const uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++; /* carry may reach inf */
    return (uint16_t)(sign | h);
}

float orc_fp16_to_fp32(uint16_t h) {
    const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    const uint32_t exp = ((uint32_t)h >> 10) & 0x1fu;
    const uint32_t man = (uint32_t)h & 0x3ffu;
    uint32_t x;
    if (exp == 0) {
        float v = ldexpf((float)man, -24); /* exact */
        return sign ? -v : v;
    } else if (exp == 31) {
        x = sign | 0x7f800000u | (man << 13);
    } else {
        x = sign | ((exp + 112u) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

void orc_fp32_to_fp16_n(const float *x, uint16_t *y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = orc_fp32_to_fp16(x[i]);
}

void orc_fp16_to_fp32_n(const uint16_t *x, float *y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = orc_fp16_to_fp32(x[i]);
}

static inline float fp16r(float f) { return orc_fp16_to_fp32(orc_fp32_to_fp16(f)); }

/* ------------------------------------------------------------------------ */
/* quantizers                                                                */
/* ------------------------------------------------------------------------ */

static void quant_q8_0_block(const float *x, uint8_t *blk) {
    float amax = 0.0f;
    for (int j = 0; j < ORC_QK; ++j) {
        const float a = fabsf(x[j]);
        if (a > amax) amax = a;
    }
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    const uint16_t dh = orc_fp32_to_fp16(d);
    memcpy(blk, &dh, 2);
    int8_t *qs = (int8_t *)(blk + 2);
    for (int j = 0; j < ORC_QK; ++j) qs[j] = (int8_t)roundf(x[j] * id);
}

void orc_quantize_q8_0(const float *x, int64_t n_rows, int64_t k, void *out) {
    orc_quantize_q8_0_padded(x, n_rows, k, k, out);
}

void orc_quantize_q8_0_padded(const float *x, int64_t n_rows, int64_t k,
                              int64_t k_pad, void *out) {
    const int64_t nb = k_pad / ORC_QK;
    uint8_t *o = (uint8_t *)out;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < n_rows; ++r) {
        float buf[ORC_QK];
        for (int64_t b = 0; b < nb; ++b) {
            for (int j = 0; j < ORC_QK; ++j) {
                const int64_t c = b * ORC_QK + j;
                buf[j] = c < k ? x[r * k + c] : 0.0f;
            }
            quant_q8_0_block(buf, o + (r * nb + b) * ORC_BLOCK_BYTES);
        }
    }
}

void orc_dequantize_q8_0(const void *blocks, int64_t n_rows, int64_t k_pad,
                         float *y) {
    const int64_t nb = k_pad / ORC_QK;
    const uint8_t *p = (const uint8_t *)blocks;
    for (int64_t r = 0; r < n_rows; ++r) {
        for (int64_t b = 0; b < nb; ++b) {
            const uint8_t *blk = p + (r * nb + b) * ORC_BLOCK_BYTES;
            uint16_t dh;
            memcpy(&dh, blk, 2);
            const float d = orc_fp16_to_fp32(dh);
            const int8_t *qs = (const int8_t *)(blk + 2);
            for (int j = 0; j < ORC_QK; ++j) y[r * k_pad + b * ORC_QK + j] = (float)qs[j] * d;
        }
    }
}

void orc_quantize_q8_1(const float *x, int64_t M, int64_t K, int64_t ldx,
                       int64_t K_pad, int8_t *qs, uint16_t *ds) {
    const int64_t nb = K_pad / ORC_QK;
#pragma omp parallel for schedule(static)
    for (int64_t m = 0; m < M; ++m) {
        for (int64_t b = 0; b < nb; ++b) {
            float v[ORC_QK];
            float amax = 0.0f;
            for (int j = 0; j < ORC_QK; ++j) {
                const int64_t c = b * ORC_QK + j;
                v[j] = c < K ? x[m * ldx + c] : 0.0f;
                const float a = fabsf(v[j]);
                if (a > amax) amax = a;
            }
            const float d = amax / 127.0f;
            const float inv = amax != 0.0f ? 127.0f / amax : 0.0f;
            int sum = 0;
            int8_t *q = qs + m * K_pad + b * ORC_QK;
            for (int j = 0; j < ORC_QK; ++j) {
                /* default mode: half-even; the conversion saturates as the
                 * reference's __float2int_rn (+inf -> 127, -inf -> -128,
                 * NaN -> 0): a block whose 127 / amax overflows (amax <
                 * 127 / FLT_MAX) forms +-inf products and 0 * inf */
                const float r = nearbyintf(v[j] * inv);
                const int iq = r != r ? 0 : r >= 127.0f ? 127 : r <= -128.0f ? -128 : (int)r;
                q[j] = (int8_t)iq;
                sum += iq;
            }
            ds[(m * nb + b) * 2 + 0] = orc_fp32_to_fp16(d);
            ds[(m * nb + b) * 2 + 1] = orc_fp32_to_fp16((float)sum * d);
        }
    }
}

/* ------------------------------------------------------------------------ */
/* GEMM                                                                      */
/* ------------------------------------------------------------------------ */

int32_t orc_block_dot(const int8_t *qa, const int8_t *qb) {
    int32_t s = 0;
    for (int j = 0; j < ORC_QK; ++j) s += (int32_t)qa[j] * (int32_t)qb[j];
    return s;
}

void orc_block_dots(const void *w, int64_t K_pad, int64_t n,
                    const int8_t *qs, int64_t m, int32_t *out) {
    const int64_t nb = K_pad / ORC_QK;
    const uint8_t *wrow = (const uint8_t *)w + n * nb * ORC_BLOCK_BYTES;
    for (int64_t b = 0; b < nb; ++b)
        out[b] = orc_block_dot((const int8_t *)(wrow + b * ORC_BLOCK_BYTES + 2),
                               qs + m * K_pad + b * ORC_QK);
}

/* Split the 34-byte blocks of W into a contiguous int8 plane and a float
 * scale plane so the inner loop vectorises; the arithmetic is unchanged. */
void orc_mul_mat_q8_0_q8_1(const void *w, int64_t K_pad, int64_t N,
                           const int8_t *qs, const uint16_t *ds, int64_t M,
                           float *y, int nthreads) {
    const int64_t nb = K_pad / ORC_QK;
    int8_t *wq = (int8_t *)malloc((size_t)(N * K_pad));
    float *wd = (float *)malloc(sizeof(float) * (size_t)(N * nb));
    float *xd = (float *)malloc(sizeof(float) * (size_t)(M * nb));
    const uint8_t *wp = (const uint8_t *)w;
    for (int64_t n = 0; n < N; ++n)
        for (int64_t b = 0; b < nb; ++b) {
            const uint8_t *blk = wp + (n * nb + b) * ORC_BLOCK_BYTES;
            uint16_t dh;
            memcpy(&dh, blk, 2);
            wd[n * nb + b] = orc_fp16_to_fp32(dh);
            memcpy(wq + n * K_pad + b * ORC_QK, blk + 2, ORC_QK);
        }
    for (int64_t i = 0; i < M * nb; ++i) xd[i] = orc_fp16_to_fp32(ds[2 * i]);

    const int nt = orc_threads(nthreads);
    /* tile over (m, n) so a W tile stays in cache across a few rows */
    const int64_t TN = 64;
    const int64_t n_tiles = (N + TN - 1) / TN;
#pragma omp parallel for schedule(dynamic, 1) num_threads(nt) collapse(2)
    for (int64_t mt = 0; mt < (M + 3) / 4; ++mt) {
        for (int64_t nt_ = 0; nt_ < n_tiles; ++nt_) {
            for (int64_t m = mt * 4; m < mt * 4 + 4 && m < M; ++m) {
                const int8_t *xr = qs + m * K_pad;
                const float *xdr = xd + m * nb;
                for (int64_t n = nt_ * TN; n < nt_ * TN + TN && n < N; ++n) {
                    const int8_t *wr = wq + n * K_pad;
                    const float *wdr = wd + n * nb;
                    float acc = 0.0f;
                    for (int64_t b = 0; b < nb; ++b) {
                        const int8_t *a = wr + b * ORC_QK;
                        const int8_t *c = xr + b * ORC_QK;
                        int32_t s = 0;
                        for (int j = 0; j < ORC_QK; ++j) s += (int32_t)a[j] * (int32_t)c[j];
                        acc = fmaf((float)s, wdr[b] * xdr[b], acc);
                    }
                    y[m * N + n] = acc;
                }
            }
        }
    }
    free(wq);
    free(wd);
    free(xd);
}

/* The CPU baseline's GEMM kernel (orc_set_gemm_kernel): 0 the loop above,
 * 1 cpu_q8.c's VNNI kernel (the same bits) where the CPU has it, with each
 * weight repacked on first use and kept (keyed by its address) */
static int gemm_kernel = 0;
#define ORC_WCACHE 512
static struct {
    const void *raw;
    int64_t K_pad, N;
    cq8_weight *w;
} wcache[ORC_WCACHE];
static int wcache_n = 0;

int orc_set_gemm_kernel(int k) {
    const int old = gemm_kernel;
    gemm_kernel = k == 1 && cq8_have_vnni() ? 1 : 0;
    return old;
}

void orc_clear_gemm_cache(void) {
    for (int i = 0; i < wcache_n; ++i) cq8_free(wcache[i].w);
    wcache_n = 0;
}

static cq8_weight *cached_weight(const void *w, int64_t K_pad, int64_t N) {
    cq8_weight *r = NULL;
#pragma omp critical(orc_wcache)
    {
        for (int i = 0; i < wcache_n && !r; ++i)
            if (wcache[i].raw == w && wcache[i].K_pad == K_pad && wcache[i].N == N) r = wcache[i].w;
        if (!r && wcache_n < ORC_WCACHE) {
            r = cq8_prepare(w, K_pad, N);
            wcache[wcache_n].raw = w;
            wcache[wcache_n].K_pad = K_pad;
            wcache[wcache_n].N = N;
            wcache[wcache_n].w = r;
            ++wcache_n;
        }
    }
    return r;
}

void orc_mul_mat_q8_0_f32(const void *w, int64_t K_pad, int64_t N,
                          const float *x, int64_t K, int64_t ldx, int64_t M,
                          float *y, int nthreads) {
    const int64_t nb = K_pad / ORC_QK;
    int8_t *qs = (int8_t *)malloc((size_t)(M * K_pad));
    uint16_t *ds = (uint16_t *)malloc(sizeof(uint16_t) * 2 * (size_t)(M * nb));
    orc_quantize_q8_1(x, M, K, ldx, K_pad, qs, ds);
    cq8_weight *cw = gemm_kernel == 1 ? cached_weight(w, K_pad, N) : NULL;
    if (cw)
        cq8_mul_mat(cw, qs, ds, M, y, orc_threads(nthreads));
    else
        orc_mul_mat_q8_0_q8_1(w, K_pad, N, qs, ds, M, y, nthreads);
    free(qs);
    free(ds);
}

void orc_mul_mat_f16_f32(const uint16_t *w, int64_t K, int64_t N, const float *x,
                         int64_t ldx, int64_t M, float *y, int nthreads) {
    const int nt = orc_threads(nthreads);
    double *xh = (double *)malloc(sizeof(double) * (size_t)(M * K));
    for (int64_t m = 0; m < M; ++m)
        for (int64_t k = 0; k < K; ++k) xh[m * K + k] = (double)fp16r(x[m * ldx + k]);
#pragma omp parallel for schedule(static) num_threads(nt)
    for (int64_t n = 0; n < N; ++n) {
        double *wr = (double *)malloc(sizeof(double) * (size_t)K);
        for (int64_t k = 0; k < K; ++k) wr[k] = (double)orc_fp16_to_fp32(w[n * K + k]);
        for (int64_t m = 0; m < M; ++m) {
            const double *xr = xh + m * K;
            double acc = 0.0;
            for (int64_t k = 0; k < K; ++k) acc += xr[k] * wr[k];
            y[m * N + n] = (float)acc;
        }
        free(wr);
    }
    free(xh);
}

/* ------------------------------------------------------------------------ */
/* LayerNorm / GELU                                                          */
/* ------------------------------------------------------------------------ */

void orc_layernorm(const float *x, int64_t M, int64_t H, int64_t ldx,
                   const float *w, const float *b, float eps, float *y,
                   int64_t ldy) {
#pragma omp parallel for schedule(static)
    for (int64_t m = 0; m < M; ++m) {
        const float *xr = x + m * ldx;
        float *yr = y + m * ldy;
        double sum = 0.0;
        for (int64_t i = 0; i < H; ++i) sum += (double)xr[i];
        const float mean = (float)(sum / (double)H);
        double sum2 = 0.0;
        for (int64_t i = 0; i < H; ++i) {
            const float v = xr[i] - mean;
            yr[i] = v;
            sum2 += (double)(v * v);
        }
        const float variance = (float)(sum2 / (double)H);
        const float scale = 1.0f / sqrtf(variance + eps);
        for (int64_t i = 0; i < H; ++i) {
            float t = yr[i] * scale;
            if (w) t = t * w[i];
            if (b) t = t + b[i];
            yr[i] = t;
        }
    }
}

/* tanh from IEEE f32 primitives only (see oracle.h), so that the CPU and
 * any other IEEE machine running the same operations agree bit for bit. */
static float exp_cw(float t) {
    const float k = rintf(t * 1.44269504088896341f);
    float r = fmaf(-k, 0.693359375f, t);
    r = fmaf(-k, -2.12194440e-4f, r);
    float p = 1.0f / 5040.0f;
    p = fmaf(p, r, 1.0f / 720.0f);
    p = fmaf(p, r, 1.0f / 120.0f);
    p = fmaf(p, r, 1.0f / 24.0f);
    p = fmaf(p, r, 1.0f / 6.0f);
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    return ldexpf(p, (int)k);
}

float orc_tanh_f32(float u) {
    const float a = fabsf(u);
    float r;
    if (a >= 9.0f) {
        r = 1.0f;
    } else if (a < 0.5f) {
        const float z = a * a;
        float p = -929569.0f / 638512875.0f;
        p = fmaf(p, z, 21844.0f / 6081075.0f);
        p = fmaf(p, z, -1382.0f / 155925.0f);
        p = fmaf(p, z, 62.0f / 2835.0f);
        p = fmaf(p, z, -17.0f / 315.0f);
        p = fmaf(p, z, 2.0f / 15.0f);
        p = fmaf(p, z, -1.0f / 3.0f);
        r = fmaf(a * z, p, a);
    } else {
        const float e = exp_cw(2.0f * a);
        r = (e - 1.0f) / (e + 1.0f);
    }
    return copysignf(r, u);
}

float orc_gelu(float x) {
    const float GELU_COEF_A = 0.044715f;
    const float SQRT_2_OVER_PI = 0.79788456080286535587989211986876f;
    const float g = SQRT_2_OVER_PI * x * (1.0f + GELU_COEF_A * x * x);
    /* the upper clamp keeps 1 + e^t below 2^126 */
    const float t = fminf(fmaxf(-2.0f * g, -100.0f), 87.0f);
    return x / (1.0f + exp_cw(t));
}

/* src/cuda/siglip2_megakernel.cu:276-280: 0.5 x (1 + tanh(g)), same g */
float orc_gelu_tanhf(float x) {
    const float GELU_COEF_A = 0.044715f;
    const float SQRT_2_OVER_PI = 0.79788456080286535587989211986876f;
    return 0.5f * x * (1.0f + tanhf(SQRT_2_OVER_PI * x * (1.0f + GELU_COEF_A * x * x)));
}

/* ggml-cpu GGML_GELU_FP16: the table is built once, on first use */
static uint16_t gelu_table[1 << 16];
static int gelu_table_ready = 0;

static void gelu_table_build(void) {
#pragma omp critical(orc_gelu_table)
    if (!gelu_table_ready) {
        for (int i = 0; i < (1 << 16); ++i)
            gelu_table[i] = orc_fp32_to_fp16(orc_gelu_tanhf(orc_fp16_to_fp32((uint16_t)i)));
        __atomic_store_n(&gelu_table_ready, 1, __ATOMIC_RELEASE);
    }
}

float orc_gelu_ggml(float x) {
    if (x <= -10.0f) return 0.0f;
    if (x >= 10.0f) return x;
    if (!__atomic_load_n(&gelu_table_ready, __ATOMIC_ACQUIRE)) gelu_table_build();
    return orc_fp16_to_fp32(gelu_table[orc_fp32_to_fp16(x)]);
}

static int gelu_mode = 0;

int orc_set_gelu_mode(int mode) {
    const int old = gelu_mode;
    gelu_mode = mode;
    return old;
}

void orc_gelu_array(int mode, const float *x, float *y, int64_t n) {
#pragma omp parallel for schedule(static) if (n > 65536)
    for (int64_t i = 0; i < n; ++i)
        y[i] = mode == 2 ? orc_gelu_ggml(x[i]) : mode == 1 ? orc_gelu_tanhf(x[i]) : orc_gelu(x[i]);
}

/* the tower restatements' GELU, per orc_set_gelu_mode */
static void gelu_n(float *u, int64_t n) {
    const int mode = gelu_mode;
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i)
        u[i] = mode == 2 ? orc_gelu_ggml(u[i]) : mode == 1 ? orc_gelu_tanhf(u[i]) : orc_gelu(u[i]);
}

/* ------------------------------------------------------------------------ */
/* attention                                                                 */
/* ------------------------------------------------------------------------ */

/* Q, K, V rounded to fp16 as they enter flash attention (see orc_attention) */
void orc_attention_1q(const float *q, const float *k, const float *v, int64_t ld,
                      int64_t n_pos, int64_t n_head, int64_t d_head, float scale,
                      float *out) {
    double *s = (double *)malloc(sizeof(double) * (size_t)(n_pos > 0 ? n_pos : 1));
    for (int64_t h = 0; h < n_head; ++h) {
        double mx = -INFINITY;
        for (int64_t j = 0; j < n_pos; ++j) {
            double acc = 0.0;
            for (int64_t d = 0; d < d_head; ++d)
                acc += (double)fp16r(q[h * d_head + d]) * (double)fp16r(k[j * ld + h * d_head + d]);
            s[j] = acc * (double)scale;
            if (s[j] > mx) mx = s[j];
        }
        double den = 0.0;
        for (int64_t j = 0; j < n_pos; ++j) {
            s[j] = exp(s[j] - mx);
            den += s[j];
        }
        for (int64_t d = 0; d < d_head; ++d) {
            double acc = 0.0;
            for (int64_t j = 0; j < n_pos; ++j) acc += s[j] * (double)fp16r(v[j * ld + h * d_head + d]);
            out[h * d_head + d] = (float)(acc / den);
        }
    }
    free(s);
}

void orc_attention(const float *qkv, int64_t n_pos, int64_t n_head,
                   int64_t d_head, float scale, const uint8_t *key_valid,
                   float *out) {
    const int64_t H = n_head * d_head;
    /* fp16-rounded K and V, as cast by the reference before FA */
    float *k16 = (float *)malloc(sizeof(float) * (size_t)(n_pos * H));
    float *v16 = (float *)malloc(sizeof(float) * (size_t)(n_pos * H));
    for (int64_t p = 0; p < n_pos; ++p)
        for (int64_t i = 0; i < H; ++i) {
            k16[p * H + i] = fp16r(qkv[p * 3 * H + H + i]);
            v16[p * H + i] = fp16r(qkv[p * 3 * H + 2 * H + i]);
        }
    /* K per head as [d][key] (kt[(h * d_head + d) * n_pos + j]): each score
     * is still summed over d in order, 8 keys side by side */
    float *kt = (float *)malloc(sizeof(float) * (size_t)(n_pos * H));
    for (int64_t p = 0; p < n_pos; ++p)
        for (int64_t i = 0; i < H; ++i) kt[i * n_pos + p] = k16[p * H + i];
#pragma omp parallel for schedule(static) collapse(2)
    for (int64_t h = 0; h < n_head; ++h) {
        for (int64_t i = 0; i < n_pos; ++i) {
            double *s = (double *)malloc(sizeof(double) * (size_t)n_pos);
            /* Q enters flash attention as fp16, as ggml's FA converts it to the
             * K vec-dot type [ggml, not in tree] */
            float q[512];
            for (int64_t d = 0; d < d_head && d < 512; ++d) q[d] = fp16r(qkv[i * 3 * H + h * d_head + d]);
            for (int64_t j0 = 0; j0 < n_pos; j0 += 8) {
                const int64_t nj = n_pos - j0 < 8 ? n_pos - j0 : 8;
                double a8[8] = {0, 0, 0, 0, 0, 0, 0, 0};
                for (int64_t d = 0; d < d_head; ++d) {
                    const float *kr = kt + (h * d_head + d) * n_pos + j0;
                    const double qd = (double)q[d];
                    if (nj == 8) {
                        for (int jj = 0; jj < 8; ++jj) a8[jj] += qd * (double)kr[jj];
                    } else {
                        for (int jj = 0; jj < nj; ++jj) a8[jj] += qd * (double)kr[jj];
                    }
                }
                for (int jj = 0; jj < nj; ++jj) s[j0 + jj] = a8[jj] * (double)scale;
            }
            double mx = -INFINITY;
            for (int64_t j = 0; j < n_pos; ++j) {
                if (key_valid && !key_valid[j]) { s[j] = -INFINITY; continue; }
                if (s[j] > mx) mx = s[j];
            }
            double den = 0.0;
            for (int64_t j = 0; j < n_pos; ++j) {
                s[j] = (s[j] == -INFINITY) ? 0.0 : exp(s[j] - mx);
                den += s[j];
            }
            /* each output's sum in key order (the d loop inside: the same
             * sums, read along V's rows) */
            double acc[512];
            for (int64_t d = 0; d < d_head; ++d) acc[d] = 0.0;
            for (int64_t j = 0; j < n_pos; ++j) {
                if (s[j] == 0.0) continue;
                const float *vr = v16 + j * H + h * d_head;
                for (int64_t d = 0; d < d_head; ++d) acc[d] += s[j] * (double)vr[d];
            }
            for (int64_t d = 0; d < d_head; ++d) out[i * H + h * d_head + d] = (float)(acc[d] / den);
            free(s);
        }
    }
    free(k16);
    free(v16);
    free(kt);
}

/* ------------------------------------------------------------------------ */
/* position embedding resize                                                 */
/* ------------------------------------------------------------------------ */

/* Per-axis anti-aliased linear filter: for output i, taps start at xmin[i],
 * count xsize[i], weights wt[i*max + j] (normalised). */
static void aa_weights(int64_t in_size, int64_t out_size, int64_t *xmin,
                       int64_t *xsize, float *wt, int64_t max_taps) {
    const float scale = (float)in_size / (float)out_size;
    const float support = scale >= 1.0f ? scale : 1.0f;
    const float invscale = scale >= 1.0f ? 1.0f / scale : 1.0f;
    for (int64_t i = 0; i < out_size; ++i) {
        const float center = scale * ((float)i + 0.5f);
        int64_t lo = (int64_t)(center - support + 0.5f);
        if (lo < 0) lo = 0;
        int64_t hi = (int64_t)(center + support + 0.5f);
        if (hi > in_size) hi = in_size;
        const int64_t n = hi - lo;
        float total = 0.0f;
        for (int64_t j = 0; j < max_taps; ++j) wt[i * max_taps + j] = 0.0f;
        for (int64_t j = 0; j < n; ++j) {
            float t = ((float)(j + lo) - center + 0.5f) * invscale;
            if (t < 0.0f) t = -t;
            const float w = t < 1.0f ? 1.0f - t : 0.0f;
            wt[i * max_taps + j] = w;
            total += w;
        }
        if (total != 0.0f)
            for (int64_t j = 0; j < n; ++j) wt[i * max_taps + j] /= total;
        xmin[i] = lo;
        xsize[i] = n;
    }
}

void orc_resize_pos_embed(const float *pos, int64_t n_side, int64_t H,
                          int64_t out_h, int64_t out_w, float *out) {
    const int64_t mt = 2 * (n_side > out_h ? n_side : out_h) + 4;
    int64_t *xmin = (int64_t *)malloc(sizeof(int64_t) * (size_t)(out_w + out_h));
    int64_t *xsz = (int64_t *)malloc(sizeof(int64_t) * (size_t)(out_w + out_h));
    float *wx = (float *)malloc(sizeof(float) * (size_t)(out_w * mt));
    float *wy = (float *)malloc(sizeof(float) * (size_t)(out_h * mt));
    aa_weights(n_side, out_w, xmin, xsz, wx, mt);
    aa_weights(n_side, out_h, xmin + out_w, xsz + out_w, wy, mt);
    /* width pass: (n_side rows, out_w cols) */
    float *tmp = (float *)malloc(sizeof(float) * (size_t)(n_side * out_w * H));
    for (int64_t y = 0; y < n_side; ++y)
        for (int64_t x = 0; x < out_w; ++x)
            for (int64_t c = 0; c < H; ++c) {
                float t = 0.0f;
                for (int64_t j = 0; j < xsz[x]; ++j)
                    t += pos[(y * n_side + xmin[x] + j) * H + c] * wx[x * mt + j];
                tmp[(y * out_w + x) * H + c] = t;
            }
    /* height pass */
    for (int64_t y = 0; y < out_h; ++y)
        for (int64_t x = 0; x < out_w; ++x)
            for (int64_t c = 0; c < H; ++c) {
                float t = 0.0f;
                for (int64_t j = 0; j < xsz[out_w + y]; ++j)
                    t += tmp[((xmin[out_w + y] + j) * out_w + x) * H + c] * wy[y * mt + j];
                out[(y * out_w + x) * H + c] = t;
            }
    free(tmp);
    free(wx);
    free(wy);
    free(xmin);
    free(xsz);
}

/* ------------------------------------------------------------------------ */
/* NaFlex front end (src/siglip2_preproc.cpp)                                */
/* ------------------------------------------------------------------------ */

/* a scaled side rounded up to whole patches, at least one (:20-24) */
static int nf_scaled(double scale, int size, int p) {
    const double v = (double)size * scale;
    const int r = (int)ceil(v / (double)p) * p;
    return r > p ? r : p;
}

/* largest scale whose grid fits max_patches, bisection to 1e-5 (:28-53) */
void orc_nf_target_size(int h, int w, int p, int max_patches, int *out_h, int *out_w) {
    const double eps = 1e-5;
    double lo = eps / 10.0, hi = 100.0;
    while (hi - lo >= eps) {
        const double mid = 0.5 * (lo + hi);
        const long long n = (long long)(nf_scaled(mid, h, p) / p) * (long long)(nf_scaled(mid, w, p) / p);
        if (n <= (long long)max_patches)
            lo = mid;
        else
            hi = mid;
    }
    *out_h = nf_scaled(lo, h, p);
    *out_w = nf_scaled(lo, w, p);
}

/* triangle filter of support max(src/dst, 1) around each output centre,
 * weights normalised to sum 1 (:76-107) */
int orc_nf_filter(int src, int dst, int fused, int *first, int *taps, float *weights, int cap) {
    const double scale = (double)src / (double)dst;
    const double r = scale > 1.0 ? scale : 1.0;
    const int mt = (int)ceil(2.0 * r) + 2;
    if (mt > cap) return -1;
    for (int i = 0; i < dst; ++i) {
        const double center = fused ? fma((double)i + 0.5, scale, -0.5) : ((double)i + 0.5) * scale - 0.5;
        const int k0 = (int)ceil(center - r), k1 = (int)floor(center + r);
        const int n = k1 - k0 + 1;
        double sum = 0.0;
        for (int t = 0; t < mt; ++t) weights[(int64_t)i * mt + t] = 0.0f;
        for (int t = 0; t < n; ++t) {
            const double d = ((double)(k0 + t) - center) / r;
            const double wv = 1.0 - fabs(d) > 0.0 ? 1.0 - fabs(d) : 0.0;
            weights[(int64_t)i * mt + t] = (float)wv;
            sum += wv;
        }
        const float inv = (float)(1.0 / sum);
        for (int t = 0; t < n; ++t) weights[(int64_t)i * mt + t] *= inv;
        first[i] = k0;
        taps[i] = n;
    }
    return mt;
}

int orc_nf_preprocess_rgb(const uint8_t *rgb, int h, int w, int max_patches, int p,
                          float rescale, const float mean[3], const float std_[3], int fused,
                          float *out, int64_t out_cap, int *n_h, int *n_w) {
    if (!rgb || h <= 0 || w <= 0 || p <= 0 || max_patches <= 0) return -1;
    int th, tw;
    orc_nf_target_size(h, w, p, max_patches, &th, &tw);
    const int nh = th / p, nw = tw / p, feat = 3 * p * p;
    if ((int64_t)nh * nw * feat > out_cap) return -1;
    const int cap_y = (int)ceil(2.0 * ((double)h / th > 1.0 ? (double)h / th : 1.0)) + 2;
    const int cap_x = (int)ceil(2.0 * ((double)w / tw > 1.0 ? (double)w / tw : 1.0)) + 2;
    int *fy0 = (int *)malloc(sizeof(int) * (size_t)th), *fyn = (int *)malloc(sizeof(int) * (size_t)th);
    int *fx0 = (int *)malloc(sizeof(int) * (size_t)tw), *fxn = (int *)malloc(sizeof(int) * (size_t)tw);
    float *wy = (float *)malloc(sizeof(float) * (size_t)th * cap_y);
    float *wx = (float *)malloc(sizeof(float) * (size_t)tw * cap_x);
    const int mty = orc_nf_filter(h, th, fused, fy0, fyn, wy, cap_y);
    const int mtx = orc_nf_filter(w, tw, fused, fx0, fxn, wx, cap_x);
    /* pass 1, along the height: (th, w, 3) floats (:120-139) */
    float *tmp = (float *)malloc(sizeof(float) * (size_t)th * w * 3);
    for (int y = 0; y < th; ++y)
        for (int x = 0; x < w; ++x)
            for (int c = 0; c < 3; ++c) {
                float a = 0.0f;
                for (int t = 0; t < fyn[y]; ++t) {
                    int sy = fy0[y] + t;
                    sy = sy < 0 ? 0 : sy >= h ? h - 1 : sy;
                    const float wt = wy[(int64_t)y * mty + t], v = (float)rgb[((int64_t)sy * w + x) * 3 + c];
                    a = fused ? fmaf(wt, v, a) : a + wt * v;
                }
                tmp[((int64_t)y * w + x) * 3 + c] = a;
            }
    /* pass 2, along the width, rounded to u8 (:141-166); then rescale,
     * normalise and the patch layout (:176-207) */
    for (int y = 0; y < th; ++y)
        for (int x = 0; x < tw; ++x)
            for (int c = 0; c < 3; ++c) {
                float a = 0.0f;
                for (int t = 0; t < fxn[x]; ++t) {
                    int sx = fx0[x] + t;
                    sx = sx < 0 ? 0 : sx >= w ? w - 1 : sx;
                    const float wt = wx[(int64_t)x * mtx + t], v = tmp[((int64_t)y * w + sx) * 3 + c];
                    a = fused ? fmaf(wt, v, a) : a + wt * v;
                }
                int iv = (int)lrintf(a);
                iv = iv < 0 ? 0 : iv > 255 ? 255 : iv;
                const float u = (float)iv;
                const float sv = fused ? fmaf(u, rescale, -mean[c]) : u * rescale - mean[c];
                const int ph = y / p, py = y % p, pw = x / p, px = x % p;
                out[((int64_t)ph * nw + pw) * feat + ((int64_t)py * p + px) * 3 + c] = sv / std_[c];
            }
    free(tmp);
    free(fy0); free(fyn); free(fx0); free(fxn); free(wy); free(wx);
    *n_h = nh;
    *n_w = nw;
    return 0;
}

/* ------------------------------------------------------------------------ */
/* model                                                                     */
/* ------------------------------------------------------------------------ */

/* y = mm(W, x) + bias  (ggml_add(ggml_mul_mat(W, x), b)) */
static void linear(const void *w, const float *bias, int64_t K, int64_t K_pad,
                   int64_t N, const float *x, int64_t ldx, int64_t M, float *y,
                   int nthreads) {
    orc_mul_mat_q8_0_f32(w, K_pad, N, x, K, ldx, M, y, nthreads);
    if (bias)
#pragma omp parallel for schedule(static)
        for (int64_t m = 0; m < M; ++m)
            for (int64_t n = 0; n < N; ++n) y[m * N + n] = y[m * N + n] + bias[n];
}

/* the down projection: Q8_0 with K padded to F_pad, or F16 rows of F */
static void linear_down(const void *w, const float *bias, int64_t F, int64_t F_pad, int64_t N,
                        const float *x, int64_t M, float *y, int down_f16, int nthreads) {
    if (!down_f16) {
        linear(w, bias, F, F_pad, N, x, F, M, y, nthreads);
        return;
    }
    orc_mul_mat_f16_f32((const uint16_t *)w, F, N, x, F, M, y, nthreads);
#pragma omp parallel for schedule(static)
    for (int64_t m = 0; m < M; ++m)
        for (int64_t n = 0; n < N; ++n) y[m * N + n] = y[m * N + n] + bias[n];
}

void orc_encoder_block(const orc_layer *L, int32_t H, int32_t F, int32_t F_pad,
                       int32_t n_head, float eps, float *x, int64_t n_pos,
                       const uint8_t *key_valid, int down_f16, int nthreads) {
    const int64_t d_head = H / n_head;
    const float kq_scale = 1.0f / sqrtf((float)d_head);
    float *h = (float *)malloc(sizeof(float) * (size_t)(n_pos * H));
    float *qkv = (float *)malloc(sizeof(float) * (size_t)(n_pos * 3 * H));
    float *att = (float *)malloc(sizeof(float) * (size_t)(n_pos * H));
    float *o = (float *)malloc(sizeof(float) * (size_t)(n_pos * H));
    float *u = (float *)malloc(sizeof(float) * (size_t)(n_pos * F));

    orc_layernorm(x, n_pos, H, H, L->ln1_w, L->ln1_b, eps, h, H);
    linear(L->qkv_w, L->qkv_b, H, H, 3 * H, h, H, n_pos, qkv, nthreads);
    orc_attention(qkv, n_pos, n_head, d_head, kq_scale, key_valid, att);
    linear(L->o_w, L->o_b, H, H, H, att, H, n_pos, o, nthreads);
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n_pos * H; ++i) x[i] = o[i] + x[i];

    orc_layernorm(x, n_pos, H, H, L->ln2_w, L->ln2_b, eps, h, H);
    linear(L->up_w, L->up_b, H, H, F, h, H, n_pos, u, nthreads);
    gelu_n(u, n_pos * F);
    linear_down(L->down_w, L->down_b, F, F_pad, H, u, n_pos, o, down_f16, nthreads);
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n_pos * H; ++i) x[i] = o[i] + x[i];

    free(h);
    free(qkv);
    free(att);
    free(o);
    free(u);
}

void orc_vision_encode(const orc_vision_model *m, const float *pixels,
                       int32_t n_h, int32_t n_w, int32_t pooling, float *out,
                       float *hidden_out, int nthreads) {
    const int64_t H = m->hidden, F = m->inter, F_pad = m->inter_pad;
    const int64_t n_pos = (int64_t)n_h * n_w;
    const int64_t d_head = H / m->n_head;
    const float kq_scale = 1.0f / sqrtf((float)d_head);
    float *x = (float *)malloc(sizeof(float) * (size_t)(n_pos * H));
    float *pos = (float *)malloc(sizeof(float) * (size_t)(n_pos * H));

    /* patch embedding + position embedding (src/siglip2_vision.cpp:676-691) */
    linear(m->patch_w, m->patch_b, m->patch_dim, m->patch_dim, H, pixels,
           m->patch_dim, n_pos, x, nthreads);
    if (n_h == m->n_side && n_w == m->n_side)
        memcpy(pos, m->pos_embd, sizeof(float) * (size_t)(n_pos * H));
    else
        orc_resize_pos_embed(m->pos_embd, m->n_side, H, n_h, n_w, pos);
    for (int64_t i = 0; i < n_pos * H; ++i) x[i] = x[i] + pos[i];

    for (int32_t l = 0; l < m->n_layer; ++l)
        orc_encoder_block(&m->layers[l], (int32_t)H, (int32_t)F, (int32_t)F_pad,
                          m->n_head, m->eps, x, n_pos, NULL, m->down_f16, nthreads);

    orc_layernorm(x, n_pos, H, H, m->post_ln_w, m->post_ln_b, m->eps, x, H);
    if (hidden_out) memcpy(hidden_out, x, sizeof(float) * (size_t)(n_pos * H));

    if (pooling == 0) {
        /* mean over patches (src/siglip2_vision.cpp:699-701) */
        for (int64_t c = 0; c < H; ++c) {
            double s = 0.0;
            for (int64_t p = 0; p < n_pos; ++p) s += (double)x[p * H + c];
            out[c] = (float)s / (float)n_pos;
        }
    } else {
        /* MAP probe head (src/siglip2_vision.cpp:249-314) */
        float *q = (float *)malloc(sizeof(float) * (size_t)H);
        float *a = (float *)malloc(sizeof(float) * (size_t)H);
        float *a2 = (float *)malloc(sizeof(float) * (size_t)H);
        float *t = (float *)malloc(sizeof(float) * (size_t)H);
        float *u = (float *)malloc(sizeof(float) * (size_t)F);
        float *k = (float *)malloc(sizeof(float) * (size_t)(n_pos * H));
        float *v = (float *)malloc(sizeof(float) * (size_t)(n_pos * H));
        linear(m->hq_w, m->hq_b, H, H, H, m->probe, H, 1, q, nthreads);
        linear(m->hk_w, m->hk_b, H, H, H, x, H, n_pos, k, nthreads);
        linear(m->hv_w, m->hv_b, H, H, H, x, H, n_pos, v, nthreads);
        /* single-query attention over the n_pos keys */
        orc_attention_1q(q, k, v, H, n_pos, m->n_head, d_head, kq_scale, t);
        linear(m->ho_w, m->ho_b, H, H, H, t, H, 1, a, nthreads);
        orc_layernorm(a, 1, H, H, m->hln_w, m->hln_b, m->eps, a2, H);
        linear(m->hup_w, m->hup_b, H, H, F, a2, H, 1, u, nthreads);
        gelu_n(u, F);
        linear_down(m->hdown_w, m->hdown_b, F, F_pad, H, u, 1, a2, m->down_f16, nthreads);
        for (int64_t i = 0; i < H; ++i) out[i] = a[i] + a2[i];
        free(q);
        free(a);
        free(a2);
        free(t);
        free(u);
        free(k);
        free(v);
    }
    free(x);
    free(pos);
}

void orc_text_encode(const orc_text_model *m, const int32_t *tokens,
                     int32_t n_tok, const int32_t *mask, float *out,
                     int nthreads) {
    if (n_tok <= 0) return;
    const int64_t H = m->hidden;
    const int64_t n_pos = n_tok;
    float *x = (float *)malloc(sizeof(float) * (size_t)(n_pos * H));
    uint8_t *kv = NULL;
    /* token rows (Q8_0 get_rows = dequantize) + position rows
     * (src/siglip2_text.cpp:649-658) */
    for (int64_t p = 0; p < n_pos; ++p) {
        const uint8_t *row = (const uint8_t *)m->tok_embd +
                             (int64_t)tokens[p] * (H / ORC_QK) * ORC_BLOCK_BYTES;
        orc_dequantize_q8_0(row, 1, H, x + p * H);
        for (int64_t c = 0; c < H; ++c) x[p * H + c] = x[p * H + c] + m->pos_embd[p * H + c];
    }
    if (mask) {
        kv = (uint8_t *)malloc((size_t)n_pos);
        for (int64_t p = 0; p < n_pos; ++p) kv[p] = mask[p] != 0;
    }
    for (int32_t l = 0; l < m->n_layer; ++l)
        orc_encoder_block(&m->layers[l], (int32_t)H, m->inter, m->inter_pad,
                          m->n_head, m->eps, x, n_pos, kv, m->down_f16, nthreads);
    orc_layernorm(x, n_pos, H, H, m->final_ln_w, m->final_ln_b, m->eps, x, H);
    /* last-token pooling + head (src/siglip2_text.cpp:667-675) */
    linear(m->head_w, m->head_b, H, H, m->proj, x + (n_pos - 1) * H, H, 1, out,
           nthreads);
    free(x);
    free(kv);
}
