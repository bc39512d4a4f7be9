/* cpu_q8.c -- TEST / BASELINE INFRASTRUCTURE ONLY (the CPU baseline of the
 * benchmark; never part of the product).  A fast CPU restatement of ggml's
 * Q8_0 x Q8_1 matrix product with the same per-block arithmetic as
 * orc_mul_mat_q8_0_q8_1 (src/cuda/siglip2_custom_mmq.cu:259-267's per-block
 * rescale, in block order), bit for bit:
 *
 *   y[m][n] = sum over blocks b, in order: acc = fmaf((float)I_b, dw[n][b] * dx[m][b], acc)
 *
 * AVX-512 VNNI (runtime-dispatched; otherwise the oracle's own loop): the
 * weights are repacked once into groups of 16 columns, block b of a group
 * as 8 vectors of 16 lanes x 4 int8 (lane c: column 16 g + c, K values
 * 4 t .. 4 t + 3), so one vpdpbusd adds 4 products to each of 16 columns'
 * block dots.  vpdpbusd multiplies unsigned by signed bytes: the
 * activation quants enter as q + 128 (q ^ 0x80) and 128 * sum_j qw[j] is
 * subtracted, exactly, in int32.  The block's f32 rescale is then one
 * vfmadd per 16 outputs: the scalar loop's fmaf lane by lane. */
#include "cpu_q8.h"
#include "oracle.h"

#include <immintrin.h>
#include <omp.h>
#include <stdlib.h>
#include <string.h>

#define QK 32
#define GC 16 /* columns per group */

struct cq8_weight {
    int64_t K_pad, N, nb, ng;
    int8_t *w;      /* [ng][nb][8][GC][4] */
    int32_t *wsum;  /* [ng][nb][GC]: 128 * sum of the block's quants */
    float *wd;      /* [ng][nb][GC]: the block scales (0 in padding columns) */
};

int cq8_have_vnni(void) {
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") &&
           __builtin_cpu_supports("avx512vnni");
}

cq8_weight *cq8_prepare(const void *w_raw, int64_t K_pad, int64_t N) {
    cq8_weight *p = (cq8_weight *)calloc(1, sizeof(cq8_weight));
    p->K_pad = K_pad;
    p->N = N;
    p->nb = K_pad / QK;
    p->ng = (N + GC - 1) / GC;
    const int64_t ng = p->ng, nb = p->nb;
    p->w = (int8_t *)aligned_alloc(64, (size_t)(ng * nb * 8 * GC * 4));
    p->wsum = (int32_t *)aligned_alloc(64, sizeof(int32_t) * (size_t)(ng * nb * GC));
    p->wd = (float *)aligned_alloc(64, sizeof(float) * (size_t)(ng * nb * GC));
    const uint8_t *raw = (const uint8_t *)w_raw;
    for (int64_t g = 0; g < ng; ++g)
        for (int64_t b = 0; b < nb; ++b)
            for (int c = 0; c < GC; ++c) {
                const int64_t n = g * GC + c;
                int8_t q[QK];
                float d = 0.0f;
                if (n < N) {
                    const uint8_t *blk = raw + (n * nb + b) * 34;
                    uint16_t dh;
                    memcpy(&dh, blk, 2);
                    d = orc_fp16_to_fp32(dh);
                    memcpy(q, blk + 2, QK);
                } else {
                    memset(q, 0, QK);
                }
                int32_t s = 0;
                for (int j = 0; j < QK; ++j) s += q[j];
                for (int t = 0; t < 8; ++t)
                    memcpy(p->w + ((((g * nb + b) * 8 + t) * GC + c) * 4), q + 4 * t, 4);
                p->wsum[(g * nb + b) * GC + c] = 128 * s;
                p->wd[(g * nb + b) * GC + c] = d;
            }
    return p;
}

void cq8_free(cq8_weight *p) {
    if (!p) return;
    free(p->w);
    free(p->wsum);
    free(p->wd);
    free(p);
}

/* 4 rows x 16 columns of one group over all blocks */
__attribute__((target("avx512f,avx512bw,avx512vnni"))) static void tile_4x16(
    const cq8_weight *p, int64_t g, const uint8_t *xu, const float *xd, int64_t rows, float *y,
    int64_t ldy) {
    const int64_t nb = p->nb;
    __m512 acc[4];
    for (int r = 0; r < 4; ++r) acc[r] = _mm512_setzero_ps();
    for (int64_t b = 0; b < nb; ++b) {
        const int8_t *wv = p->w + (g * nb + b) * 8 * GC * 4;
        __m512i I[4];
        for (int r = 0; r < 4; ++r) I[r] = _mm512_setzero_si512();
        for (int t = 0; t < 8; ++t) {
            const __m512i w = _mm512_load_si512((const void *)(wv + t * GC * 4));
            for (int r = 0; r < 4; ++r) {
                int32_t x4;
                memcpy(&x4, xu + (r * nb + b) * QK + 4 * t, 4);
                I[r] = _mm512_dpbusd_epi32(I[r], _mm512_set1_epi32(x4), w);
            }
        }
        const __m512i ws = _mm512_load_si512((const void *)(p->wsum + (g * nb + b) * GC));
        const __m512 wd = _mm512_load_ps(p->wd + (g * nb + b) * GC);
        for (int r = 0; r < 4; ++r) {
            const __m512 If = _mm512_cvtepi32_ps(_mm512_sub_epi32(I[r], ws));
            const __m512 s = _mm512_mul_ps(wd, _mm512_set1_ps(xd[r * nb + b]));
            acc[r] = _mm512_fmadd_ps(If, s, acc[r]);
        }
    }
    const int64_t n0 = g * GC;
    const __mmask16 keep = (__mmask16)(p->N - n0 >= GC ? 0xFFFF : ((1u << (p->N - n0)) - 1));
    for (int64_t r = 0; r < rows; ++r) _mm512_mask_storeu_ps(y + r * ldy + n0, keep, acc[r]);
}

void cq8_mul_mat(const cq8_weight *p, const int8_t *qs, const uint16_t *ds, int64_t M, float *y,
                 int nthreads) {
    const int64_t nb = p->nb, K_pad = p->K_pad, N = p->N;
    /* activation quants biased to unsigned (q + 128) and scales widened */
    uint8_t *xu = (uint8_t *)malloc((size_t)((M + 3) * K_pad));
    float *xd = (float *)malloc(sizeof(float) * (size_t)((M + 3) * nb));
    for (int64_t i = 0; i < M * K_pad; ++i) xu[i] = (uint8_t)qs[i] ^ 0x80u;
    memset(xu + M * K_pad, 0x80, (size_t)(3 * K_pad));
    for (int64_t i = 0; i < M * nb; ++i) xd[i] = orc_fp16_to_fp32(ds[2 * i]);
    for (int64_t i = M * nb; i < (M + 3) * nb; ++i) xd[i] = 0.0f;
    const int64_t mt = (M + 3) / 4;
#pragma omp parallel for schedule(dynamic, 1) collapse(2) num_threads(nthreads > 0 ? nthreads : omp_get_max_threads())
    for (int64_t i = 0; i < mt; ++i)
        for (int64_t g = 0; g < p->ng; ++g) {
            const int64_t m = i * 4;
            tile_4x16(p, g, xu + m * K_pad, xd + m * nb, M - m < 4 ? M - m : 4, y + m * N, N);
        }
    free(xu);
    free(xd);
}
