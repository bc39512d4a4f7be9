/* cpu_q8.h -- TEST / BASELINE INFRASTRUCTURE ONLY: the CPU baseline's Q8_0 x
 * Q8_1 matrix product (AVX-512 VNNI), bit-identical to the oracle's
 * orc_mul_mat_q8_0_q8_1.  See cpu_q8.c. */
#pragma once
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct cq8_weight cq8_weight;

/* 1 if this CPU runs the AVX-512 VNNI kernel */
int cq8_have_vnni(void);
/* repack raw Q8_0 blocks (K_pad, N) once */
cq8_weight *cq8_prepare(const void *w_raw, int64_t K_pad, int64_t N);
void cq8_free(cq8_weight *w);
/* y[m*N + n] for M rows of Q8_1 activations (qs [M][K_pad], ds [M][K_pad/32]
 * as (d, s) fp16 pairs); needs cq8_have_vnni() */
void cq8_mul_mat(const cq8_weight *w, const int8_t *qs, const uint16_t *ds, int64_t M,
                 float *y, int nthreads);

#ifdef __cplusplus
}
#endif
