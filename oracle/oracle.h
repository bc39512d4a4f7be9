/*
 * oracle.h -- CPU restatement of the SigLIP2 Q8_0 matmul hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (the HIP library, the
 * C++ encoders, the Python bindings) may include, link or call this code.
 * Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg use it,
 * and only as the parity reference / the timed CPU baseline.
 *
 * The reference runs this path through ggml (dbrain/ggml fork, a git
 * submodule that is empty in the reference tree, commit unrecorded).  ggml's
 * sources are not available, so every function here restates the semantics
 * from the reference's own call sites and kernels, cited per function:
 *
 *   src/cuda/siglip2_custom_mmq.cu      activation quantizer + GEMM math
 *   src/cuda/siglip2_megakernel.cu      LN / GELU / residual / QKV layout
 *   src/siglip2_vision.cpp              vision graph, MAP head, pooling
 *   src/siglip2_text.cpp                text graph
 *   src/siglip2_preproc.cpp             anti-aliased bilinear filter
 *   tools/siglip2-quantize/main.cpp     Q8_0 K padding
 *
 * Where ggml's own CPU semantics are restated from its public (MIT) source
 * rather than from a file in the reference tree, the comment says
 * "[ggml, not in tree]".
 *
 * Layout conventions (ggml ne order, innermost first, i.e. row-major rows):
 *   weights W (K, N)  : N rows of K_pad/32 block_q8_0 (34 B: fp16 d, int8 qs[32])
 *   activations X (K, M): M rows of K floats, row m at x + m*ldx
 *   GEMM output Y (N, M): y[m*N + n]
 */
#ifndef S2X_ORACLE_H
#define S2X_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORC_QK 32

/* ---- fp16 ------------------------------------------------------------- */
uint16_t orc_fp32_to_fp16(float f);       /* IEEE binary16, round-nearest-even */
float    orc_fp16_to_fp32(uint16_t h);
void     orc_fp32_to_fp16_n(const float *x, uint16_t *y, int64_t n);
void     orc_fp16_to_fp32_n(const uint16_t *x, float *y, int64_t n);

/* ---- quantizers --------------------------------------------------------- */
/* Q8_0 weights, ggml quantize_row_q8_0_ref semantics [ggml, not in tree]:
 * d = amax/127, id = d ? 1/d : 0, q = roundf(x*id), store fp16(d).
 * x: n_rows rows of k floats (k % 32 == 0); out: n_rows*k/32 34-byte blocks. */
void orc_quantize_q8_0(const float *x, int64_t n_rows, int64_t k, void *out);

/* Same, but zero-pads each row from k to k_pad (k_pad % 32 == 0) first
 * (tools/siglip2-quantize/main.cpp:174-186). */
void orc_quantize_q8_0_padded(const float *x, int64_t n_rows, int64_t k,
                              int64_t k_pad, void *out);

/* Dequantize Q8_0 rows (ggml dequantize_row_q8_0: y = q * fp16->f32(d)). */
void orc_dequantize_q8_0(const void *blocks, int64_t n_rows, int64_t k_pad,
                         float *y);

/* Q8_1 activations (src/cuda/siglip2_custom_mmq.cu:63-76, plus the Q8_1 sum):
 * per 32-block: amax = max|x|; d = amax/127; inv = amax ? 127/amax : 0;
 * q = rint_half_even(x*inv) clamped to [-128,127];
 * ds[2*b+0] = fp16(d); ds[2*b+1] = fp16((float)sum(q) * d).
 * Columns k in [K, K_pad) are treated as zeros.
 * qs: M rows of K_pad int8; ds: M rows of K_pad/32 (d, s) fp16 pairs. */
void orc_quantize_q8_1(const float *x, int64_t M, int64_t K, int64_t ldx,
                       int64_t K_pad, int8_t *qs, uint16_t *ds);

/* ---- GEMM ---------------------------------------------------------------- */
/* Exact per-block integer dot: I = sum_{k<32} qa[k]*qb[k]. */
int32_t orc_block_dot(const int8_t *qa, const int8_t *qb);

/* Per-block dots of one (m, n) pair: out[kb] for kb < K_pad/32. */
void orc_block_dots(const void *w, int64_t K_pad, int64_t n,
                    const int8_t *qs, int64_t m, int32_t *out);

/* Y = W(Q8_0) x X(Q8_1):  y[m*N+n] = sum over kb, in order, of
 *   acc = fmaf((float)I_kb, fp16(dw)*fp16(dx), acc)     (acc starts at 0)
 * which is ggml-cpu's generic vec_dot_q8_0_q8_0 accumulation with
 * contraction [ggml, not in tree].  nthreads <= 0 uses all cores. */
void orc_mul_mat_q8_0_q8_1(const void *w, int64_t K_pad, int64_t N,
                           const int8_t *qs, const uint16_t *ds, int64_t M,
                           float *y, int nthreads);

/* GGML_OP_MUL_MAT(Q8_0 W, F32 X): quantize X to Q8_1 (zero-padding K to
 * K_pad, src/siglip2_vision.cpp:99-107) and multiply. */
void orc_mul_mat_q8_0_f32(const void *w, int64_t K_pad, int64_t N,
                          const float *x, int64_t K, int64_t ldx, int64_t M,
                          float *y, int nthreads);

/* ---- pointwise / normalisation -------------------------------------------- */
/* ggml_norm + ggml_mul(w) + ggml_add(b) [ggml, not in tree]:
 * double-precision sum for the mean, two-pass double sum of (x-mean)^2 for
 * the variance, scale = 1/sqrtf(var+eps), y = (((x-mean)*scale)*w)+b with a
 * float rounding after every operation (src/siglip2_vision.cpp:79-88).
 * w or b may be NULL. */
void orc_layernorm(const float *x, int64_t M, int64_t H, int64_t ldx,
                   const float *w, const float *b, float eps, float *y,
                   int64_t ldy);

/* tanh in f32 from IEEE primitives only (mul, add, fma, divide, rint,
 * ldexp): |u| < 0.5 Maclaurin series through u^15 (exact series
 * coefficients), |u| < 9 (e - 1)/(e + 1) with e = e^(2|u|) by Cody-Waite
 * reduction and a degree-7 Taylor polynomial, else +-1.  Any IEEE machine
 * running these operations in this order gets the same bits. */
float orc_tanh_f32(float u);

/* GELU tanh form of src/cuda/siglip2_megakernel.cu:276-280 with the same
 * inner argument g = sqrt(2/pi) * x * (1 + 0.044715 x^2), evaluated through
 * the identity 0.5 * x * (1 + tanh(g)) = x / (1 + e^(-2g)): one exp (the
 * Cody-Waite exp of orc_tanh_f32, argument clamped to +-100) and one IEEE
 * division, no branch.  ggml's CPU path instead looks GELU up in an fp16
 * table [ggml, not in tree]; this restatement keeps the f32 formula the
 * reference's CUDA epilogue uses. */
float orc_gelu(float x);

/* The reference CUDA epilogue's own formula, 0.5 x (1 + tanhf(g))
 * (src/cuda/siglip2_megakernel.cu:276-280), with the host libm's tanhf in
 * place of CUDA's: the "exact fp32" mode, for measuring how far orc_gelu
 * is from the formula as written. */
float orc_gelu_tanhf(float x);

/* ggml-cpu's default GELU (GGML_GELU_FP16) [ggml fork dbrain/ggml, commit
 * not recorded; not in tree], restated from its published source: x <= -10
 * gives 0, x >= 10 gives x, otherwise the fp16 table entry of fp16(x), the
 * table holding fp16(ggml_gelu_f32(h)) for every fp16 h, ggml_gelu_f32 the
 * tanhf form above.  The "ggml-faithful" mode. */
float orc_gelu_ggml(float x);

/* The GELU the tower restatements apply: 0 orc_gelu (default; the GPU's
 * formulation, bit for bit), 1 orc_gelu_tanhf, 2 orc_gelu_ggml.  Process-
 * wide; returns the previous mode. */
int orc_set_gelu_mode(int mode);

/* y[i] = the mode's GELU of x[i] (modes as orc_set_gelu_mode) */
void orc_gelu_array(int mode, const float *x, float *y, int64_t n);

/* The GEMM kernel of orc_mul_mat_q8_0_f32 (and so of the towers): 0 the
 * scalar loop of orc_mul_mat_q8_0_q8_1 (default), 1 the AVX-512 VNNI kernel
 * of cpu_q8.c where the CPU has it (the same bits; for the CPU baseline).
 * Returns the previous kernel.  orc_clear_gemm_cache frees the repacked
 * weights kernel 1 keeps per weight address. */
int orc_set_gemm_kernel(int k);
void orc_clear_gemm_cache(void);

/* ---- attention ------------------------------------------------------------ */
/* The MAP probe head's single-query attention (src/siglip2_vision.cpp:
 * 249-314): for each head h, softmax_j(f16(q_h) . f16(k_j,h) * scale) .
 * f16(v_j,h) over n_pos keys, in double (as orc_attention).  k, v: n_pos
 * rows of stride ld floats, head h at h*d_head; out: H floats. */
void orc_attention_1q(const float *q, const float *k, const float *v, int64_t ld,
                      int64_t n_pos, int64_t n_head, int64_t d_head, float scale,
                      float *out);

/* softmax(Q K^T * scale [+ mask]) V for one image/sequence, all heads.
 * qkv: n_pos rows of 3*H floats laid out [q | k | v], head h at h*d_head
 * (src/siglip2_vision.cpp:201-206).  K and V are rounded to fp16 first, as
 * the reference casts them before flash attention (src/siglip2_vision.cpp:
 * 164-167); Q is rounded to fp16 as ggml's flash attention converts it to
 * the K vec-dot type [ggml, not in tree].  Scores, softmax and PV then run
 * in double (ggml's CPU kernel accumulates V*p in fp16; this restatement
 * keeps that sum exact instead).
 * key_valid: NULL (all valid) or n_pos flags; invalid keys get weight 0.
 * out: n_pos rows of H floats, head-major within the row. */
void orc_attention(const float *qkv, int64_t n_pos, int64_t n_head,
                   int64_t d_head, float scale, const uint8_t *key_valid,
                   float *out);

/* ---- position embedding resize -------------------------------------------- */
/* Anti-aliased bilinear resize of an (n_side x n_side x H) grid to
 * (out_h x out_w x H), PyTorch F.interpolate(mode="bilinear",
 * align_corners=False, antialias=True) semantics as HF Siglip2 uses it
 * (triangle filter, support max(scale,1), window clipped to the image and
 * renormalised).  Separable: width pass, then height pass.
 * Filter design restated from src/siglip2_preproc.cpp:53-107. */
void orc_resize_pos_embed(const float *pos, int64_t n_side, int64_t H,
                          int64_t out_h, int64_t out_w, float *out);

/* ---- NaFlex front end ----------------------------------------------------- */
/* src/siglip2_preproc.cpp: target grid by binary search over the scale
 * (:20-53), separable anti-aliased bilinear resize of RGB u8 with a float
 * intermediate and lrintf rounding (:68-167), rescale + normalise +
 * patchify to (n_h*n_w, p*p*3) channel-last patches (:169-207).
 * `fused` = 1 restates the reference as its release build compiles it
 * (GCC -O3 -march=native, default -ffp-contract=fast: every a*b+c of the
 * file is one fused multiply-add, in double for the filter centres and in
 * float for the filter passes and the rescale); 0 rounds each product. */
void orc_nf_target_size(int h, int w, int p, int max_patches, int *out_h, int *out_w);
/* Filter of one axis: first source index, tap count and max_taps weights per
 * output pixel; returns max_taps (<= cap) or -1. */
int orc_nf_filter(int src, int dst, int fused, int *first, int *taps, float *weights, int cap);
/* Returns 0 and fills out (n_h*n_w*3*p*p floats, <= out_cap) and n_h, n_w;
 * -1 on bad arguments or a too small out_cap. */
int orc_nf_preprocess_rgb(const uint8_t *rgb, int h, int w, int max_patches, int p,
                          float rescale, const float mean[3], const float std_[3], int fused,
                          float *out, int64_t out_cap, int *n_h, int *n_w);

/* ---- model ---------------------------------------------------------------- */
typedef struct {
    const float *ln1_w, *ln1_b;
    const void  *qkv_w;  const float *qkv_b;   /* K=H,     N=3H */
    const void  *o_w;    const float *o_b;     /* K=H,     N=H  */
    const float *ln2_w, *ln2_b;
    const void  *up_w;   const float *up_b;    /* K=H,     N=F  */
    const void  *down_w; const float *down_b;  /* K=F_pad, N=H  */
} orc_layer;

typedef struct {
    int32_t hidden, inter, inter_pad, n_head, n_layer;
    int32_t patch_dim, n_side;                 /* 768, 16 */
    float   eps;
    const void  *patch_w; const float *patch_b; /* K=patch_dim, N=H */
    const float *pos_embd;                      /* n_side*n_side rows of H */
    const float *post_ln_w, *post_ln_b;
    /* MAP probe head (src/siglip2_vision.cpp:249-314) */
    const float *probe;                         /* H */
    const void  *hq_w, *hk_w, *hv_w, *ho_w;     /* K=H, N=H */
    const float *hq_b, *hk_b, *hv_b, *ho_b;
    const float *hln_w, *hln_b;
    const void  *hup_w; const float *hup_b;     /* K=H, N=F */
    const void  *hdown_w; const float *hdown_b; /* K=F_pad, N=H */
    const orc_layer *layers;
    /* 1: down_w / hdown_w are F16 rows (N=H rows of K=F halves), the
     * converter's type for K % 32 != 0; 0: Q8_0 with K padded to F_pad */
    int32_t down_f16;
} orc_vision_model;

typedef struct {
    int32_t hidden, inter, inter_pad, n_head, n_layer, vocab, max_pos, proj;
    float   eps;
    const void  *tok_embd;                      /* vocab rows, Q8_0 K=H */
    const float *pos_embd;                      /* max_pos rows of H */
    const float *final_ln_w, *final_ln_b;
    const void  *head_w; const float *head_b;   /* K=H, N=proj */
    const orc_layer *layers;
    int32_t down_f16;                           /* as in orc_vision_model */
} orc_text_model;

/* One pre-LN encoder block in place on x (n_pos rows of H), following
 * build_block (src/siglip2_vision.cpp:181-244). */
void orc_encoder_block(const orc_layer *L, int32_t H, int32_t F, int32_t F_pad,
                       int32_t n_head, float eps, float *x, int64_t n_pos,
                       const uint8_t *key_valid, int down_f16, int nthreads);

/* GGML_OP_MUL_MAT with an F16 weight W (N rows of K halves) and an F32
 * activation X (M rows, stride ldx): X rounded to f16 (round to nearest
 * even, ggml's F32 -> F16 of the vec-dot operand), each product of two f16
 * values exact in double, summed in double in k order, rounded to f32 once
 * (any f32 accumulation order lies within K * 2^-24 of it). */
void orc_mul_mat_f16_f32(const uint16_t *w, int64_t K, int64_t N, const float *x,
                         int64_t ldx, int64_t M, float *y, int nthreads);

/* Vision tower for ONE image of n_h x n_w patches (src/siglip2_vision.cpp:
 * 601-758).  pooling: 0 = mean, 1 = probe.  out: H floats.
 * hidden_out (optional): post-LN hidden states, n_h*n_w rows of H. */
void orc_vision_encode(const orc_vision_model *m, const float *pixels,
                       int32_t n_h, int32_t n_w, int32_t pooling, float *out,
                       float *hidden_out, int nthreads);

/* Text tower for ONE prompt of n_tok tokens (src/siglip2_text.cpp:564-739).
 * mask: NULL or n_tok flags (1 = valid).  out: proj floats. */
void orc_text_encode(const orc_text_model *m, const int32_t *tokens,
                     int32_t n_tok, const int32_t *mask, float *out,
                     int nthreads);

#ifdef __cplusplus
}
#endif
#endif
