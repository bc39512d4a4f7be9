/*
 * s2x.h -- C-ABI of the MI355X (gfx950) SigLIP2 Q8_0 matmul hot path.
 *
 * Plain C: pointers, sizes and status codes; no C++ or torch types.
 * Device pointers are HIP device memory owned by the caller unless stated.
 * `stream` is a hipStream_t passed as void* (NULL = the null stream).
 * Every function returns an s2x_status; on failure a message is available
 * from s2x_last_error() on the calling thread.  Launch functions are
 * asynchronous on `stream`; they neither allocate nor synchronise unless
 * stated.  The library keeps no global mutable state besides the per-thread
 * error message and the scratch array of s2x_mul_mat_q8_0_f32_static, so
 * concurrent calls on different streams are safe, except calls of that one
 * entry point on the same GPU.
 *
 * Layouts use the reference's ggml order (innermost first): an activation
 * X (K, M) is M rows of K floats (row stride ldx floats), a GEMM output
 * Y (N, M) is y[m*N + n].
 */
#ifndef S2X_H
#define S2X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    S2X_OK = 0,
    S2X_ERR_INVALID_ARG = 1,   /* bad shape / null pointer / misalignment */
    S2X_ERR_UNSUPPORTED = 2,   /* shape or feature the library does not handle */
    S2X_ERR_HIP = 3,           /* a HIP runtime call failed */
    S2X_ERR_WORKSPACE = 4,     /* caller workspace too small */
    S2X_ERR_OOM = 5,           /* device allocation failed */
    S2X_ERR_NOT_LOADED = 6     /* encoder used before load */
} s2x_status;

const char *s2x_status_string(int status);
const char *s2x_last_error(void);
/* Library version string, e.g. "s2x 0.1 gfx950". */
const char *s2x_version(void);

/* ------------------------------------------------------------------------ */
/* a1  F32 -> Q8_1 activation quantizer                                      */
/* Replaces siglip2_custom_mmq::launch_quantize_activation                   */
/* (src/cuda/siglip2_custom_mmq.cuh:63-67) and ggml-cuda's quantize_mmq_q8_1. */
/* Per 32-value block: d = amax/127; q = rint_half_even(x*127/amax) clamped  */
/* to [-128,127]; ds = (fp16(d), fp16(sum(q)*d)).  Columns K..K_pad-1 are     */
/* zero (the K padding of src/siglip2_vision.cpp:99-107).                     */
/*   x  : M rows, stride ldx floats, K valid columns                          */
/*   qs : M rows of K_pad int8 (K_pad % 32 == 0, K <= K_pad)                  */
/*   ds : M rows of K_pad/32 (fp16 d, fp16 s) pairs                           */
/* ------------------------------------------------------------------------ */
int s2x_quantize_q8_1(const float *x, int64_t K, int64_t M, int64_t ldx,
                      int64_t K_pad, void *qs, void *ds, void *stream);

/* ------------------------------------------------------------------------ */
/* a2  Q8_0 weights, repacked once for the MFMA GEMM                          */
/* A raw Q8_0 matrix W (K_pad, N) is N rows of K_pad/32 34-byte block_q8_0    */
/* (fp16 d then int8 qs[32]; bench/microbench_mmq.cpp:322-343).  The repack  */
/* is lossless: an int8 plane (N rows of K_pad) and the fp16 scales          */
/* transposed (K_pad/32 rows of N).                                           */
/* ------------------------------------------------------------------------ */
typedef struct s2x_weight s2x_weight;

/* Bytes of device memory a prepared (K_pad, N) weight occupies. */
size_t s2x_weight_bytes(int64_t K_pad, int64_t N);
/* Repack raw Q8_0 blocks (host memory if `raw_is_host`, else device) into a
 * new device-resident weight.  Allocates; synchronises `stream`. */
int s2x_weight_create(const void *raw, int raw_is_host, int64_t K_pad,
                      int64_t N, void *stream, s2x_weight **out);
/* Same, into caller memory `dev_buf` of s2x_weight_bytes() bytes (no
 * allocation; asynchronous on `stream`; raw must be device memory). */
int s2x_weight_create_in(const void *raw_dev, int64_t K_pad, int64_t N,
                         void *dev_buf, void *stream, s2x_weight **out);
void s2x_weight_destroy(s2x_weight *w);
int64_t s2x_weight_k(const s2x_weight *w);
int64_t s2x_weight_n(const s2x_weight *w);

/* ------------------------------------------------------------------------ */
/* a3  Q8_0 x Q8_1 GEMM on int8 MFMA                                          */
/* Y[m*ldy+n] = epilogue(acc), acc = sum over 32-blocks kb, in order, of       */
/*   acc = fmaf((float)I_kb, d_w * d_x, acc),  I_kb = sum q_w*q_x (exact)     */
/* Replaces ggml-cuda mul_mat_q<Q8_0> behind GGML_OP_MUL_MAT(Q8_0, F32) and   */
/* siglip2_custom_mmq::launch_custom_mmq (src/cuda/siglip2_custom_mmq.cuh:    */
/* 96-103); the epilogues replace the fused tails of                          */
/* src/cuda/siglip2_megakernel.cuh:117-132 (bias + GELU, bias + residual) and */
/* the GELU output's re-quantization for the next GEMM.                       */
/* The activation is Q8_1 as s2x_quantize_q8_1 writes it: qs (M rows of K_pad */
/* int8, 16-byte aligned) and ds (M rows of K_pad/32 (fp16 d, fp16 s)).       */
/* One kernel serves every entry point below and the encoders.                */
/* ------------------------------------------------------------------------ */
typedef enum {
    S2X_EPI_NONE = 0,        /* y = acc                                      */
    S2X_EPI_BIAS = 1,        /* y = acc + bias[n]                            */
    S2X_EPI_BIAS_GELU = 2,   /* y = gelu_tanh(acc + bias[n])                 */
    S2X_EPI_BIAS_RESID = 3,  /* y = (acc + bias[n]) + resid[r(m)*ld_resid+n] */
    S2X_EPI_GELU_Q81 = 4,    /* no y: gelu_tanh(acc + bias[n]) quantized to  */
                             /* Q8_1 over rows of q_kpad values (columns     */
                             /* N..q_kpad-1 zero): q_out (M rows of q_kpad   */
                             /* int8, 16-byte aligned) and q_ds (M rows of   */
                             /* q_kpad/32 words), = s2x_quantize_q8_1 of the */
                             /* BIAS_GELU output, bit for bit                */
    S2X_EPI_GELU_F16 = 5     /* no y: f16(gelu_tanh(acc + bias[n])) in M rows */
                             /* of q_kpad halves at q_out (columns N..q_kpad */
                             /* -1 zero; q_ds unused): the activation of an  */
                             /* F16 weight (s2x_mul_mat_f16_f32's X in f16)  */
} s2x_epilogue_kind;

typedef struct {
    int32_t      kind;        /* s2x_epilogue_kind */
    const float *bias;        /* N floats, required unless kind == NONE */
    const float *resid;       /* BIAS_RESID only; may alias y             */
    int64_t      ld_resid;    /* row stride of resid in floats            */
    int64_t      resid_rows;  /* 0: r(m) = m; > 0: r(m) = m % resid_rows  */
    void        *q_out;       /* GELU_Q81, GELU_F16                        */
    void        *q_ds;        /* GELU_Q81 only                            */
    int64_t      q_kpad;      /* GELU_*: N <= q_kpad < N + 32, % 32 == 0   */
} s2x_epilogue;

int s2x_mul_mat_q8_0_q8_1(const s2x_weight *w, const void *qs, const void *ds,
                          int64_t M, float *y, int64_t ldy,
                          const s2x_epilogue *epi, void *stream);

/* s2x_mul_mat_q8_0_q8_1 with the K blocks in n_split contiguous ranges of
 * whole 4-block stages, summed separately (each in block order from zero)
 * and then added in range order: y = ((p_0 + p_1) + ...) [+ bias]
 * [+ resid].  Epilogue NONE or BIAS_RESID (resid_rows 0); workspace: n_split
 * * M * N floats, 16-byte aligned.  No counterpart in the reference: the
 * form the text encoder runs for its long-K GEMMs, whose few rows give one
 * launch per K range too few workgroups; its bits depend on K and n_split,
 * not on M. */
int s2x_mul_mat_q8_0_q8_1_split_k(const s2x_weight *w, const void *qs, const void *ds,
                                  int64_t M, float *y, int64_t ldy,
                                  const s2x_epilogue *epi, int32_t n_split,
                                  void *workspace, size_t ws_bytes, void *stream);

/* Drop-in GGML_OP_MUL_MAT(W: Q8_0 raw device blocks (K_pad, N), X: F32
 * (K, M)) -> Y: F32 (N, M).  X is quantized to Q8_1 (K zero-padded to K_pad)
 * and W repacked inside `workspace`, whose size s2x_mul_mat_workspace_size()
 * gives.  No allocation. */
size_t s2x_mul_mat_workspace_size(int64_t K_pad, int64_t N, int64_t M);
int s2x_mul_mat_q8_0_f32(const void *w_raw, int64_t K_pad, int64_t N,
                         const float *x, int64_t K, int64_t ldx, int64_t M,
                         float *y, void *workspace, size_t ws_bytes,
                         void *stream);

/* Drop-in GGML_OP_MUL_MAT(W: F16 (K, N), X: F32 (K, M)) -> Y: F32 (N, M),
 * the reference's path for weights its converter stores as F16 (matrices
 * whose K is not a multiple of 32: ffn_down, scripts/convert_siglip2_to_
 * gguf.py:241-290, kept F16 by src/siglip2_vision.cpp:496-556).  X is
 * rounded to f16 (as ggml converts the F32 operand of an F16 dot) and the
 * products accumulate in f32 on f16 MFMA.  w_raw: N rows of K halves on the
 * device.  K is zero-padded to a multiple of 32 inside `workspace`
 * (s2x_mul_mat_f16_workspace_size() bytes, 256-byte aligned).  No
 * allocation. */
size_t s2x_mul_mat_f16_workspace_size(int64_t K, int64_t N, int64_t M);
int s2x_mul_mat_f16_f32(const void *w_raw, int64_t K, int64_t N, const float *x,
                        int64_t ldx, int64_t M, float *y, void *workspace,
                        size_t ws_bytes, void *stream);

/* Allocation-free variant of s2x_mul_mat_q8_0_f32: same arguments without
 * the workspace, same results bit for bit.  No counterpart in the reference;
 * it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Its
 * workspace is a static device array of S2X_STATIC_SCRATCH_BYTES that each
 * GPU the library runs on holds until the process ends.  A shape whose
 * s2x_mul_mat_workspace_size() exceeds it returns S2X_ERR_UNSUPPORTED before
 * any launch (64 MiB: the so400m fc2 shape, K_pad 4320 x N 1152, up to
 * M = 12,720 rows, the K = 1152 shapes up to M = 47,713).  Every call on a
 * GPU shares that GPU's array:
 * calls that overlap on one GPU (other streams, other threads) race. */
#define S2X_STATIC_SCRATCH_BYTES ((size_t)64 << 20)
int s2x_mul_mat_q8_0_f32_static(const void *w_raw, int64_t K_pad, int64_t N,
                                const float *x, int64_t K, int64_t ldx,
                                int64_t M, float *y, void *stream);

/* Debug view of the GEMM's integer stage: out[m*N+n] = I_kb (the exact
 * int32 block dot of block `kb`) from the same kernel's MFMA data path. */
int s2x_block_dots(const s2x_weight *w, const void *qs, int64_t M, int64_t kb,
                   int32_t *out, void *stream);

/* QKV projection fused with the attention staging: the Q8_0 x Q8_1 product
 * with W_qkv (N = 3*n_head*d_head, rows [q;k;v]) plus qkv_bias, rounded to
 * f16 and written straight into the staging workspace `ws` in the layout
 * s2x_attn_prep produces (ws of s2x_attn_workspace_size() bytes).  Equals
 * s2x_mul_mat_q8_0_q8_1 followed by s2x_attn_prep, bit for bit; replaces
 * that pair and the reference's launch_fused_qkv_prep
 * (src/cuda/siglip2_megakernel.cuh:75-100) after its MUL_MAT.  Rows of the
 * GEMM are the packed segment rows (M = sum of seg_len).  The padding slots
 * of ws are cleared first. */
int s2x_mul_mat_qkv_attn_prep(const s2x_weight *w, const void *qs, const void *ds,
                              int64_t M, const float *qkv_bias,
                              const int32_t *seg_start_dev, const int32_t *seg_len_dev,
                              int64_t n_seg, int64_t max_len, int64_t n_head,
                              int64_t d_head, void *ws, size_t ws_bytes, void *stream);

/* ------------------------------------------------------------------------ */
/* a4  LayerNorm(+affine), alone and fused with the Q8_1 quantizer           */
/* Replaces siglip2_megakernel::launch_fused_layernorm_affine                */
/* (src/cuda/siglip2_megakernel.cuh:50-58) and ggml_norm/mul/add.             */
/* y = ((x - mean) * (1/sqrtf(var + eps))) * w + b, every op rounded in f32, */
/* mean and var from a two-pass row reduction.  H % 32 == 0, H <= 2048.       */
/* ------------------------------------------------------------------------ */
int s2x_layernorm(const float *x, int64_t H, int64_t M, int64_t ldx,
                  const float *w, const float *b, float eps, float *y,
                  int64_t ldy, void *stream);
/* Fused: writes Q8_1 (qs: M rows of H int8, ds: M rows of H/32 pairs) and,
 * if y != NULL, the f32 LayerNorm output as well. */
int s2x_layernorm_quantize_q8_1(const float *x, int64_t H, int64_t M,
                                int64_t ldx, const float *w, const float *b,
                                float eps, void *qs, void *ds, float *y,
                                int64_t ldy, void *stream);

/* ------------------------------------------------------------------------ */
/* a5  standalone epilogues (src/cuda/siglip2_megakernel.cuh:117-132)        */
/* ------------------------------------------------------------------------ */
/* y = (mm + bias[h]) + resid, both adds rounded in f32 */
int s2x_bias_residual(const float *mm, const float *bias, const float *resid,
                      float *y, int64_t H, int64_t n_pos, void *stream);
/* y = gelu_tanh(mm + bias[h]) */
int s2x_bias_gelu(const float *mm, const float *bias, float *y, int64_t H,
                  int64_t n_pos, void *stream);

/* ------------------------------------------------------------------------ */
/* a6/a7  attention                                                          */
/* Replaces launch_qkv_copy_to_scratch + launch_fused_qkv_prep               */
/* (src/cuda/siglip2_megakernel.cuh:75-100), ggml_flash_attn_ext             */
/* (src/siglip2_vision.cpp:141-175) and launch_fused_post_fa_cont            */
/* (src/cuda/siglip2_megakernel.cuh:148-155).                                 */
/*                                                                            */
/* Sequences are segments of a packed token array: segment s covers rows     */
/* seg_start[s] .. seg_start[s]+seg_len[s]-1.  Attention never crosses a     */
/* segment.  key_valid (optional, one byte per packed row) drops keys.       */
/* ------------------------------------------------------------------------ */
/* Bytes of the f16 Q/K/V staging buffer for n_seg segments of at most
 * max_len tokens with n_head heads of d_head. */
size_t s2x_attn_workspace_size(int64_t n_seg, int64_t max_len, int64_t n_head,
                               int64_t d_head);
/* qkv: packed rows of 3*H floats [q | k | v] (no bias yet); adds qkv_bias
 * and stages Q, K (f16, d zero-padded) and V^T (f16) into `ws`. */
int s2x_attn_prep(const float *qkv, int64_t ld_qkv, const float *qkv_bias,
                  const int32_t *seg_start_dev, const int32_t *seg_len_dev,
                  int64_t n_seg, int64_t max_len, int64_t n_head,
                  int64_t d_head, void *ws, size_t ws_bytes, void *stream);
/* softmax(Q K^T * scale) V per segment and head; out: packed rows of
 * H = n_head*d_head floats, head-major within the row. */
int s2x_attn_run(const void *ws, size_t ws_bytes, const int32_t *seg_start_dev,
                 const int32_t *seg_len_dev, const uint8_t *key_valid,
                 int64_t n_seg, int64_t max_len, int64_t n_head,
                 int64_t d_head, float scale, float *out, int64_t ld_out,
                 void *stream);

/* s2x_attn_run followed by s2x_quantize_q8_1 of its output (K = H), in
 * one pass for 72-wide heads in groups of four (n_head % 4 == 0): the
 * post-attention contiguous copy and the activation quantizer of the
 * out-projection (siglip2_vision.cpp:148 launch_fused_post_fa_cont,
 * siglip2_custom_mmq.cuh:63 launch_quantize_activation).  qs [n_rows][H]
 * int8, ds [n_rows][ld_ds] words as s2x_quantize_q8_1 writes them, the same
 * bits.  `out` (f32 [n_rows][ld_out], 16-byte aligned) is scratch: at most
 * the columns of Q8_1 blocks that straddle two heads are written.  The segments
 * must cover rows 0 .. n_rows - 1. */
int s2x_attn_run_q8_1(const void *ws, size_t ws_bytes, const int32_t *seg_start_dev,
                      const int32_t *seg_len_dev, const uint8_t *key_valid,
                      int64_t n_seg, int64_t max_len, int64_t n_head,
                      int64_t d_head, float scale, int64_t n_rows, void *qs,
                      void *ds, int64_t ld_ds, float *out, int64_t ld_out,
                      void *stream);

/* fp64 attention straight from the QKV rows (bias added in f32, Q/K/V
 * rounded to f16 as the reference casts them, then scores, softmax and PV in
 * double in a fixed key order).  Needs no staging workspace; meant for short
 * sequences such as the 64-token text prompts.  d_head <= 80. */
int s2x_attn_fp64(const float *qkv, int64_t ld_qkv, const float *qkv_bias,
                  const int32_t *seg_start_dev, const int32_t *seg_len_dev,
                  const uint8_t *key_valid, int64_t n_seg, int64_t max_len,
                  int64_t n_head, int64_t d_head, float scale, float *out,
                  int64_t ld_out, void *stream);

/* a9: the MAP probe head's attention, one query over each segment's keys
 * (the pooling head's ggml_flash_attn_ext with a single query row,
 * src/siglip2_vision.cpp:249-314): out[s*H + h*d_head + d] =
 * sum_j softmax_j(f16(q_h) . f16(k_j,h) * scale) * f16(v_j,h)[d], over rows
 * seg_start[s] .. seg_start[s] + seg_len[s] - 1 of k and v (row stride ld
 * floats; H = n_head * d_head).  q: H floats shared by every segment.  The
 * scores and softmax in f32, the PV sums in key-group partials.
 * seg_len[s] <= max_len <= 4096, d_head <= 128. */
int s2x_attn_1q(const float *q, const float *k, const float *v, int64_t ld,
                const int32_t *seg_start_dev, const int32_t *seg_len_dev, int64_t n_seg,
                int64_t max_len, int64_t n_head, int64_t d_head, float scale, float *out,
                void *stream);

/* ------------------------------------------------------------------------ */
/* a8  position-embedding resize (replaces ggml_interpolate(BILINEAR |       */
/* ANTIALIAS) at src/siglip2_vision.cpp:680-690): anti-aliased bilinear,     */
/* PyTorch F.interpolate(antialias=True, align_corners=False) semantics.      */
/* pos: n_side*n_side rows of H; out: out_h*out_w rows of H (device).         */
/* ------------------------------------------------------------------------ */
int s2x_resize_pos_embed(const float *pos, int64_t n_side, int64_t H,
                         int64_t out_h, int64_t out_w, float *out,
                         void *stream);

/* ------------------------------------------------------------------------ */
/* NaFlex front end (replaces siglip2::preprocess_image_rgb,                   */
/* src/siglip2_preproc.h:44-55 / src/siglip2_preproc.cpp:209-244, on the GPU; */
/* same grid, anti-aliased resize, rounding and normalisation, bit for bit    */
/* with the reference's release build).                                       */
/* s2x_nf_target_size: the (target_h, target_w) the image is resized to, both */
/* multiples of patch (host function, no GPU).                                */
/* s2x_nf_preprocess_rgb_dev: rgb = h*w*3 u8 channel-last (device); out =     */
/* n_h*n_w rows of 3*patch*patch floats (device, out_cap floats available);   */
/* mean / std: 3 floats each (host); workspace: device memory of              */
/* s2x_nf_workspace_size() bytes.  n_h / n_w (host) receive the grid.         */
/* ------------------------------------------------------------------------ */
int s2x_nf_target_size(int32_t h, int32_t w, int32_t patch, int32_t max_num_patches,
                       int32_t *target_h, int32_t *target_w);
size_t s2x_nf_workspace_size(int32_t h, int32_t w, int32_t patch, int32_t max_num_patches);
int s2x_nf_preprocess_rgb_dev(const uint8_t *rgb, int32_t h, int32_t w,
                              int32_t max_num_patches, int32_t patch, float rescale,
                              const float *mean, const float *std_, float *out,
                              int64_t out_cap, int32_t *n_h, int32_t *n_w,
                              void *workspace, size_t ws_bytes, void *stream);
/* s2x_nf_preprocess_rgb_batch_dev: n_img same-size images in one call (one  */
/* launch per pass): rgb = n_img contiguous h*w*3 u8 images, out = n_img     */
/* contiguous blocks of n_h*n_w*3*patch*patch floats (out_cap: floats per    */
/* image available, >= one block), workspace >= n_img *                     */
/* s2x_nf_workspace_size() bytes; each image's output equals                 */
/* s2x_nf_preprocess_rgb_dev's.  No counterpart in the reference, which      */
/* preprocesses one image per call (src/siglip2_preproc.cpp:217-251).        */
int s2x_nf_preprocess_rgb_batch_dev(const uint8_t *rgb, int32_t n_img, int32_t h, int32_t w,
                                    int32_t max_num_patches, int32_t patch, float rescale,
                                    const float *mean, const float *std_, float *out,
                                    int64_t out_cap, int32_t *n_h, int32_t *n_w,
                                    void *workspace, size_t ws_bytes, void *stream);

/* ------------------------------------------------------------------------ */
/* a11  Q8_0 get_rows (replaces ggml_get_rows on the Q8_0 token table,        */
/* src/siglip2_text.cpp:649-658): out[i] = dequant(table row ids[i]) (+ add  */
/* row i % add_rows of `add` when add != NULL).                               */
/* ------------------------------------------------------------------------ */
int s2x_get_rows_q8_0(const void *table_raw, int64_t K, int64_t n_rows_table,
                      const int32_t *ids, int64_t n_ids, const float *add,
                      int64_t add_rows, float *out, void *stream);

/* ------------------------------------------------------------------------ */
/* a10  encoders (replace siglip2::VisionEncoder / TextEncoder,               */
/* src/siglip2_vision.h:37-68, src/siglip2_text.h:25-75).                     */
/* Weights come from host memory: raw Q8_0 blocks for every matrix, f32 for  */
/* biases, LayerNorms, position embeddings and the probe -- except, with     */
/* down_f16 = 1, the ffn_down matrices (layers and MAP head): F16 rows (H    */
/* rows of F halves), the type the reference's converter writes for a K not  */
/* a multiple of 32 and its encoder keeps (src/siglip2_vision.cpp:496-556).  */
/* ------------------------------------------------------------------------ */
typedef struct {
    const float *ln1_w, *ln1_b;
    const void  *qkv_w;  const float *qkv_b;   /* Q8_0 (H, 3H), rows [q;k;v] */
    const void  *o_w;    const float *o_b;     /* Q8_0 (H, H)                */
    const float *ln2_w, *ln2_b;
    const void  *up_w;   const float *up_b;    /* Q8_0 (H, F)                */
    const void  *down_w; const float *down_b;  /* Q8_0 (F_pad, H) or F16 (F, H) */
} s2x_layer_weights;

typedef struct {
    int32_t hidden, inter, inter_pad, n_head, n_layer;
    int32_t patch_dim, n_side;                  /* 768, 16 */
    float   eps;
    const void  *patch_w; const float *patch_b; /* Q8_0 (patch_dim, H)    */
    const float *pos_embd;                      /* n_side^2 rows of H     */
    const float *post_ln_w, *post_ln_b;
    const float *probe;                         /* H                      */
    const void  *hq_w, *hk_w, *hv_w, *ho_w;     /* Q8_0 (H, H)            */
    const float *hq_b, *hk_b, *hv_b, *ho_b;
    const float *hln_w, *hln_b;
    const void  *hup_w; const float *hup_b;     /* Q8_0 (H, F)            */
    const void  *hdown_w; const float *hdown_b; /* as the layers' down_w  */
    const s2x_layer_weights *layers;            /* n_layer entries        */
    int32_t down_f16;                           /* 0: Q8_0, 1: F16 ffn_down */
} s2x_vision_weights;

typedef struct {
    int32_t hidden, inter, inter_pad, n_head, n_layer, vocab, max_pos, proj;
    float   eps;
    const void  *tok_embd;                      /* Q8_0 (H, vocab)        */
    const float *pos_embd;                      /* max_pos rows of H      */
    const float *final_ln_w, *final_ln_b;
    const void  *head_w; const float *head_b;   /* Q8_0 (H, proj)         */
    const s2x_layer_weights *layers;
    int32_t down_f16;                           /* 0: Q8_0, 1: F16 ffn_down */
} s2x_text_weights;

/* ------------------------------------------------------------------------ */
/* GGUF weight files (replaces the reference's loader path into the          */
/* encoders, src/gguf_loader.cpp:205-337 and the tensor binding of           */
/* VisionEncoder::load / TextEncoder::load, src/siglip2_vision.cpp:424-560,  */
/* src/siglip2_text.cpp:424-540).  Host only: the file is mapped read-only, */
/* tensors are bound by the converter's names                                 */
/* (scripts/convert_siglip2_to_gguf.py:7-35) and the siglip2.vision.* /      */
/* siglip2.text.* metadata.  Q8_0 and F32 tensors are used in place, F16    */
/* vectors are widened, F16 / F32 matrices are quantized to Q8_0 on load     */
/* (K zero-padded to a multiple of 32).  The filled struct points into the   */
/* handle and stays valid until s2x_gguf_close.                               */
/* ------------------------------------------------------------------------ */
typedef struct s2x_gguf s2x_gguf;
int s2x_gguf_open(const char *path, s2x_gguf **out);
void s2x_gguf_close(s2x_gguf *g);
int s2x_gguf_vision_weights(s2x_gguf *g, s2x_vision_weights *out);
int s2x_gguf_text_weights(s2x_gguf *g, s2x_text_weights *out);
/* The contrastive head's scalars mm.logit_scale (exponentiated by the
 * scorer) and mm.logit_bias (read_score_params,
 * src/siglip2_score.cpp:17-74). */
int s2x_gguf_score_params(s2x_gguf *g, float *logit_scale, float *logit_bias);

typedef struct s2x_vision s2x_vision;
typedef struct s2x_text s2x_text;

enum { S2X_POOL_MEAN = 0, S2X_POOL_PROBE = 1 };

/* Upload + repack all weights to the current HIP device; the encoder owns
 * its own HIP stream (default priority). */
int s2x_vision_create(const s2x_vision_weights *w, s2x_vision **out);
void s2x_vision_destroy(s2x_vision *v);
/* Run on the encoder's stream (NULL) or a caller stream. */
int s2x_vision_set_stream(s2x_vision *v, void *stream);
/* Attention precision: 0 (default) = f16-MFMA flash attention with f32
 * softmax and an exact f16 hi/lo split of P; 1 = s2x_attn_fp64. */
int s2x_vision_set_attention_fp64(s2x_vision *v, int enable);
/* HIP graph replay of encodes of at most 8,192 packed rows (1 = default,
 * 0 = plain launches).  The reference turns on ggml's CUDA graphs with one
 * graph per shape in its encoders (CMakeLists.txt:59-64); here the second
 * encode with the same sizes and buffers is captured into a HIP graph and
 * later ones replay it (up to 4 shapes per encoder).  Results are the same
 * bits either way. */
int s2x_vision_set_graphs(s2x_vision *v, int enable);
/* EXPERIMENTAL, outside the parity tolerance: the embeddings it gives reach
 * cosine 0.9998 of the block-order CPU restatement, below the 0.9999 that
 * the default path meets.
 * 1 = the vision tower's plain and residual GEMMs of 32+ K blocks (out,
 * fc2, the head's) run as s2x_mul_mat_q8_0_q8_1_split_k (2 ranges, 4 from
 * 96 blocks), for latency at batch 1; 0 (default) = one block-order sum per
 * output, the oracle's.  No counterpart in the reference (whose GPU GEMMs
 * split K by stream-K); an image's bits do not depend on its batch either
 * way.  Batch 32 runs slower with it (partial sums of 4 x 107 MB per fc2). */
int s2x_vision_set_split_k(s2x_vision *v, int enable);
/* Reference signature (VisionEncoder::encode): one image, host pixels
 * [n_h*n_w, patch_dim], host output `hidden` floats. Synchronous. */
int s2x_vision_encode(s2x_vision *v, const float *pixels_host, int32_t n_h,
                      int32_t n_w, int32_t pooling, float *out_host);

/* Batched, device-resident: n_img images of the same n_h x n_w grid,
 * pixels_dev [n_img*n_h*n_w, patch_dim], out_dev [n_img, hidden].
 * Asynchronous on the encoder's stream. */
int s2x_vision_encode_batch_dev(s2x_vision *v, const float *pixels_dev,
                                int32_t n_img, int32_t n_h, int32_t n_w,
                                int32_t pooling, float *out_dev);

/* Ragged (NaFlex) device-resident batch in the HF padded convention:
 * pixels_dev [n_img, max_patches, patch_dim], image i's h*w valid patches
 * first (row-major over its h x w grid) then padding, shapes_host
 * [n_img][2] = (h, w).  The valid rows are packed and attention runs per
 * image, which equals HF's key-masked attention over the padded batch.
 * out_dev [n_img, hidden].  Asynchronous. */
int s2x_vision_encode_ragged_dev(s2x_vision *v, const float *pixels_dev,
                                 const int32_t *shapes_host, int32_t n_img,
                                 int32_t max_patches, int32_t pooling,
                                 float *out_dev);

/* Raw images to embeddings on the device (the reference server's
 * preprocess_image_rgb + VisionEncoder::encode per image,
 * src/siglip2_server.cpp:336-366, as one batch): rgb_dev[i] = image i as
 * h*w*3 u8 channel-last (device), hw_host[i] = (h, w).  Each image goes
 * through the NaFlex front end (s2x_nf_preprocess_rgb_dev semantics,
 * max_num_patches, rescale, mean[3], std[3] on the host) straight into
 * the packed rows of the ragged batch.  out_dev [n_img, hidden].
 * Asynchronous. */
int s2x_vision_encode_rgb_batch_dev(s2x_vision *v, const uint8_t *const *rgb_dev,
                                    const int32_t *hw_host, int32_t n_img,
                                    int32_t max_num_patches, float rescale,
                                    const float *mean, const float *std_,
                                    int32_t pooling, float *out_dev);

/* Per-kernel GPU timing of the MFMA GEMM launches (HIP events on the
 * encoder's stream) for roofline reporting.  enable != 0 turns recording
 * on; s2x_vision_gemm_stats returns the summed milliseconds and op count
 * (2*M*N*K_logical) of the GEMMs recorded since the last reset, plus the
 * launch count.  Synchronises the encoder stream. */
int s2x_vision_gemm_timing(s2x_vision *v, int enable);
int s2x_vision_gemm_stats(s2x_vision *v, double *ms, double *ops,
                          int64_t *launches, int reset);

int s2x_text_create(const s2x_text_weights *w, s2x_text **out);
void s2x_text_destroy(s2x_text *t);
int s2x_text_set_stream(s2x_text *t, void *stream);
/* Attention precision for the text tower: 1 (default) = s2x_attn_fp64 (the
 * oracle's arithmetic to within 1 ulp), 0 = the f16-MFMA flash kernel. */
int s2x_text_set_attention_fp64(s2x_text *t, int enable);
/* As s2x_vision_set_graphs, for the text tower. */
int s2x_text_set_graphs(s2x_text *t, int enable);
/* EXPERIMENTAL, outside the parity tolerance (cosine 0.99988 of the
 * block-order CPU restatement on the so400m text tower, below 0.9999).
 * 1 = the text tower's plain and residual GEMMs of 32+ K blocks run as
 * s2x_mul_mat_q8_0_q8_1_split_k (2 ranges, 4 from 96 blocks); 0 (default) =
 * one block-order sum per output, the oracle's.  No counterpart in the
 * reference (whose GPU GEMMs split K by stream-K); a prompt's bits do not
 * depend on its batch either way. */
int s2x_text_set_split_k(s2x_text *t, int enable);
/* TextEncoder::encode: one prompt of n_tok ids (host), optional host mask
 * (1 = valid), out_host proj floats.  Synchronous. */
int s2x_text_encode(s2x_text *t, const int32_t *ids_host, int32_t n_tok,
                    const int32_t *mask_host, float *out_host);
/* TextEncoder::encode_batch: n_batch prompts of n_tok ids each (host, batch
 * major), no mask (the reference rejects one, src/siglip2_text.cpp:769-772);
 * out_host n_batch*proj floats.  Synchronous. */
int s2x_text_encode_batch(s2x_text *t, const int32_t *ids_host, int32_t n_tok,
                          int32_t n_batch, float *out_host);

#ifdef __cplusplus
}
#endif
#endif /* S2X_H */
