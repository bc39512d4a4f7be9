// s2x_kernels.h -- host-side launchers of the gfx950 kernels (internal).
//
// All launchers are asynchronous on `stream`, validate nothing (the C-ABI
// layer in s2x_abi.cpp does) and return hipError_t from the launch.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace s2x {

// Longest attention segment (tokens per image / prompt) the kernels accept.
constexpr int64_t MAX_SEG_LEN = 4096;

// Device view of a repacked Q8_0 weight (K_pad, N).
struct WeightView {
    const int8_t *qs;     // N rows of K_pad int8 (16-byte aligned)
    // KB rows of ldT fp16 bits of d (transposed); within each group of 64
    // columns, column c + j (j < 32) sits at 2 j and c + 32 + j at 2 j + 1,
    // so one 32-bit word holds the scales of columns j and j + 32
    const uint16_t *dT;
    int64_t ldT;          // >= round_up(N, GEMM_BN)
    int64_t K_pad;        // multiple of 32
    int64_t N;
};

// Column tile of the GEMM; the transposed weight scales are padded to it.
constexpr int64_t GEMM_BN = 128;
inline int64_t gemm_ld_dw(int64_t N) { return (N + GEMM_BN - 1) / GEMM_BN * GEMM_BN; }

// Destination planes of a Q8_1 quantization: int8 quants [M][K_pad] and the
// block_q8_1 scale words [M][ld_ds] (fp16 d | fp16 s << 16), ld_ds >= K_pad/32.
struct Q81Out {
    int8_t   *qs = nullptr;
    uint32_t *ds = nullptr;
    int64_t   ld_ds = 0;  // 0: K_pad / 32
};

enum EpiKind {
    EPI_NONE = 0, EPI_BIAS = 1, EPI_BIAS_GELU = 2, EPI_BIAS_RESID = 3, EPI_DUMP_I = 4,
    EPI_QKV = 5,       // (mm + bias) -> f16 Q / K / V^T in the attention layout
    EPI_GELU_Q81 = 6,  // GELU(mm + bias) quantized to Q8_1 (int8 quants + ds words)
    EPI_GELU_F16 = 7,  // GELU(mm + bias) rounded to f16 (rows of h_kpad halves)
};

// row map entry of a GEMM row that no segment covers
constexpr int32_t ROW_NONE = -1;

struct EpiParams {
    int          kind;
    const float *bias;
    const float *resid;
    int64_t      ld_resid;
    int64_t      resid_rows;  // 0: row m; >0: row m % resid_rows
    int64_t      dump_kb;     // EPI_DUMP_I: the block whose int32 dot is written
    // EPI_QKV: output columns [q | k | v] (n_head x d_head each); row m is
    // position rowmap[m] & 0xffff of segment rowmap[m] >> 16, or no
    // position at all (nothing stored) where rowmap[m] is ROW_NONE
    _Float16      *q, *k, *vt;
    const int32_t *rowmap;
    int            n_head, d_head, d_pad, dv_pad, len_pad;
    // EPI_GELU_Q81: quants [M][q_kpad] (columns N..q_kpad-1 quantize zeros)
    // and ds words [M][q_ldds]
    int8_t   *q_out8;
    uint32_t *q_ds;
    int64_t   q_kpad, q_ldds;
    // EPI_GELU_F16: f16 rows [M][h_ld], columns N..h_kpad-1 written as zero
    _Float16 *h_out;
    int64_t   h_ld, h_kpad;
    // K split (EPI_NONE only; set by launch_gemm_split_k): workgroup row
    // blockIdx.y sums blocks [kb_split * y, min(KB, kb_split * (y + 1)))
    // into the outputs at y + blockIdx.y * y_split
    int       kb_split;
    int64_t   y_split;
};

// a1: F32 -> Q8_1 into the planes of `out`.
hipError_t launch_quantize_q8_1(const float *x, int64_t K, int64_t M, int64_t ldx,
                                int64_t K_pad, const Q81Out &out, hipStream_t stream);

// a2: raw block_q8_0 (N rows of K_pad/32 34-byte blocks, device) -> WeightView
// planes
hipError_t launch_repack_q8_0(const void *raw, int64_t K_pad, int64_t N, int8_t *qs,
                              uint16_t *dT, int64_t ldT, hipStream_t stream);

// a3: Y = W x X(Q8_1) with epilogue, on int8 MFMA (s2x_gemm.hip).  xq: int8
// quants [M][K_pad] (16-byte aligned), xds: ds words [M][ld_ds].
hipError_t launch_gemm(const WeightView &w, const int8_t *xq, const uint32_t *xds, int64_t ld_ds,
                       int64_t M, float *y, int64_t ldy, const EpiParams &epi,
                       hipStream_t stream);

// F16 weights (the converter's type for matrices whose K is not a multiple
// of 32, e.g. ffn_down): Y = W16 x f16(X) with f32 accumulation on f16 MFMA.
// w16: N rows of K_pad halves, x16: M rows of K_pad halves (both zero past
// K, 16-byte aligned rows); epilogues NONE, BIAS, BIAS_RESID.
// The same product as launch_gemm with EPI_NONE / EPI_BIAS_RESID, its K
// blocks in n_split contiguous ranges of whole 4-block stages (a function of
// K alone): each range's sum, in block order from zero, goes to a partial
// plane of `part` (n_split x M x N floats) in one launch of
// n_split x the tiles, then y = ((p_0 + p_1) + ...) [+ bias] [+ resid] in
// that order.  For GEMMs of too few tiles to fill the chip (a text batch);
// the bits depend on K and n_split, not on M.
hipError_t launch_gemm_split_k(const WeightView &w, const int8_t *xq, const uint32_t *xds,
                               int64_t ld_ds, int64_t M, float *y, int64_t ldy,
                               const EpiParams &epi, int n_split, float *part,
                               hipStream_t stream);

hipError_t launch_gemm_f16(const _Float16 *w16, int64_t K_pad, int64_t N, const _Float16 *x16,
                           int64_t M, float *y, int64_t ldy, const EpiParams &epi,
                           hipStream_t stream);
// f32 rows (K valid of ldx) -> f16 rows of K_pad halves, zeros past K
hipError_t launch_f32_to_f16(const float *x, int64_t K, int64_t M, int64_t ldx, int64_t K_pad,
                             _Float16 *y, hipStream_t stream);
// raw F16 weight rows (N rows of K halves, device) -> N rows of K_pad halves
hipError_t launch_repack_f16(const void *raw, int64_t K, int64_t N, int64_t K_pad, _Float16 *w16,
                             hipStream_t stream);

// a4: LayerNorm (+ Q8_1).  q may be null (no quantized output), y may be
// null (no f32 output); at least one is set.
hipError_t launch_layernorm(const float *x, int64_t H, int64_t M, int64_t ldx,
                            const float *w, const float *b, float eps, const Q81Out *q,
                            float *y, int64_t ldy, hipStream_t stream);

// a5: standalone epilogues
hipError_t launch_bias_residual(const float *mm, const float *bias, const float *resid,
                                float *y, int64_t H, int64_t n_pos, hipStream_t stream);
hipError_t launch_bias_gelu(const float *mm, const float *bias, float *y, int64_t H,
                            int64_t n_pos, hipStream_t stream);

// a6/a7: attention staging + flash attention over packed segments
struct AttnLayout {
    int64_t n_seg, max_len, n_head, d_head;
    int64_t d_pad;     // d_head rounded up to 16 (Q/K row length)
    int64_t dv_pad;    // d_head rounded up to 32 (V^T rows)
    int64_t len_pad;   // max_len rounded up to 128 (query tile)
    size_t q_off, k_off, vt_off, planes_bytes;  // Q, K, V^T planes
    size_t rowmap_off, bytes;  // + n_seg * max_len int32 (fused QKV entry point)
    // softmax probabilities enter the PV product as an exact f16 pair
    // (hi + lo, ~22 bits) instead of one f16 (11 bits)
    bool p_split = true;
};
AttnLayout attn_layout(int64_t n_seg, int64_t max_len, int64_t n_head, int64_t d_head);
hipError_t launch_attn_prep(const float *qkv, int64_t ld_qkv, const float *qkv_bias,
                            const int32_t *seg_start, const int32_t *seg_len,
                            const AttnLayout &L, void *ws, hipStream_t stream);
// Row -> (segment << 16 | position) table of packed segments, for EPI_QKV
// (rows outside [0, n_rows) are not written).
hipError_t launch_rowmap(const int32_t *seg_start, const int32_t *seg_len, int64_t n_seg,
                         int64_t max_len, int32_t *rowmap, int64_t n_rows, hipStream_t stream);
// EPI_QKV destination planes of layout L in workspace ws.
EpiParams epi_qkv(const AttnLayout &L, void *ws, const float *qkv_bias, const int32_t *rowmap);
// With qo: the output's Q8_1 (K = n_head * d_head) instead of the whole f32
// output -- at most the columns of Q8_1 blocks that straddle two heads are
// written to `out` -- over the packed rows 0 .. n_rows - 1 (every row a
// segment's); needs attn_q81_fusable.
hipError_t launch_attn(const void *ws, const int32_t *seg_start, const int32_t *seg_len,
                       const uint8_t *key_valid, const AttnLayout &L, float scale,
                       float *out, int64_t ld_out, hipStream_t stream,
                       const Q81Out *qo = nullptr, int64_t n_rows = 0);
// 72-wide heads in groups of four: whole Q8_1 blocks per group of heads
inline bool attn_q81_fusable(int64_t n_head, int64_t d_head) {
    return d_head == 72 && n_head % 4 == 0;
}
// fp64 attention straight from the QKV GEMM rows (+bias), fixed summation
// order; for short sequences (the text tower).
hipError_t launch_attn_f64(const float *qkv, int64_t ld_qkv, const float *qkv_bias,
                           const int32_t *seg_start, const int32_t *seg_len,
                           const uint8_t *key_valid, int64_t n_seg, int64_t max_len,
                           int64_t n_head, int64_t d_head, float scale, float *out,
                           int64_t ld_out, hipStream_t stream);
// Single-query attention (MAP probe head): q [H] shared by all segments,
// k/v packed rows (ld floats), out [n_seg][H].
hipError_t launch_attn_1q(const float *q, const float *k, const float *v, int64_t ld,
                          const int32_t *seg_start, const int32_t *seg_len,
                          int64_t n_seg, int64_t n_head, int64_t d_head, float scale,
                          float *out, hipStream_t stream);

// a8: anti-aliased bilinear resize of the position-embedding grid
hipError_t launch_resize_pos_embed(const float *pos, int64_t n_side, int64_t H,
                                   int64_t out_h, int64_t out_w, float *out,
                                   hipStream_t stream);

// a11: Q8_0 get_rows (+ optional add of row i % add_rows)
hipError_t launch_get_rows_q8_0(const void *table_raw, int64_t K, int64_t n_rows,
                                const int32_t *ids, int64_t n_ids, const float *add,
                                int64_t add_rows, float *out, hipStream_t stream);

// Pooling helpers
// out[s][c] = mean over the rows of segment s (double accumulation)
hipError_t launch_mean_pool(const float *x, int64_t H, const int32_t *seg_start,
                            const int32_t *seg_len, int64_t n_seg, float *out,
                            hipStream_t stream);
// out[i][c] = x[rows[i]][c]
hipError_t launch_gather_rows(const float *x, int64_t H, const int32_t *rows,
                              int64_t n, float *out, hipStream_t stream);
// packed[t] = padded[img(t)][pos(t)] for the valid (first seg_len) rows
hipError_t launch_pack_rows(const float *padded, int64_t row_len, int64_t max_rows,
                            const int32_t *seg_start, const int32_t *seg_len,
                            int64_t n_seg, float *packed, hipStream_t stream);
// bytes of zeros (16-byte aligned p), a kernel (no memset node in captured graphs)
hipError_t launch_fill_zero(void *p, size_t bytes, hipStream_t stream);
// y[i] = a[i] + b[i]
hipError_t launch_add(const float *a, const float *b, float *y, int64_t n,
                      hipStream_t stream);

// NaFlex front end (s2x_naflex.hip): target grid, anti-aliased resize,
// rescale + normalise + patchify of one RGB u8 image (device pointers).
void nf_target_size(int h, int w, int p, int max_patches, int *out_h, int *out_w);
size_t nf_workspace_bytes(int h, int w, int p, int max_patches);
hipError_t launch_nf_preprocess(const uint8_t *rgb, int h, int w, int max_patches, int p,
                                float rescale, const float mean[3], const float stdv[3],
                                float *out, int64_t out_cap, int *n_h, int *n_w, void *ws,
                                size_t ws_bytes, hipStream_t stream);
// n_img same-size images, rgb contiguous (h*w*3 bytes each), out contiguous
// (n_h*n_w*3*p*p floats each, out_cap >= that), ws >= n_img x
// nf_workspace_bytes(): one launch per pass for the whole batch
hipError_t launch_nf_preprocess_batch(const uint8_t *rgb, int n_img, int h, int w,
                                      int max_patches, int p, float rescale, const float mean[3],
                                      const float stdv[3], float *out, int64_t out_cap, int *n_h,
                                      int *n_w, void *ws, size_t ws_bytes, hipStream_t stream);

}  // namespace s2x
