// s2x_abi.cpp -- the extern "C" boundary (include/s2x.h): argument checks,
// status codes, weight objects and the op-level entry points.
#include "s2x.h"

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <string>

#include "s2x_internal.h"
#include "s2x_kernels.h"

namespace s2x {

static thread_local std::string g_last_error;

int fail(int status, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return status;
}

int hip_fail(hipError_t e, const char *what) {
    return fail(S2X_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

bool aligned(const void *p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

WeightView view_of(const s2x_weight *w) { return w->view; }

}  // namespace s2x

using namespace s2x;

extern "C" {

const char *s2x_status_string(int status) {
    switch (status) {
    case S2X_OK: return "ok";
    case S2X_ERR_INVALID_ARG: return "invalid argument";
    case S2X_ERR_UNSUPPORTED: return "unsupported";
    case S2X_ERR_HIP: return "HIP runtime error";
    case S2X_ERR_WORKSPACE: return "workspace too small";
    case S2X_ERR_OOM: return "out of device memory";
    case S2X_ERR_NOT_LOADED: return "encoder not loaded";
    default: return "unknown status";
    }
}

const char *s2x_last_error(void) { return g_last_error.c_str(); }

const char *s2x_version(void) { return "s2x 0.1 gfx950"; }

// ---------------------------------------------------------------------------
// a1
// ---------------------------------------------------------------------------
int s2x_quantize_q8_1(const float *x, int64_t K, int64_t M, int64_t ldx, int64_t K_pad,
                      void *qs, void *ds, void *stream) {
    if (M < 0 || K < 0 || K_pad <= 0 || K_pad % QK_ != 0 || K > K_pad || ldx < K)
        return fail(S2X_ERR_INVALID_ARG, "quantize_q8_1: bad shape K=%lld K_pad=%lld ldx=%lld M=%lld",
                    (long long)K, (long long)K_pad, (long long)ldx, (long long)M);
    if (M == 0) return S2X_OK;
    if (!x || !qs || !ds) return fail(S2X_ERR_INVALID_ARG, "quantize_q8_1: null pointer");
    if (!aligned(qs, 4) || !aligned(ds, 4) || !aligned(x, 4))
        return fail(S2X_ERR_INVALID_ARG, "quantize_q8_1: qs/ds/x must be 4-byte aligned");
    Q81Out o;
    o.qs = (int8_t *)qs;
    o.ds = (uint32_t *)ds;
    hipError_t e = launch_quantize_q8_1(x, K, M, ldx, K_pad, o, (hipStream_t)stream);
    return e == hipSuccess ? S2X_OK : hip_fail(e, "quantize_q8_1 launch");
}

// ---------------------------------------------------------------------------
// a2
// ---------------------------------------------------------------------------
size_t s2x_weight_bytes(int64_t K_pad, int64_t N) {
    if (K_pad <= 0 || N <= 0 || K_pad % QK_ != 0) return 0;
    return weight_planes_bytes(K_pad, N);
}

int s2x_weight_create_in(const void *raw_dev, int64_t K_pad, int64_t N, void *dev_buf,
                         void *stream, s2x_weight **out) {
    if (!out) return fail(S2X_ERR_INVALID_ARG, "weight_create_in: out is null");
    *out = nullptr;
    if (K_pad <= 0 || N <= 0 || K_pad % QK_ != 0)
        return fail(S2X_ERR_INVALID_ARG, "weight_create_in: bad shape K_pad=%lld N=%lld",
                    (long long)K_pad, (long long)N);
    if (!raw_dev || !dev_buf || !aligned(raw_dev, 2) || !aligned(dev_buf, 256))
        return fail(S2X_ERR_INVALID_ARG,
                    "weight_create_in: raw must be 2-byte and dev_buf 256-byte aligned");
    s2x_weight *w = new s2x_weight();
    w->mem = dev_buf;
    w->owns = false;
    w->view = planes_view(dev_buf, K_pad, N);
    hipError_t e = repack_into(raw_dev, w->view, (hipStream_t)stream);
    if (e != hipSuccess) {
        delete w;
        return hip_fail(e, "repack launch");
    }
    *out = w;
    return S2X_OK;
}

int s2x_weight_create(const void *raw, int raw_is_host, int64_t K_pad, int64_t N, void *stream,
                      s2x_weight **out) {
    if (!out) return fail(S2X_ERR_INVALID_ARG, "weight_create: out is null");
    *out = nullptr;
    if (K_pad <= 0 || N <= 0 || K_pad % QK_ != 0 || !raw)
        return fail(S2X_ERR_INVALID_ARG, "weight_create: bad shape K_pad=%lld N=%lld",
                    (long long)K_pad, (long long)N);
    int st = weight_upload(raw, raw_is_host != 0, K_pad, N, (hipStream_t)stream, out);
    if (st != S2X_OK) return st;
    hipError_t e = hipStreamSynchronize((hipStream_t)stream);
    if (e != hipSuccess) {
        s2x_weight_destroy(*out);
        *out = nullptr;
        return hip_fail(e, "weight_create sync");
    }
    return S2X_OK;
}

void s2x_weight_destroy(s2x_weight *w) {
    if (!w) return;
    if (w->owns && w->mem) (void)hipFree(w->mem);
    delete w;
}

int64_t s2x_weight_k(const s2x_weight *w) { return w ? w->view.K_pad : 0; }
int64_t s2x_weight_n(const s2x_weight *w) { return w ? w->view.N : 0; }

// ---------------------------------------------------------------------------
// a3
// ---------------------------------------------------------------------------
static int check_epi(const s2x_epilogue *epi, int64_t N, EpiParams &p) {
    p = EpiParams{EPI_NONE, nullptr, nullptr, 0, 0, 0};
    if (!epi) return S2X_OK;
    p.kind = epi->kind;
    p.bias = epi->bias;
    p.resid = epi->resid;
    p.ld_resid = epi->ld_resid;
    p.resid_rows = epi->resid_rows;
    switch (epi->kind) {
    case S2X_EPI_NONE: return S2X_OK;
    case S2X_EPI_BIAS:
    case S2X_EPI_BIAS_GELU:
        if (!epi->bias) return fail(S2X_ERR_INVALID_ARG, "epilogue: bias is null");
        return S2X_OK;
    case S2X_EPI_BIAS_RESID:
        if (!epi->bias || !epi->resid || epi->ld_resid < N || epi->resid_rows < 0)
            return fail(S2X_ERR_INVALID_ARG, "epilogue: bias/resid/ld_resid invalid");
        return S2X_OK;
    case S2X_EPI_GELU_Q81:
        if (!epi->bias || !epi->q_out || !epi->q_ds || epi->q_kpad % QK_ || epi->q_kpad < N ||
            epi->q_kpad - N >= QK_)
            return fail(S2X_ERR_INVALID_ARG, "epilogue GELU_Q81: bias/q_out/q_ds/q_kpad invalid");
        if (!aligned(epi->q_out, 16) || !aligned(epi->q_ds, 4))
            return fail(S2X_ERR_INVALID_ARG, "epilogue GELU_Q81: q_out must be 16-byte aligned");
        p.kind = EPI_GELU_Q81;
        p.q_out8 = (int8_t *)epi->q_out;
        p.q_ds = (uint32_t *)epi->q_ds;
        p.q_kpad = epi->q_kpad;
        p.q_ldds = epi->q_kpad / QK_;
        return S2X_OK;
    case S2X_EPI_GELU_F16:
        if (!epi->bias || !epi->q_out || epi->q_kpad % QK_ || epi->q_kpad < N ||
            epi->q_kpad - N >= QK_ || !aligned(epi->q_out, 2))
            return fail(S2X_ERR_INVALID_ARG, "epilogue GELU_F16: bias/q_out/q_kpad invalid");
        p.kind = EPI_GELU_F16;
        p.h_out = (_Float16 *)epi->q_out;
        p.h_ld = p.h_kpad = epi->q_kpad;
        return S2X_OK;
    default: return fail(S2X_ERR_INVALID_ARG, "epilogue: unknown kind %d", epi->kind);
    }
}

static int check_q81_input(const s2x_weight *w, const void *qs, const void *ds, int64_t M,
                           const char *who) {
    if (!w) return fail(S2X_ERR_INVALID_ARG, "%s: weight is null", who);
    if (M < 0) return fail(S2X_ERR_INVALID_ARG, "%s: M < 0", who);
    if (M > (1 << 30)) return fail(S2X_ERR_UNSUPPORTED, "%s: M too large", who);
    if (M > 0 && (!qs || !ds)) return fail(S2X_ERR_INVALID_ARG, "%s: null qs/ds", who);
    if (!aligned(qs, 16) || !aligned(ds, 4))
        return fail(S2X_ERR_INVALID_ARG, "%s: qs must be 16-byte and ds 4-byte aligned", who);
    return S2X_OK;
}

int s2x_mul_mat_q8_0_q8_1(const s2x_weight *w, const void *qs, const void *ds, int64_t M,
                          float *y, int64_t ldy, const s2x_epilogue *epi, void *stream) {
    int st = check_q81_input(w, qs, ds, M, "mul_mat_q8_0_q8_1");
    if (st != S2X_OK) return st;
    EpiParams p;
    st = check_epi(epi, w->view.N, p);
    if (st != S2X_OK) return st;
    if (p.kind != EPI_GELU_Q81 && p.kind != EPI_GELU_F16 && (!y || ldy < w->view.N || !aligned(y, 4)))
        return fail(S2X_ERR_INVALID_ARG, "mul_mat_q8_0_q8_1: y null/misaligned or ldy=%lld < N=%lld",
                    (long long)ldy, (long long)w->view.N);
    if (M == 0) return S2X_OK;
    hipError_t e = launch_gemm(w->view, (const int8_t *)qs, (const uint32_t *)ds,
                               w->view.K_pad / QK_, M, y, ldy, p, (hipStream_t)stream);
    return e == hipSuccess ? S2X_OK : hip_fail(e, "gemm launch");
}

int s2x_mul_mat_q8_0_q8_1_split_k(const s2x_weight *w, const void *qs, const void *ds, int64_t M,
                                  float *y, int64_t ldy, const s2x_epilogue *epi, int32_t n_split,
                                  void *workspace, size_t ws_bytes, void *stream) {
    int st = check_q81_input(w, qs, ds, M, "mul_mat_q8_0_q8_1_split_k");
    if (st != S2X_OK) return st;
    EpiParams p;
    st = check_epi(epi, w->view.N, p);
    if (st != S2X_OK) return st;
    if ((p.kind != EPI_NONE && p.kind != EPI_BIAS_RESID) || p.resid_rows != 0)
        return fail(S2X_ERR_UNSUPPORTED,
                    "mul_mat_q8_0_q8_1_split_k: epilogue NONE or BIAS_RESID (resid_rows 0) only");
    if (n_split < 1 || n_split > 64)
        return fail(S2X_ERR_INVALID_ARG, "mul_mat_q8_0_q8_1_split_k: n_split=%d not in 1..64",
                    (int)n_split);
    if (!y || ldy < w->view.N || !aligned(y, 4))
        return fail(S2X_ERR_INVALID_ARG, "mul_mat_q8_0_q8_1_split_k: y null/misaligned or ldy < N");
    const size_t need = sizeof(float) * (size_t)n_split * (size_t)M * (size_t)w->view.N;
    if (!workspace || !aligned(workspace, 16) || ws_bytes < need)
        return fail(S2X_ERR_INVALID_ARG,
                    "mul_mat_q8_0_q8_1_split_k: workspace of n_split * M * N floats needed (%zu bytes, "
                    "16-byte aligned)", need);
    if (M == 0) return S2X_OK;
    hipError_t e = launch_gemm_split_k(w->view, (const int8_t *)qs, (const uint32_t *)ds,
                                       w->view.K_pad / QK_, M, y, ldy, p, n_split,
                                       (float *)workspace, (hipStream_t)stream);
    return e == hipSuccess ? S2X_OK : hip_fail(e, "split-k gemm launch");
}

size_t s2x_mul_mat_workspace_size(int64_t K_pad, int64_t N, int64_t M) {
    if (K_pad <= 0 || N <= 0 || M < 0 || K_pad % QK_ != 0) return 0;
    return mul_mat_ws_layout(K_pad, N, M).total;
}

int s2x_mul_mat_q8_0_f32(const void *w_raw, int64_t K_pad, int64_t N, const float *x, int64_t K,
                         int64_t ldx, int64_t M, float *y, void *workspace, size_t ws_bytes,
                         void *stream) {
    if (K_pad <= 0 || N <= 0 || K_pad % QK_ != 0 || K <= 0 || K > K_pad || ldx < K || M < 0)
        return fail(S2X_ERR_INVALID_ARG,
                    "mul_mat_q8_0_f32: bad shape K=%lld K_pad=%lld N=%lld M=%lld ldx=%lld",
                    (long long)K, (long long)K_pad, (long long)N, (long long)M, (long long)ldx);
    if (M == 0) return S2X_OK;
    if (M > (1 << 30)) return fail(S2X_ERR_UNSUPPORTED, "mul_mat_q8_0_f32: M too large");
    if (!w_raw || !x || !y || !workspace)
        return fail(S2X_ERR_INVALID_ARG, "mul_mat_q8_0_f32: null pointer");
    const MulMatWs L = mul_mat_ws_layout(K_pad, N, M);
    if (ws_bytes < L.total)
        return fail(S2X_ERR_WORKSPACE, "mul_mat_q8_0_f32: workspace %zu < %zu bytes", ws_bytes,
                    L.total);
    if (!aligned(workspace, 256) || !aligned(w_raw, 2) || !aligned(x, 4) || !aligned(y, 4))
        return fail(S2X_ERR_INVALID_ARG, "mul_mat_q8_0_f32: misaligned pointer");
    uint8_t *ws = (uint8_t *)workspace;
    hipStream_t s = (hipStream_t)stream;
    const WeightView wv = planes_view(ws + L.w_off, K_pad, N);
    hipError_t e = repack_into(w_raw, wv, s);
    if (e != hipSuccess) return hip_fail(e, "repack launch");
    Q81Out o;
    o.qs = (int8_t *)(ws + L.xq_off);
    o.ds = (uint32_t *)(ws + L.ds_off);
    o.ld_ds = K_pad / QK_;
    e = launch_quantize_q8_1(x, K, M, ldx, K_pad, o, s);
    if (e != hipSuccess) return hip_fail(e, "quantize launch");
    EpiParams p{EPI_NONE, nullptr, nullptr, 0, 0, 0};
    e = launch_gemm(wv, o.qs, o.ds, o.ld_ds, M, y, N, p, s);
    return e == hipSuccess ? S2X_OK : hip_fail(e, "gemm launch");
}

static MulMatWs mul_mat_f16_ws_layout(int64_t K, int64_t N, int64_t M) {
    const int64_t K_pad = round_up_i(K, QK_);
    MulMatWs L;
    L.w_off = 0;
    L.xq_off = (size_t)round_up_i(N * K_pad * 2, 256);
    L.ds_off = L.xq_off;
    L.total = L.xq_off + (size_t)round_up_i(M * K_pad * 2, 256);
    return L;
}

size_t s2x_mul_mat_f16_workspace_size(int64_t K, int64_t N, int64_t M) {
    if (K <= 0 || N <= 0 || M < 0) return 0;
    return mul_mat_f16_ws_layout(K, N, M).total;
}

int s2x_mul_mat_f16_f32(const void *w_raw, int64_t K, int64_t N, const float *x, int64_t ldx,
                        int64_t M, float *y, void *workspace, size_t ws_bytes, void *stream) {
    if (K <= 0 || N <= 0 || M < 0 || ldx < K)
        return fail(S2X_ERR_INVALID_ARG, "mul_mat_f16_f32: bad shape K=%lld N=%lld M=%lld ldx=%lld",
                    (long long)K, (long long)N, (long long)M, (long long)ldx);
    if (M == 0) return S2X_OK;
    if (M > (1 << 30) || N > (1 << 30) || K > (1 << 24))
        return fail(S2X_ERR_UNSUPPORTED, "mul_mat_f16_f32: shape too large");
    if (!w_raw || !x || !y || !workspace)
        return fail(S2X_ERR_INVALID_ARG, "mul_mat_f16_f32: null pointer");
    const MulMatWs L = mul_mat_f16_ws_layout(K, N, M);
    if (ws_bytes < L.total)
        return fail(S2X_ERR_WORKSPACE, "mul_mat_f16_f32: workspace %zu < %zu bytes", ws_bytes, L.total);
    if (!aligned(workspace, 256) || !aligned(w_raw, 2) || !aligned(x, 4) || !aligned(y, 4))
        return fail(S2X_ERR_INVALID_ARG, "mul_mat_f16_f32: misaligned pointer");
    const int64_t K_pad = round_up_i(K, QK_);
    uint8_t *ws = (uint8_t *)workspace;
    hipStream_t s = (hipStream_t)stream;
    _Float16 *w16 = (_Float16 *)(ws + L.w_off), *x16 = (_Float16 *)(ws + L.xq_off);
    hipError_t e = launch_repack_f16(w_raw, K, N, K_pad, w16, s);
    if (e != hipSuccess) return hip_fail(e, "repack launch");
    e = launch_f32_to_f16(x, K, M, ldx, K_pad, x16, s);
    if (e != hipSuccess) return hip_fail(e, "convert launch");
    EpiParams p{EPI_NONE, nullptr, nullptr, 0, 0, 0};
    e = launch_gemm_f16(w16, K_pad, N, x16, M, y, N, p, s);
    return e == hipSuccess ? S2X_OK : hip_fail(e, "gemm launch");
}

int s2x_block_dots(const s2x_weight *w, const void *qs, int64_t M, int64_t kb, int32_t *out,
                   void *stream) {
    if (!w || !qs || !out) return fail(S2X_ERR_INVALID_ARG, "block_dots: null pointer");
    if (M <= 0 || M > (1 << 30) || kb < 0 || kb >= w->view.K_pad / QK_)
        return fail(S2X_ERR_INVALID_ARG, "block_dots: bad M=%lld or kb=%lld", (long long)M,
                    (long long)kb);
    if (!aligned(qs, 16)) return fail(S2X_ERR_INVALID_ARG, "block_dots: qs must be 16-byte aligned");
    // the integer stage reads no activation scales (the DMA of a null plane
    // returns zeros)
    EpiParams p{EPI_DUMP_I, nullptr, nullptr, 0, 0, kb};
    hipError_t e = launch_gemm(w->view, (const int8_t *)qs, nullptr, 0, M,
                               reinterpret_cast<float *>(out), w->view.N, p, (hipStream_t)stream);
    return e == hipSuccess ? S2X_OK : hip_fail(e, "block dots launch");
}

// ---------------------------------------------------------------------------
// a4 / a5
// ---------------------------------------------------------------------------
static int check_ln(const float *x, int64_t H, int64_t M, int64_t ldx, const char *who) {
    if (H <= 0 || H % QK_ != 0 || H > 2048 || M < 0 || ldx < H)
        return fail(S2X_ERR_INVALID_ARG, "%s: bad shape H=%lld M=%lld ldx=%lld", who,
                    (long long)H, (long long)M, (long long)ldx);
    if (M > 0 && !x) return fail(S2X_ERR_INVALID_ARG, "%s: x is null", who);
    return S2X_OK;
}

int s2x_layernorm(const float *x, int64_t H, int64_t M, int64_t ldx, const float *w,
                  const float *b, float eps, float *y, int64_t ldy, void *stream) {
    int st = check_ln(x, H, M, ldx, "layernorm");
    if (st != S2X_OK) return st;
    if (M == 0) return S2X_OK;
    if (!y || ldy < H) return fail(S2X_ERR_INVALID_ARG, "layernorm: y null or ldy < H");
    hipError_t e = launch_layernorm(x, H, M, ldx, w, b, eps, nullptr, y, ldy, (hipStream_t)stream);
    return e == hipSuccess ? S2X_OK : hip_fail(e, "layernorm launch");
}

int s2x_layernorm_quantize_q8_1(const float *x, int64_t H, int64_t M, int64_t ldx,
                                const float *w, const float *b, float eps, void *qs, void *ds,
                                float *y, int64_t ldy, void *stream) {
    int st = check_ln(x, H, M, ldx, "layernorm_quantize");
    if (st != S2X_OK) return st;
    if (M == 0) return S2X_OK;
    if (!qs || !ds || !aligned(qs, 4) || !aligned(ds, 4))
        return fail(S2X_ERR_INVALID_ARG, "layernorm_quantize: qs/ds null or misaligned");
    if (y && ldy < H) return fail(S2X_ERR_INVALID_ARG, "layernorm_quantize: ldy < H");
    Q81Out o;
    o.qs = (int8_t *)qs;
    o.ds = (uint32_t *)ds;
    hipError_t e = launch_layernorm(x, H, M, ldx, w, b, eps, &o, y, ldy, (hipStream_t)stream);
    return e == hipSuccess ? S2X_OK : hip_fail(e, "layernorm_quantize launch");
}

int s2x_bias_residual(const float *mm, const float *bias, const float *resid, float *y,
                      int64_t H, int64_t n_pos, void *stream) {
    if (H <= 0 || n_pos < 0) return fail(S2X_ERR_INVALID_ARG, "bias_residual: bad shape");
    if (n_pos == 0) return S2X_OK;
    if (!mm || !bias || !resid || !y) return fail(S2X_ERR_INVALID_ARG, "bias_residual: null");
    hipError_t e = launch_bias_residual(mm, bias, resid, y, H, n_pos, (hipStream_t)stream);
    return e == hipSuccess ? S2X_OK : hip_fail(e, "bias_residual launch");
}

int s2x_bias_gelu(const float *mm, const float *bias, float *y, int64_t H, int64_t n_pos,
                  void *stream) {
    if (H <= 0 || n_pos < 0) return fail(S2X_ERR_INVALID_ARG, "bias_gelu: bad shape");
    if (n_pos == 0) return S2X_OK;
    if (!mm || !bias || !y) return fail(S2X_ERR_INVALID_ARG, "bias_gelu: null");
    hipError_t e = launch_bias_gelu(mm, bias, y, H, n_pos, (hipStream_t)stream);
    return e == hipSuccess ? S2X_OK : hip_fail(e, "bias_gelu launch");
}

// ---------------------------------------------------------------------------
// a6 / a7
// ---------------------------------------------------------------------------
static int check_attn_shape(int64_t n_seg, int64_t max_len, int64_t n_head, int64_t d_head,
                            const char *who) {
    if (n_seg < 0 || max_len <= 0 || n_head <= 0 || d_head <= 0)
        return fail(S2X_ERR_INVALID_ARG, "%s: bad shape", who);
    const AttnLayout L = attn_layout(n_seg, max_len, n_head, d_head);
    if (L.d_pad != 80 || L.dv_pad != 96 || d_head % 4 != 0)
        return fail(S2X_ERR_UNSUPPORTED, "%s: d_head %lld not supported (needs 65..80, %%4)", who,
                    (long long)d_head);
    return S2X_OK;
}

size_t s2x_attn_workspace_size(int64_t n_seg, int64_t max_len, int64_t n_head, int64_t d_head) {
    if (n_seg < 0 || max_len <= 0 || n_head <= 0 || d_head <= 0) return 0;
    return attn_layout(n_seg, max_len, n_head, d_head).bytes;
}

int s2x_attn_prep(const float *qkv, int64_t ld_qkv, const float *qkv_bias,
                  const int32_t *seg_start_dev, const int32_t *seg_len_dev, int64_t n_seg,
                  int64_t max_len, int64_t n_head, int64_t d_head, void *ws, size_t ws_bytes,
                  void *stream) {
    int st = check_attn_shape(n_seg, max_len, n_head, d_head, "attn_prep");
    if (st != S2X_OK) return st;
    if (n_seg == 0) return S2X_OK;
    const AttnLayout L = attn_layout(n_seg, max_len, n_head, d_head);
    if (!qkv || !qkv_bias || !seg_start_dev || !seg_len_dev || !ws)
        return fail(S2X_ERR_INVALID_ARG, "attn_prep: null pointer");
    if (ws_bytes < L.bytes) return fail(S2X_ERR_WORKSPACE, "attn_prep: workspace too small");
    if (ld_qkv < 3 * n_head * d_head || !aligned(ws, 256))
        return fail(S2X_ERR_INVALID_ARG, "attn_prep: ld_qkv < 3H or ws misaligned");
    hipError_t e = launch_attn_prep(qkv, ld_qkv, qkv_bias, seg_start_dev, seg_len_dev, L, ws,
                                    (hipStream_t)stream);
    return e == hipSuccess ? S2X_OK : hip_fail(e, "attn_prep launch");
}

int s2x_mul_mat_qkv_attn_prep(const s2x_weight *w, const void *qs, const void *ds, int64_t M,
                              const float *qkv_bias, const int32_t *seg_start_dev,
                              const int32_t *seg_len_dev, int64_t n_seg, int64_t max_len,
                              int64_t n_head, int64_t d_head, void *ws, size_t ws_bytes,
                              void *stream) {
    int st = check_attn_shape(n_seg, max_len, n_head, d_head, "mul_mat_qkv_attn_prep");
    if (st != S2X_OK) return st;
    st = check_q81_input(w, qs, ds, M, "mul_mat_qkv_attn_prep");
    if (st != S2X_OK) return st;
    if (w->view.N != 3 * n_head * d_head)
        return fail(S2X_ERR_INVALID_ARG, "mul_mat_qkv_attn_prep: W has N=%lld, not 3*%lld*%lld",
                    (long long)w->view.N, (long long)n_head, (long long)d_head);
    if (n_seg > 32767 || max_len > 65535 || max_len > MAX_SEG_LEN)
        return fail(S2X_ERR_UNSUPPORTED, "mul_mat_qkv_attn_prep: n_seg or max_len too large");
    if (M > n_seg * max_len)
        return fail(S2X_ERR_INVALID_ARG, "mul_mat_qkv_attn_prep: M > n_seg * max_len");
    if (n_seg == 0 || M == 0) return S2X_OK;
    if (!qkv_bias || !seg_start_dev || !seg_len_dev || !ws)
        return fail(S2X_ERR_INVALID_ARG, "mul_mat_qkv_attn_prep: null pointer");
    const AttnLayout L = attn_layout(n_seg, max_len, n_head, d_head);
    if (ws_bytes < L.bytes)
        return fail(S2X_ERR_WORKSPACE, "mul_mat_qkv_attn_prep: workspace %zu < %zu bytes", ws_bytes,
                    L.bytes);
    if (!aligned(ws, 256)) return fail(S2X_ERR_INVALID_ARG, "mul_mat_qkv_attn_prep: ws misaligned");
    hipStream_t s = (hipStream_t)stream;
    uint8_t *base = (uint8_t *)ws;
    // padding slots zero, and rows no segment covers map to (0, 0)
    hipError_t e = launch_fill_zero(ws, L.bytes, s);
    if (e != hipSuccess) return hip_fail(e, "fill launch");
    int32_t *rowmap = reinterpret_cast<int32_t *>(base + L.rowmap_off);
    e = launch_rowmap(seg_start_dev, seg_len_dev, n_seg, max_len, rowmap, M, s);
    if (e != hipSuccess) return hip_fail(e, "rowmap launch");
    e = launch_gemm(w->view, (const int8_t *)qs, (const uint32_t *)ds, w->view.K_pad / QK_, M,
                    nullptr, 0, epi_qkv(L, ws, qkv_bias, rowmap), s);
    return e == hipSuccess ? S2X_OK : hip_fail(e, "gemm launch");
}

int s2x_attn_run(const void *ws, size_t ws_bytes, const int32_t *seg_start_dev,
                 const int32_t *seg_len_dev, const uint8_t *key_valid, int64_t n_seg,
                 int64_t max_len, int64_t n_head, int64_t d_head, float scale, float *out,
                 int64_t ld_out, void *stream) {
    int st = check_attn_shape(n_seg, max_len, n_head, d_head, "attn_run");
    if (st != S2X_OK) return st;
    if (n_seg == 0) return S2X_OK;
    const AttnLayout L = attn_layout(n_seg, max_len, n_head, d_head);
    if (!ws || !seg_start_dev || !seg_len_dev || !out)
        return fail(S2X_ERR_INVALID_ARG, "attn_run: null pointer");
    if (ws_bytes < L.bytes) return fail(S2X_ERR_WORKSPACE, "attn_run: workspace too small");
    if (ld_out < n_head * d_head || ld_out % 4 != 0 || !aligned(out, 16))
        return fail(S2X_ERR_INVALID_ARG, "attn_run: out must be 16-byte aligned, ld_out %% 4 == 0");
    hipError_t e = launch_attn(ws, seg_start_dev, seg_len_dev, key_valid, L, scale, out, ld_out,
                               (hipStream_t)stream);
    return e == hipSuccess ? S2X_OK : hip_fail(e, "attn launch");
}

int s2x_attn_run_q8_1(const void *ws, size_t ws_bytes, const int32_t *seg_start_dev,
                      const int32_t *seg_len_dev, const uint8_t *key_valid, int64_t n_seg,
                      int64_t max_len, int64_t n_head, int64_t d_head, float scale,
                      int64_t n_rows, void *qs, void *ds, int64_t ld_ds, float *out,
                      int64_t ld_out, void *stream) {
    int st = check_attn_shape(n_seg, max_len, n_head, d_head, "attn_run_q8_1");
    if (st != S2X_OK) return st;
    if (!attn_q81_fusable(n_head, d_head))
        return fail(S2X_ERR_UNSUPPORTED, "attn_run_q8_1: needs d_head 72 and n_head %% 4 == 0");
    if (n_seg == 0 || n_rows == 0) return S2X_OK;
    const AttnLayout L = attn_layout(n_seg, max_len, n_head, d_head);
    const int64_t H = n_head * d_head;
    if (!ws || !seg_start_dev || !seg_len_dev || !out || !qs || !ds || n_rows < 0)
        return fail(S2X_ERR_INVALID_ARG, "attn_run_q8_1: null pointer or negative rows");
    if (ws_bytes < L.bytes) return fail(S2X_ERR_WORKSPACE, "attn_run_q8_1: workspace too small");
    if (ld_out < H || ld_out % 4 != 0 || !aligned(out, 16) || ld_ds < H / 32 || !aligned(qs, 4) ||
        !aligned(ds, 4))
        return fail(S2X_ERR_INVALID_ARG,
                    "attn_run_q8_1: out 16-byte aligned with ld_out %% 4 == 0, ld_ds >= H / 32");
    Q81Out o;
    o.qs = reinterpret_cast<int8_t *>(qs);
    o.ds = reinterpret_cast<uint32_t *>(ds);
    o.ld_ds = ld_ds;
    hipError_t e = launch_attn(ws, seg_start_dev, seg_len_dev, key_valid, L, scale, out, ld_out,
                               (hipStream_t)stream, &o, n_rows);
    return e == hipSuccess ? S2X_OK : hip_fail(e, "attn launch");
}

int s2x_attn_fp64(const float *qkv, int64_t ld_qkv, const float *qkv_bias,
                  const int32_t *seg_start_dev, const int32_t *seg_len_dev,
                  const uint8_t *key_valid, int64_t n_seg, int64_t max_len, int64_t n_head,
                  int64_t d_head, float scale, float *out, int64_t ld_out, void *stream) {
    if (n_seg < 0 || max_len <= 0 || n_head <= 0 || d_head <= 0 || d_head > 80)
        return fail(S2X_ERR_INVALID_ARG, "attn_fp64: bad shape (d_head <= 80)");
    if (n_seg == 0) return S2X_OK;
    if (!qkv || !qkv_bias || !seg_start_dev || !seg_len_dev || !out)
        return fail(S2X_ERR_INVALID_ARG, "attn_fp64: null pointer");
    if (ld_qkv < 3 * n_head * d_head || ld_out < n_head * d_head)
        return fail(S2X_ERR_INVALID_ARG, "attn_fp64: ld_qkv < 3H or ld_out < H");
    hipError_t e = launch_attn_f64(qkv, ld_qkv, qkv_bias, seg_start_dev, seg_len_dev, key_valid,
                                   n_seg, max_len, n_head, d_head, scale, out, ld_out,
                                   (hipStream_t)stream);
    return e == hipSuccess ? S2X_OK : hip_fail(e, "attn_fp64 launch");
}

int s2x_attn_1q(const float *q, const float *k, const float *v, int64_t ld,
                const int32_t *seg_start_dev, const int32_t *seg_len_dev, int64_t n_seg,
                int64_t max_len, int64_t n_head, int64_t d_head, float scale, float *out,
                void *stream) {
    if (n_seg < 0 || max_len <= 0 || n_head <= 0 || d_head <= 0)
        return fail(S2X_ERR_INVALID_ARG, "attn_1q: bad shape");
    if (d_head > 128 || max_len > MAX_SEG_LEN || n_seg > 65535 || n_head > 65535)
        return fail(S2X_ERR_UNSUPPORTED, "attn_1q: d_head <= 128, max_len <= %lld",
                    (long long)MAX_SEG_LEN);
    if (n_seg == 0) return S2X_OK;
    if (!q || !k || !v || !seg_start_dev || !seg_len_dev || !out)
        return fail(S2X_ERR_INVALID_ARG, "attn_1q: null pointer");
    if (ld < n_head * d_head) return fail(S2X_ERR_INVALID_ARG, "attn_1q: ld < H");
    hipError_t e = launch_attn_1q(q, k, v, ld, seg_start_dev, seg_len_dev, n_seg, n_head, d_head,
                                  scale, out, (hipStream_t)stream);
    return e == hipSuccess ? S2X_OK : hip_fail(e, "attn_1q launch");
}

// ---------------------------------------------------------------------------
// a8 / a11
// ---------------------------------------------------------------------------
int s2x_resize_pos_embed(const float *pos, int64_t n_side, int64_t H, int64_t out_h,
                         int64_t out_w, float *out, void *stream) {
    if (n_side <= 0 || H <= 0 || out_h <= 0 || out_w <= 0 || !pos || !out)
        return fail(S2X_ERR_INVALID_ARG, "resize_pos_embed: bad arguments");
    if (2 * n_side > out_h * 32 || 2 * n_side > out_w * 32)
        return fail(S2X_ERR_UNSUPPORTED, "resize_pos_embed: downscale factor too large");
    hipError_t e = launch_resize_pos_embed(pos, n_side, H, out_h, out_w, out, (hipStream_t)stream);
    return e == hipSuccess ? S2X_OK : hip_fail(e, "resize launch");
}

// ---------------------------------------------------------------------------
// NaFlex front end
// ---------------------------------------------------------------------------
static int check_nf(int32_t h, int32_t w, int32_t patch, int32_t max_num_patches,
                    const char *who) {
    if (h <= 0 || w <= 0 || patch <= 0 || max_num_patches <= 0 || h > 65535 || w > 65535 ||
        patch > 256 || max_num_patches > (1 << 20))
        return fail(S2X_ERR_INVALID_ARG, "%s: bad size %dx%d, patch %d, max_num_patches %d", who,
                    h, w, patch, max_num_patches);
    return S2X_OK;
}

int s2x_nf_target_size(int32_t h, int32_t w, int32_t patch, int32_t max_num_patches,
                       int32_t *target_h, int32_t *target_w) {
    if (int st = check_nf(h, w, patch, max_num_patches, "nf_target_size")) return st;
    if (!target_h || !target_w) return fail(S2X_ERR_INVALID_ARG, "nf_target_size: null output");
    int th = 0, tw = 0;
    nf_target_size(h, w, patch, max_num_patches, &th, &tw);
    *target_h = th;
    *target_w = tw;
    return S2X_OK;
}

size_t s2x_nf_workspace_size(int32_t h, int32_t w, int32_t patch, int32_t max_num_patches) {
    if (h <= 0 || w <= 0 || patch <= 0 || max_num_patches <= 0 || h > 65535 || w > 65535 ||
        patch > 256 || max_num_patches > (1 << 20))
        return 0;
    return nf_workspace_bytes(h, w, patch, max_num_patches);
}

int s2x_nf_preprocess_rgb_dev(const uint8_t *rgb, int32_t h, int32_t w, int32_t max_num_patches,
                              int32_t patch, float rescale, const float *mean, const float *std_,
                              float *out, int64_t out_cap, int32_t *n_h, int32_t *n_w,
                              void *workspace, size_t ws_bytes, void *stream) {
    if (int st = check_nf(h, w, patch, max_num_patches, "nf_preprocess_rgb_dev")) return st;
    if (!rgb || !mean || !std_ || !out || !n_h || !n_w || !workspace)
        return fail(S2X_ERR_INVALID_ARG, "nf_preprocess_rgb_dev: null pointer");
    const size_t need = nf_workspace_bytes(h, w, patch, max_num_patches);
    if (ws_bytes < need)
        return fail(S2X_ERR_WORKSPACE, "nf_preprocess_rgb_dev: workspace %zu < %zu bytes", ws_bytes,
                    need);
    int32_t th = 0, tw = 0;
    nf_target_size(h, w, patch, max_num_patches, &th, &tw);
    const int64_t need_out = (int64_t)(th / patch) * (tw / patch) * 3 * patch * patch;
    if (out_cap < need_out)
        return fail(S2X_ERR_INVALID_ARG, "nf_preprocess_rgb_dev: out_cap %lld < %lld floats",
                    (long long)out_cap, (long long)need_out);
    int nh = 0, nw = 0;
    hipError_t e = launch_nf_preprocess(rgb, h, w, max_num_patches, patch, rescale, mean, std_,
                                        out, out_cap, &nh, &nw, workspace, ws_bytes,
                                        (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "nf_preprocess launch");
    *n_h = nh;
    *n_w = nw;
    return S2X_OK;
}

int s2x_nf_preprocess_rgb_batch_dev(const uint8_t *rgb, int32_t n_img, int32_t h, int32_t w,
                                    int32_t max_num_patches, int32_t patch, float rescale,
                                    const float *mean, const float *std_, float *out,
                                    int64_t out_cap, int32_t *n_h, int32_t *n_w, void *workspace,
                                    size_t ws_bytes, void *stream) {
    if (int st = check_nf(h, w, patch, max_num_patches, "nf_preprocess_rgb_batch_dev")) return st;
    if (n_img <= 0 || n_img > 65535)
        return fail(S2X_ERR_INVALID_ARG, "nf_preprocess_rgb_batch_dev: n_img %d not in 1..65535",
                    n_img);
    if (!rgb || !mean || !std_ || !out || !n_h || !n_w || !workspace)
        return fail(S2X_ERR_INVALID_ARG, "nf_preprocess_rgb_batch_dev: null pointer");
    const size_t need = (size_t)n_img * nf_workspace_bytes(h, w, patch, max_num_patches);
    if (ws_bytes < need)
        return fail(S2X_ERR_WORKSPACE, "nf_preprocess_rgb_batch_dev: workspace %zu < %zu bytes",
                    ws_bytes, need);
    int32_t th = 0, tw = 0;
    nf_target_size(h, w, patch, max_num_patches, &th, &tw);
    const int64_t need_out = (int64_t)(th / patch) * (tw / patch) * 3 * patch * patch;
    if (out_cap < need_out)
        return fail(S2X_ERR_INVALID_ARG,
                    "nf_preprocess_rgb_batch_dev: out_cap %lld < %lld floats per image",
                    (long long)out_cap, (long long)need_out);
    int nh = 0, nw = 0;
    hipError_t e = launch_nf_preprocess_batch(rgb, n_img, h, w, max_num_patches, patch, rescale,
                                              mean, std_, out, out_cap, &nh, &nw, workspace,
                                              ws_bytes, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "nf_preprocess_batch launch");
    *n_h = nh;
    *n_w = nw;
    return S2X_OK;
}

int s2x_get_rows_q8_0(const void *table_raw, int64_t K, int64_t n_rows_table, const int32_t *ids,
                      int64_t n_ids, const float *add, int64_t add_rows, float *out,
                      void *stream) {
    if (K <= 0 || K % QK_ != 0 || n_rows_table <= 0 || n_ids < 0 || (add && add_rows <= 0))
        return fail(S2X_ERR_INVALID_ARG, "get_rows_q8_0: bad shape");
    if (n_ids == 0) return S2X_OK;
    if (!table_raw || !ids || !out) return fail(S2X_ERR_INVALID_ARG, "get_rows_q8_0: null");
    hipError_t e = launch_get_rows_q8_0(table_raw, K, n_rows_table, ids, n_ids, add, add_rows, out,
                                        (hipStream_t)stream);
    return e == hipSuccess ? S2X_OK : hip_fail(e, "get_rows launch");
}

}  // extern "C"
