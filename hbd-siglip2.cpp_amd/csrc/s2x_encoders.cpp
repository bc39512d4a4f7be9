// s2x_encoders.cpp -- the SigLIP2 vision and text towers on the gfx950
// kernels, behind the s2x_vision_* / s2x_text_* C-ABI.
//
// Graph (src/siglip2_vision.cpp:181-244, 601-758; src/siglip2_text.cpp:
// 115-205, 564-932), restated as a fixed launch sequence per block:
//   LN1+Q8_1 -> QKV GEMM -> attention staging (bias, f16, V^T) -> flash
//   attention -> Q8_1 -> O GEMM (+bias +residual, in place) -> LN2+Q8_1 ->
//   FC1 GEMM (+bias, GELU) -> Q8_1 (K padded 4304 -> 4320) -> FC2 GEMM
//   (+bias +residual, in place)
// Tokens of all images are packed into one row range (M = sum of patch
// counts); attention runs per image segment, so a batch of 32 images is one
// GEMM of M = 23328 rows per weight.
#include <hip/hip_runtime.h>

#include <cmath>
#include <algorithm>
#include <cstring>
#include <map>
#include <utility>
#include <vector>

#include "s2x.h"
#include "s2x_internal.h"
#include "s2x_kernels.h"

namespace s2x {

#define S2X_HIP_TRY(expr)                                       \
    do {                                                        \
        hipError_t e__ = (expr);                                \
        if (e__ != hipSuccess) return hip_fail(e__, #expr);     \
    } while (0)

#define S2X_TRY(expr)                                           \
    do {                                                        \
        int s__ = (expr);                                       \
        if (s__ != S2X_OK) return s__;                          \
    } while (0)

int weight_upload(const void *raw, bool is_host, int64_t K_pad, int64_t N, hipStream_t stream,
                  s2x_weight **out) {
    *out = nullptr;
    const size_t raw_bytes = (size_t)(N * (K_pad / QK_)) * 34;
    const void *src = raw;
    void *tmp = nullptr;
    if (is_host) {
        if (hipMalloc(&tmp, raw_bytes) != hipSuccess)
            return fail(S2X_ERR_OOM, "weight upload: hipMalloc(%zu) failed", raw_bytes);
        hipError_t e = hipMemcpy(tmp, raw, raw_bytes, hipMemcpyHostToDevice);
        if (e != hipSuccess) {
            (void)hipFree(tmp);
            return hip_fail(e, "weight upload copy");
        }
        src = tmp;
    }
    void *planes = nullptr;
    if (hipMalloc(&planes, weight_planes_bytes(K_pad, N)) != hipSuccess) {
        if (tmp) (void)hipFree(tmp);
        return fail(S2X_ERR_OOM, "weight upload: hipMalloc planes failed");
    }
    s2x_weight *w = new s2x_weight();
    w->mem = planes;
    w->owns = true;
    w->view = planes_view(planes, K_pad, N);
    hipError_t e = repack_into(src, w->view, stream);
    if (e == hipSuccess && tmp) e = hipStreamSynchronize(stream);
    if (tmp) (void)hipFree(tmp);
    if (e != hipSuccess) {
        (void)hipFree(planes);
        delete w;
        return hip_fail(e, "weight repack");
    }
    *out = w;
    return S2X_OK;
}

namespace {

struct DevBuf {
    void *p = nullptr;
    size_t n = 0;
    ~DevBuf() {
        if (p) (void)hipFree(p);
    }
    template <class T> T *as() const { return reinterpret_cast<T *>(p); }
};

// Encodes of at most this many packed rows run as HIP graph replays, of up
// to GRAPH_CACHE distinct shapes per encoder.
constexpr int64_t GRAPH_MAX_ROWS = 8192;
constexpr size_t GRAPH_CACHE = 4;

// Grow a device buffer; waits for `stream` before releasing the old one.
int ensure(DevBuf &b, size_t bytes, hipStream_t stream) {
    if (b.n >= bytes && b.p) return S2X_OK;
    if (b.p) {
        S2X_HIP_TRY(hipStreamSynchronize(stream));
        (void)hipFree(b.p);
        b.p = nullptr;
        b.n = 0;
    }
    const size_t n = (size_t)round_up_i((int64_t)bytes, 4096);
    if (hipMalloc(&b.p, n) != hipSuccess) {
        b.p = nullptr;
        return fail(S2X_ERR_OOM, "hipMalloc(%zu) failed", n);
    }
    b.n = n;
    return S2X_OK;
}

int upload_f32(const float *host, int64_t n, float **dev, const char *what) {
    *dev = nullptr;
    if (!host) return fail(S2X_ERR_INVALID_ARG, "missing tensor %s", what);
    if (hipMalloc(reinterpret_cast<void **>(dev), sizeof(float) * (size_t)n) != hipSuccess)
        return fail(S2X_ERR_OOM, "hipMalloc for %s failed", what);
    S2X_HIP_TRY(hipMemcpy(*dev, host, sizeof(float) * (size_t)n, hipMemcpyHostToDevice));
    return S2X_OK;
}

int upload_q8(const void *raw, int64_t K_pad, int64_t N, hipStream_t s, s2x_weight **w,
              const char *what) {
    if (!raw) return fail(S2X_ERR_INVALID_ARG, "missing tensor %s", what);
    return weight_upload(raw, true, K_pad, N, s, w);
}

// F16 matrix (N rows of K halves, host) -> device rows of K_pad halves, zero
// past K
int upload_f16(const void *raw, int64_t K, int64_t K_pad, int64_t N, _Float16 **dev,
               const char *what) {
    *dev = nullptr;
    if (!raw) return fail(S2X_ERR_INVALID_ARG, "missing tensor %s", what);
    const size_t bytes = sizeof(_Float16) * (size_t)(N * K_pad);
    if (hipMalloc(reinterpret_cast<void **>(dev), bytes) != hipSuccess)
        return fail(S2X_ERR_OOM, "hipMalloc for %s failed", what);
    S2X_HIP_TRY(hipMemset(*dev, 0, bytes));
    S2X_HIP_TRY(hipMemcpy2D(*dev, (size_t)K_pad * 2, raw, (size_t)K * 2, (size_t)K * 2, (size_t)N,
                            hipMemcpyHostToDevice));
    return S2X_OK;
}

// ffn_down: a Q8_0 weight, or F16 rows (the converter's type for K % 32 != 0)
struct DownW {
    s2x_weight *q8 = nullptr;
    _Float16 *f16 = nullptr;  // N rows of K_pad halves
    void release() {
        s2x_weight_destroy(q8);
        if (f16) (void)hipFree(f16);
    }
    int upload(const void *raw, bool as_f16, int64_t K, int64_t K_pad, int64_t N, hipStream_t s,
               const char *what) {
        return as_f16 ? upload_f16(raw, K, K_pad, N, &f16, what) : upload_q8(raw, K_pad, N, s, &q8, what);
    }
};

struct DevLayer {
    s2x_weight *qkv = nullptr, *o = nullptr, *up = nullptr;
    DownW down;
    float *ln1_w = nullptr, *ln1_b = nullptr, *qkv_b = nullptr, *o_b = nullptr;
    float *ln2_w = nullptr, *ln2_b = nullptr, *up_b = nullptr, *down_b = nullptr;
    void release() {
        s2x_weight_destroy(qkv);
        s2x_weight_destroy(o);
        s2x_weight_destroy(up);
        down.release();
        for (float *p : {ln1_w, ln1_b, qkv_b, o_b, ln2_w, ln2_b, up_b, down_b})
            if (p) (void)hipFree(p);
    }
};

// hipEvent pairs around GEMM launches, for the roofline report
struct GemmTiming {
    bool on = false;
    struct Rec {
        hipEvent_t a, b;
        double ops;
    };
    std::vector<Rec> pending;
    std::vector<hipEvent_t> pool;
    double ms = 0.0, ops = 0.0;
    int64_t launches = 0;
    hipEvent_t get() {
        if (!pool.empty()) {
            hipEvent_t e = pool.back();
            pool.pop_back();
            return e;
        }
        hipEvent_t e = nullptr;
        (void)hipEventCreate(&e);
        return e;
    }
    int collect(hipStream_t s) {
        if (pending.empty()) return S2X_OK;
        S2X_HIP_TRY(hipStreamSynchronize(s));
        for (auto &r : pending) {
            float t = 0.0f;
            S2X_HIP_TRY(hipEventElapsedTime(&t, r.a, r.b));
            ms += t;
            ops += r.ops;
            launches += 1;
            pool.push_back(r.a);
            pool.push_back(r.b);
        }
        pending.clear();
        return S2X_OK;
    }
    ~GemmTiming() {
        for (auto &r : pending) {
            (void)hipEventDestroy(r.a);
            (void)hipEventDestroy(r.b);
        }
        for (auto e : pool) (void)hipEventDestroy(e);
    }
};

// The transformer stack shared by both towers.
struct Tower {
    int64_t H = 0, F = 0, F_pad = 0, n_head = 0, d_head = 0, n_layer = 0;
    float eps = 1e-6f;
    std::vector<DevLayer> layers;
    hipStream_t own = nullptr, stream = nullptr;
    // x: residual stream f32 [M][H]; qs / ds: Q8_1 of the current GEMM input
    // ([M][kmax] int8, [M][kmax/32] ds words); qs2 / ds2: the fc1 epilogue's
    // Q8_1 output (fc2 input, K = F_pad); h16: its f16 output instead, for
    // an F16 ffn_down ([M][F_pad] halves)
    DevBuf x, qs, ds, qs2, ds2, h16, qkv, att, attn_ws, seg, rowmap, part;
    bool down_f16 = false;
    GemmTiming timing;
    // attention in fp64 (k_attn_f64, from an f32 QKV GEMM output) instead of
    // the f16-MFMA flash kernel fed by the QKV GEMM's attention-layout epilogue
    bool attn_f64 = false;
    // K-split GEMMs (launch_gemm_split_k) for the plain and residual
    // epilogues, an option of both towers for encodes of few rows (text
    // prompts, one image), whose long-K GEMMs (fc2: 135 blocks) otherwise
    // get only tens of workgroups.  The split is a function of K, so an
    // input's bits do not depend on the batch it is in (with the option set
    // the same way); off by default, since the sums' new order moves a
    // 27-layer random-weight embedding to cosine ~0.9999 against the
    // block-order oracle.
    bool split_k = false;
    int splits(int64_t KB, const EpiParams &e) const {
        if (!split_k || (e.kind != EPI_NONE && e.kind != EPI_BIAS_RESID) || e.resid_rows != 0)
            return 1;
        return KB >= 96 ? 4 : KB >= 32 ? 2 : 1;
    }
    // HIP graphs of recent encodes' launch sequences (see launch_seq)
    bool graphs = true;
    struct GraphEntry {
        std::vector<int64_t> key;
        hipGraphExec_t exec = nullptr;  // null: seen once, not captured yet
    };
    std::vector<GraphEntry> gcache;  // most recently used last

    ~Tower() {
        for (auto &g : gcache)
            if (g.exec) (void)hipGraphExecDestroy(g.exec);
        for (auto &L : layers) L.release();
        if (own) (void)hipStreamDestroy(own);
    }

    // Launch-bound encodes (M <= GRAPH_MAX_ROWS: batch 1, text prompts) run
    // ~250 short kernels whose launch gaps are a large share of the time.
    // body() issues an encode's kernels on `stream` and nothing else (no
    // allocation, copy from host memory or synchronisation: every buffer it
    // uses is already sized).  The first call with a given key runs body()
    // as it is; the second call with that key captures body() into a HIP
    // graph and launches it; later calls replay the graph.  Up to
    // GRAPH_CACHE keys are kept (least recently used dropped), as the
    // reference's encoders cache one graph per shape.  The key holds every
    // size and device address the kernels take (the caller's and the
    // tower's buffers), so a replay launches exactly the kernels, arguments
    // and order that body() would.
    template <class Body>
    int launch_seq(std::vector<int64_t> key, int64_t M, Body &&body) {
        if (!graphs || timing.on || M > GRAPH_MAX_ROWS || stream == nullptr) return body();
        for (const DevBuf *b : {&x, &qs, &ds, &qs2, &ds2, &h16, &qkv, &att, &attn_ws, &seg, &rowmap, &part})
            key.push_back((int64_t)(uintptr_t)b->p);
        key.push_back((int64_t)(uintptr_t)stream);
        key.push_back(attn_f64);
        key.push_back(split_k);
        size_t i = 0;
        while (i < gcache.size() && gcache[i].key != key) ++i;
        if (i == gcache.size()) {  // first call with this key
            if (gcache.size() >= GRAPH_CACHE) {
                if (gcache.front().exec) {
                    S2X_HIP_TRY(hipStreamSynchronize(stream));
                    (void)hipGraphExecDestroy(gcache.front().exec);
                }
                gcache.erase(gcache.begin());
            }
            gcache.push_back({key, nullptr});
            return body();
        }
        GraphEntry g = gcache[i];
        gcache.erase(gcache.begin() + (long)i);
        if (!g.exec) {
            S2X_HIP_TRY(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal));
            const int st = body();
            hipGraph_t gr = nullptr;
            const hipError_t e = hipStreamEndCapture(stream, &gr);
            if (st != S2X_OK || e != hipSuccess) {
                if (gr) (void)hipGraphDestroy(gr);
                return st != S2X_OK ? st : hip_fail(e, "graph capture");
            }
            const hipError_t ei = hipGraphInstantiate(&g.exec, gr, nullptr, nullptr, 0);
            (void)hipGraphDestroy(gr);
            if (ei != hipSuccess) return hip_fail(ei, "graph instantiate");
        }
        gcache.push_back(g);
        S2X_HIP_TRY(hipGraphLaunch(g.exec, stream));
        return S2X_OK;
    }

    int init_stream() {
        S2X_HIP_TRY(hipStreamCreateWithFlags(&own, hipStreamNonBlocking));
        stream = own;
        return S2X_OK;
    }

    int load_layers(const s2x_layer_weights *lw, int64_t n) {
        if (!lw) return fail(S2X_ERR_INVALID_ARG, "layers array is null");
        layers.resize((size_t)n);
        for (int64_t l = 0; l < n; ++l) {
            const s2x_layer_weights &s = lw[l];
            DevLayer &d = layers[(size_t)l];
            S2X_TRY(upload_f32(s.ln1_w, H, &d.ln1_w, "ln1.weight"));
            S2X_TRY(upload_f32(s.ln1_b, H, &d.ln1_b, "ln1.bias"));
            S2X_TRY(upload_q8(s.qkv_w, H, 3 * H, stream, &d.qkv, "attn_qkv.weight"));
            S2X_TRY(upload_f32(s.qkv_b, 3 * H, &d.qkv_b, "attn_qkv.bias"));
            S2X_TRY(upload_q8(s.o_w, H, H, stream, &d.o, "attn_o.weight"));
            S2X_TRY(upload_f32(s.o_b, H, &d.o_b, "attn_o.bias"));
            S2X_TRY(upload_f32(s.ln2_w, H, &d.ln2_w, "ln2.weight"));
            S2X_TRY(upload_f32(s.ln2_b, H, &d.ln2_b, "ln2.bias"));
            S2X_TRY(upload_q8(s.up_w, H, F, stream, &d.up, "ffn_up.weight"));
            S2X_TRY(upload_f32(s.up_b, F, &d.up_b, "ffn_up.bias"));
            S2X_TRY(d.down.upload(s.down_w, down_f16, F, F_pad, H, stream, "ffn_down.weight"));
            S2X_TRY(upload_f32(s.down_b, H, &d.down_b, "ffn_down.bias"));
        }
        return S2X_OK;
    }

    // GEMM over the Q8_1 rows in qs / ds (or qs2 / ds2), with optional event
    // timing; k_logical excludes the K padding.
    int gemm(const s2x_weight *w, int64_t M, float *y, int64_t ldy, const EpiParams &e,
             int64_t k_logical, bool from_qs2 = false) {
        const DevBuf &xq = from_qs2 ? qs2 : qs, &xd = from_qs2 ? ds2 : ds;
        hipEvent_t a = nullptr, b = nullptr;
        if (timing.on) {
            a = timing.get();
            b = timing.get();
            S2X_HIP_TRY(hipEventRecord(a, stream));
        }
        const int ns = splits(w->view.K_pad / QK_, e);
        const hipError_t err =
            ns > 1 ? launch_gemm_split_k(w->view, xq.as<int8_t>(), xd.as<uint32_t>(),
                                         w->view.K_pad / QK_, M, y, ldy, e, ns, part.as<float>(), stream)
                   : launch_gemm(w->view, xq.as<int8_t>(), xd.as<uint32_t>(), w->view.K_pad / QK_,
                                 M, y, ldy, e, stream);
        if (err != hipSuccess) return hip_fail(err, "gemm launch");
        if (timing.on) {
            S2X_HIP_TRY(hipEventRecord(b, stream));
            timing.pending.push_back({a, b, 2.0 * (double)M * (double)w->view.N * (double)k_logical});
        }
        return S2X_OK;
    }

    // The MLP of a block or of the MAP head on M rows whose LN2 + Q8_1 is in
    // qs / ds: fc1 (+bias, GELU, and Q8_1 -- or f16 for an F16 ffn_down --
    // of the result), then fc2 (+bias + resid) into y.
    int ffn(const s2x_weight *up, const float *up_b, const DownW &down, const float *down_b,
            int64_t M, float *y, const float *resid) {
        if (down.f16) {
            EpiParams ep{EPI_GELU_F16, up_b, nullptr, 0, 0, 0};
            ep.h_out = h16.as<_Float16>();
            ep.h_ld = ep.h_kpad = F_pad;
            S2X_TRY(gemm(up, M, nullptr, 0, ep, H));
            const hipError_t e = launch_gemm_f16(down.f16, F_pad, H, h16.as<_Float16>(), M, y, H,
                                                 EpiParams{EPI_BIAS_RESID, down_b, resid, H, 0, 0},
                                                 stream);
            return e == hipSuccess ? S2X_OK : hip_fail(e, "f16 gemm launch");
        }
        EpiParams ep{EPI_GELU_Q81, up_b, nullptr, 0, 0, 0};
        ep.q_out8 = qs2.as<int8_t>();
        ep.q_ds = ds2.as<uint32_t>();
        ep.q_kpad = F_pad;
        ep.q_ldds = F_pad / QK_;
        S2X_TRY(gemm(up, M, nullptr, 0, ep, H));
        return gemm(down.q8, M, y, H, EpiParams{EPI_BIAS_RESID, down_b, resid, H, 0, 0}, F, true);
    }

    // Q8_1 planes of the GEMM input buffers for rows of K_pad values
    Q81Out qout(int64_t K_pad) {
        Q81Out o;
        o.qs = qs.as<int8_t>();
        o.ds = ds.as<uint32_t>();
        o.ld_ds = K_pad / QK_;
        return o;
    }

    int quantize(const float *src, int64_t K, int64_t M, int64_t ldx, int64_t K_pad) {
        hipError_t e = launch_quantize_q8_1(src, K, M, ldx, K_pad, qout(K_pad), stream);
        return e == hipSuccess ? S2X_OK : hip_fail(e, "quantize launch");
    }

    int layernorm_q(const float *src, int64_t M, const float *w, const float *b, float *y) {
        const Q81Out o = qout(H);
        hipError_t e = launch_layernorm(src, H, M, H, w, b, eps, &o, y, H, stream);
        return e == hipSuccess ? S2X_OK : hip_fail(e, "layernorm launch");
    }

    // Buffers for M packed rows; kmax: the widest GEMM input (patch_dim for
    // the vision patch embedding).
    int reserve(int64_t M, int64_t n_seg, int64_t max_len, int64_t kmax_in = 0) {
        const int64_t kmax = std::max<int64_t>(H, kmax_in);
        S2X_TRY(ensure(x, sizeof(float) * (size_t)(M * H), stream));
        S2X_TRY(ensure(qs, (size_t)(M * kmax), stream));
        S2X_TRY(ensure(ds, sizeof(uint32_t) * (size_t)(M * (kmax / QK_)), stream));
        if (down_f16) {
            S2X_TRY(ensure(h16, sizeof(_Float16) * (size_t)(M * F_pad), stream));
        } else {
            S2X_TRY(ensure(qs2, (size_t)(M * F_pad), stream));
            S2X_TRY(ensure(ds2, sizeof(uint32_t) * (size_t)(M * (F_pad / QK_)), stream));
        }
        S2X_TRY(ensure(att, sizeof(float) * (size_t)(M * H), stream));
        if (attn_f64)
            S2X_TRY(ensure(qkv, sizeof(float) * (size_t)(M * 3 * H), stream));
        else
            S2X_TRY(ensure(attn_ws, attn_layout(n_seg, max_len, n_head, d_head).bytes, stream));
        S2X_TRY(ensure(seg, sizeof(int32_t) * (size_t)(2 * n_seg), stream));
        S2X_TRY(ensure(rowmap, sizeof(int32_t) * (size_t)M, stream));
        // partial sums of a split GEMM: at most 4 x H (fc2) or 2 x 3 H (QKV)
        if (split_k) S2X_TRY(ensure(part, sizeof(float) * (size_t)(M * 6 * H), stream));
        return S2X_OK;
    }

    // The attention workspace's padding slots (d_head..d_pad of Q / K rows,
    // positions past a segment's length) must hold zeros; the QKV GEMM
    // epilogue writes real slots only, so the workspace is cleared whenever
    // its layout or address changes.
    void *attn_zeroed_at = nullptr;
    int64_t attn_zeroed_key[3] = {-1, -1, -1};
    int attn_ws_ready(const AttnLayout &AL) {
        const int64_t key[3] = {AL.n_seg, AL.len_pad, AL.n_head};
        if (attn_zeroed_at == attn_ws.p && std::equal(key, key + 3, attn_zeroed_key)) return S2X_OK;
        hipError_t e = launch_fill_zero(attn_ws.p, AL.planes_bytes, stream);
        if (e != hipSuccess) return hip_fail(e, "fill launch");
        attn_zeroed_at = attn_ws.p;
        std::copy(key, key + 3, attn_zeroed_key);
        return S2X_OK;
    }

    // Upload the segment table (starts then lengths) to `seg` and build the
    // row map; skipped when the table is the one already there (steady-state
    // batches stay asynchronous).
    std::vector<int32_t> seg_host;
    void *seg_dev_at = nullptr, *rowmap_at = nullptr;
    int64_t rowmap_rows = -1;
    int set_segments(const std::vector<int32_t> &start, const std::vector<int32_t> &len, int64_t M) {
        const size_t n = start.size();
        std::vector<int32_t> tab(2 * n);
        std::memcpy(tab.data(), start.data(), n * 4);
        std::memcpy(tab.data() + n, len.data(), n * 4);
        if (tab == seg_host && seg_dev_at == seg.p && rowmap_at == rowmap.p && rowmap_rows == M)
            return S2X_OK;
        S2X_HIP_TRY(hipMemcpyAsync(seg.p, tab.data(), 8 * n, hipMemcpyHostToDevice, stream));
        S2X_HIP_TRY(hipStreamSynchronize(stream));  // `tab` is pageable host memory
        const int64_t max_len = n ? *std::max_element(len.begin(), len.end()) : 0;
        hipError_t e = launch_rowmap(seg_start(), seg_len((int64_t)n), (int64_t)n, max_len,
                                     rowmap.as<int32_t>(), M, stream);
        if (e != hipSuccess) return hip_fail(e, "rowmap launch");
        seg_host = std::move(tab);
        seg_dev_at = seg.p;
        rowmap_at = rowmap.p;
        rowmap_rows = M;
        return S2X_OK;
    }
    const int32_t *seg_start() const { return seg.as<int32_t>(); }
    const int32_t *seg_len(int64_t n_seg) const { return seg.as<int32_t>() + n_seg; }

    // The encoder blocks in place on x (M packed rows, n_seg segments):
    //   LN1+Q8_1 -> QKV GEMM -> attention -> Q8_1 (folded into the flash
    //   attention for 72-wide heads in groups of four) -> O GEMM (+bias +residual,
    //   in place) -> LN2+Q8_1 -> FC1 GEMM (+bias, GELU, Q8_1 of the result
    //   with K padded to F_pad) -> FC2 GEMM (+bias +residual, in place)
    // The QKV GEMM writes the flash kernel's operands itself (EPI_QKV); with
    // fp64 attention it writes f32 rows for k_attn_f64 instead.
    int run_layers(int64_t M, int64_t n_seg, int64_t max_len, const uint8_t *key_valid) {
        const AttnLayout AL = attn_layout(n_seg, max_len, n_head, d_head);
        const float kq_scale = 1.0f / std::sqrt((float)d_head);
        float *xp = x.as<float>();
        if (!attn_f64) S2X_TRY(attn_ws_ready(AL));
        hipError_t e;
        for (auto &L : layers) {
            S2X_TRY(layernorm_q(xp, M, L.ln1_w, L.ln1_b, nullptr));
            if (attn_f64) {
                S2X_TRY(gemm(L.qkv, M, qkv.as<float>(), 3 * H,
                             EpiParams{EPI_NONE, nullptr, nullptr, 0, 0, 0}, H));
                e = launch_attn_f64(qkv.as<float>(), 3 * H, L.qkv_b, seg_start(), seg_len(n_seg),
                                    key_valid, n_seg, max_len, n_head, d_head, kq_scale,
                                    att.as<float>(), H, stream);
                if (e != hipSuccess) return hip_fail(e, "attn_f64 launch");
            } else {
                S2X_TRY(gemm(L.qkv, M, nullptr, 0, epi_qkv(AL, attn_ws.p, L.qkv_b, rowmap.as<int32_t>()), H));
                if (attn_q81_fusable(n_head, d_head)) {
                    // the out-projection's Q8_1 input straight from attention
                    const Q81Out o = qout(H);
                    e = launch_attn(attn_ws.p, seg_start(), seg_len(n_seg), key_valid, AL, kq_scale,
                                    att.as<float>(), H, stream, &o, M);
                    if (e != hipSuccess) return hip_fail(e, "attn launch");
                    S2X_TRY(gemm(L.o, M, xp, H, EpiParams{EPI_BIAS_RESID, L.o_b, xp, H, 0, 0}, H));
                    S2X_TRY(layernorm_q(xp, M, L.ln2_w, L.ln2_b, nullptr));
                    S2X_TRY(ffn(L.up, L.up_b, L.down, L.down_b, M, xp, xp));
                    continue;
                }
                e = launch_attn(attn_ws.p, seg_start(), seg_len(n_seg), key_valid, AL, kq_scale,
                                att.as<float>(), H, stream);
                if (e != hipSuccess) return hip_fail(e, "attn launch");
            }
            S2X_TRY(quantize(att.as<float>(), H, M, H, H));
            S2X_TRY(gemm(L.o, M, xp, H, EpiParams{EPI_BIAS_RESID, L.o_b, xp, H, 0, 0}, H));
            S2X_TRY(layernorm_q(xp, M, L.ln2_w, L.ln2_b, nullptr));
            S2X_TRY(ffn(L.up, L.up_b, L.down, L.down_b, M, xp, xp));
        }
        return S2X_OK;
    }
};

int check_dims(int64_t H, int64_t F, int64_t F_pad, int64_t n_head, int64_t n_layer) {
    if (H <= 0 || H % 32 != 0 || H > 2048 || n_head <= 0 || H % n_head != 0 || n_layer < 0 ||
        F <= 0 || F_pad < F || F_pad % 32 != 0 || F_pad - F >= 32)
        return fail(S2X_ERR_INVALID_ARG, "bad config H=%lld F=%lld F_pad=%lld heads=%lld layers=%lld",
                    (long long)H, (long long)F, (long long)F_pad, (long long)n_head,
                    (long long)n_layer);
    const int64_t dh = H / n_head;
    if (dh < 65 || dh > 80 || dh % 4 != 0)
        return fail(S2X_ERR_UNSUPPORTED, "head dim %lld unsupported (attention kernel: 65..80, %%4)",
                    (long long)dh);
    return S2X_OK;
}

}  // namespace
}  // namespace s2x

using namespace s2x;

// ---------------------------------------------------------------------------
// vision
// ---------------------------------------------------------------------------
struct s2x_vision {
    Tower t;
    int64_t patch_dim = 0, n_side = 0;
    s2x_weight *patch = nullptr, *hkv = nullptr, *ho = nullptr, *hup = nullptr;
    DownW hdown;
    float *patch_b = nullptr, *pos_embd = nullptr, *post_ln_w = nullptr, *post_ln_b = nullptr;
    float *probe_q = nullptr, *hkv_b = nullptr, *ho_b = nullptr, *hln_w = nullptr,
          *hln_b = nullptr, *hup_b = nullptr, *hdown_b = nullptr;
    std::vector<std::pair<std::pair<int, int>, float *>> pos_cache;  // LRU of resized grids
    DevBuf pix, pos_packed, kv, hq, ha, hout, hid, nf_ws;

    ~s2x_vision() {
        for (s2x_weight *w : {patch, hkv, ho, hup}) s2x_weight_destroy(w);
        hdown.release();
        for (float *p : {patch_b, pos_embd, post_ln_w, post_ln_b, probe_q, hkv_b, ho_b, hln_w,
                         hln_b, hup_b, hdown_b})
            if (p) (void)hipFree(p);
        for (auto &e : pos_cache) (void)hipFree(e.second);
    }

    // position embeddings for an n_h x n_w grid (cached, LRU of 4 shapes)
    int pos_for(int n_h, int n_w, const float **out) {
        if (n_h == n_side && n_w == n_side) {
            *out = pos_embd;
            return S2X_OK;
        }
        for (size_t i = 0; i < pos_cache.size(); ++i)
            if (pos_cache[i].first == std::make_pair(n_h, n_w)) {
                auto e = pos_cache[i];
                pos_cache.erase(pos_cache.begin() + (long)i);
                pos_cache.push_back(e);
                *out = e.second;
                return S2X_OK;
            }
        if (pos_cache.size() >= 4) {
            S2X_HIP_TRY(hipStreamSynchronize(t.stream));
            (void)hipFree(pos_cache.front().second);
            pos_cache.erase(pos_cache.begin());
        }
        float *buf = nullptr;
        if (hipMalloc(reinterpret_cast<void **>(&buf), sizeof(float) * (size_t)(n_h * n_w * t.H)) != hipSuccess)
            return fail(S2X_ERR_OOM, "pos cache alloc");
        hipError_t e = launch_resize_pos_embed(pos_embd, n_side, t.H, n_h, n_w, buf, t.stream);
        if (e != hipSuccess) {
            (void)hipFree(buf);
            return hip_fail(e, "resize launch");
        }
        pos_cache.push_back({{n_h, n_w}, buf});
        *out = buf;
        return S2X_OK;
    }

    // launch_seq key of an encode: its path, sizes, the device addresses it
    // reads and writes, and the vision tower's own buffers
    std::vector<int64_t> seq_key(int64_t path, int64_t M, int64_t n_img, int64_t max_len,
                                 int32_t pooling, const void *in, const void *out_dev,
                                 const void *pos) const {
        std::vector<int64_t> k{path, M, n_img, max_len, pooling, (int64_t)(uintptr_t)in,
                               (int64_t)(uintptr_t)out_dev, (int64_t)(uintptr_t)pos};
        for (const DevBuf *b : {&pix, &pos_packed, &kv, &hq, &ha, &hid})
            k.push_back((int64_t)(uintptr_t)b->p);
        return k;
    }

    // After the packed, position-embedded patch rows are in t.x: the blocks,
    // post-LN and pooling into out_dev [n_img][H].
    int tail(int64_t M, int64_t n_img, int64_t max_len, int32_t pooling, float *out_dev) {
        const int64_t H = t.H;
        S2X_TRY(t.run_layers(M, n_img, max_len, nullptr));
        if (pooling == S2X_POOL_MEAN) {
            S2X_TRY(ensure(hid, sizeof(float) * (size_t)(M * H), t.stream));
            hipError_t e = launch_layernorm(t.x.as<float>(), H, M, H, post_ln_w, post_ln_b, t.eps,
                                            nullptr, hid.as<float>(), H, t.stream);
            if (e != hipSuccess) return hip_fail(e, "post-LN launch");
            e = launch_mean_pool(hid.as<float>(), H, t.seg_start(), t.seg_len(n_img), n_img,
                                 out_dev, t.stream);
            return e == hipSuccess ? S2X_OK : hip_fail(e, "mean pool launch");
        }
        // MAP probe head (src/siglip2_vision.cpp:249-314)
        S2X_TRY(t.layernorm_q(t.x.as<float>(), M, post_ln_w, post_ln_b, nullptr));
        S2X_TRY(ensure(kv, sizeof(float) * (size_t)(M * 2 * H), t.stream));
        S2X_TRY(ensure(hq, sizeof(float) * (size_t)(n_img * H), t.stream));
        S2X_TRY(ensure(ha, sizeof(float) * (size_t)(n_img * H), t.stream));
        S2X_TRY(t.gemm(hkv, M, kv.as<float>(), 2 * H, EpiParams{EPI_BIAS, hkv_b, nullptr, 0, 0, 0}, H));
        hipError_t e = launch_attn_1q(probe_q, kv.as<float>(), kv.as<float>() + H, 2 * H,
                                      t.seg_start(), t.seg_len(n_img), n_img, t.n_head, t.d_head,
                                      1.0f / std::sqrt((float)t.d_head), hq.as<float>(), t.stream);
        if (e != hipSuccess) return hip_fail(e, "probe attention launch");
        S2X_TRY(t.quantize(hq.as<float>(), H, n_img, H, H));
        S2X_TRY(t.gemm(ho, n_img, ha.as<float>(), H, EpiParams{EPI_BIAS, ho_b, nullptr, 0, 0, 0}, H));
        S2X_TRY(t.layernorm_q(ha.as<float>(), n_img, hln_w, hln_b, nullptr));
        return t.ffn(hup, hup_b, hdown, hdown_b, n_img, out_dev, ha.as<float>());
    }
};

extern "C" {

int s2x_vision_create(const s2x_vision_weights *w, s2x_vision **out) {
    if (!out) return fail(S2X_ERR_INVALID_ARG, "vision_create: out is null");
    *out = nullptr;
    if (!w) return fail(S2X_ERR_INVALID_ARG, "vision_create: weights are null");
    S2X_TRY(check_dims(w->hidden, w->inter, w->inter_pad, w->n_head, w->n_layer));
    if (w->patch_dim <= 0 || w->patch_dim % 32 != 0 || w->n_side <= 0)
        return fail(S2X_ERR_INVALID_ARG, "vision_create: bad patch_dim/n_side");
    if (w->down_f16 != 0 && w->down_f16 != 1)
        return fail(S2X_ERR_INVALID_ARG, "vision_create: down_f16 must be 0 or 1");
    s2x_vision *v = new s2x_vision();
    Tower &t = v->t;
    t.H = w->hidden;
    t.F = w->inter;
    t.F_pad = w->inter_pad;
    t.n_head = w->n_head;
    t.d_head = t.H / t.n_head;
    t.n_layer = w->n_layer;
    t.eps = w->eps;
    t.down_f16 = w->down_f16 != 0;
    v->patch_dim = w->patch_dim;
    v->n_side = w->n_side;
    auto bail = [&](int st) {
        delete v;
        return st;
    };
    int st = t.init_stream();
    if (st) return bail(st);
    const int64_t H = t.H, F = t.F, F_pad = t.F_pad;
    hipStream_t s = t.stream;
    if ((st = upload_q8(w->patch_w, v->patch_dim, H, s, &v->patch, "patch_embd.weight")) ||
        (st = upload_f32(w->patch_b, H, &v->patch_b, "patch_embd.bias")) ||
        (st = upload_f32(w->pos_embd, v->n_side * v->n_side * H, &v->pos_embd, "position_embd")) ||
        (st = upload_f32(w->post_ln_w, H, &v->post_ln_w, "post_ln.weight")) ||
        (st = upload_f32(w->post_ln_b, H, &v->post_ln_b, "post_ln.bias")) ||
        (st = t.load_layers(w->layers, w->n_layer)))
        return bail(st);
    // probe head: K and V projections share one GEMM (rows [k; v])
    if (!w->hk_w || !w->hv_w || !w->hk_b || !w->hv_b || !w->probe || !w->hq_w || !w->hq_b)
        return bail(fail(S2X_ERR_INVALID_ARG, "vision_create: probe head tensors missing"));
    {
        const size_t rb = (size_t)(H * (H / QK_)) * 34;
        std::vector<uint8_t> kvraw(2 * rb);
        std::memcpy(kvraw.data(), w->hk_w, rb);
        std::memcpy(kvraw.data() + rb, w->hv_w, rb);
        std::vector<float> kvb(2 * (size_t)H);
        std::memcpy(kvb.data(), w->hk_b, sizeof(float) * (size_t)H);
        std::memcpy(kvb.data() + H, w->hv_b, sizeof(float) * (size_t)H);
        if ((st = upload_q8(kvraw.data(), H, 2 * H, s, &v->hkv, "head.attn_kv")) ||
            (st = upload_f32(kvb.data(), 2 * H, &v->hkv_b, "head.attn_kv.bias")))
            return bail(st);
    }
    if ((st = upload_q8(w->ho_w, H, H, s, &v->ho, "head.attn_o.weight")) ||
        (st = upload_f32(w->ho_b, H, &v->ho_b, "head.attn_o.bias")) ||
        (st = upload_f32(w->hln_w, H, &v->hln_w, "head.ln.weight")) ||
        (st = upload_f32(w->hln_b, H, &v->hln_b, "head.ln.bias")) ||
        (st = upload_q8(w->hup_w, H, F, s, &v->hup, "head.ffn_up.weight")) ||
        (st = upload_f32(w->hup_b, F, &v->hup_b, "head.ffn_up.bias")) ||
        (st = v->hdown.upload(w->hdown_w, t.down_f16, F, F_pad, H, s, "head.ffn_down.weight")) ||
        (st = upload_f32(w->hdown_b, H, &v->hdown_b, "head.ffn_down.bias")))
        return bail(st);
    // The probe query is image independent: q = mm(W_q, probe) + b_q, once.
    {
        s2x_weight *hq = nullptr;
        float *probe = nullptr, *hq_b = nullptr;
        if ((st = upload_q8(w->hq_w, H, H, s, &hq, "head.attn_q.weight")) ||
            (st = upload_f32(w->probe, H, &probe, "head.probe")) ||
            (st = upload_f32(w->hq_b, H, &hq_b, "head.attn_q.bias"))) {
            s2x_weight_destroy(hq);
            if (probe) (void)hipFree(probe);
            if (hq_b) (void)hipFree(hq_b);
            return bail(st);
        }
        if (hipMalloc(reinterpret_cast<void **>(&v->probe_q), sizeof(float) * (size_t)H) != hipSuccess)
            st = fail(S2X_ERR_OOM, "probe_q alloc");
        if (!st) st = ensure(t.qs, (size_t)H, s);
        if (!st) st = ensure(t.ds, sizeof(uint32_t) * (size_t)(H / QK_), s);
        if (!st) st = t.quantize(probe, H, 1, H, H);
        if (!st) st = t.gemm(hq, 1, v->probe_q, H, EpiParams{EPI_BIAS, hq_b, nullptr, 0, 0, 0}, H);
        if (!st && hipStreamSynchronize(s) != hipSuccess) st = fail(S2X_ERR_HIP, "probe sync");
        s2x_weight_destroy(hq);
        (void)hipFree(probe);
        (void)hipFree(hq_b);
        if (st) return bail(st);
    }
    if (hipStreamSynchronize(s) != hipSuccess) return bail(fail(S2X_ERR_HIP, "create sync"));
    *out = v;
    return S2X_OK;
}

void s2x_vision_destroy(s2x_vision *v) {
    if (!v) return;
    (void)hipStreamSynchronize(v->t.stream);
    delete v;
}

int s2x_vision_set_stream(s2x_vision *v, void *stream) {
    if (!v) return fail(S2X_ERR_NOT_LOADED, "vision: not created");
    v->t.stream = stream ? (hipStream_t)stream : v->t.own;
    return S2X_OK;
}

int s2x_vision_set_attention_fp64(s2x_vision *v, int enable) {
    if (!v) return fail(S2X_ERR_NOT_LOADED, "vision: not created");
    v->t.attn_f64 = enable != 0;
    return S2X_OK;
}

int s2x_vision_set_split_k(s2x_vision *v, int enable) {
    if (!v) return fail(S2X_ERR_NOT_LOADED, "vision: not created");
    v->t.split_k = enable != 0;
    return S2X_OK;
}

int s2x_vision_set_graphs(s2x_vision *v, int enable) {
    if (!v) return fail(S2X_ERR_NOT_LOADED, "vision: not created");
    v->t.graphs = enable != 0;
    return S2X_OK;
}

int s2x_vision_encode_batch_dev(s2x_vision *v, const float *pixels_dev, int32_t n_img, int32_t n_h,
                                int32_t n_w, int32_t pooling, float *out_dev) {
    if (!v) return fail(S2X_ERR_NOT_LOADED, "vision: not created");
    if (n_img <= 0 || n_h <= 0 || n_w <= 0 || !pixels_dev || !out_dev ||
        (pooling != S2X_POOL_MEAN && pooling != S2X_POOL_PROBE))
        return fail(S2X_ERR_INVALID_ARG, "vision_encode_batch: bad arguments");
    const int64_t n_pos = (int64_t)n_h * n_w;
    if (n_pos > MAX_SEG_LEN) return fail(S2X_ERR_UNSUPPORTED, "vision: more than 4096 patches");
    Tower &t = v->t;
    const int64_t M = n_pos * n_img;
    S2X_TRY(t.reserve(M, n_img, n_pos, v->patch_dim));
    std::vector<int32_t> st((size_t)n_img), ln((size_t)n_img, (int32_t)n_pos);
    for (int i = 0; i < n_img; ++i) st[(size_t)i] = (int32_t)(i * n_pos);
    S2X_TRY(t.set_segments(st, ln, M));
    const float *pos = nullptr;
    S2X_TRY(v->pos_for(n_h, n_w, &pos));
    return t.launch_seq(v->seq_key(1, M, n_img, n_pos, pooling, pixels_dev, out_dev, pos), M, [&] {
        S2X_TRY(t.quantize(pixels_dev, v->patch_dim, M, v->patch_dim, v->patch_dim));
        S2X_TRY(t.gemm(v->patch, M, t.x.as<float>(), t.H,
                       EpiParams{EPI_BIAS_RESID, v->patch_b, pos, t.H, n_pos, 0}, v->patch_dim));
        return v->tail(M, n_img, n_pos, pooling, out_dev);
    });
}

int s2x_vision_encode(s2x_vision *v, const float *pixels_host, int32_t n_h, int32_t n_w,
                      int32_t pooling, float *out_host) {
    if (!v) return fail(S2X_ERR_NOT_LOADED, "vision: not created");
    if (!pixels_host || !out_host || n_h <= 0 || n_w <= 0)
        return fail(S2X_ERR_INVALID_ARG, "vision_encode: bad arguments");
    const size_t pix_bytes = sizeof(float) * (size_t)((int64_t)n_h * n_w * v->patch_dim);
    S2X_TRY(ensure(v->pix, pix_bytes, v->t.stream));
    S2X_TRY(ensure(v->hout, sizeof(float) * (size_t)v->t.H, v->t.stream));
    S2X_HIP_TRY(hipMemcpyAsync(v->pix.p, pixels_host, pix_bytes, hipMemcpyHostToDevice, v->t.stream));
    S2X_TRY(s2x_vision_encode_batch_dev(v, v->pix.as<float>(), 1, n_h, n_w, pooling, v->hout.as<float>()));
    S2X_HIP_TRY(hipMemcpyAsync(out_host, v->hout.p, sizeof(float) * (size_t)v->t.H,
                               hipMemcpyDeviceToHost, v->t.stream));
    S2X_HIP_TRY(hipStreamSynchronize(v->t.stream));
    return S2X_OK;
}

int s2x_vision_encode_ragged_dev(s2x_vision *v, const float *pixels_dev,
                                 const int32_t *shapes_host, int32_t n_img, int32_t max_patches,
                                 int32_t pooling, float *out_dev) {
    if (!v) return fail(S2X_ERR_NOT_LOADED, "vision: not created");
    if (n_img <= 0 || max_patches <= 0 || !pixels_dev || !shapes_host || !out_dev ||
        (pooling != S2X_POOL_MEAN && pooling != S2X_POOL_PROBE))
        return fail(S2X_ERR_INVALID_ARG, "vision_encode_ragged: bad arguments");
    if (max_patches > MAX_SEG_LEN)
        return fail(S2X_ERR_UNSUPPORTED, "vision: more than 4096 patches");
    Tower &t = v->t;
    std::vector<int32_t> st((size_t)n_img), ln((size_t)n_img);
    int64_t M = 0, max_len = 0;
    for (int i = 0; i < n_img; ++i) {
        const int32_t h = shapes_host[2 * i], w = shapes_host[2 * i + 1];
        if (h <= 0 || w <= 0 || (int64_t)h * w > max_patches)
            return fail(S2X_ERR_INVALID_ARG, "vision_encode_ragged: image %d shape %dx%d invalid", i, h, w);
        st[(size_t)i] = (int32_t)M;
        ln[(size_t)i] = h * w;
        M += (int64_t)h * w;
        if (h * w > max_len) max_len = h * w;
    }
    S2X_TRY(t.reserve(M, n_img, max_len, v->patch_dim));
    S2X_TRY(t.set_segments(st, ln, M));
    S2X_TRY(ensure(v->pix, sizeof(float) * (size_t)(M * v->patch_dim), t.stream));
    S2X_TRY(ensure(v->pos_packed, sizeof(float) * (size_t)(M * t.H), t.stream));
    hipError_t e = launch_pack_rows(pixels_dev, v->patch_dim, max_patches, t.seg_start(),
                                    t.seg_len(n_img), n_img, v->pix.as<float>(), t.stream);
    if (e != hipSuccess) return hip_fail(e, "pack launch");
    for (int i = 0; i < n_img; ++i) {
        const float *pos = nullptr;
        S2X_TRY(v->pos_for(shapes_host[2 * i], shapes_host[2 * i + 1], &pos));
        S2X_HIP_TRY(hipMemcpyAsync(v->pos_packed.as<float>() + (int64_t)st[(size_t)i] * t.H, pos,
                                   sizeof(float) * (size_t)(ln[(size_t)i] * t.H),
                                   hipMemcpyDeviceToDevice, t.stream));
    }
    return t.launch_seq(v->seq_key(2, M, n_img, max_len, pooling, nullptr, out_dev, nullptr), M, [&] {
        S2X_TRY(t.quantize(v->pix.as<float>(), v->patch_dim, M, v->patch_dim, v->patch_dim));
        S2X_TRY(t.gemm(v->patch, M, t.x.as<float>(), t.H,
                       EpiParams{EPI_BIAS_RESID, v->patch_b, v->pos_packed.as<float>(), t.H, 0, 0},
                       v->patch_dim));
        return v->tail(M, n_img, max_len, pooling, out_dev);
    });
}

int s2x_vision_encode_rgb_batch_dev(s2x_vision *v, const uint8_t *const *rgb_dev,
                                    const int32_t *hw_host, int32_t n_img,
                                    int32_t max_num_patches, float rescale, const float *mean,
                                    const float *std_, int32_t pooling, float *out_dev) {
    if (!v) return fail(S2X_ERR_NOT_LOADED, "vision: not created");
    if (n_img <= 0 || max_num_patches <= 0 || !rgb_dev || !hw_host || !mean || !std_ ||
        !out_dev || (pooling != S2X_POOL_MEAN && pooling != S2X_POOL_PROBE))
        return fail(S2X_ERR_INVALID_ARG, "vision_encode_rgb_batch: bad arguments");
    if (max_num_patches > MAX_SEG_LEN)
        return fail(S2X_ERR_UNSUPPORTED, "vision: more than 4096 patches");
    int p = 1;
    while (3 * p * p < v->patch_dim) ++p;
    if (3 * p * p != v->patch_dim)
        return fail(S2X_ERR_UNSUPPORTED, "vision_encode_rgb_batch: patch_dim %lld is not 3*p*p",
                    (long long)v->patch_dim);
    Tower &t = v->t;
    std::vector<int32_t> st((size_t)n_img), ln((size_t)n_img), shp(2 * (size_t)n_img);
    int64_t M = 0, max_len = 0;
    size_t ws_bytes = 0;
    for (int i = 0; i < n_img; ++i) {
        const int32_t h = hw_host[2 * i], w = hw_host[2 * i + 1];
        if (h <= 0 || w <= 0 || h > 65535 || w > 65535 || !rgb_dev[i])
            return fail(S2X_ERR_INVALID_ARG, "vision_encode_rgb_batch: image %d (%dx%d) invalid", i, h, w);
        int th = 0, tw = 0;
        nf_target_size(h, w, p, max_num_patches, &th, &tw);
        shp[2 * (size_t)i] = th / p;
        shp[2 * (size_t)i + 1] = tw / p;
        st[(size_t)i] = (int32_t)M;
        ln[(size_t)i] = (th / p) * (tw / p);
        M += ln[(size_t)i];
        max_len = std::max<int64_t>(max_len, ln[(size_t)i]);
        ws_bytes = std::max(ws_bytes, nf_workspace_bytes(h, w, p, max_num_patches));
    }
    if (max_len > MAX_SEG_LEN) return fail(S2X_ERR_UNSUPPORTED, "vision: more than 4096 patches");
    S2X_TRY(t.reserve(M, n_img, max_len, v->patch_dim));
    S2X_TRY(t.set_segments(st, ln, M));
    S2X_TRY(ensure(v->pix, sizeof(float) * (size_t)(M * v->patch_dim), t.stream));
    S2X_TRY(ensure(v->pos_packed, sizeof(float) * (size_t)(M * t.H), t.stream));
    S2X_TRY(ensure(v->nf_ws, ws_bytes, t.stream));
    // each image's patches land straight in its packed row range
    for (int i = 0; i < n_img; ++i) {
        int nh = 0, nw = 0;
        hipError_t e = launch_nf_preprocess(
            rgb_dev[i], hw_host[2 * i], hw_host[2 * i + 1], max_num_patches, p, rescale, mean,
            std_, v->pix.as<float>() + (int64_t)st[(size_t)i] * v->patch_dim,
            (int64_t)ln[(size_t)i] * v->patch_dim, &nh, &nw, v->nf_ws.p, ws_bytes, t.stream);
        if (e != hipSuccess) return hip_fail(e, "nf_preprocess launch");
        const float *pos = nullptr;
        S2X_TRY(v->pos_for(nh, nw, &pos));
        S2X_HIP_TRY(hipMemcpyAsync(v->pos_packed.as<float>() + (int64_t)st[(size_t)i] * t.H, pos,
                                   sizeof(float) * (size_t)(ln[(size_t)i] * t.H),
                                   hipMemcpyDeviceToDevice, t.stream));
    }
    return t.launch_seq(v->seq_key(2, M, n_img, max_len, pooling, nullptr, out_dev, nullptr), M, [&] {
        S2X_TRY(t.quantize(v->pix.as<float>(), v->patch_dim, M, v->patch_dim, v->patch_dim));
        S2X_TRY(t.gemm(v->patch, M, t.x.as<float>(), t.H,
                       EpiParams{EPI_BIAS_RESID, v->patch_b, v->pos_packed.as<float>(), t.H, 0, 0},
                       v->patch_dim));
        return v->tail(M, n_img, max_len, pooling, out_dev);
    });
}

int s2x_vision_gemm_timing(s2x_vision *v, int enable) {
    if (!v) return fail(S2X_ERR_NOT_LOADED, "vision: not created");
    S2X_TRY(v->t.timing.collect(v->t.stream));
    v->t.timing.on = enable != 0;
    return S2X_OK;
}

int s2x_vision_gemm_stats(s2x_vision *v, double *ms, double *ops, int64_t *launches, int reset) {
    if (!v) return fail(S2X_ERR_NOT_LOADED, "vision: not created");
    S2X_TRY(v->t.timing.collect(v->t.stream));
    if (ms) *ms = v->t.timing.ms;
    if (ops) *ops = v->t.timing.ops;
    if (launches) *launches = v->t.timing.launches;
    if (reset) {
        v->t.timing.ms = 0.0;
        v->t.timing.ops = 0.0;
        v->t.timing.launches = 0;
    }
    return S2X_OK;
}

}  // extern "C"

// ---------------------------------------------------------------------------
// text
// ---------------------------------------------------------------------------
struct s2x_text {
    Tower t;
    int64_t vocab = 0, max_pos = 0, proj = 0;
    void *tok = nullptr;  // raw Q8_0 token table (device)
    float *pos_embd = nullptr, *fln_w = nullptr, *fln_b = nullptr, *head_b = nullptr;
    s2x_weight *head = nullptr;
    DevBuf ids, rows, pooled, out, kv8;
    ~s2x_text() {
        s2x_weight_destroy(head);
        for (void *p : {tok, (void *)pos_embd, (void *)fln_w, (void *)fln_b, (void *)head_b})
            if (p) (void)hipFree(p);
    }

    // n_batch prompts of n_tok ids already in `ids`; out_host n_batch*proj
    int run(int32_t n_tok, int32_t n_batch, const uint8_t *key_valid_dev, float *out_host) {
        const int64_t H = t.H, M = (int64_t)n_tok * n_batch;
        std::vector<int32_t> st((size_t)n_batch), ln((size_t)n_batch, n_tok), last((size_t)n_batch);
        for (int b = 0; b < n_batch; ++b) {
            st[(size_t)b] = b * n_tok;
            last[(size_t)b] = b * n_tok + n_tok - 1;
        }
        S2X_TRY(t.set_segments(st, ln, M));
        S2X_TRY(ensure(rows, sizeof(int32_t) * (size_t)n_batch, t.stream));
        S2X_TRY(ensure(pooled, sizeof(float) * (size_t)(n_batch * H), t.stream));
        S2X_TRY(ensure(out, sizeof(float) * (size_t)(n_batch * proj), t.stream));
        S2X_HIP_TRY(hipMemcpyAsync(rows.p, last.data(), 4 * (size_t)n_batch, hipMemcpyHostToDevice, t.stream));
        const std::vector<int64_t> key{3, n_tok, n_batch, (int64_t)(uintptr_t)key_valid_dev,
                                       (int64_t)(uintptr_t)ids.p, (int64_t)(uintptr_t)rows.p,
                                       (int64_t)(uintptr_t)pooled.p, (int64_t)(uintptr_t)out.p};
        S2X_TRY(t.launch_seq(key, M, [&] {
            hipError_t e = launch_get_rows_q8_0(tok, H, vocab, ids.as<int32_t>(), M, pos_embd, n_tok,
                                                t.x.as<float>(), t.stream);
            if (e != hipSuccess) return hip_fail(e, "get_rows launch");
            S2X_TRY(t.run_layers(M, n_batch, n_tok, key_valid_dev));
            e = launch_layernorm(t.x.as<float>(), H, M, H, fln_w, fln_b, t.eps, nullptr,
                                 t.x.as<float>(), H, t.stream);
            if (e != hipSuccess) return hip_fail(e, "final LN launch");
            e = launch_gather_rows(t.x.as<float>(), H, rows.as<int32_t>(), n_batch, pooled.as<float>(), t.stream);
            if (e != hipSuccess) return hip_fail(e, "gather launch");
            S2X_TRY(t.quantize(pooled.as<float>(), H, n_batch, H, H));
            return t.gemm(head, n_batch, out.as<float>(), proj, EpiParams{EPI_BIAS, head_b, nullptr, 0, 0, 0}, H);
        }));
        S2X_HIP_TRY(hipMemcpyAsync(out_host, out.p, sizeof(float) * (size_t)(n_batch * proj),
                                   hipMemcpyDeviceToHost, t.stream));
        S2X_HIP_TRY(hipStreamSynchronize(t.stream));
        return S2X_OK;
    }

    int put_ids(const int32_t *ids_host, int64_t n) {
        for (int64_t i = 0; i < n; ++i)
            if (ids_host[i] < 0 || ids_host[i] >= vocab)
                return fail(S2X_ERR_INVALID_ARG, "token id %d out of range [0, %lld)", ids_host[i],
                            (long long)vocab);
        S2X_TRY(ensure(ids, sizeof(int32_t) * (size_t)n, t.stream));
        S2X_HIP_TRY(hipMemcpyAsync(ids.p, ids_host, 4 * (size_t)n, hipMemcpyHostToDevice, t.stream));
        S2X_HIP_TRY(hipStreamSynchronize(t.stream));
        return S2X_OK;
    }
};

extern "C" {

int s2x_text_create(const s2x_text_weights *w, s2x_text **out) {
    if (!out) return fail(S2X_ERR_INVALID_ARG, "text_create: out is null");
    *out = nullptr;
    if (!w) return fail(S2X_ERR_INVALID_ARG, "text_create: weights are null");
    S2X_TRY(check_dims(w->hidden, w->inter, w->inter_pad, w->n_head, w->n_layer));
    if (w->vocab <= 0 || w->max_pos <= 0 || w->proj <= 0 || !w->tok_embd)
        return fail(S2X_ERR_INVALID_ARG, "text_create: bad vocab/max_pos/proj");
    if (w->down_f16 != 0 && w->down_f16 != 1)
        return fail(S2X_ERR_INVALID_ARG, "text_create: down_f16 must be 0 or 1");
    s2x_text *x = new s2x_text();
    Tower &t = x->t;
    t.H = w->hidden;
    t.F = w->inter;
    t.F_pad = w->inter_pad;
    t.n_head = w->n_head;
    t.d_head = t.H / t.n_head;
    t.n_layer = w->n_layer;
    t.eps = w->eps;
    t.down_f16 = w->down_f16 != 0;
    x->vocab = w->vocab;
    x->max_pos = w->max_pos;
    x->proj = w->proj;
    // short prompts: exact-order fp64 attention (k_attn_f64_short), whose
    // embeddings stay the oracle's to cosine 0.99999+; the flash kernel's
    // f32 scores shift the 27-layer text embedding to ~0.99988
    t.attn_f64 = true;
    auto bail = [&](int st) {
        delete x;
        return st;
    };
    int st = t.init_stream();
    if (st) return bail(st);
    const size_t tok_bytes = (size_t)(x->vocab * (t.H / QK_)) * 34;
    if (hipMalloc(&x->tok, tok_bytes) != hipSuccess) return bail(fail(S2X_ERR_OOM, "token table alloc"));
    if (hipMemcpy(x->tok, w->tok_embd, tok_bytes, hipMemcpyHostToDevice) != hipSuccess)
        return bail(fail(S2X_ERR_HIP, "token table upload"));
    if ((st = upload_f32(w->pos_embd, x->max_pos * t.H, &x->pos_embd, "position_embd")) ||
        (st = upload_f32(w->final_ln_w, t.H, &x->fln_w, "final_ln.weight")) ||
        (st = upload_f32(w->final_ln_b, t.H, &x->fln_b, "final_ln.bias")) ||
        (st = upload_q8(w->head_w, t.H, x->proj, t.stream, &x->head, "head.weight")) ||
        (st = upload_f32(w->head_b, x->proj, &x->head_b, "head.bias")) ||
        (st = t.load_layers(w->layers, w->n_layer)))
        return bail(st);
    if (hipStreamSynchronize(t.stream) != hipSuccess) return bail(fail(S2X_ERR_HIP, "create sync"));
    *out = x;
    return S2X_OK;
}

void s2x_text_destroy(s2x_text *x) {
    if (!x) return;
    (void)hipStreamSynchronize(x->t.stream);
    delete x;
}

int s2x_text_set_stream(s2x_text *x, void *stream) {
    if (!x) return fail(S2X_ERR_NOT_LOADED, "text: not created");
    x->t.stream = stream ? (hipStream_t)stream : x->t.own;
    return S2X_OK;
}

int s2x_text_set_attention_fp64(s2x_text *x, int enable) {
    if (!x) return fail(S2X_ERR_NOT_LOADED, "text: not created");
    x->t.attn_f64 = enable != 0;
    return S2X_OK;
}

int s2x_text_set_split_k(s2x_text *x, int enable) {
    if (!x) return fail(S2X_ERR_NOT_LOADED, "text: not created");
    x->t.split_k = enable != 0;
    return S2X_OK;
}

int s2x_text_set_graphs(s2x_text *x, int enable) {
    if (!x) return fail(S2X_ERR_NOT_LOADED, "text: not created");
    x->t.graphs = enable != 0;
    return S2X_OK;
}

int s2x_text_encode(s2x_text *x, const int32_t *ids_host, int32_t n_tok, const int32_t *mask_host,
                    float *out_host) {
    if (!x) return fail(S2X_ERR_NOT_LOADED, "text: not created");
    if (!ids_host || !out_host || n_tok <= 0 || n_tok > x->max_pos)
        return fail(S2X_ERR_INVALID_ARG, "n_tokens must be in (0, %lld], got %d",
                    (long long)x->max_pos, n_tok);
    S2X_TRY(x->t.reserve(n_tok, 1, n_tok));
    S2X_TRY(x->put_ids(ids_host, n_tok));
    const uint8_t *kv = nullptr;
    if (mask_host) {
        std::vector<uint8_t> m((size_t)n_tok);
        for (int i = 0; i < n_tok; ++i) m[(size_t)i] = mask_host[i] != 0;
        S2X_TRY(ensure(x->kv8, (size_t)n_tok, x->t.stream));
        S2X_HIP_TRY(hipMemcpyAsync(x->kv8.p, m.data(), (size_t)n_tok, hipMemcpyHostToDevice, x->t.stream));
        S2X_HIP_TRY(hipStreamSynchronize(x->t.stream));
        kv = x->kv8.as<uint8_t>();
    }
    return x->run(n_tok, 1, kv, out_host);
}

int s2x_text_encode_batch(s2x_text *x, const int32_t *ids_host, int32_t n_tok, int32_t n_batch,
                          float *out_host) {
    if (!x) return fail(S2X_ERR_NOT_LOADED, "text: not created");
    if (n_batch <= 0) return fail(S2X_ERR_INVALID_ARG, "n_batch must be > 0");
    if (!ids_host || !out_host || n_tok <= 0 || n_tok > x->max_pos)
        return fail(S2X_ERR_INVALID_ARG, "n_tokens must be in (0, %lld], got %d",
                    (long long)x->max_pos, n_tok);
    const int64_t M = (int64_t)n_tok * n_batch;
    S2X_TRY(x->t.reserve(M, n_batch, n_tok));
    S2X_TRY(x->put_ids(ids_host, M));
    return x->run(n_tok, n_batch, nullptr, out_host);
}

}  // extern "C"
