"""The GEMM's fused epilogues through the C-ABI, at the vision shapes and at
batch-32 row counts (M = 23,328 = 32 x 729): GELU -> Q8_1 re-quantization of
the fc1 output, the QKV projection written straight into the attention
staging planes, the in-place residual and the position-row residual.  Every
comparison is bit for bit: against the oracle on the rows it can afford, and
against the unfused GPU chain (GEMM to f32, then the standalone stage) on
every row."""
import ctypes

import numpy as np
import pytest
import torch

import s2x
from s2x import synth
from gpu_util import assert_same, dev, empty, host, ptr, say, stream

pytestmark = pytest.mark.gpu

N_HEAD, D_HEAD, H = 16, 72, 1152
INTER, INTER_PAD = 4304, 4320


def _quant_gpu(x, k_pad):
    M, K = x.shape
    xd = dev(x)
    qs = empty((M, k_pad), torch.int8)
    ds = empty((M, k_pad // 32, 2), torch.int16)
    s2x.call("s2x_quantize_q8_1", ptr(xd), K, M, K, k_pad, ptr(qs), ptr(ds), stream())
    return qs, ds


def _weight(raw, k_pad, n):
    w = ctypes.c_void_p()
    s2x.call("s2x_weight_create", raw.ctypes.data, 1, k_pad, n, None, ctypes.byref(w))
    return w


def _mm(w, qs, ds, M, N, epi=None, y=None):
    if y is None:
        y = empty((M, N), torch.float32)
    s2x.call("s2x_mul_mat_q8_0_q8_1", w, ptr(qs), ptr(ds), M, ptr(y), N,
             ctypes.byref(epi) if epi is not None else None, stream())
    return y


def _rows(M, n, seed):
    """n random rows plus the last 40 (the partial last row tile)."""
    r = np.random.default_rng(seed).choice(M - 40, n, replace=False)
    return np.sort(np.concatenate([r, np.arange(M - 40, M)]))


@pytest.fixture(scope="module")
def weights():
    out = {}
    for label, N, K, K_pad in [("qkv", 3 * H, H, H), ("out", H, H, H), ("fc1", INTER, H, H),
                               ("fc2", H, INTER, INTER_PAD)]:
        rng = np.random.default_rng(N * 7 + K)
        raw = synth.quantize_q8_0(rng.normal(0, 0.02, (N, K)).astype(np.float32), K_pad)
        bias = rng.normal(0, 0.5, N).astype(np.float32)
        out[label] = (raw, N, K, K_pad, bias)
    return out


# ------------------------------------------------------------ all shapes ----
@pytest.mark.timeout(300)
@pytest.mark.parametrize("label", ["qkv", "out", "fc1", "fc2"])
def test_batch32_rows_match_oracle(orc, weights, label):
    # M = 23328: 182 full 128-row tiles + one of 32 rows; sampled rows and
    # the last 40 against the oracle, bit for bit
    raw, N, K, K_pad, _ = weights[label]
    M = 32 * 729
    say(f"gemm {label} M={M}")
    x = np.random.default_rng(31).standard_normal((M, K)).astype(np.float32)
    qs, ds = _quant_gpu(x, K_pad)
    w = _weight(raw, K_pad, N)
    try:
        yg = host(_mm(w, qs, ds, M, N))
    finally:
        s2x.lib.s2x_weight_destroy(w)
    rows = _rows(M, 48, 32)
    rq, rd = orc.quantize_q8_1(x[rows], K_pad)
    assert_same(yg[rows], orc.mul_mat_q8_0_q8_1(raw, K_pad, N, rq, rd), f"{label} M={M}")


# ------------------------------------------------------- GELU -> Q8_1 -------
@pytest.mark.timeout(300)
@pytest.mark.parametrize("M", [729, 32 * 729])
def test_gelu_q81_epilogue(orc, weights, M):
    raw, N, K, K_pad, bias = weights["fc1"]
    # output columns 64..95 (one Q8_1 block): zero weights and bias -10, so
    # every row's block is GELU(-10) ~ -1.2e-37, below 127 / FLT_MAX: its
    # 127 / amax overflows and the quants saturate (-128), as the
    # reference's __float2int_rn does
    raw, bias = raw.copy(), bias.copy()
    raw[64:96] = 0
    bias[64:96] = -10.0
    say(f"fc1 GELU->Q8_1 epilogue M={M}")
    x = np.random.default_rng(33).standard_normal((M, K)).astype(np.float32)
    qs, ds = _quant_gpu(x, K_pad)
    bd = dev(bias)
    q_out = torch.full((M, INTER_PAD), 0x55, dtype=torch.int8, device="cuda:0")
    q_ds = torch.full((M, INTER_PAD // 32, 2), 0x5555, dtype=torch.int16, device="cuda:0")
    w = _weight(raw, K_pad, N)
    try:
        e = s2x.Epilogue()
        e.kind, e.bias = s2x.EPI_GELU_Q81, bd.data_ptr()
        e.q_out, e.q_ds, e.q_kpad = q_out.data_ptr(), q_ds.data_ptr(), INTER_PAD
        s2x.call("s2x_mul_mat_q8_0_q8_1", w, ptr(qs), ptr(ds), M, None, 0, ctypes.byref(e),
                 stream())
        # the unfused chain on every row: BIAS_GELU to f32, then the quantizer
        e2 = s2x.Epilogue()
        e2.kind, e2.bias = s2x.EPI_BIAS_GELU, bd.data_ptr()
        g = _mm(w, qs, ds, M, N, e2)
        q2, d2 = empty((M, INTER_PAD), torch.int8), empty((M, INTER_PAD // 32, 2), torch.int16)
        s2x.call("s2x_quantize_q8_1", ptr(g), N, M, N, INTER_PAD, ptr(q2), ptr(d2), stream())
        gq, gd = host(q_out), host(q_ds).view(np.uint16)
        assert_same(gq, host(q2), "GELU_Q81 quants vs quantize(BIAS_GELU)")
        assert_same(gd, host(d2).view(np.uint16), "GELU_Q81 scales vs quantize(BIAS_GELU)")
        assert not gq[:, N:].any()  # columns N..q_kpad-1 quantize zeros
        assert (gq[:, 64:96] == -128).all()  # the saturated block
    finally:
        s2x.lib.s2x_weight_destroy(w)
    rows = np.arange(M) if M <= 729 else _rows(M, 48, 34)
    rq, rd = orc.quantize_q8_1(x[rows], K_pad)
    ref_q, ref_d = orc.quantize_q8_1(orc.gelu(orc.mul_mat_q8_0_q8_1(raw, K_pad, N, rq, rd) + bias),
                                     INTER_PAD)
    assert_same(gq[rows], ref_q, "GELU_Q81 quants vs oracle")
    assert_same(gd[rows], ref_d, "GELU_Q81 scales vs oracle")


def test_gelu_q81_rejects_bad_arguments(weights):
    raw, N, K, K_pad, bias = weights["fc1"]
    M = 64
    x = np.random.default_rng(35).standard_normal((M, K)).astype(np.float32)
    qs, ds = _quant_gpu(x, K_pad)
    bd = dev(bias)
    q_out = empty((M * INTER_PAD + 16,), torch.int8)
    q_ds = empty((M, INTER_PAD // 32, 2), torch.int16)
    w = _weight(raw, K_pad, N)
    try:
        for kpad, off in [(INTER_PAD, 1), (4304 + 32 + 16, 0), (4288, 0), (4330, 0)]:
            e = s2x.Epilogue()
            e.kind, e.bias = s2x.EPI_GELU_Q81, bd.data_ptr()
            e.q_out, e.q_ds, e.q_kpad = q_out.data_ptr() + off, q_ds.data_ptr(), kpad
            st = s2x.lib.s2x_mul_mat_q8_0_q8_1(w, ptr(qs), ptr(ds), M, None, 0, ctypes.byref(e),
                                               stream())
            assert st == 1, (kpad, off)  # S2X_ERR_INVALID_ARG, before any launch
    finally:
        s2x.lib.s2x_weight_destroy(w)


# ----------------------------------------------- QKV -> attention planes ----
def _layout(n_seg, max_len):
    up = lambda a, b: (a + b - 1) // b * b  # noqa: E731
    d_pad, dv_pad, len_pad = up(D_HEAD, 16), up(D_HEAD, 32), up(max_len, 128)
    qk = n_seg * N_HEAD * len_pad * d_pad * 2
    vt = n_seg * N_HEAD * dv_pad * len_pad * 2
    k_off = up(qk, 256)
    vt_off = k_off + up(qk, 256)
    return dict(d_pad=d_pad, dv_pad=dv_pad, len_pad=len_pad, k_off=k_off, vt_off=vt_off,
                planes=vt_off + up(vt, 256))


def _segment_planes(L, planes, sg):
    """Q, K, V^T of segment sg (n_head x ...) cut out of the raw planes."""
    q = planes[:L["k_off"]].view(np.float16)
    k = planes[L["k_off"]:L["vt_off"]].view(np.float16)
    vt = planes[L["vt_off"]:].view(np.float16)
    lp, dp, dvp = L["len_pad"], L["d_pad"], L["dv_pad"]
    q = q.reshape(-1, N_HEAD, lp, dp)[sg]
    k = k.reshape(-1, N_HEAD, lp, dp)[sg]
    vt = vt.reshape(-1, N_HEAD, dvp, lp)[sg]
    return q, k, vt


def _expected_segment(L, y16):
    """Planes of one segment from its (length, 3H) f16 QKV rows."""
    length = y16.shape[0]
    lp, dp, dvp = L["len_pad"], L["d_pad"], L["dv_pad"]
    q = np.zeros((N_HEAD, lp, dp), np.float16)
    k = np.zeros((N_HEAD, lp, dp), np.float16)
    vt = np.zeros((N_HEAD, dvp, lp), np.float16)
    for h in range(N_HEAD):
        q[h, :length, :D_HEAD] = y16[:, h * D_HEAD:(h + 1) * D_HEAD]
        k[h, :length, :D_HEAD] = y16[:, H + h * D_HEAD:H + (h + 1) * D_HEAD]
        vt[h, :D_HEAD, :length] = y16[:, 2 * H + h * D_HEAD:2 * H + (h + 1) * D_HEAD].T
    return q, k, vt


QKV_CASES = {
    "one_729": [729],
    "naflex_4": [256, 576, 729, 1024],
    # segments shorter than, straddling and ending inside 32-row GEMM windows
    "ragged_small": [1, 64, 130, 255, 33, 729, 2],
    "batch32": [729] * 32,
}
# padded layouts: segment s starts at s * stride, so rows between a
# segment's end and the next start belong to no segment (the fused
# epilogue must store nothing for them)
QKV_STRIDES = {"gapped_padded": 128}
QKV_CASES["gapped_padded"] = [100, 128, 1, 77]


@pytest.mark.timeout(300)
@pytest.mark.parametrize("case", list(QKV_CASES))
def test_qkv_attn_prep(orc, weights, case):
    raw, N, K, K_pad, bias = weights["qkv"]
    lens = np.asarray(QKV_CASES[case], np.int32)
    if case in QKV_STRIDES:
        stride = QKV_STRIDES[case]
        starts = (np.arange(len(lens)) * stride).astype(np.int32)
        M = int(stride * (len(lens) - 1) + lens[-1])
    else:
        starts = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.int32)
        M = int(lens.sum())
    n_seg, max_len = len(lens), int(lens.max())
    say(f"QKV -> attention planes: {case}, M={M}, {n_seg} segments")
    x = np.random.default_rng(36).standard_normal((M, K)).astype(np.float32)
    qs, ds = _quant_gpu(x, K_pad)
    bd, sd, ld = dev(bias), dev(starts), dev(lens)
    wsb = s2x.lib.s2x_attn_workspace_size(n_seg, max_len, N_HEAD, D_HEAD)
    L = _layout(n_seg, max_len)
    assert wsb >= L["planes"] + n_seg * max_len * 4
    # both workspaces start as garbage: every padding slot must be written
    ws_f = torch.full((wsb,), 0x5A, dtype=torch.uint8, device="cuda:0")
    ws_u = torch.full((wsb,), 0xA5, dtype=torch.uint8, device="cuda:0")
    w = _weight(raw, K_pad, N)
    try:
        s2x.call("s2x_mul_mat_qkv_attn_prep", w, ptr(qs), ptr(ds), M, ptr(bd), ptr(sd), ptr(ld),
                 n_seg, max_len, N_HEAD, D_HEAD, ptr(ws_f), ctypes.c_size_t(wsb), stream())
        y = _mm(w, qs, ds, M, N)
        s2x.call("s2x_attn_prep", ptr(y), N, ptr(bd), ptr(sd), ptr(ld), n_seg, max_len, N_HEAD,
                 D_HEAD, ptr(ws_u), ctypes.c_size_t(wsb), stream())
        fused = host(ws_f)[:L["planes"]]
        assert_same(fused, host(ws_u)[:L["planes"]], "fused QKV planes vs GEMM + attn_prep")
    finally:
        s2x.lib.s2x_weight_destroy(w)
    # against the oracle: f16(mm + bias) placed per segment and head, zero
    # padding, for the first, the longest and the last segment
    for sg in sorted({0, int(np.argmax(lens)), n_seg - 1}):
        s, n = int(starts[sg]), int(lens[sg])
        rq, rd = orc.quantize_q8_1(x[s:s + n], K_pad)
        y16 = (orc.mul_mat_q8_0_q8_1(raw, K_pad, N, rq, rd) + bias).astype(np.float16)
        got = _segment_planes(L, fused, sg)
        for name, g, r in zip("Q K Vt".split(), got, _expected_segment(L, y16)):
            assert_same(g.view(np.uint16), r.view(np.uint16), f"{case} segment {sg} {name}")


def test_qkv_attn_prep_rejects_bad_arguments(weights):
    raw, N, K, K_pad, bias = weights["qkv"]
    lens = np.asarray([100, 50], np.int32)
    starts = np.asarray([0, 100], np.int32)
    x = np.random.default_rng(37).standard_normal((150, K)).astype(np.float32)
    qs, ds = _quant_gpu(x, K_pad)
    bd, sd, ld = dev(bias), dev(starts), dev(lens)
    wsb = s2x.lib.s2x_attn_workspace_size(2, 100, N_HEAD, D_HEAD)
    ws = empty((wsb,), torch.uint8)
    w = _weight(raw, K_pad, N)
    try:
        f = s2x.lib.s2x_mul_mat_qkv_attn_prep
        assert f(w, ptr(qs), ptr(ds), 150, ptr(bd), ptr(sd), ptr(ld), 2, 100, N_HEAD, D_HEAD,
                 ptr(ws), ctypes.c_size_t(wsb - 1), stream()) == 4   # workspace too small
        assert f(w, ptr(qs), ptr(ds), 201, ptr(bd), ptr(sd), ptr(ld), 2, 100, N_HEAD, D_HEAD,
                 ptr(ws), ctypes.c_size_t(wsb), stream()) == 1       # M > n_seg * max_len
        assert f(w, ptr(qs), ptr(ds), 150, ptr(bd), ptr(sd), ptr(ld), 2, 100, 8, D_HEAD,
                 ptr(ws), ctypes.c_size_t(wsb), stream()) == 1       # N != 3 * 8 * 72
        assert f(w, ptr(qs), ptr(ds), 150, ptr(bd), ptr(sd), ptr(ld), 2, 100, N_HEAD, D_HEAD,
                 ptr(ws), ctypes.c_size_t(wsb), stream()) == 0
    finally:
        s2x.lib.s2x_weight_destroy(w)


# ------------------------------------------------ at most 8 rows ------------
@pytest.mark.timeout(300)
@pytest.mark.parametrize("label", ["out", "fc1", "fc2"])
@pytest.mark.parametrize("M", [1, 3, 8])
def test_small_m_gemm_epilogues(orc, weights, label, M):
    # GEMMs of at most 8 rows (the pooling head's one query per image, the
    # text head) take the form that computes the block dots side by side and
    # runs each output's fma chain in one thread: plain, bias, GELU, the
    # in-place residual and (fc1) GELU -> Q8_1, against the oracle bit for
    # bit, and the plain rows equal to the same rows of a 9-row GEMM (the
    # MFMA latency form)
    raw, N, K, K_pad, bias = weights[label]
    say(f"small-M gemm {label} M={M}")
    rng = np.random.default_rng(40 + M)
    x = rng.standard_normal((9, K)).astype(np.float32)
    qs, ds = _quant_gpu(x, K_pad)  # M-row GEMMs read the first M rows of the 9
    bd = dev(bias)
    res = rng.standard_normal((M, N)).astype(np.float32)
    rdv = dev(res)
    w = _weight(raw, K_pad, N)
    try:
        yg = host(_mm(w, qs, ds, M, N))
        y9 = host(_mm(w, qs, ds, 9, N))
        e = s2x.Epilogue()
        e.kind, e.bias = s2x.EPI_BIAS, bd.data_ptr()
        yb = host(_mm(w, qs, ds, M, N, e))
        e.kind = s2x.EPI_BIAS_GELU
        yq = host(_mm(w, qs, ds, M, N, e))
        e.kind, e.resid, e.ld_resid = s2x.EPI_BIAS_RESID, rdv.data_ptr(), N
        _mm(w, qs, ds, M, N, e, rdv)  # in place on the residual rows
        yr = host(rdv)
        if label == "fc1":
            q_out = torch.full((M, INTER_PAD), 0x55, dtype=torch.int8, device="cuda:0")
            q_ds = torch.full((M, INTER_PAD // 32, 2), 0x5555, dtype=torch.int16, device="cuda:0")
            e = s2x.Epilogue()
            e.kind, e.bias = s2x.EPI_GELU_Q81, bd.data_ptr()
            e.q_out, e.q_ds, e.q_kpad = q_out.data_ptr(), q_ds.data_ptr(), INTER_PAD
            s2x.call("s2x_mul_mat_q8_0_q8_1", w, ptr(qs), ptr(ds), M, None, 0, ctypes.byref(e),
                     stream())
            gq, gd = host(q_out), host(q_ds).view(np.uint16)
    finally:
        s2x.lib.s2x_weight_destroy(w)
    rq, rd = orc.quantize_q8_1(x[:M], K_pad)
    ref = orc.mul_mat_q8_0_q8_1(raw, K_pad, N, rq, rd)
    assert_same(yg, ref, f"{label} M={M} plain vs oracle")
    assert_same(yg, y9[:M], f"{label} M={M} plain vs the 9-row GEMM")
    assert_same(yb, ref + bias, f"{label} M={M} bias")
    assert_same(yq, orc.gelu(ref + bias), f"{label} M={M} bias + GELU")
    assert_same(yr, (ref + bias) + res, f"{label} M={M} in-place residual")
    if label == "fc1":
        ref_q, ref_d = orc.quantize_q8_1(orc.gelu(ref + bias), INTER_PAD)
        assert_same(gq, ref_q, f"fc1 M={M} GELU_Q81 quants")
        assert_same(gd, ref_d, f"fc1 M={M} GELU_Q81 scales")


# ------------------------------------------------------------- residuals ----
@pytest.mark.timeout(300)
@pytest.mark.parametrize("M", [729, 32 * 729])
@pytest.mark.parametrize("kind", ["inplace", "pos_rows"])
def test_residual_epilogues_h1152(orc, weights, kind, M):
    # the out-projection / fc2 tail: y = (acc + bias) + r, r the residual
    # stream updated in place, or position rows repeated every 729 rows
    raw, N, K, K_pad, bias = weights["out"]
    say(f"residual epilogue {kind} M={M}")
    rng = np.random.default_rng(38)
    x = rng.standard_normal((M, K)).astype(np.float32)
    qs, ds = _quant_gpu(x, K_pad)
    bd = dev(bias)
    if kind == "inplace":
        res = rng.standard_normal((M, N)).astype(np.float32)
        rdv = dev(res)
        y, r_rows = rdv, 0
    else:
        res = rng.standard_normal((729, N)).astype(np.float32)
        rdv = dev(res)
        y, r_rows = empty((M, N), torch.float32), 729
    w = _weight(raw, K_pad, N)
    try:
        mm = host(_mm(w, qs, ds, M, N))
        e = s2x.Epilogue()
        e.kind, e.bias, e.resid, e.ld_resid, e.resid_rows = (s2x.EPI_BIAS_RESID, bd.data_ptr(),
                                                             rdv.data_ptr(), N, r_rows)
        _mm(w, qs, ds, M, N, e, y)
        yg = host(y)
    finally:
        s2x.lib.s2x_weight_destroy(w)
    rr = res if r_rows == 0 else res[np.arange(M) % 729]
    assert_same(yg, (mm + bias) + rr, f"residual {kind} M={M} vs GEMM + numpy tail")
    rows = np.arange(M) if M <= 729 else _rows(M, 32, 39)
    rq, rd = orc.quantize_q8_1(x[rows], K_pad)
    assert_same(mm[rows], orc.mul_mat_q8_0_q8_1(raw, K_pad, N, rq, rd), f"GEMM rows M={M}")


# --------------------------------------------- F16 weights (ffn_down) -------
def _f16_terms_abs(w16, x):
    xh = np.abs(x.astype(np.float16).astype(np.float64))
    return xh @ np.abs(w16.astype(np.float64)).T


@pytest.mark.timeout(300)
@pytest.mark.parametrize("M", [1, 333, 729, 32 * 729])
def test_mul_mat_f16_matches_oracle(orc, M):
    # the converter's F16 ffn_down: K = 4304 (not a multiple of 32), N = 1152
    from gpu_util import h5_rel
    K, N = INTER, H
    rng = np.random.default_rng(50)
    w16 = (rng.standard_normal((N, K)) * 0.02).astype(np.float16)
    x = rng.standard_normal((M, K)).astype(np.float32)
    say(f"F16 mul_mat M={M}")
    wd, xd = dev(w16.view(np.uint16)), dev(x)
    wsb = s2x.lib.s2x_mul_mat_f16_workspace_size(K, N, M)
    ws = empty((wsb,), torch.uint8)
    y = empty((M, N), torch.float32)
    s2x.call("s2x_mul_mat_f16_f32", ptr(wd), K, N, ptr(xd), K, M, ptr(y), ptr(ws),
             ctypes.c_size_t(wsb), stream())
    yg = host(y)
    rows = np.arange(M) if M <= 729 else _rows(M, 48, 51)
    ref = orc.mul_mat_f16_f32(w16, x[rows])
    rel = h5_rel(yg[rows], ref.astype(np.float64), _f16_terms_abs(w16, x[rows]))
    say(f"  max rel err (tau = 1e-3 rms) {rel:.2e}")
    assert rel <= 1e-4
    assert s2x.lib.s2x_mul_mat_f16_f32(ptr(wd), K, N, ptr(xd), K, M, ptr(y), ptr(ws),
                                       ctypes.c_size_t(wsb - 1), stream()) == 4


@pytest.mark.parametrize("M", [729, 32 * 729])
def test_gelu_f16_epilogue(orc, weights, M):
    # fc1 with its output rounded to f16 for an F16 ffn_down: bit for bit
    # f16(gelu(mm + b)) of the oracle, columns 4304..4319 zero
    raw, N, K, K_pad, bias = weights["fc1"]
    say(f"fc1 GELU->f16 epilogue M={M}")
    x = np.random.default_rng(52).standard_normal((M, K)).astype(np.float32)
    qs, ds = _quant_gpu(x, K_pad)
    bd = dev(bias)
    h = torch.full((M, INTER_PAD), 7.0, dtype=torch.float16, device="cuda:0")
    w = _weight(raw, K_pad, N)
    try:
        e = s2x.Epilogue()
        e.kind, e.bias = s2x.EPI_GELU_F16, bd.data_ptr()
        e.q_out, e.q_kpad = h.data_ptr(), INTER_PAD
        s2x.call("s2x_mul_mat_q8_0_q8_1", w, ptr(qs), ptr(ds), M, None, 0, ctypes.byref(e),
                 stream())
        hg = host(h)
    finally:
        s2x.lib.s2x_weight_destroy(w)
    assert not hg[:, N:].view(np.uint16).any()
    rows = np.arange(M) if M <= 729 else _rows(M, 48, 53)
    rq, rd = orc.quantize_q8_1(x[rows], K_pad)
    ref = orc.gelu(orc.mul_mat_q8_0_q8_1(raw, K_pad, N, rq, rd) + bias).astype(np.float16)
    assert_same(hg[rows, :N].view(np.uint16), ref.view(np.uint16), "GELU_F16 vs oracle")
