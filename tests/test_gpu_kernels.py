"""Kernel-level parity on the GPU, through the C-ABI, against the CPU oracle
on identical seeded inputs.  Integer/byte stages are compared bit for bit."""
import ctypes

import numpy as np
import pytest
import torch

import s2x
from s2x import synth
from gpu_util import assert_same, cos, dev, empty, host, ptr, say, stream, zeros

pytestmark = pytest.mark.gpu

SHAPES = [  # (label, N, K, K_pad) -- the vision layer GEMMs
    ("qkv", 3456, 1152, 1152),
    ("out", 1152, 1152, 1152),
    ("fc1", 4304, 1152, 1152),
    ("fc2", 1152, 4304, 4320),
]


def _quant_gpu(x, k_pad):
    M, K = x.shape
    xd = dev(x)
    qs = empty((M, k_pad), torch.int8)
    ds = empty((M, k_pad // 32, 2), torch.int16)
    s2x.call("s2x_quantize_q8_1", ptr(xd), K, M, K, k_pad, ptr(qs), ptr(ds), stream())
    return qs, ds


@pytest.mark.parametrize("M,K,K_pad", [(729, 1152, 1152), (23328, 1152, 1152), (729, 4304, 4320),
                                       (100, 768, 768), (1, 1152, 1152), (3, 32, 64)])
def test_quantize_q8_1_bit_exact(orc, M, K, K_pad):
    say(f"quantize M={M} K={K} K_pad={K_pad}")
    rng = np.random.default_rng(M + K)
    x = (rng.standard_normal((M, K)) * rng.uniform(0.01, 30, (M, 1))).astype(np.float32)
    x[0, :64] = 0.0
    if K >= 64:
        x[min(1, M - 1), :32] = np.float32(127.0)
        x[min(1, M - 1), 1:9] = [2.5, 3.5, -2.5, -3.5, 0.5, 1.5, -0.5, 126.5]
    if K >= 96:
        # a block whose 127 / amax overflows (amax < 127 / FLT_MAX): the
        # saturating conversion (+inf -> 127, -inf -> -128, 0 * inf -> 0)
        x[min(2, M - 1), 64:96] = 0.0
        x[min(2, M - 1), 64:68] = [1e-38, -1e-38, 2e-38, -3e-38]
    qs, ds = _quant_gpu(x, K_pad)
    rq, rd = orc.quantize_q8_1(x, K_pad)
    assert_same(host(qs), rq, "qs")
    assert_same(host(ds).view(np.uint16), rd, "ds")


def test_quantize_strided_input(orc):
    rng = np.random.default_rng(1)
    full = rng.standard_normal((50, 4400)).astype(np.float32)
    xd = dev(full)
    qs = empty((50, 4320), torch.int8)
    ds = empty((50, 135, 2), torch.int16)
    s2x.call("s2x_quantize_q8_1", ptr(xd), 4304, 50, 4400, 4320, ptr(qs), ptr(ds), stream())
    rq, rd = orc.quantize_q8_1(np.ascontiguousarray(full[:, :4304]), 4320)
    assert np.array_equal(host(qs), rq) and np.array_equal(host(ds).view(np.uint16), rd)


# (M, H, ldx, affine w, affine b): 13001 rows exceed one pass of the
# row-striding grid (4 x 3072 rows); ldx = H + 1 takes the unaligned loads
LN_CASES = [(729, 1152, 1152, True, True), (13001, 1152, 1152, True, True),
            (37, 768, 769, True, False), (5, 96, 96, False, True), (3, 2048, 2048, False, False)]


@pytest.mark.parametrize("M,H,ldx,has_w,has_b", LN_CASES)
def test_layernorm_quantize(orc, M, H, ldx, has_w, has_b):
    say(f"layernorm M={M} H={H} ldx={ldx} w={has_w} b={has_b}")
    rng = np.random.default_rng(2 + M)
    xs = (rng.standard_normal((M, ldx)) * 2 + 0.3).astype(np.float32)
    x = np.ascontiguousarray(xs[:, :H])
    w = rng.normal(1, 0.02, H).astype(np.float32) if has_w else None
    b = rng.normal(0, 0.02, H).astype(np.float32) if has_b else None
    xd = dev(xs)
    wd = dev(w) if has_w else None
    bd = dev(b) if has_b else None
    wp = ptr(wd) if has_w else None
    bp = ptr(bd) if has_b else None
    qs = empty((M, H), torch.int8)
    ds = empty((M, H // 32, 2), torch.int16)
    y = empty((M, H), torch.float32)
    s2x.call("s2x_layernorm_quantize_q8_1", ptr(xd), H, M, ldx, wp, bp, ctypes.c_float(1e-6),
             ptr(qs), ptr(ds), ptr(y), H, stream())
    yg = host(y)
    ref = orc.layernorm(x, w, b, 1e-6)
    # double-accumulated mean/variance as the CPU: the LN output is the same
    assert_same(yg, ref, "layernorm")
    # the fused quantizer is bit-exact on the GPU's own LN output
    rq, rd = orc.quantize_q8_1(yg)
    assert_same(host(qs), rq, "ln qs")
    assert_same(host(ds).view(np.uint16), rd, "ln ds")
    # LN alone
    y2 = empty((M, H), torch.float32)
    s2x.call("s2x_layernorm", ptr(xd), H, M, ldx, wp, bp, ctypes.c_float(1e-6), ptr(y2), H,
             stream())
    assert np.array_equal(host(y2), yg)


def _same_or_both_nan(a, b):
    return np.array_equal(a, b, equal_nan=True)


def test_quantize_q8_1_nan_and_inf_blocks(orc):
    """Blocks with NaNs (one, or all 32: amax 0, as a running max from 0
    takes it), infinities and values whose 127 / amax overflows."""
    x = np.random.default_rng(11).standard_normal((6, 256)).astype(np.float32)
    x[0, 0:32] = np.nan
    x[1, 32 + 5] = np.nan
    x[2, 64 + 7] = np.inf
    x[3, 96 + 1] = -np.inf
    x[4, 128:160] = 0.0
    x[4, 128:132] = [1e-38, -2e-38, 3e-39, 0.0]
    x[5, 160:192] = -0.0
    x[5, 192:224] = np.float32(2.0 ** -110)
    qs, ds = _quant_gpu(x, 256)
    rq, rd = orc.quantize_q8_1(x, 256)
    assert_same(host(qs), rq, "qs")
    assert_same(host(ds).view(np.uint16), rd, "ds")


def test_layernorm_quantize_special_blocks(orc):
    """LayerNorm + Q8_1 where blocks leave the fast form's domain -- a NaN
    input row, w = inf and w = NaN columns, blocks of w = 0 with tiny or
    zero b (amax below 2^-100, or 127 / amax overflowing) -- next to
    ordinary rows: the same bytes as the oracle's LayerNorm then quantizer."""
    H, M = 1152, 40
    rng = np.random.default_rng(12)
    x = (rng.standard_normal((M, H)) * 2 + 0.3).astype(np.float32)
    w = rng.normal(1, 0.02, H).astype(np.float32)
    b = rng.normal(0, 0.02, H).astype(np.float32)
    x[3, 100] = np.nan
    w[200] = np.inf
    w[300] = np.nan
    w[320:352] = 0.0
    b[320:352] = 0.0
    b[321] = 1e-38
    w[352:384] = 0.0
    b[352:384] = np.float32(2.0 ** -110)
    w[384:416] = 0.0
    b[384:416] = 0.0
    for m_rows in (M, 5000):  # registers for w and b; w and b in LDS
        xs = np.ascontiguousarray(np.tile(x, (m_rows // M + 1, 1))[:m_rows])
        say(f"layernorm special blocks M={m_rows}")
        xd, wd, bd = dev(xs), dev(w), dev(b)
        qs = empty((m_rows, H), torch.int8)
        ds = empty((m_rows, H // 32, 2), torch.int16)
        y = empty((m_rows, H), torch.float32)
        s2x.call("s2x_layernorm_quantize_q8_1", ptr(xd), H, m_rows, H, ptr(wd), ptr(bd),
                 ctypes.c_float(1e-6), ptr(qs), ptr(ds), ptr(y), H, stream())
        yg = host(y)
        ref = orc.layernorm(xs, w, b, 1e-6)
        assert _same_or_both_nan(yg, ref), "layernorm"
        rq, rd = orc.quantize_q8_1(ref)
        assert_same(host(qs), rq, "ln qs")
        assert_same(host(ds).view(np.uint16), rd, "ln ds")


def _weight(raw, k_pad, n):
    w = ctypes.c_void_p()
    s2x.call("s2x_weight_create", raw.ctypes.data, 1, k_pad, n, None, ctypes.byref(w))
    return w


@pytest.fixture(scope="module")
def gemm_data():
    data = {}
    for label, N, K, K_pad in SHAPES:
        rng = np.random.default_rng(N * 7 + K)
        wf = rng.normal(0, 0.02, (N, K)).astype(np.float32)
        raw = synth.quantize_q8_0(wf, K_pad)
        data[label] = (raw, N, K, K_pad)
    return data


@pytest.mark.parametrize("label", [s[0] for s in SHAPES])
def test_block_dots_bit_exact(orc, gemm_data, label):
    raw, N, K, K_pad = gemm_data[label]
    say(f"block dots {label}")
    M = 729
    x = np.random.default_rng(3).standard_normal((M, K)).astype(np.float32)
    qs, ds = _quant_gpu(x, K_pad)
    rq, _ = orc.quantize_q8_1(x, K_pad)
    w = _weight(raw, K_pad, N)
    try:
        wq = raw.reshape(N, K_pad // 32, 34)[:, :, 2:].copy().view(np.int8).astype(np.int64)
        KB = K_pad // 32
        for kb in sorted({0, KB // 2, KB - 1}):
            out = empty((M, N), torch.int32)
            s2x.call("s2x_block_dots", w, ptr(qs), M, kb, ptr(out), stream())
            ref = rq[:, kb * 32:(kb + 1) * 32].astype(np.int64) @ wq[:, kb, :].T
            assert np.array_equal(host(out), ref), f"kb={kb}"
    finally:
        s2x.lib.s2x_weight_destroy(w)


def _gemm_terms_abs(orc, raw, N, K_pad, rq, rd):
    wq = raw.reshape(N, K_pad // 32, 34)[:, :, 2:].copy().view(np.int8).astype(np.float32)
    dw = orc.fp16_to_fp32(raw.reshape(N, K_pad // 32, 34)[:, :, :2].copy().view(np.uint16)[..., 0])
    dx = orc.fp16_to_fp32(rd[..., 0])
    # sum_kb |I| dw dx, for the tolerance floor
    M = rq.shape[0]
    acc = np.zeros((M, N), np.float64)
    for kb in range(K_pad // 32):
        I = rq[:, kb * 32:(kb + 1) * 32].astype(np.float32) @ wq[:, kb, :].T
        acc += np.abs(I) * dx[:, kb:kb + 1] * dw[None, :, kb]
    return acc


@pytest.mark.parametrize("label", [s[0] for s in SHAPES])
def test_gemm_matches_oracle(orc, gemm_data, label):
    raw, N, K, K_pad = gemm_data[label]
    M = 729
    say(f"gemm {label} M={M}")
    x = np.random.default_rng(4).standard_normal((M, K)).astype(np.float32)
    qs, ds = _quant_gpu(x, K_pad)
    rq, rd = orc.quantize_q8_1(x, K_pad)
    ref = orc.mul_mat_q8_0_q8_1(raw, K_pad, N, rq, rd)
    w = _weight(raw, K_pad, N)
    try:
        y = empty((M, N), torch.float32)
        s2x.call("s2x_mul_mat_q8_0_q8_1", w, ptr(qs), ptr(ds), M, ptr(y), N, None, stream())
        yg = host(y)
    finally:
        s2x.lib.s2x_weight_destroy(w)
    from gpu_util import h5_rel
    rel = h5_rel(yg, ref.astype(np.float64), _gemm_terms_abs(orc, raw, N, K_pad, rq, rd))
    n_diff = int((yg != ref).sum())
    say(f"  max rel err (tau=1e-3 rms) {rel:.3e}, differing elements {n_diff}")
    assert rel <= 1e-4
    assert n_diff == 0  # same per-block fma order as the oracle: bit-exact


# K blocks 1..7 and 13: stage rings of several blocks end part-filled
# (fewer than 4 blocks: one partial stage; otherwise the last stage is
# fetched as the window of the last 4 blocks); ragged N and M leave partial
# edge tiles.  "small": 6 tiles, the latency form; "wide": 520 tiles of
# 128 x 128, the throughput form (sampled rows, the last tile's included);
# "rows5": 5 rows, the form of block dots side by side and one fma chain per
# output, with N = 203 ending on a partial group of 8 columns.
@pytest.mark.parametrize("form", ["small", "wide", "rows5"])
@pytest.mark.parametrize("KB", [1, 2, 3, 4, 5, 7, 13])
def test_gemm_short_k(orc, KB, form):
    M, N = {"small": (300, 200), "wide": (8300, 1000), "rows5": (5, 203)}[form]
    K_pad = 32 * KB
    K = K_pad - (5 if KB > 1 else 0)
    say(f"gemm short K: KB={KB} M={M} N={N}")
    rng = np.random.default_rng(40 + KB)
    raw = synth.quantize_q8_0(rng.normal(0, 0.02, (N, K)).astype(np.float32), K_pad)
    x = rng.standard_normal((M, K)).astype(np.float32)
    qs, ds = _quant_gpu(x, K_pad)
    rows = np.arange(M) if form != "wide" else np.unique(np.concatenate(
        [rng.choice(M, 200, replace=False), np.arange(M - 44, M)]))
    rq, rd = orc.quantize_q8_1(x[rows], K_pad)
    ref = orc.mul_mat_q8_0_q8_1(raw, K_pad, N, rq, rd)
    w = _weight(raw, K_pad, N)
    try:
        y = empty((M, N), torch.float32)
        s2x.call("s2x_mul_mat_q8_0_q8_1", w, ptr(qs), ptr(ds), M, ptr(y), N, None, stream())
        assert_same(host(y)[rows], ref, f"gemm KB={KB} {form}")
    finally:
        s2x.lib.s2x_weight_destroy(w)


def test_gemm_large_m_batch_invariant(orc, gemm_data):
    raw, N, K, K_pad = gemm_data["fc2"]
    M = 23328
    say("gemm fc2 M=23328")
    x = np.random.default_rng(5).standard_normal((M, K)).astype(np.float32)
    qs, ds = _quant_gpu(x, K_pad)
    w = _weight(raw, K_pad, N)
    try:
        y = empty((M, N), torch.float32)
        s2x.call("s2x_mul_mat_q8_0_q8_1", w, ptr(qs), ptr(ds), M, ptr(y), N, None, stream())
        yg = host(y)
        sub = 729
        y1 = empty((sub, N), torch.float32)
        s2x.call("s2x_mul_mat_q8_0_q8_1", w, ptr(qs[M - sub:]), ptr(ds[M - sub:]), sub, ptr(y1), N,
                 None, stream())
        assert np.array_equal(host(y1), yg[M - sub:])
    finally:
        s2x.lib.s2x_weight_destroy(w)
    rows = np.random.default_rng(6).choice(M, 64, replace=False)
    rq, rd = orc.quantize_q8_1(x[rows], K_pad)
    assert np.array_equal(orc.mul_mat_q8_0_q8_1(raw, K_pad, N, rq, rd), yg[rows])


@pytest.mark.parametrize("label", ["fc1", "out"])
def test_drop_in_large_m(orc, gemm_data, label):
    # batch-32 row count through the drop-in (int8) GEMM: partial last row
    # tile (23328 = 182 * 128 + 32), partial column tile for fc1 (4304 =
    # 33 * 128 + 80), a partly filled last round of tiles.  The checked rows
    # include the last 40
    raw, N, K, K_pad = gemm_data[label]
    M = 23328
    say(f"drop-in {label} M=23328")
    x = np.random.default_rng(8).standard_normal((M, K)).astype(np.float32)
    wd, xd = dev(raw), dev(x)
    y = empty((M, N), torch.float32)
    ws_bytes = s2x.lib.s2x_mul_mat_workspace_size(K_pad, N, M)
    ws = empty((ws_bytes,), torch.uint8)
    s2x.call("s2x_mul_mat_q8_0_f32", ptr(wd), K_pad, N, ptr(xd), K, K, M, ptr(y), ptr(ws),
             ctypes.c_size_t(ws_bytes), stream())
    yg = host(y)
    rows = np.concatenate([np.arange(M - 40, M), np.random.default_rng(9).choice(M - 40, 40,
                                                                                   replace=False)])
    assert_same(yg[rows], orc.mul_mat_q8_0_f32(raw, K_pad, N, x[rows]), f"drop-in {label} M=23328")


@pytest.mark.parametrize("label", [s[0] for s in SHAPES])
def test_drop_in_mul_mat_f32(orc, gemm_data, label):
    # the drop-in op runs the int8 GEMM; rows 0-7 carry tiny values so
    # their activation scales are fp16 subnormals (amax/127 < 6.1e-5)
    raw, N, K, K_pad = gemm_data[label]
    M = 333
    x = np.random.default_rng(7).standard_normal((M, K)).astype(np.float32)
    x[:8] *= np.float32(1e-4)
    wd, xd = dev(raw), dev(x)
    y = empty((M, N), torch.float32)
    ws_bytes = s2x.lib.s2x_mul_mat_workspace_size(K_pad, N, M)
    ws = empty((ws_bytes,), torch.uint8)
    s2x.call("s2x_mul_mat_q8_0_f32", ptr(wd), K_pad, N, ptr(xd), K, K, M, ptr(y), ptr(ws),
             ctypes.c_size_t(ws_bytes), stream())
    ref = orc.mul_mat_q8_0_f32(raw, K_pad, N, x)
    assert np.abs(ref[:8]).max() > 0
    assert_same(host(y), ref, f"drop-in {label}")
    small = ctypes.c_size_t(ws_bytes - 1)
    assert s2x.lib.s2x_mul_mat_q8_0_f32(ptr(wd), K_pad, N, ptr(xd), K, K, M, ptr(y), ptr(ws), small,
                                        stream()) == 4


@pytest.mark.parametrize("kind", ["bias", "gelu", "resid", "resid_rows", "resid_inplace"])
def test_gemm_epilogues(orc, gemm_data, kind):
    raw, N, K, K_pad = gemm_data["out"]
    M = 300
    rng = np.random.default_rng(8)
    x = rng.standard_normal((M, K)).astype(np.float32)
    bias = rng.normal(0, 0.02, N).astype(np.float32)
    res = rng.standard_normal((M, N)).astype(np.float32)
    pos = rng.standard_normal((100, N)).astype(np.float32)
    qs, ds = _quant_gpu(x, K_pad)
    rq, rd = orc.quantize_q8_1(x, K_pad)
    mm = orc.mul_mat_q8_0_q8_1(raw, K_pad, N, rq, rd)
    bd, rdv, pd = dev(bias), dev(res), dev(pos)
    y = empty((M, N), torch.float32)
    e = s2x.Epilogue()
    e.bias = bd.data_ptr()
    if kind == "bias":
        e.kind, ref = s2x.EPI_BIAS, mm + bias
    elif kind == "gelu":
        e.kind, ref = s2x.EPI_BIAS_GELU, orc.gelu(mm + bias)
    elif kind == "resid":
        e.kind, e.resid, e.ld_resid = s2x.EPI_BIAS_RESID, rdv.data_ptr(), N
        ref = (mm + bias) + res
    elif kind == "resid_rows":
        e.kind, e.resid, e.ld_resid, e.resid_rows = s2x.EPI_BIAS_RESID, pd.data_ptr(), N, 100
        ref = (mm + bias) + pos[np.arange(M) % 100]
    else:
        y = rdv
        e.kind, e.resid, e.ld_resid = s2x.EPI_BIAS_RESID, rdv.data_ptr(), N
        ref = (mm + bias) + res
    w = _weight(raw, K_pad, N)
    try:
        s2x.call("s2x_mul_mat_q8_0_q8_1", w, ptr(qs), ptr(ds), M, ptr(y), N, ctypes.byref(e), stream())
        yg = host(y)
    finally:
        s2x.lib.s2x_weight_destroy(w)
    # GELU included: both sides evaluate the same f32 tanh from IEEE primitives
    assert_same(yg, ref.astype(np.float32), f"epilogue {kind}")


def _split_ref(orc, raw, N, K_pad, rq, rd, n_split):
    """The split form restated on the oracle: each K range's product from
    the oracle's own block-order GEMM on that slice, then added in range
    order in f32."""
    KB = K_pad // 32
    per = ((KB + n_split - 1) // n_split + 3) // 4 * 4
    blocks = raw.reshape(N, KB, 34)
    acc = None
    for a in range(0, KB, per):
        b = min(KB, a + per)
        p = orc.mul_mat_q8_0_q8_1(np.ascontiguousarray(blocks[:, a:b]).reshape(-1), (b - a) * 32, N,
                                  np.ascontiguousarray(rq[:, a * 32:b * 32]),
                                  np.ascontiguousarray(rd[:, a:b]))
        acc = p if acc is None else (acc + p).astype(np.float32)
    return acc, (KB + per - 1) // per


# fc2 (135 blocks) in 4 ranges, out (36) in 2, a 13-block K in 3 requested
# (2 ranges of whole stages); M = 320 (a 5 x 64 text batch) and its first 64
# rows alone, which must give the same bits
@pytest.mark.parametrize("case", [("fc2", 4, "resid"), ("out", 2, "resid"), ("out", 2, "none"),
                                  ("k13", 3, "resid")])
def test_gemm_split_k_bit_exact(orc, gemm_data, case):
    label, n_split, kind = case
    if label == "k13":
        N, K_pad = 200, 13 * 32
        K = K_pad - 5
        raw = synth.quantize_q8_0(np.random.default_rng(41).normal(0, 0.02, (N, K)).astype(np.float32), K_pad)
    else:
        raw, N, K, K_pad = gemm_data[label]
    rng = np.random.default_rng(9)
    bias = rng.normal(0, 0.02, N).astype(np.float32)
    say(f"split-K gemm {label} n_split={n_split} {kind}")
    outs = {}
    for M in (320, 64):
        x = np.random.default_rng(12).standard_normal((320, K)).astype(np.float32)[:M]
        res = np.random.default_rng(13).standard_normal((320, N)).astype(np.float32)[:M]
        qs, ds = _quant_gpu(x, K_pad)
        rq, rd = orc.quantize_q8_1(x, K_pad)
        ref, splits = _split_ref(orc, raw, N, K_pad, rq, rd, n_split)
        e = s2x.Epilogue()
        bd, rdv = dev(bias), dev(res)
        if kind == "resid":
            e.kind, e.bias, e.resid, e.ld_resid = s2x.EPI_BIAS_RESID, bd.data_ptr(), rdv.data_ptr(), N
            ref = (ref + bias) + res
        else:
            e.kind = s2x.EPI_NONE
        y = rdv if kind == "resid" else empty((M, N), torch.float32)  # in place on the residual
        ws = empty((n_split * M * N,), torch.float32)
        w = _weight(raw, K_pad, N)
        try:
            s2x.call("s2x_mul_mat_q8_0_q8_1_split_k", w, ptr(qs), ptr(ds), M, ptr(y), N, ctypes.byref(e),
                     n_split, ptr(ws), ws.numel() * 4, stream())
            outs[M] = host(y)
        finally:
            s2x.lib.s2x_weight_destroy(w)
        assert splits > 1
        assert_same(outs[M], ref.astype(np.float32), f"split-K {label} M={M}")
    assert np.array_equal(outs[64], outs[320][:64])


def test_standalone_epilogues(orc):
    rng = np.random.default_rng(9)
    H, n = 4304, 37
    mm = rng.standard_normal((n, H)).astype(np.float32)
    b = rng.normal(0, 0.02, H).astype(np.float32)
    r = rng.standard_normal((n, H)).astype(np.float32)
    md, bd, rd = dev(mm), dev(b), dev(r)
    y = empty((n, H), torch.float32)
    s2x.call("s2x_bias_residual", ptr(md), ptr(bd), ptr(rd), ptr(y), H, n, stream())
    assert np.array_equal(host(y), (mm + b) + r)
    s2x.call("s2x_bias_gelu", ptr(md), ptr(bd), ptr(y), H, n, stream())
    assert_same(host(y), orc.gelu(mm + b), "bias_gelu")


# Every float whose GELU goes through a division by y = 1 + e^t other than
# y = 2 (|x| < 2^-30) or y = 1 (x >= 2^7), plus a stretch of the clamped
# y = 1 + e^87: [2^-30, 2^7), its negatives and [-2^10, -2^7).
GELU_RANGES = [(0x30800000, 0x43000000), (0xB0800000, 0xC3000000), (0xC3000000, 0xC4800000)]


def test_gelu_every_float_in_the_division_domain(orc):
    """The GPU GELU (its division is Markstein's, on v_rcp_f32) equals the
    oracle's (an IEEE division) bit for bit on 645 M floats: all of them
    in the ranges where the quotient is not a division by 1 or 2."""
    chunk = 1 << 25
    zero = zeros((1,), torch.float32)
    y = empty((chunk,), torch.float32)
    total = bad = 0
    for lo, hi in GELU_RANGES:
        for a in range(lo, hi, chunk):
            b = min(a + chunk, hi)
            x = np.arange(a, b, dtype=np.uint32).view(np.float32)
            xd = dev(x)
            s2x.call("s2x_bias_gelu", ptr(xd), ptr(zero), ptr(y), 1, b - a, stream())
            got = host(y[:b - a]).view(np.uint32)
            ref = orc.gelu_mode(orc.GELU_EXACT, x).view(np.uint32)
            miss = np.flatnonzero(got != ref)
            if len(miss):
                say(f"gelu: {len(miss)} of {b - a} differ from 0x{a:08x}; first "
                    f"x={x[miss[0]]!r} got 0x{got[miss[0]]:08x} ref 0x{ref[miss[0]]:08x}")
            total += b - a
            bad += len(miss)
            del xd
    say(f"gelu: {total} floats, {bad} differ")
    assert total == sum(hi - lo for lo, hi in GELU_RANGES) == 645_922_816
    assert bad == 0


def _attn_case(orc, lens, n_head=16, dh=72, key_valid=None, seed=10):
    H = n_head * dh
    rng = np.random.default_rng(seed)
    M = int(sum(lens))
    qkv = (rng.standard_normal((M, 3 * H)) * 1.5).astype(np.float32)
    bias = rng.normal(0, 0.5, 3 * H).astype(np.float32)
    starts = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.int32)
    lens = np.asarray(lens, np.int32)
    max_len = int(lens.max())
    ws_bytes = s2x.lib.s2x_attn_workspace_size(len(lens), max_len, n_head, dh)
    ws = zeros((ws_bytes,), torch.uint8)
    qd, bd, sd, ld = dev(qkv), dev(bias), dev(starts), dev(lens)
    kv = dev(key_valid) if key_valid is not None else None
    out = empty((M, H), torch.float32)
    scale = np.float32(1.0 / np.sqrt(np.float32(dh)))
    s2x.call("s2x_attn_prep", ptr(qd), 3 * H, ptr(bd), ptr(sd), ptr(ld), len(lens), max_len, n_head,
             dh, ptr(ws), ctypes.c_size_t(ws_bytes), stream())
    s2x.call("s2x_attn_run", ptr(ws), ctypes.c_size_t(ws_bytes), ptr(sd), ptr(ld), ptr(kv),
             len(lens), max_len, n_head, dh, ctypes.c_float(scale), ptr(out), H, stream())
    og = host(out)
    biased = qkv + bias
    errs = []
    for s, L in zip(starts, lens):
        kvs = None if key_valid is None else key_valid[s:s + L]
        ref = orc.attention(biased[s:s + L], n_head, dh, scale, kvs)
        errs.append(np.abs(og[s:s + L] - ref).max() / np.abs(ref).max())
        assert cos(og[s:s + L], ref) > 0.99999
    return max(errs)


def test_attention_segments(orc):
    e = _attn_case(orc, [729, 1, 64, 130, 255, 128])
    say(f"attention max err / max|out| = {e:.2e}")
    # Q, K, V rounded to f16 on both sides; the scores, the softmax and the
    # f16 hi+lo probability pair keep the rest near f32 (measured 7.3e-7)
    assert e < 1e-5


def test_attention_key_mask(orc):
    lens = [64, 200]
    kv = np.ones(264, np.uint8)
    kv[40:64] = 0
    kv[64 + 150:] = 0
    assert _attn_case(orc, lens, key_valid=kv, seed=11) < 1e-5


@pytest.mark.parametrize("case", ["ragged", "masked", "batch32", "one", "ragged40", "masked36"])
def test_attention_q8_1_equals_attention_then_quantize(case):
    """s2x_attn_run_q8_1 (Q8_1 of whole blocks in the attention epilogue;
    the blocks that straddle two heads in a second pass, or, from 256
    four-head workgroups up -- batch32, ragged40, masked36 -- by the
    workgroup that runs the group's four heads in turn) gives exactly the
    bytes of s2x_attn_run followed by s2x_quantize_q8_1."""
    n_head, dh = 16, 72
    H = n_head * dh
    rng = np.random.default_rng(17)
    ragged40 = [int(x) for x in rng.choice([1, 33, 64, 130, 255, 384, 385, 500, 729], 39)] + [729]
    lens = {"ragged": [729, 1, 64, 130, 255, 128, 33], "masked": [64, 200],
            "batch32": [729] * 32, "one": [729], "ragged40": ragged40,
            "masked36": [729] * 36}[case]
    M = int(sum(lens))
    qkv = (rng.standard_normal((M, 3 * H)) * 1.5).astype(np.float32)
    bias = rng.normal(0, 0.5, 3 * H).astype(np.float32)
    starts = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.int32)
    lens = np.asarray(lens, np.int32)
    max_len = int(lens.max())
    kv = None
    if case == "masked":
        kv = np.ones(M, np.uint8)
        kv[40:64] = 0
        kv[64 + 150:] = 0
    if case == "masked36":  # a tenth of the keys masked, each segment's first kept
        kv = (rng.random(M) >= 0.1).astype(np.uint8)
        kv[starts] = 1
    say(f"attention + Q8_1: {case}, M={M}")
    wsb = s2x.lib.s2x_attn_workspace_size(len(lens), max_len, n_head, dh)
    ws = zeros((wsb,), torch.uint8)
    qd, bd, sd, ld = dev(qkv), dev(bias), dev(starts), dev(lens)
    kd = dev(kv) if kv is not None else None
    scale = ctypes.c_float(np.float32(1.0 / np.sqrt(np.float32(dh))))
    s2x.call("s2x_attn_prep", ptr(qd), 3 * H, ptr(bd), ptr(sd), ptr(ld), len(lens), max_len,
             n_head, dh, ptr(ws), ctypes.c_size_t(wsb), stream())
    out = empty((M, H), torch.float32)
    s2x.call("s2x_attn_run", ptr(ws), ctypes.c_size_t(wsb), ptr(sd), ptr(ld), ptr(kd), len(lens),
             max_len, n_head, dh, scale, ptr(out), H, stream())
    qs_r = zeros((M, H), torch.int8)
    ds_r = zeros((M, H // 32), torch.int32)
    s2x.call("s2x_quantize_q8_1", ptr(out), H, M, H, H, ptr(qs_r), ptr(ds_r), stream())
    # the fused path, into garbage-filled buffers (every byte must be written)
    qs_f = torch.full((M, H), 0x5A, dtype=torch.int8, device="cuda:0")
    ds_f = torch.full((M, H // 32), 0x5A5A5A5A, dtype=torch.int32, device="cuda:0")
    scratch = torch.full((M, H), float("nan"), dtype=torch.float32, device="cuda:0")
    s2x.call("s2x_attn_run_q8_1", ptr(ws), ctypes.c_size_t(wsb), ptr(sd), ptr(ld), ptr(kd),
             len(lens), max_len, n_head, dh, scale, M, ptr(qs_f), ptr(ds_f), H // 32, ptr(scratch),
             H, stream())
    assert_same(host(qs_f), host(qs_r), f"{case} quants")
    assert_same(host(ds_f), host(ds_r), f"{case} scale words")


@pytest.mark.parametrize("masked", [False, True])
def test_attention_fp64_matches_oracle(orc, masked):
    n_head, dh = 16, 72
    H = n_head * dh
    lens = [64, 64, 17, 130]
    rng = np.random.default_rng(16)
    M = sum(lens)
    qkv = (rng.standard_normal((M, 3 * H)) * 1.5).astype(np.float32)
    bias = rng.normal(0, 0.5, 3 * H).astype(np.float32)
    starts = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.int32)
    kv = None
    if masked:
        kv = np.ones(M, np.uint8)
        kv[40:64] = 0
        kv[64 + 5] = 0
    qd, bd, sd, ld = dev(qkv), dev(bias), dev(starts), dev(np.asarray(lens, np.int32))
    kd = dev(kv) if kv is not None else None
    out = empty((M, H), torch.float32)
    scale = np.float32(1.0 / np.sqrt(np.float32(dh)))
    s2x.call("s2x_attn_fp64", ptr(qd), 3 * H, ptr(bd), ptr(sd), ptr(ld), ptr(kd), len(lens),
             max(lens), n_head, dh, ctypes.c_float(scale), ptr(out), H, stream())
    og = host(out)
    biased = qkv + bias
    ref = np.concatenate([orc.attention(biased[s:s + L], n_head, dh, scale,
                                        None if kv is None else kv[s:s + L])
                          for s, L in zip(starts, lens)])
    n_diff = int((og != ref).sum())
    say(f"fp64 attention: {n_diff} of {og.size} outputs differ from the oracle, max ulp "
        f"{(np.abs(og - ref) / np.spacing(np.abs(ref))).max():.1f}")
    assert (np.abs(og - ref) <= np.spacing(np.abs(ref))).all()  # at most 1 ulp (exp())
    assert n_diff <= og.size // 100000


def _attn_fp64(qkv, bias, lens, n_head, dh, kv=None):
    H = n_head * dh
    starts = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.int32)
    qd, bd, sd, ld = dev(qkv), dev(bias), dev(starts), dev(np.asarray(lens, np.int32))
    kd = dev(kv) if kv is not None else None
    out = empty((int(sum(lens)), H), torch.float32)
    scale = np.float32(1.0 / np.sqrt(np.float32(dh)))
    s2x.call("s2x_attn_fp64", ptr(qd), 3 * H, ptr(bd), ptr(sd), ptr(ld), ptr(kd), len(lens),
             max(lens), n_head, dh, ctypes.c_float(scale), ptr(out), H, stream())
    return host(out), starts, scale


@pytest.mark.parametrize("masked", [False, True])
def test_attention_fp64_short_segments(orc, masked):
    # segments of <= 64 tokens take the workgroup-per-head kernel: the bits of
    # the one-lane-per-query kernel (run here through a batch that also holds
    # a 100-token segment) and within 1 ulp of the oracle
    n_head, dh = 16, 72
    lens = [64, 17, 1, 40, 64]
    rng = np.random.default_rng(17)
    M = sum(lens) + 100
    qkv = (rng.standard_normal((M, 3 * n_head * dh)) * 1.5).astype(np.float32)
    bias = rng.normal(0, 0.5, 3 * n_head * dh).astype(np.float32)
    kv = None
    if masked:
        kv = np.ones(M, np.uint8)
        kv[5:9] = 0
        kv[64 + 17 + 1 + 30:64 + 17 + 1 + 40] = 0
    n_short = sum(lens)
    short, starts, scale = _attn_fp64(qkv[:n_short], bias, lens, n_head, dh,
                                      None if kv is None else kv[:n_short])
    long_, _, _ = _attn_fp64(qkv, bias, lens + [100], n_head, dh, kv)
    assert np.array_equal(short, long_[:n_short])
    ref = np.concatenate([orc.attention((qkv + bias)[s:s + L], n_head, dh, scale,
                                        None if kv is None else kv[s:s + L])
                          for s, L in zip(starts, lens)])
    assert (np.abs(short - ref) <= np.spacing(np.abs(ref))).all()


@pytest.mark.parametrize("hw", [(27, 27), (8, 32), (16, 16), (32, 32)])
def test_resize_pos_embed(orc, hw):
    h, w = hw
    pos = np.random.default_rng(12).normal(0, 0.02, (256, 1152)).astype(np.float32)
    pd = dev(pos)
    out = empty((h * w, 1152), torch.float32)
    s2x.call("s2x_resize_pos_embed", ptr(pd), 16, 1152, h, w, ptr(out), stream())
    assert np.array_equal(host(out), orc.resize_pos_embed(pos, 16, h, w))


def test_get_rows_q8_0(orc):
    rng = np.random.default_rng(13)
    table = synth.quantize_q8_0(rng.normal(0, 0.02, (500, 1152)).astype(np.float32))
    ids = rng.integers(0, 500, 70).astype(np.int32)
    pos = rng.normal(0, 0.02, (64, 1152)).astype(np.float32)
    td, idd, pd = dev(table), dev(ids), dev(pos)
    out = empty((70, 1152), torch.float32)
    s2x.call("s2x_get_rows_q8_0", ptr(td), 1152, 500, ptr(idd), 70, ptr(pd), 35, ptr(out), stream())
    deq = orc.dequantize_q8_0(table, 500, 1152)
    assert np.array_equal(host(out), deq[ids] + pos[np.arange(70) % 35])


# --------------------------------------------------- MAP head attention ----
@pytest.mark.parametrize("lens", [[256], [729], [1024], [729, 1, 64, 130, 1024, 255, 576]],
                         ids=["n256", "n729", "n1024", "ragged"])
def test_attention_1q_vs_oracle(orc, lens):
    """k_attn_1q (the probe head's one-query attention) through s2x_attn_1q,
    keys and values in rows of stride 2H as the head's K/V GEMM writes them,
    against the oracle's single-query attention (Q, K, V rounded to f16,
    float64 softmax): within 1e-5 of max|out| per segment."""
    n_head, dh = 16, 72
    H = n_head * dh
    rng = np.random.default_rng(sum(lens))
    M = int(sum(lens))
    q = rng.standard_normal(H).astype(np.float32)
    kv = (rng.standard_normal((M, 2 * H)) * 1.5).astype(np.float32)
    starts = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.int32)
    L = np.asarray(lens, np.int32)
    say(f"attn_1q: segments {lens}")
    qd, kvd, sd, ld = dev(q), dev(kv), dev(starts), dev(L)
    out = empty((len(lens), H), torch.float32)
    scale = np.float32(1.0 / np.sqrt(np.float32(dh)))
    kp = kvd.data_ptr()
    s2x.call("s2x_attn_1q", ptr(qd), ctypes.c_void_p(kp), ctypes.c_void_p(kp + 4 * H), 2 * H, ptr(sd),
             ptr(ld), len(lens), int(L.max()), n_head, dh, ctypes.c_float(scale), ptr(out), stream())
    og = host(out)
    for i, (s, n) in enumerate(zip(starts, L)):
        ref = orc.attention_1q(q, kv[s:s + n, :H], kv[s:s + n, H:], n_head, dh, scale)
        err = np.abs(og[i] - ref).max() / np.abs(ref).max()
        assert err <= 1e-5, (i, n, err)


def test_attention_1q_rejects_bad_arguments():
    f = s2x.lib.s2x_attn_1q
    t = empty((16,), torch.float32)
    p = ptr(t)
    assert f(p, p, p, 1152, p, p, 1, 4097, 16, 72, ctypes.c_float(0.1), p, stream()) != 0  # max_len
    assert f(p, p, p, 1152, p, p, 1, 100, 4, 129, ctypes.c_float(0.1), p, stream()) != 0   # d_head
    assert f(p, p, p, 1151, p, p, 1, 100, 16, 72, ctypes.c_float(0.1), p, stream()) != 0   # ld < H
    assert f(p, p, p, 1152, p, p, 0, 100, 16, 72, ctypes.c_float(0.1), p, stream()) == 0   # no segments
