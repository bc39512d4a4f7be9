"""Pins the CPU oracle's primitives against closed forms, brute force and
library routines (numpy float16 rounding, float64 evaluation).  CPU only."""
import numpy as np
import pytest


# ---------------------------------------------------------------- fp16 ----
def test_fp16_roundtrip_all_values(orc):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f = orc.fp16_to_fp32(h)
    ref = h.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(f), nan)
    assert np.array_equal(f[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    back = orc.fp32_to_fp16(f[~nan])
    assert np.array_equal(back, h[~nan])


def test_fp16_rounding_matches_numpy(orc):
    rng = np.random.default_rng(7)
    x = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 6, 200000),
        np.array([65504, 65519.99, 65520, 1e6, -70000, 6.1e-5, 6.0e-8, 2.98e-8, 2.99e-8,
                  5.96e-8, 1e-10, 0.0, -0.0, np.inf, -np.inf], np.float32),
    ]).astype(np.float32)
    # exact ties: midpoints between consecutive fp16 values
    base = np.arange(0x0001, 0x7bff, 7, dtype=np.uint16).view(np.float16).astype(np.float64)
    nxt = (np.arange(0x0001, 0x7bff, 7, dtype=np.uint16) + 1).view(np.float16).astype(np.float64)
    ties = ((base + nxt) / 2).astype(np.float32)
    x = np.concatenate([x, ties, -ties])
    ours = orc.fp32_to_fp16(x)
    ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(ours, ref)


# ------------------------------------------------------------ Q8_1 -------
def _q81(orc, row):
    qs, ds = orc.quantize_q8_1(np.asarray(row, np.float32)[None, :])
    return qs[0], orc.fp16_to_fp32(ds[0])


def test_q8_1_zero_block(orc):
    q, ds = _q81(orc, np.zeros(32))
    assert not q.any() and not ds.any()


def test_q8_1_amax_maps_to_127(orc):
    row = np.linspace(-3.0, 2.0, 32).astype(np.float32)
    q, ds = _q81(orc, row)
    assert q[0] == -127 and q.max() < 127
    assert ds[0, 0] == np.float32(np.float16(np.float32(3.0) / np.float32(127)))


def test_q8_1_half_even_ties(orc):
    # amax = 127 -> inv = 1 exactly, so q = rint(x): ties go to even
    row = np.zeros(32, np.float32)
    row[0] = 127.0
    row[1:9] = [2.5, 3.5, -2.5, -3.5, 0.5, 1.5, -0.5, 126.5]
    q, ds = _q81(orc, row)
    assert list(q[:9]) == [127, 2, 4, -2, -4, 0, 2, 0, 126]
    assert ds[0, 1] == np.float32(np.float16(np.float32(q.astype(np.int32).sum()) * np.float32(1.0)))


def test_q8_1_single_nonzero_and_sum(orc):
    row = np.zeros(64, np.float32)
    row[5] = -0.3
    row[40] = 7.0
    q, ds = _q81(orc, row)
    assert q[5] == -127 and q[40] == 127 and np.count_nonzero(q) == 2
    d0 = np.float32(0.3) / np.float32(127)
    assert ds[0, 0] == np.float32(np.float16(d0))
    assert ds[0, 1] == np.float32(np.float16(np.float32(-127) * d0))


def test_q8_1_padding_tail_is_zero(orc):
    x = np.random.default_rng(3).standard_normal((5, 4304)).astype(np.float32)
    qs, ds = orc.quantize_q8_1(x, 4320)
    assert not qs[:, 4304:].any()
    qs2, ds2 = orc.quantize_q8_1(np.concatenate([x, np.zeros((5, 16), np.float32)], 1))
    assert np.array_equal(qs, qs2) and np.array_equal(ds, ds2)


def test_q8_1_brute_force_double(orc):
    rng = np.random.default_rng(11)
    x = (rng.standard_normal((64, 256)) * rng.uniform(0.01, 50, (64, 1))).astype(np.float32)
    qs, ds = orc.quantize_q8_1(x)
    b = x.reshape(64, 8, 32).astype(np.float64)
    amax = np.abs(b).max(2, keepdims=True)
    qd = np.clip(np.rint(b * (127.0 / amax)), -128, 127)
    diff = np.abs(qd.reshape(64, 256) - qs)
    # f32 evaluation of x*(127/amax) may cross a .5 boundary in rare cases
    assert diff.max() <= 1 and (diff > 0).mean() < 1e-3
    d = orc.fp16_to_fp32(ds[..., 0])
    assert np.array_equal(d, (amax[..., 0] / 127.0).astype(np.float32).astype(np.float16).astype(np.float32))


def test_q8_1_fp16_overflow_of_d(orc):
    row = np.zeros(32, np.float32)
    row[0] = 1e8  # amax/127 > 65504
    q, ds = _q81(orc, row)
    assert q[0] == 127 and np.isinf(ds[0, 0])


# ------------------------------------------------------------ Q8_0 -------
def test_q8_1_tiny_amax_saturates(orc):
    # amax = 1e-38 < 127 / FLT_MAX: 127 / amax overflows to inf, and the
    # reference's __float2int_rn saturates the +-inf products (0 * inf -> 0)
    row = np.zeros(32, np.float32)
    row[0], row[1], row[2] = 1e-38, -1e-38, 5e-39
    q, ds = _q81(orc, row)
    assert q[0] == 127 and q[1] == -128 and q[2] == 127 and (q[3:] == 0).all()
    assert ds[0, 0] == 0.0  # d = amax / 127 is below the f16 range


def test_q8_round_by_magic_add_equals_rint():
    """The device kernels round x * (127 / amax) to int8 by adding 1.5 * 2^23
    to the f32 product and keeping the low bits (s2x_device.h q8_round).
    That equals rint (half to even) and never needs the [-128, 127] clamp
    for every product a Q8_1 block can form: all f32 values of magnitude up
    to 127.0001 near each half-integer and integer (ties, their float
    neighbours), plus random products x * inv with |x| <= amax."""
    magic = np.float32(12582912.0)

    def by_magic(p):
        s = (p.astype(np.float32) + magic).astype(np.float32)
        return (s.view(np.uint32).astype(np.int64) - 0x4B400000).astype(np.int64)

    h = np.arange(-255, 256, dtype=np.float64) / 2.0  # -127.5 .. 127.5 step 0.5
    pts = h.astype(np.float32)
    near = [pts]
    for _ in range(4):  # 4 float steps either side of every point
        near.append(np.nextafter(near[-1], np.float32(np.inf)))
    below = [pts]
    for _ in range(4):
        below.append(np.nextafter(below[-1], np.float32(-np.inf)))
    p = np.concatenate(near + below)
    p = p[np.abs(p) <= np.float32(127.0001)]
    assert np.array_equal(by_magic(p), np.rint(p).astype(np.int64))
    rng = np.random.default_rng(5)
    x = rng.standard_normal((20000, 32)).astype(np.float32)
    x[:100] *= np.float32(1e-30)  # tiny blocks
    x[100:200] *= np.float32(1e30)
    amax = np.abs(x).max(axis=1, keepdims=True)
    inv = (np.float32(127.0) / amax).astype(np.float32)
    prod = (x * inv).astype(np.float32)
    q = by_magic(prod)
    assert np.array_equal(q, np.rint(prod).astype(np.int64))
    assert q.min() >= -127 and q.max() <= 127


def test_q8_0_roundf_half_away(orc):
    w = np.zeros((1, 32), np.float32)
    w[0, 0] = 127.0            # d = 1, id = 1
    w[0, 1:5] = [2.5, -2.5, 0.5, 125.5]
    raw = orc.quantize_q8_0(w)
    q = raw[0, 2:34].view(np.int8)
    assert list(q[:5]) == [127, 3, -3, 1, 126]


def test_q8_0_dequant_error_bound(orc):
    w = np.random.default_rng(5).normal(0, 0.02, (16, 4304)).astype(np.float32)
    raw = orc.quantize_q8_0(w, 4320)
    deq = orc.dequantize_q8_0(raw, 16, 4320)
    d = orc.fp16_to_fp32(raw.reshape(16, 135, 34)[:, :, :2].copy().view(np.uint16)[..., 0])
    err = np.abs(deq[:, :4304] - w)
    bound = np.repeat(d, 32, axis=1)[:, :4304] * 0.5 + np.abs(w) * 2e-3
    assert (err <= bound).all()
    assert not deq[:, 4304:].any()


def test_synth_quantizer_matches_oracle(orc):
    from s2x import synth
    w = np.random.default_rng(9).normal(0, 0.02, (37, 4304)).astype(np.float32)
    w[0, :32] = 0
    w[1, 0] = 127.0
    w[1, 1:5] = [2.5, -2.5, 0.5, 125.5]
    assert np.array_equal(synth.quantize_q8_0(w, 4320), orc.quantize_q8_0(w, 4320))


# ------------------------------------------------------------ GEMM -------
def _rand_gemm(orc, M, N, K, K_pad=None, seed=0):
    rng = np.random.default_rng(seed)
    K_pad = K_pad or K
    w = rng.normal(0, 0.02, (N, K)).astype(np.float32)
    x = rng.standard_normal((M, K)).astype(np.float32)
    return orc.quantize_q8_0(w, K_pad), x, K_pad


def test_block_dots_brute_force(orc):
    raw, x, K_pad = _rand_gemm(orc, 7, 9, 4304, 4320)
    qs, _ = orc.quantize_q8_1(x, K_pad)
    wq = raw.reshape(9, 135, 34)[:, :, 2:].copy().view(np.int8).reshape(9, -1).astype(np.int64)
    for m, n in [(0, 0), (3, 8), (6, 4)]:
        ref = (wq[n].reshape(135, 32) * qs[m].astype(np.int64).reshape(135, 32)).sum(1)
        assert np.array_equal(orc.block_dots(raw, K_pad, n, qs, m), ref)


def test_gemm_single_block_is_one_rounding(orc):
    raw, x, K_pad = _rand_gemm(orc, 33, 17, 32)
    qs, ds = orc.quantize_q8_1(x)
    y = orc.mul_mat_q8_0_q8_1(raw, 32, 17, qs, ds)
    wq = raw[:, 2:].copy().view(np.int8).astype(np.int64)
    dw = orc.fp16_to_fp32(raw[:, :2].copy().view(np.uint16)[:, 0])
    dx = orc.fp16_to_fp32(ds[:, 0, 0])
    I = qs.astype(np.int64) @ wq.T
    ref = (I.astype(np.float32) * (dw[None, :] * dx[:, None])).astype(np.float32)
    assert np.array_equal(y, ref)


def test_gemm_float64_tolerance(orc):
    raw, x, K_pad = _rand_gemm(orc, 40, 70, 4304, 4320, seed=2)
    qs, ds = orc.quantize_q8_1(x, K_pad)
    y = orc.mul_mat_q8_0_q8_1(raw, K_pad, 70, qs, ds)
    wq = raw.reshape(70, 135, 34)[:, :, 2:].copy().view(np.int8).astype(np.float64)
    dw = orc.fp16_to_fp32(raw.reshape(70, 135, 34)[:, :, :2].copy().view(np.uint16)[..., 0]).astype(np.float64)
    dx = orc.fp16_to_fp32(ds[..., 0]).astype(np.float64)
    I = np.einsum("mbk,nbk->mnb", qs.reshape(40, 135, 32).astype(np.float64), wq)
    terms = I * dw[None] * dx[:, None]
    ref = terms.sum(2)
    tau = np.abs(terms).sum(2)
    assert (np.abs(y - ref) <= 1e-5 * tau + 1e-30).all()


def test_gemm_power_of_two_scaling_is_exact(orc):
    raw, x, K_pad = _rand_gemm(orc, 12, 33, 1152, seed=4)
    y1 = orc.mul_mat_q8_0_f32(raw, K_pad, 33, x)
    y2 = orc.mul_mat_q8_0_f32(raw, K_pad, 33, x * np.float32(4.0))
    assert np.array_equal(y2, y1 * np.float32(4.0))


def test_gemm_rows_independent(orc):
    raw, x, K_pad = _rand_gemm(orc, 20, 48, 1152, seed=8)
    y = orc.mul_mat_q8_0_f32(raw, K_pad, 48, x)
    perm = np.random.default_rng(1).permutation(20)
    assert np.array_equal(orc.mul_mat_q8_0_f32(raw, K_pad, 48, x[perm]), y[perm])
    x0 = x.copy()
    x0[3] = 0
    assert not orc.mul_mat_q8_0_f32(raw, K_pad, 48, x0)[3].any()


def test_mul_mat_f32_pads_k(orc):
    raw, x, K_pad = _rand_gemm(orc, 9, 40, 4304, 4320, seed=6)
    y = orc.mul_mat_q8_0_f32(raw, K_pad, 40, x)
    qs, ds = orc.quantize_q8_1(x, K_pad)
    assert np.array_equal(y, orc.mul_mat_q8_0_q8_1(raw, K_pad, 40, qs, ds))
    deq = orc.dequantize_q8_0(raw, 40, K_pad)[:, :4304].astype(np.float64)
    ref = x.astype(np.float64) @ deq.T
    assert np.abs(y - ref).max() < 0.02 * np.abs(ref).max()


# ------------------------------------------------------------ LN / GELU --
def test_mul_mat_f16_integers_exact(orc):
    # small integers: every f16 value, product and partial sum is exact, so
    # the result is the integer dot product itself (a transposed operand or a
    # dropped term cannot pass)
    rng = np.random.default_rng(40)
    M, N, K = 7, 9, 4304
    x = rng.integers(-8, 9, (M, K)).astype(np.float32)
    w = rng.integers(-8, 9, (N, K)).astype(np.float16)
    y = orc.mul_mat_f16_f32(w, x)
    assert np.array_equal(y, (x.astype(np.int64) @ w.astype(np.int64).T).astype(np.float32))


def test_mul_mat_f16_rounds_x_to_f16_and_sums_in_double(orc):
    rng = np.random.default_rng(41)
    M, N, K = 33, 20, 1000
    x = rng.standard_normal((M, K)).astype(np.float32)
    x[0, :4] = [1 + 2.0 ** -11, 1 + 3 * 2.0 ** -11, -(1 + 2.0 ** -11), 65520.0]  # ties; overflow
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float16)
    y = orc.mul_mat_f16_f32(w, x)
    xh = x.astype(np.float16).astype(np.float64)  # numpy: round to nearest even
    assert xh[0, 0] == 1.0 and xh[0, 1] == 1 + 2.0 ** -9 and np.isinf(xh[0, 3])
    ref = xh @ w.astype(np.float64).T
    fin = np.isfinite(ref)
    assert not fin[0].any() and fin[1:].all()
    # double sums in another order round to the same f32 but for rare ties
    d = np.abs(y[fin].astype(np.float64) - ref[fin].astype(np.float32).astype(np.float64))
    assert (d <= np.spacing(np.abs(ref[fin]).astype(np.float32))).all()
    assert (y[fin] == ref[fin].astype(np.float32)).mean() > 0.999


def test_layernorm_float64(orc):
    rng = np.random.default_rng(12)
    x = (rng.standard_normal((50, 1152)) * 3 + 0.5).astype(np.float32)
    w = rng.normal(1, 0.02, 1152).astype(np.float32)
    b = rng.normal(0, 0.02, 1152).astype(np.float32)
    y = orc.layernorm(x, w, b, 1e-6)
    xd = x.astype(np.float64)
    ref = (xd - xd.mean(1, keepdims=True)) / np.sqrt(xd.var(1, keepdims=True) + 1e-6) * w + b
    assert np.abs(y - ref).max() < 2e-6 * np.abs(ref).max()


def test_layernorm_constant_row(orc):
    x = np.full((2, 64), 3.25, np.float32)
    y = orc.layernorm(x, None, np.full(64, 0.5, np.float32), 1e-6)
    assert np.array_equal(y, np.full((2, 64), 0.5, np.float32))


def test_tanh_f32_accuracy(orc):
    x = np.concatenate([np.linspace(-12, 12, 120001), np.logspace(-10, 1.2, 20001),
                        -np.logspace(-10, 1.2, 20001), [0.0, 0.5, -0.5, 9.0, -9.0]]).astype(np.float32)
    t = orc.tanh_f32(x)
    ref = np.tanh(x.astype(np.float64))
    ulp = np.abs(t - ref) / np.spacing(np.abs(ref).astype(np.float32)).astype(np.float64)
    assert ulp.max() <= 3.0
    assert np.array_equal(orc.tanh_f32(-x), -t)  # odd
    assert orc.tanh_f32(np.float32(0.0)) == 0.0


def test_gelu_closed_form(orc):
    x = np.linspace(-12, 12, 4001).astype(np.float32)
    g = orc.gelu(x)
    xd = x.astype(np.float64)
    ref = 0.5 * xd * (1 + np.tanh(np.sqrt(2 / np.pi) * (xd + 0.044715 * xd ** 3)))
    assert np.abs(g - ref).max() < 1e-5
    assert orc.gelu(np.float32(0.0)) == 0.0
    assert orc.gelu(np.float32(20.0)) == np.float32(20.0)
    # far left: x / (1 + e^87) (the exponent clamped at 87: e^87 = 6.08e37)
    g20 = orc.gelu(np.float32(-20.0))
    assert -3.4e-37 < g20 < -3.2e-37


# ------------------------------------------------------------ attention --
def _attn_ref(qkv, n_head, dh, scale, valid=None):
    H = n_head * dh
    q = qkv[:, :H].astype(np.float16).astype(np.float64)
    k = qkv[:, H:2 * H].astype(np.float16).astype(np.float64)
    v = qkv[:, 2 * H:].astype(np.float16).astype(np.float64)
    out = np.zeros((qkv.shape[0], H))
    for h in range(n_head):
        sl = slice(h * dh, (h + 1) * dh)
        s = q[:, sl] @ k[:, sl].T * scale
        if valid is not None:
            s[:, ~valid.astype(bool)] = -np.inf
        s -= s.max(1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(1, keepdims=True)
        out[:, sl] = p @ v[:, sl]
    return out


def test_attention_float64(orc):
    rng = np.random.default_rng(13)
    qkv = rng.standard_normal((70, 3 * 4 * 72)).astype(np.float32)
    scale = np.float32(1 / np.sqrt(72))
    out = orc.attention(qkv, 4, 72, scale)
    assert np.abs(out - _attn_ref(qkv, 4, 72, scale)).max() < 1e-6


def test_attention_mask_drops_keys(orc):
    rng = np.random.default_rng(14)
    qkv = rng.standard_normal((40, 3 * 2 * 72)).astype(np.float32)
    valid = np.ones(40, np.uint8)
    valid[25:] = 0
    scale = np.float32(0.1)
    out = orc.attention(qkv, 2, 72, scale, valid)
    assert np.abs(out - _attn_ref(qkv, 2, 72, scale, valid)).max() < 1e-6
    # masking equals dropping the rows as keys
    sub = orc.attention(qkv[:25], 2, 72, scale)
    assert np.abs(out[:25] - sub).max() < 1e-6


def test_attention_single_key_returns_v(orc):
    qkv = np.random.default_rng(15).standard_normal((1, 3 * 72)).astype(np.float32)
    out = orc.attention(qkv, 1, 72, np.float32(0.3))
    assert np.array_equal(out[0], qkv[0, 144:].astype(np.float16).astype(np.float32))


def test_attention_1q_float64_and_multi_query(orc):
    """The MAP head's single-query attention: against the float64 softmax
    reference, and equal to the multi-query restatement's row whose query it
    is (keys and values taken from rows of stride ld = 2H, as the head lays
    them out)."""
    rng = np.random.default_rng(16)
    n_head, dh, n = 4, 72, 300
    H = n_head * dh
    q = rng.standard_normal(H).astype(np.float32)
    kv = (rng.standard_normal((n, 2 * H)) * 1.3).astype(np.float32)
    scale = np.float32(1 / np.sqrt(72))
    out = orc.attention_1q(q, kv[:, :H], kv[:, H:], n_head, dh, scale)
    qkv = np.concatenate([np.tile(q, (n, 1)), kv], axis=1)
    assert np.abs(out - _attn_ref(qkv, n_head, dh, scale)[0]).max() < 1e-6
    assert np.array_equal(out, orc.attention(qkv, n_head, dh, scale)[0])
    # one key: the output is that key's f16 value row
    one = orc.attention_1q(q, kv[:1, :H], kv[:1, H:], n_head, dh, scale)
    assert np.array_equal(one, kv[0, H:].astype(np.float16).astype(np.float32))
