"""The oracle's three GELU modes (CPU).

  GELU_EXACT  orc_gelu: x / (1 + e^(-2g)), the GPU's formulation bit for bit
  GELU_TANHF  0.5 x (1 + tanhf(g)): src/cuda/siglip2_megakernel.cu:276-280 as
              written, host libm tanhf
  GELU_GGML   ggml-cpu's default fp16-table GELU (GGML_GELU_FP16) [ggml, not in
              the reference tree]: clamps at +-10, else table[fp16(x)]

Each is pinned against float64 mathematics or an independent numpy
construction here; the divergence figures between them are measured in
test_gelu_mode_divergence."""
import numpy as np
import pytest

import pyoracle as po

G = np.sqrt(2.0 / np.pi)


def gelu64(x):
    """GELU tanh form in float64, through the well-conditioned identity."""
    x = np.asarray(x, np.float64)
    return x / (1.0 + np.exp(-2.0 * G * x * (1.0 + 0.044715 * x * x)))


def test_ggml_table_clamps_and_known_values():
    x = np.array([-1e6, -10.0, -10.0001, 10.0, 10.5, 1e6, 0.0], np.float32)
    y = po.gelu_mode(po.GELU_GGML, x)
    assert np.array_equal(y[:3], [0.0, 0.0, 0.0])           # x <= -10 -> 0
    assert np.array_equal(y[3:6], x[3:6])                     # x >= 10 -> x
    assert y[6] == 0.0


def test_ggml_table_equals_independent_fp16_table():
    """Every fp16 input in (-10, 10): the table value must be fp16 of the
    tanh-form GELU of that fp16 value.  numpy's float32 tanh is another
    implementation than libm's tanhf: where 1 + tanh(g) cancels (x below
    about -1.8) a 1-ulp difference between the two is amplified and may
    move the fp16 rounding of the (small) result by a few f16 ulps; above
    that every entry must agree."""
    h = np.arange(0, 1 << 16, dtype=np.uint32).astype(np.uint16).view(np.float16)
    x = h.astype(np.float32)
    x = x[np.isfinite(x) & (x > -10) & (x < 10)]
    got = po.gelu_mode(po.GELU_GGML, x)
    x32 = x.astype(np.float32)
    ref = (np.float32(0.5) * x32 * (np.float32(1.0) + np.tanh(np.float32(G) * x32 *
           (np.float32(1.0) + np.float32(0.044715) * x32 * x32)))).astype(np.float16).astype(np.float32)
    same = got == ref
    tail = x < -1.75
    assert same[~tail].all(), x[~tail][~same[~tail]][:8]
    assert same[tail].mean() > 0.85, same[tail].mean()  # measured 0.908
    gi = got.astype(np.float16).view(np.int16).astype(np.int32)
    ri = ref.astype(np.float16).view(np.int16).astype(np.int32)
    assert np.abs(gi - ri)[~same].max(initial=0) <= 4
    assert np.abs(got - ref).max() < 1e-4


def test_modes_against_float64():
    """Where |GELU| >= 2^-10 (away from the negative tail, where 1 + tanh(g)
    cancels): the exact mode within 2e-6 relative, the tanhf form within
    1e-4, the fp16 table within fp16's half-ulp 2^-11 (5e-3 with the fp16
    rounding of the input)."""
    x = np.linspace(-12, 12, 1 << 20, dtype=np.float32)
    ref = gelu64(x)
    big = np.abs(ref) >= 2.0 ** -10
    for mode, tol in ((po.GELU_EXACT, 2e-6), (po.GELU_TANHF, 1e-4), (po.GELU_GGML, 5e-3)):
        y = po.gelu_mode(mode, x).astype(np.float64)
        rel = np.abs(y - ref)[big] / np.abs(ref[big])
        assert rel.max() < tol, (mode, rel.max())
        # absolute error everywhere, scaled by max(|x|, 1)
        assert (np.abs(y - ref) / np.maximum(np.abs(x), 1.0)).max() < max(tol, 2e-7), mode


def test_exact_mode_is_the_gpu_formulation():
    """GELU_EXACT is orc_gelu itself (the per-element entry point)."""
    x = np.random.default_rng(3).normal(0, 3, 2000).astype(np.float32)
    assert np.array_equal(po.gelu_mode(po.GELU_EXACT, x), po.gelu(x))


def test_gelu_mode_divergence():
    """How far the GPU's formulation is from the reference CUDA formula and
    from ggml-cpu's table, on fc1-like pre-activations (N(0, 0.7) + a bias
    N(0, 0.02), rows of 4,320): the share of Q8_1 blocks whose quants or
    scales change when each is quantized.  Measured: 0.016 % (tanhf form),
    64 % (fp16 table)."""
    rng = np.random.default_rng(5)
    M, F = 512, 4320
    pre = (rng.standard_normal((M, F)) * 0.7 + rng.normal(0, 0.02, F)).astype(np.float32)
    q = {}
    for mode in (po.GELU_EXACT, po.GELU_TANHF, po.GELU_GGML):
        qs, ds = po.quantize_q8_1(po.gelu_mode(mode, pre), F)
        q[mode] = (np.asarray(qs).reshape(M, F // 32, 32), np.asarray(ds).reshape(M, F // 32, -1))

    def changed(a, b):
        return (np.any(q[a][0] != q[b][0], axis=2) | np.any(q[a][1] != q[b][1], axis=2)).mean()
    assert changed(po.GELU_EXACT, po.GELU_TANHF) < 1e-3
    assert 0.3 < changed(po.GELU_EXACT, po.GELU_GGML) < 0.9


def test_mode_switch_reaches_the_tower():
    """The tower restatements use the selected mode (a small tower: the
    ggml table moves the embedding, slightly), and the switch restores."""
    from s2x import synth
    cfg = synth.VisionConfig(hidden=288, inter=1076, n_head=4, n_layer=2)
    m = po.vision_model(synth.vision_model(cfg, seed=3))
    px = synth.pixels(1, 256, seed=4)
    e0 = po.vision_encode(m, px, 16, 16, pooling=1)
    prev = po.set_gelu_mode(po.GELU_GGML)
    try:
        e2 = po.vision_encode(m, px, 16, 16, pooling=1)
    finally:
        assert po.set_gelu_mode(prev) == po.GELU_GGML
    assert not np.array_equal(e0, e2)
    cos = float(np.dot(e0, e2) / np.linalg.norm(e0) / np.linalg.norm(e2))
    assert cos > 0.999, cos
    assert np.array_equal(po.vision_encode(m, px, 16, 16, pooling=1), e0)
