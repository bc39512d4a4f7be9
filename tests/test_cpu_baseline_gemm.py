"""The CPU baseline's AVX-512 VNNI Q8_0 x Q8_1 kernel (oracle/cpu_q8.c)
must give the oracle's block-order GEMM bit for bit: ragged shapes (N not a
multiple of 16, M not a multiple of 4, K of 1 to 135 blocks), extreme
quants (-128), and whole towers run with either kernel.  CPU only; skipped
on a CPU without AVX-512 VNNI (the baseline then runs the oracle's loop)."""
import time

import numpy as np
import pytest

from s2x import synth

pytestmark = pytest.mark.filterwarnings("ignore")


@pytest.fixture(scope="module")
def vnni(orc):
    if not orc.have_vnni():
        pytest.skip("no AVX-512 VNNI on this CPU")
    return orc


@pytest.mark.parametrize("M,N,KB", [(1, 16, 1), (5, 37, 3), (64, 1152, 36), (33, 4304, 36),
                                    (9, 1152, 135), (4, 3, 2)])
def test_vnni_gemm_bit_exact(vnni, M, N, KB):
    orc = vnni
    rng = np.random.default_rng(M * 1000 + N + KB)
    K_pad = 32 * KB
    K = K_pad - (7 if KB > 1 else 0)
    raw = synth.quantize_q8_0(rng.normal(0, 0.02, (N, K)).astype(np.float32), K_pad)
    if N > 2:  # a block of -128 quants (raw files may hold them)
        blk = raw.reshape(N, KB, 34)
        blk[2, 0, 2:] = np.uint8(0x80)
    x = rng.standard_normal((M, K)).astype(np.float32) * 3
    prev = orc.set_gemm_kernel(0)
    try:
        ref = orc.mul_mat_q8_0_f32(raw, K_pad, N, x)
        orc.set_gemm_kernel(1)
        got = orc.mul_mat_q8_0_f32(raw, K_pad, N, x)
        got2 = orc.mul_mat_q8_0_f32(raw, K_pad, N, x)  # the cached repack
    finally:
        orc.set_gemm_kernel(prev)
        orc.lib().orc_clear_gemm_cache()
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    assert np.array_equal(got2.view(np.uint32), ref.view(np.uint32))


def test_vnni_tower_equals_oracle_tower(vnni):
    orc = vnni
    cfg = synth.VisionConfig(hidden=288, inter=1076, n_head=4, n_layer=2)
    m = orc.vision_model(synth.vision_model(cfg, seed=21))
    px = synth.pixels(1, 256, seed=22)
    prev = orc.set_gemm_kernel(0)
    try:
        ref = orc.vision_encode(m, px, 16, 16, pooling=1)
        orc.set_gemm_kernel(1)
        got = orc.vision_encode(m, px, 16, 16, pooling=1)
    finally:
        orc.set_gemm_kernel(prev)
        orc.lib().orc_clear_gemm_cache()
    assert np.array_equal(got, ref)


def test_vnni_gemm_is_faster(vnni):
    """The point of the kernel: the so400m fc1 shape (729 x 4304 x 1152)."""
    orc = vnni
    rng = np.random.default_rng(1)
    raw = synth.quantize_q8_0(rng.normal(0, 0.02, (4304, 1152)).astype(np.float32), 1152)
    x = rng.standard_normal((729, 1152)).astype(np.float32)
    t = {}
    prev = orc.set_gemm_kernel(0)
    try:
        for k in (0, 1):
            orc.set_gemm_kernel(k)
            orc.mul_mat_q8_0_f32(raw, 1152, 4304, x)
            t0 = time.perf_counter()
            orc.mul_mat_q8_0_f32(raw, 1152, 4304, x)
            t[k] = time.perf_counter() - t0
    finally:
        orc.set_gemm_kernel(prev)
        orc.lib().orc_clear_gemm_cache()
    print(f"fc1 729x4304x1152: loop {t[0] * 1e3:.1f} ms, VNNI {t[1] * 1e3:.1f} ms")
    assert t[1] < t[0]
