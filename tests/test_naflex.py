"""NaFlex front end (src/siglip2_preproc.cpp), host side: the oracle's
restatement is pinned to the reference's own code -- src/siglip2_preproc.cpp
compiled from the reference tree with its release flags into oracle/_ref/
(`make -C oracle ref`) -- bit for bit on a spread of image sizes, aspect
ratios, down- and up-sampling and patch budgets; the same restatement with
every product rounded on its own must NOT match (the reference's build fuses
them), so the comparison is known to discriminate.  The library's host-side
grid search is checked against the oracle and against the invariants of the
grid; argument checks need no GPU."""
import ctypes

import numpy as np
import pytest

import pyoracle
import s2x

CASES = [  # (h, w, max_num_patches)
    (480, 640, 256), (1000, 300, 729), (432, 432, 729), (100, 100, 1024), (33, 700, 576),
    (512, 512, 256), (2000, 1500, 729), (17, 23, 256), (640, 480, 1024), (300, 1000, 576),
    (1, 1, 729), (1, 1500, 256), (1500, 2, 729), (224, 224, 196), (720, 1280, 729),
]


def _image(h, w, seed):
    rng = np.random.default_rng(seed)
    if seed % 2:
        return rng.integers(0, 256, (h, w, 3), dtype=np.uint8)
    # smooth gradients + noise: many filter sums land near .5 steps
    yy, xx = np.mgrid[0:h, 0:w]
    base = (yy * 255.0 / max(h - 1, 1))[..., None] * np.array([1.0, 0.3, 0.7]) + \
        (xx * 255.0 / max(w - 1, 1))[..., None] * np.array([0.0, 0.7, 0.3])
    return np.clip(base + rng.normal(0, 3, (h, w, 3)), 0, 255).astype(np.uint8)


need_ref = pytest.mark.skipif(pyoracle.ref_preprocess_lib() is None,
                              reason="oracle/_ref/libref_preproc.so absent (reference tree not present)")


@need_ref
@pytest.mark.parametrize("i", range(len(CASES)))
def test_oracle_preprocess_equals_reference_build(i):
    h, w, mp = CASES[i]
    img = _image(h, w, i)
    ref, nh, nw = pyoracle.ref_preprocess_rgb(img, mp)
    got, gh, gw = pyoracle.nf_preprocess_rgb(img, mp, fused=1)
    assert (gh, gw) == (nh, nw)
    assert np.array_equal(got, ref)


@need_ref
def test_unfused_restatement_is_caught():
    # a plausible mistake (products rounded before the adds) must fail the
    # comparison above on these inputs
    mismatches = 0
    for i in range(4):
        h, w, mp = CASES[i]
        img = _image(h, w, i)
        ref, _, _ = pyoracle.ref_preprocess_rgb(img, mp)
        got, _, _ = pyoracle.nf_preprocess_rgb(img, mp, fused=0)
        mismatches += not np.array_equal(got, ref)
    assert mismatches == 4


@pytest.mark.parametrize("h,w,p,mp", [(480, 640, 16, 256), (1, 1, 16, 729), (7, 4000, 16, 729),
                                      (4000, 7, 14, 576), (432, 432, 16, 729), (999, 1001, 16, 1024),
                                      (300, 300, 32, 64)])
def test_target_size(h, w, p, mp):
    th, tw = ctypes.c_int32(), ctypes.c_int32()
    s2x.call("s2x_nf_target_size", h, w, p, mp, ctypes.byref(th), ctypes.byref(tw))
    assert (th.value, tw.value) == pyoracle.nf_target_size(h, w, p, mp)
    assert th.value % p == 0 and tw.value % p == 0 and th.value >= p and tw.value >= p
    assert (th.value // p) * (tw.value // p) <= mp or (th.value, tw.value) == (p, p)


def test_preprocess_rejects_bad_arguments():
    th, tw = ctypes.c_int32(), ctypes.c_int32()
    assert s2x.lib.s2x_nf_target_size(0, 10, 16, 256, ctypes.byref(th), ctypes.byref(tw)) == 1
    assert s2x.lib.s2x_nf_target_size(10, 10, 0, 256, ctypes.byref(th), ctypes.byref(tw)) == 1
    assert s2x.lib.s2x_nf_workspace_size(10, 10, 16, 0) == 0
    out = ctypes.c_void_p(16)
    st = s2x.lib.s2x_nf_preprocess_rgb_dev(None, 10, 10, 256, 16, ctypes.c_float(1 / 255), None,
                                           None, out, 10, None, None, None, 0, None)
    assert st == 1
