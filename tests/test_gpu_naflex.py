"""NaFlex front end on the GPU, through the C-ABI, against the oracle's
restatement of src/siglip2_preproc.cpp (itself pinned to the reference's own
build in test_naflex.py): bit-exact patches and grids for down- and
up-sampling, extreme aspect ratios, a 1x1 image and several patch budgets."""
import ctypes

import numpy as np
import pytest
import torch

import pyoracle
import s2x
from gpu_util import dev, empty, host, ptr, say, stream

pytestmark = pytest.mark.gpu

MEAN = np.array([0.5, 0.5, 0.5], np.float32)
STD = np.array([0.5, 0.5, 0.5], np.float32)


def _gpu_preprocess(img, mp, p=16, rescale=1.0 / 255.0, mean=MEAN, std=STD):
    h, w = img.shape[:2]
    d = dev(np.ascontiguousarray(img))
    cap = mp * 3 * p * p
    out = empty((cap,), torch.float32)
    wsb = s2x.lib.s2x_nf_workspace_size(h, w, p, mp)
    ws = empty((wsb,), torch.uint8)
    nh, nw = ctypes.c_int32(), ctypes.c_int32()
    s2x.call("s2x_nf_preprocess_rgb_dev", ptr(d), h, w, mp, p, ctypes.c_float(rescale),
             mean.ctypes.data, std.ctypes.data, ptr(out), cap, ctypes.byref(nh), ctypes.byref(nw),
             ptr(ws), ctypes.c_size_t(wsb), stream())
    n = nh.value * nw.value
    return host(out)[: n * 3 * p * p].reshape(n, 3 * p * p), nh.value, nw.value


@pytest.mark.parametrize("h,w,mp,p,seed", [
    (480, 640, 256, 16, 1), (1000, 300, 729, 16, 2), (432, 432, 729, 16, 3), (100, 100, 1024, 16, 4),
    (2000, 1500, 729, 16, 5), (17, 23, 256, 16, 6), (1, 1, 729, 16, 7), (1, 1500, 256, 16, 8),
    (720, 1280, 729, 14, 9), (3000, 4000, 1024, 16, 10),
])
def test_preprocess_matches_oracle(h, w, mp, p, seed):
    say(f"naflex {h}x{w} max_patches={mp} p={p}")
    img = np.random.default_rng(seed).integers(0, 256, (h, w, 3), dtype=np.uint8)
    got, nh, nw = _gpu_preprocess(img, mp, p)
    ref, rh, rw = pyoracle.nf_preprocess_rgb(img, mp, p=p, fused=1)
    assert (nh, nw) == (rh, rw)
    assert np.array_equal(got, ref)


def test_preprocess_other_normalisation():
    img = np.random.default_rng(11).integers(0, 256, (300, 500, 3), dtype=np.uint8)
    mean = np.array([0.48145466, 0.4578275, 0.40821073], np.float32)
    std = np.array([0.26862954, 0.26130258, 0.27577711], np.float32)
    got, nh, nw = _gpu_preprocess(img, 576, mean=mean, std=std)
    ref, _, _ = pyoracle.nf_preprocess_rgb(img, 576, mean=mean, std=std, fused=1)
    assert np.array_equal(got, ref)


def test_preprocess_workspace_and_capacity_errors():
    img = dev(np.zeros((64, 64, 3), np.uint8))
    out = empty((16 * 768,), torch.float32)
    need = s2x.lib.s2x_nf_workspace_size(64, 64, 16, 16)
    ws = empty((need,), torch.uint8)
    nh, nw = ctypes.c_int32(), ctypes.c_int32()
    args = lambda cap, wsb: (ptr(img), 64, 64, 16, 16, ctypes.c_float(1 / 255), MEAN.ctypes.data,  # noqa: E731
                             STD.ctypes.data, ptr(out), cap, ctypes.byref(nh), ctypes.byref(nw),
                             ptr(ws), ctypes.c_size_t(wsb), stream())
    assert s2x.lib.s2x_nf_preprocess_rgb_dev(*args(16 * 768, need - 4)) == 4  # S2X_ERR_WORKSPACE
    assert s2x.lib.s2x_nf_preprocess_rgb_dev(*args(16 * 768 - 1, need)) == 1
    assert s2x.lib.s2x_nf_preprocess_rgb_dev(*args(16 * 768, need)) == 0
    torch.cuda.synchronize()
    assert (nh.value, nw.value) == (4, 4)


@pytest.mark.parametrize("h,w,mp,n_img", [(480, 640, 729, 5), (17, 23, 256, 3), (1000, 300, 729, 1)])
def test_preprocess_batch_matches_per_image(h, w, mp, n_img):
    # one call for n_img same-size images: each image's patches equal the
    # single-image entry point's (and so the oracle's)
    say(f"naflex batch {n_img} x {h}x{w} max_patches={mp}")
    p = 16
    rng = np.random.default_rng(20 + n_img)
    imgs = rng.integers(0, 256, (n_img, h, w, 3), dtype=np.uint8)
    d = dev(imgs)
    th, tw = ctypes.c_int32(), ctypes.c_int32()
    s2x.call("s2x_nf_target_size", h, w, p, mp, ctypes.byref(th), ctypes.byref(tw))
    per = (th.value // p) * (tw.value // p) * 3 * p * p
    out = empty((n_img * per,), torch.float32)
    wsb = n_img * s2x.lib.s2x_nf_workspace_size(h, w, p, mp)
    ws = empty((wsb,), torch.uint8)
    nh, nw = ctypes.c_int32(), ctypes.c_int32()
    s2x.call("s2x_nf_preprocess_rgb_batch_dev", ptr(d), n_img, h, w, mp, p,
             ctypes.c_float(1.0 / 255.0), MEAN.ctypes.data, STD.ctypes.data, ptr(out), per,
             ctypes.byref(nh), ctypes.byref(nw), ptr(ws), ctypes.c_size_t(wsb), stream())
    got = host(out).reshape(n_img, per)
    for i in range(n_img):
        one, oh, ow = _gpu_preprocess(imgs[i], mp, p)
        assert (nh.value, nw.value) == (oh, ow)
        assert np.array_equal(got[i], one.reshape(-1)), f"image {i}"
    # a workspace one byte short of n_img images is rejected before any launch
    st = s2x.lib.s2x_nf_preprocess_rgb_batch_dev(
        ptr(d), n_img, h, w, mp, p, ctypes.c_float(1.0 / 255.0), MEAN.ctypes.data,
        STD.ctypes.data, ptr(out), per, ctypes.byref(nh), ctypes.byref(nw), ptr(ws),
        ctypes.c_size_t(wsb - 1), stream())
    assert st != 0
