"""The reference-shaped C++ classes (include/siglip2_vision.h, siglip2_text.h,
siglip2_preproc.h) executed by a program compiled against them
(tests/cpp/drop_in_driver, built by build()): VisionEncoder::load + encode,
TextEncoder::load + encode / encode_batch and preprocess_image_rgb must give
the C-ABI's results bit for bit (and the oracle's NaFlex patches)."""
import ctypes
import os
import subprocess

import numpy as np
import pytest
import torch

import pyoracle
import s2x
from s2x import synth
from gguf_util import text_tensors, vision_tensors, write_gguf
from gpu_util import dev, empty, host, ptr, say

pytestmark = pytest.mark.gpu

DRIVER = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "drop_in_driver")
SMALL_V = synth.VisionConfig(hidden=288, inter=1076, n_head=4, n_layer=2)
SMALL_T = synth.TextConfig(hidden=288, inter=1076, n_head=4, n_layer=2, vocab=1000, max_pos=64,
                           proj=288)


def _run(*args):
    say("drop_in_driver " + " ".join(str(a) for a in args[:2]))
    r = subprocess.run([DRIVER, *[str(a) for a in args]], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0, r.stderr
    return r.stdout


@pytest.fixture(scope="module", autouse=True)
def _driver_built():
    if not os.access(DRIVER, os.X_OK):
        pytest.fail("tests/cpp/drop_in_driver is not built (run __graft_entry__.build())")


@pytest.mark.parametrize("down_f16", [False, True])
def test_vision_encoder_class(tmp_path, down_f16):
    hm = synth.vision_model(SMALL_V, seed=61, down_f16=down_f16)
    path = tmp_path / "v.gguf"
    write_gguf(path, *vision_tensors(hm))
    g = ctypes.c_void_p()
    s2x.call("s2x_gguf_open", str(path).encode(), ctypes.byref(g))
    try:
        w = s2x.VisionWeights()
        s2x.call("s2x_gguf_vision_weights", g, ctypes.byref(w))
        h = ctypes.c_void_p()
        s2x.call("s2x_vision_create", ctypes.byref(w), ctypes.byref(h))
    finally:
        s2x.lib.s2x_gguf_close(g)
    try:
        for (n_h, n_w), pool in [((27, 27), 1), ((12, 20), 0)]:
            px = synth.pixels(1, n_h * n_w, seed=62 + n_h)
            want = np.empty(SMALL_V.hidden, np.float32)
            s2x.call("s2x_vision_encode", h, px.ctypes.data, n_h, n_w, pool, want.ctypes.data)
            (tmp_path / "px.f32").write_bytes(px.tobytes())
            _run("vision", path, tmp_path / "px.f32", n_h, n_w, pool, tmp_path / "out.f32")
            got = np.fromfile(tmp_path / "out.f32", np.float32)
            assert np.array_equal(got, want), (n_h, n_w, pool)
    finally:
        s2x.lib.s2x_vision_destroy(h)
    out = _run("badload", tmp_path / "missing.gguf")
    assert "missing.gguf" in out


def test_text_encoder_class(tmp_path):
    hm = synth.text_model(SMALL_T, seed=63)
    path = tmp_path / "t.gguf"
    write_gguf(path, *text_tensors(hm))
    g = ctypes.c_void_p()
    s2x.call("s2x_gguf_open", str(path).encode(), ctypes.byref(g))
    try:
        w = s2x.TextWeights()
        s2x.call("s2x_gguf_text_weights", g, ctypes.byref(w))
        h = ctypes.c_void_p()
        s2x.call("s2x_text_create", ctypes.byref(w), ctypes.byref(h))
    finally:
        s2x.lib.s2x_gguf_close(g)
    try:
        ids, _ = synth.text_tokens(4, 64, vocab=SMALL_T.vocab, seed=64)
        ids = np.ascontiguousarray(ids, np.int32)
        want = np.empty((4, SMALL_T.proj), np.float32)
        s2x.call("s2x_text_encode_batch", h, ids.ctypes.data, 64, 4, want.ctypes.data)
        (tmp_path / "ids.i32").write_bytes(ids.tobytes())
        _run("text", path, tmp_path / "ids.i32", 64, 4, tmp_path / "out.f32")
        assert np.array_equal(np.fromfile(tmp_path / "out.f32", np.float32).reshape(4, -1), want)
        one = np.ascontiguousarray(ids[2, :23])
        want1 = np.empty(SMALL_T.proj, np.float32)
        s2x.call("s2x_text_encode", h, one.ctypes.data, 23, None, want1.ctypes.data)
        (tmp_path / "one.i32").write_bytes(one.tobytes())
        _run("text", path, tmp_path / "one.i32", 23, 1, tmp_path / "one.f32")
        assert np.array_equal(np.fromfile(tmp_path / "one.f32", np.float32), want1)
    finally:
        s2x.lib.s2x_text_destroy(h)


@pytest.mark.parametrize("h,w,mp", [(480, 640, 729), (300, 1000, 256), (17, 23, 576)])
def test_preprocess_image_rgb(tmp_path, h, w, mp):
    img = np.random.default_rng(h + w).integers(0, 256, (h, w, 3), dtype=np.uint8)
    (tmp_path / "rgb.u8").write_bytes(img.tobytes())
    out = _run("preproc", tmp_path / "rgb.u8", h, w, mp, tmp_path / "px.f32")
    nh, nw = (int(v) for v in out.split())
    ref, rh, rw = pyoracle.nf_preprocess_rgb(img, mp, p=16, fused=1)
    assert (nh, nw) == (rh, rw)
    assert np.array_equal(np.fromfile(tmp_path / "px.f32", np.float32).reshape(ref.shape), ref)


# ---------------------------------------------------------------- CLIs ----
BIN = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "hbd-siglip2.cpp_amd",
                   "bin")


def _cli(name, *args, rc=0):
    say(f"{name} " + " ".join(str(a) for a in args[:4]))
    r = subprocess.run([os.path.join(BIN, name), *[str(a) for a in args]], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == rc, (r.returncode, r.stderr)
    return r


def test_vision_cli(tmp_path):
    """siglip2-cli with the reference's raw-file contract: --pixel-values on
    a given and on the default grid, --rgb through the GPU front end, each
    --out equal to the C-ABI's encode bit for bit; --image fails (no image
    decoder) with exit code 1, as a failed preprocess does."""
    hm = synth.vision_model(SMALL_V, seed=71)
    path = tmp_path / "v.gguf"
    write_gguf(path, *vision_tensors(hm))
    h = ctypes.c_void_p()
    s2x.call("s2x_vision_create", ctypes.byref(hm.struct), ctypes.byref(h))
    try:
        for (n_h, n_w), pool, args in [((12, 20), 0, ["--shape", "12,20", "--pooling", "mean"]),
                                       ((16, 16), 1, [])]:
            px = synth.pixels(1, n_h * n_w, seed=72 + n_h)
            (tmp_path / "px.f32").write_bytes(px.tobytes())
            want = np.empty(SMALL_V.hidden, np.float32)
            s2x.call("s2x_vision_encode", h, px.ctypes.data, n_h, n_w, pool, want.ctypes.data)
            _cli("siglip2-cli", "--model", path, "--pixel-values", tmp_path / "px.f32", *args,
                 "--out", tmp_path / "out.f32")
            assert np.array_equal(np.fromfile(tmp_path / "out.f32", np.float32), want), (n_h, n_w)
        img = np.random.default_rng(73).integers(0, 256, (300, 500, 3), dtype=np.uint8)
        (tmp_path / "img.rgb").write_bytes(img.tobytes())
        r = _cli("siglip2-cli", "--model", path, "--rgb", tmp_path / "img.rgb", "--rgb-shape",
                 "300,500", "--max-num-patches", "256", "--out", tmp_path / "rgb.f32")
        ref, nh, nw = pyoracle.nf_preprocess_rgb(img, 256, p=16, fused=1)
        assert f"grid={nh}x{nw}" in r.stderr
        want = np.empty(SMALL_V.hidden, np.float32)
        ref = np.ascontiguousarray(ref, np.float32)
        s2x.call("s2x_vision_encode", h, ref.ctypes.data, nh, nw, 1, want.ctypes.data)
        assert np.array_equal(np.fromfile(tmp_path / "rgb.f32", np.float32), want)
        r = _cli("siglip2-cli", "--model", path, "--image", tmp_path / "img.png", rc=1)
        assert "preprocess failed" in r.stderr
        r = _cli("siglip2-cli", "--model", path, "--pixel-values", tmp_path / "px.f32",
                 "--shape", "8,8", rc=1)
        assert "size mismatch" in r.stderr
    finally:
        s2x.lib.s2x_vision_destroy(h)


def test_text_cli(tmp_path):
    """siglip2-text-cli --token-ids / --attention-mask (int32 files of one
    length) equal to the C-ABI's masked encode bit for bit."""
    hm = synth.text_model(SMALL_T, seed=74)
    path = tmp_path / "t.gguf"
    write_gguf(path, *text_tensors(hm))
    h = ctypes.c_void_p()
    s2x.call("s2x_text_create", ctypes.byref(hm.struct), ctypes.byref(h))
    try:
        ids, _ = synth.text_tokens(1, 40, vocab=SMALL_T.vocab, seed=75)
        ids = np.ascontiguousarray(ids[0], np.int32)
        mask = np.ones(40, np.int32)
        mask[33:] = 0
        (tmp_path / "ids.i32").write_bytes(ids.tobytes())
        (tmp_path / "mask.i32").write_bytes(mask.tobytes())
        want = np.empty(SMALL_T.proj, np.float32)
        s2x.call("s2x_text_encode", h, ids.ctypes.data, 40, mask.ctypes.data, want.ctypes.data)
        _cli("siglip2-text-cli", "--model", path, "--token-ids", tmp_path / "ids.i32",
             "--attention-mask", tmp_path / "mask.i32", "--out", tmp_path / "out.f32")
        assert np.array_equal(np.fromfile(tmp_path / "out.f32", np.float32), want)
        (tmp_path / "short.i32").write_bytes(mask[:7].tobytes())
        r = _cli("siglip2-text-cli", "--model", path, "--token-ids", tmp_path / "ids.i32",
                 "--attention-mask", tmp_path / "short.i32", rc=1)
        assert "size mismatch" in r.stderr
    finally:
        s2x.lib.s2x_text_destroy(h)
