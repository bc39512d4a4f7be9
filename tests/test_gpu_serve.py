"""The service on the GPU: a server process (python -m s2x_serve, worker
isolation on: the GPU work runs in its worker process) over a small
two-tower GGUF and a SentencePiece model, its answers against libs2x called
directly in this process on the same decoded images and tokens -- the same
bits -- and its unload (the worker's end) and reload."""
import ctypes
import http.client
import io
import json
import os
import subprocess
import sys
import threading
import time
import uuid

import numpy as np
import pytest
import torch

import s2x
from s2x import synth
from gpu_util import say
from s2x_serve.engine import MEAN, RESCALE, STD, decode_image
from s2x_serve.scoring import l2_normalize, score_image_text
from s2x_serve.tokenizer import Tokenizer

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "hbd-siglip2.cpp_amd")
SMALL_V = synth.VisionConfig(hidden=288, inter=1076, n_head=4, n_layer=2)
SMALL_T = synth.TextConfig(hidden=288, inter=1076, n_head=4, n_layer=2, vocab=1000, max_pos=64, proj=288)
SCALE, BIAS = 2.302585, -3.5


def _images():
    from PIL import Image
    rng = np.random.default_rng(77)
    out = []
    for (h, w), fmt in (((48, 64), "PNG"), ((100, 80), "JPEG"), ((33, 129), "PNG")):
        im = Image.fromarray(rng.integers(0, 256, (h, w, 3), dtype=np.uint8))
        b = io.BytesIO()
        im.save(b, format=fmt)
        out.append(b.getvalue())
    return out


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    from gguf_util import score_tensors, text_tensors, vision_tensors, write_gguf
    import sentencepiece as spm
    d = tmp_path_factory.mktemp("serve")
    kv_v, ts_v = vision_tensors(synth.vision_model(SMALL_V, seed=31))
    kv_t, ts_t = text_tensors(synth.text_model(SMALL_T, seed=32))
    gguf = d / "model.gguf"
    write_gguf(gguf, kv_v + kv_t, ts_v + ts_t + score_tensors(SCALE, BIAS))
    corpus = d / "corpus.txt"
    corpus.write_text("\n".join(["a photo of a cat", "a photo of a dog", "a red car on the road",
                                 "two birds in the sky", "the quick brown fox jumps over the lazy dog",
                                 "siglip encodes images and text into one space"] * 20))
    spm.SentencePieceTrainer.train(input=str(corpus), model_prefix=str(d / "tok"), vocab_size=32,
                                   model_type="unigram", minloglevel=2)
    return str(gguf), str(d / "tok.model")


@pytest.fixture(scope="module")
def server(model):
    gguf, tok = model
    env = dict(os.environ)
    env["PYTHONPATH"] = PKG + os.pathsep + env.get("PYTHONPATH", "")
    say("serve: starting python -m s2x_serve (worker isolation on)")
    proc = subprocess.Popen([sys.executable, "-m", "s2x_serve", "--model", gguf, "--tokenizer", tok,
                             "--host", "127.0.0.1", "--port", "0"], env=env, stderr=subprocess.PIPE,
                            text=True)
    lines, port = [], []
    ready = threading.Event()

    def read():
        for line in proc.stderr:
            lines.append(line.rstrip())
            if "listening on" in line:
                port.append(int(line.split("listening on ")[1].split()[0].rsplit(":", 1)[1]))
                ready.set()
        ready.set()

    threading.Thread(target=read, daemon=True).start()
    ready.wait(timeout=300)
    if not port:
        proc.kill()
        pytest.fail("server did not start: " + " | ".join(lines[-10:]))
    say(f"serve: listening on port {port[0]}")
    yield port[0]
    proc.terminate()
    proc.wait(timeout=60)


def _post(port, path, body, ctype):
    c = http.client.HTTPConnection("127.0.0.1", port, timeout=300)
    c.request("POST", path, body=body, headers={"Content-Type": ctype} if ctype else {})
    r = c.getresponse()
    return r.status, json.loads(r.read())


def _get(port, path):
    c = http.client.HTTPConnection("127.0.0.1", port, timeout=60)
    c.request("GET", path)
    r = c.getresponse()
    return r.status, json.loads(r.read())


def _form(files=(), fields=()):
    bd = uuid.uuid4().hex
    parts = [f"--{bd}\r\nContent-Disposition: form-data; name=\"{n}\"; filename=\"i\"\r\n\r\n".encode()
             + d + b"\r\n" for n, d in files]
    parts += [f"--{bd}\r\nContent-Disposition: form-data; name=\"{n}\"\r\n\r\n{v}\r\n".encode()
              for n, v in fields]
    return b"".join(parts) + f"--{bd}--\r\n".encode(), f"multipart/form-data; boundary={bd}"


@pytest.fixture(scope="module")
def direct(model):
    """The towers built in this process from the same file."""
    gguf, tok = model
    g = ctypes.c_void_p()
    s2x.call("s2x_gguf_open", gguf.encode(), ctypes.byref(g))
    try:
        vw, tw = s2x.VisionWeights(), s2x.TextWeights()
        s2x.call("s2x_gguf_vision_weights", g, ctypes.byref(vw))
        s2x.call("s2x_gguf_text_weights", g, ctypes.byref(tw))
        v, t = ctypes.c_void_p(), ctypes.c_void_p()
        s2x.call("s2x_vision_create", ctypes.byref(vw), ctypes.byref(v))
        s2x.call("s2x_text_create", ctypes.byref(tw), ctypes.byref(t))
        # the vision encoder on torch's stream: torch.cuda.synchronize() waits for it
        s2x.call("s2x_vision_set_stream", v, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    finally:
        s2x.lib.s2x_gguf_close(g)
    tk = Tokenizer(tok)

    def images(blobs, pooling, mnp):
        ims = [decode_image(b) for b in blobs]
        devs = [torch.from_numpy(im).to("cuda:0") for im in ims]
        ptrs = (ctypes.c_void_p * len(devs))(*[d.data_ptr() for d in devs])
        hw = np.array([[im.shape[0], im.shape[1]] for im in ims], np.int32)
        out = torch.empty((len(ims), SMALL_V.hidden), dtype=torch.float32, device="cuda:0")
        torch.cuda.synchronize()
        s2x.call("s2x_vision_encode_rgb_batch_dev", v, ptrs, hw.ctypes.data, len(ims), mnp,
                 ctypes.c_float(RESCALE), (ctypes.c_float * 3)(*MEAN), (ctypes.c_float * 3)(*STD),
                 pooling, ctypes.c_void_p(out.data_ptr()))
        torch.cuda.synchronize()
        return out.cpu().numpy()

    def texts(prompts):
        ids = np.array([tk.encode(p, SMALL_T.max_pos)[0] for p in prompts], np.int32)
        out = np.empty((len(prompts), SMALL_T.proj), np.float32)
        s2x.call("s2x_text_encode_batch", t, ids.ctypes.data, SMALL_T.max_pos, len(prompts),
                 out.ctypes.data)
        return out

    yield images, texts
    s2x.lib.s2x_vision_destroy(v)
    s2x.lib.s2x_text_destroy(t)


def test_serve_equals_direct_calls(server, direct):
    images, texts = direct
    blobs = _images()
    prompts = ["a photo of a cat", "a red car", "two birds in the sky over a lake at dawn"]
    port = server
    st, h = _get(port, "/health")
    say(f"serve: health {h}")
    assert st == 200 and h["model_loaded"] is True and h["worker_pid"] > 0
    say("serve: /v1/embeddings (probe, default 729 patches; mean, 256)")
    st, body = _post(port, "/v1/embeddings", *_form([("images", b) for b in blobs]))
    assert st == 200, body
    want = l2_normalize(images(blobs, s2x.POOL_PROBE, 729))
    assert np.array_equal(np.float32(body["embeddings"]), want)
    st, body = _post(port, "/v1/embeddings?pooling=mean&max_num_patches=256", *_form([("images", blobs[1])]))
    assert st == 200 and np.array_equal(np.float32(body["embeddings"]),
                                        l2_normalize(images(blobs[1:2], s2x.POOL_MEAN, 256)))
    say("serve: /v1/text_embeddings")
    st, body = _post(port, "/v1/text_embeddings", *_form(fields=[("prompts", p) for p in prompts]))
    assert st == 200 and np.array_equal(np.float32(body["embeddings"]), l2_normalize(texts(prompts)))
    say("serve: /v1/classify")
    st, body = _post(port, "/v1/classify?return_logits=true",
                     *_form([("images", b) for b in blobs], [("prompts", p) for p in prompts]))
    assert st == 200
    logits, probs = score_image_text(images(blobs, s2x.POOL_PROBE, 729), texts(prompts), SCALE, BIAS)
    assert np.array_equal(np.float32(body["scores"]), probs)
    assert np.array_equal(np.float32(body["logits"]), logits)
    say("serve: /v1/classify_from_embeddings")
    emb = l2_normalize(images(blobs, s2x.POOL_PROBE, 729))
    st, body = _post(port, "/v1/classify_from_embeddings",
                     json.dumps({"image_embeddings": emb.tolist(), "prompts": prompts}).encode(),
                     "application/json")
    assert st == 200
    assert np.array_equal(np.float32(body["scores"]), score_image_text(emb, texts(prompts), SCALE, BIAS)[1])
    st, body = _post(port, "/v1/embeddings", *_form([("images", b"not an image")]))
    assert st == 500 and "decode" in body["error"]


def test_serve_unload_ends_worker_and_reload_gives_same_bits(server, direct):
    images, _ = direct
    port = server
    pid = _get(port, "/health")[1]["worker_pid"]
    say(f"serve: unload (worker pid {pid})")
    st, body = _post(port, "/v1/admin/unload", b"", None)
    assert st == 200 and body["unloaded"] is True and body["model_loaded"] is False
    t0 = time.monotonic()
    while time.monotonic() - t0 < 30:
        try:
            os.kill(pid, 0)
        except ProcessLookupError:
            break
        time.sleep(0.1)
    with pytest.raises(ProcessLookupError):
        os.kill(pid, 0)
    assert _get(port, "/health")[1]["model_loaded"] is False
    say("serve: reload through a request")
    blobs = _images()[:1]
    st, body = _post(port, "/v1/embeddings", *_form([("images", blobs[0])]))
    assert st == 200
    assert np.array_equal(np.float32(body["embeddings"]), l2_normalize(images(blobs, s2x.POOL_PROBE, 729)))
    assert _get(port, "/health")[1]["worker_pid"] not in (pid, -1)
