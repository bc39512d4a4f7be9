"""The SigLIP2 service (s2x_serve) on the CPU: worker frames, the
tokenizer's reference semantics, the scores' formula, the configuration,
every route through a real HTTP socket against a stand-in engine
(tests/serve_stub.py), in-process and through worker processes (spawn,
unload = kill, restart after an unload or a crash, errors carried back),
and the idle unload.  The GPU engine itself is tested in
tests/test_gpu_serve.py."""
import http.client
import json
import os
import socket
import sys
import threading
import time
import uuid

import numpy as np
import pytest

from s2x_serve import frames
from s2x_serve.frames import Frame, FrameError
from s2x_serve.scoring import l2_normalize, score_image_text, sigmoid
from s2x_serve.server import Config, HelpRequested, Service, UsageError, make_server, parse_config

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
from serve_stub import StubEngine  # noqa: E402


# ------------------------------------------------------------------ frames --
def test_frames_roundtrip_and_errors():
    a, b = socket.socketpair()
    try:
        frames.send_frame(a, Frame.LOAD_REQ, 7, {"model_path": "m"})
        frames.send_frame(a, Frame.PING, 8)
        t, rid, p = frames.recv_frame(b)
        assert (t, rid, frames.as_json(p)) == (Frame.LOAD_REQ, 7, {"model_path": "m"})
        assert frames.recv_frame(b) == (Frame.PING, 8, b"")
        x = np.random.default_rng(0).standard_normal(37).astype(np.float32)
        meta, y = frames.unpack_floats(frames.pack_floats({"n": 1}, x))
        assert meta == {"n": 1} and np.array_equal(x, y)
        blobs = [b"", b"\x00\xff" * 1000, b"png"]
        meta, got = frames.unpack_blobs(frames.pack_blobs({"k": [1, 2]}, blobs))
        assert meta == {"k": [1, 2]} and got == blobs
        with pytest.raises(FrameError) as e:
            frames.unpack_blobs(frames.pack_blobs({}, [b"abc"])[:-1])
        assert e.value.kind == "protocol"
        # a header promising more than the cap
        a.sendall(frames.HEADER.pack(Frame.ERR, frames.MAX_PAYLOAD + 1, 1))
        with pytest.raises(FrameError) as e:
            frames.recv_frame(b)
        assert e.value.kind == "too-big"
        # a peer that closes mid-frame, then one that closes between frames
        a.sendall(frames.HEADER.pack(Frame.ERR, 10, 2) + b"12345")
        a.close()
        with pytest.raises(FrameError) as e:
            frames.recv_frame(b)
        assert e.value.kind == "eof-mid-frame"
    finally:
        b.close()
    a, b = socket.socketpair()
    a.close()
    with pytest.raises(FrameError) as e:
        frames.recv_frame(b)
    assert e.value.kind == "eof"
    b.close()


# --------------------------------------------------------------- tokenizer --
@pytest.fixture(scope="module")
def spm_models(tmp_path_factory):
    import sentencepiece as spm
    d = tmp_path_factory.mktemp("spm")
    corpus = d / "corpus.txt"
    words = ["a photo of a cat", "a photo of a dog", "the quick brown fox", "jumps over the lazy dog",
             "siglip two encodes images and text", "one two three four five six seven"]
    corpus.write_text("\n".join(words * 20))
    out = {}
    for name, extra in (("nopad", {}), ("pad", {"pad_id": 3, "unk_id": 0, "bos_id": 1, "eos_id": 2})):
        spm.SentencePieceTrainer.train(input=str(corpus), model_prefix=str(d / name), vocab_size=40,
                                       model_type="unigram", minloglevel=2, **extra)
        out[name] = str(d / f"{name}.model")
    return out


def test_tokenizer_reference_semantics(spm_models):
    from s2x_serve.tokenizer import Tokenizer
    t = Tokenizer(spm_models["nopad"])
    assert t.pad_id == 0 and t.eos_id >= 0  # no pad id in the model: 0
    pieces = list(t.sp.encode("a photo of a cat"))
    ids, mask = t.encode("a photo of a cat", 64)
    assert ids[:len(pieces) + 1] == pieces + [t.eos_id]
    assert ids[len(pieces) + 1:] == [0] * (64 - len(pieces) - 1)
    assert mask == [1] * (len(pieces) + 1) + [0] * (64 - len(pieces) - 1)
    long = " ".join(["the quick brown fox"] * 20)
    ids, mask = t.encode(long, 8)
    assert len(ids) == 8 and ids[-1] == t.eos_id and mask == [1] * 8
    assert ids[:7] == list(t.sp.encode(long))[:7]
    ids, mask = t.encode("a dog", 0)  # natural length
    assert ids == list(t.sp.encode("a dog")) + [t.eos_id] and mask == [1] * len(ids)
    t2 = Tokenizer(spm_models["pad"])
    ids, _ = t2.encode("a cat", 16)
    assert t2.pad_id == 3 and ids[-1] == 3


# ----------------------------------------------------------------- scores --
def test_scores_formula():
    rng = np.random.default_rng(1)
    img = rng.standard_normal((3, 16)).astype(np.float32) * 5
    txt = rng.standard_normal((4, 16)).astype(np.float32)
    logits, probs = score_image_text(img, txt, np.float32(2.3), np.float32(-10.0))
    i64 = img.astype(np.float64) / np.linalg.norm(img.astype(np.float64), axis=1, keepdims=True)
    t64 = txt.astype(np.float64) / np.linalg.norm(txt.astype(np.float64), axis=1, keepdims=True)
    ref = i64 @ t64.T * np.exp(2.3) - 10.0
    assert logits.shape == (3, 4) and logits.dtype == np.float32
    assert np.abs(logits - ref).max() < 1e-5
    assert np.abs(probs - 1 / (1 + np.exp(-ref))).max() < 1e-6
    # the split form: no overflow at large |logit|
    assert sigmoid(np.float32([-1000.0]))[0] == 0.0 and sigmoid(np.float32([1000.0]))[0] == 1.0
    n = l2_normalize(img)
    assert np.allclose(np.linalg.norm(n, axis=1), 1.0, atol=1e-6)


# ----------------------------------------------------------------- config --
def test_parse_config():
    c = parse_config([], {"MODEL_PATH": "m.gguf", "PORT": "9000", "LAZY_LOAD": "1", "VISION_ONLY": "true"})
    assert (c.model_path, c.port, c.lazy_load, c.vision_only, c.worker_isolation) == (
        "m.gguf", 9000, True, True, True)
    c = parse_config(["--model", "x", "--port", "1234", "--text-only", "--idle-unload-seconds", "5"],
                     {"MODEL_PATH": "m", "SIGLIP2_WORKER_ISOLATION": "0"})
    assert (c.model_path, c.port, c.text_only, c.idle_unload_seconds, c.worker_isolation) == (
        "x", 1234, True, 5, False)
    assert parse_config([], {"LAZY_LOAD": "false"}).lazy_load is False
    for bad in (["--vision-only", "--text-only"], ["--port", "x"], ["--bogus"], ["--model"]):
        with pytest.raises(UsageError):
            parse_config(bad, {})
    with pytest.raises(HelpRequested):
        parse_config(["--model", "m", "-h"], {})


# ------------------------------------------------------------------- HTTP --
def _multipart(files=(), fields=()):
    boundary = uuid.uuid4().hex
    out = []
    for name, data in files:
        out.append(f"--{boundary}\r\nContent-Disposition: form-data; name=\"{name}\"; "
                   f"filename=\"f.bin\"\r\nContent-Type: application/octet-stream\r\n\r\n".encode()
                   + data + b"\r\n")
    for name, value in fields:
        out.append(f"--{boundary}\r\nContent-Disposition: form-data; name=\"{name}\"\r\n\r\n"
                   f"{value}\r\n".encode())
    out.append(f"--{boundary}--\r\n".encode())
    return b"".join(out), f"multipart/form-data; boundary={boundary}"


class Client:
    def __init__(self, port):
        self.c = http.client.HTTPConnection("127.0.0.1", port, timeout=60)

    def req(self, method, path, body=None, ctype=None, headers=None):
        h = dict(headers or {})
        if ctype:
            h["Content-Type"] = ctype
        self.c.request(method, path, body=body, headers=h)
        r = self.c.getresponse()
        data = r.read()
        return r.status, json.loads(data)

    def post_form(self, path, files=(), fields=()):
        body, ctype = _multipart(files, fields)
        return self.req("POST", path, body, ctype)


@pytest.fixture
def serve():
    started = []

    def start(**kw):
        cfg = Config(host="127.0.0.1", port=0, lazy_load=True, **kw)
        svc = Service(cfg, engine_factory=StubEngine if not cfg.worker_isolation else None)
        httpd = make_server(svc)
        th = threading.Thread(target=httpd.serve_forever, daemon=True)
        th.start()
        started.append((httpd, svc))
        return Client(httpd.server_address[1]), svc

    yield start
    for httpd, svc in started:
        httpd.shutdown()
        httpd.server_close()
        svc.unload()


IMAGES = [b"\x89PNG first image", b"second image bytes" * 7]


def _check_routes(cl, stub, worker):
    st, body = cl.req("GET", "/health")
    assert st == 200 and body["status"] == "ok" and body["model_loaded"] is False
    # embeddings: pooling and max_num_patches travel with the request
    st, body = cl.post_form("/v1/embeddings", files=[("images", b) for b in IMAGES],
                            fields=[("pooling", "mean"), ("max_num_patches", "256")])
    assert st == 200
    assert np.array_equal(np.float32(body["embeddings"]), stub.encode_images(IMAGES, "mean", 256))
    st, body = cl.post_form("/v1/embeddings?pooling=pooler", files=[("images", IMAGES[0])])
    assert st == 200
    assert np.array_equal(np.float32(body["embeddings"]), stub.encode_images(IMAGES[:1], "probe", 729))
    assert cl.req("GET", "/health")[1]["model_loaded"] is True
    if worker:
        assert cl.req("GET", "/health")[1]["worker_pid"] > 0
    assert cl.post_form("/v1/embeddings", fields=[("pooling", "mean")]) == (400, {"error": "No images provided"})
    st, body = cl.post_form("/v1/embeddings", files=[("images", IMAGES[0])], fields=[("pooling", "max")])
    assert st == 400 and "pooling must be one of" in body["error"]
    st, body = cl.post_form("/v1/embeddings?return_last_hidden=true", files=[("images", IMAGES[0])])
    assert st == 501
    st, body = cl.post_form("/v1/embeddings?max_num_patches=many", files=[("images", IMAGES[0])])
    assert st == 400
    # text: urlencoded and multipart, repeated fields
    st, body = cl.req("POST", "/v1/text_embeddings", b"prompts=a+cat&prompts=a%20dog",
                      "application/x-www-form-urlencoded")
    assert st == 200
    assert np.array_equal(np.float32(body["embeddings"]), stub.encode_texts(["a cat", "a dog"]))
    st, body = cl.post_form("/v1/text_embeddings", fields=[("prompts", "x"), ("prompts", "y z")])
    assert st == 200 and np.array_equal(np.float32(body["embeddings"]), stub.encode_texts(["x", "y z"]))
    assert cl.req("POST", "/v1/text_embeddings", b"", "application/x-www-form-urlencoded")[0] == 400
    st, body = cl.post_form("/v1/text_embeddings", fields=[("prompts", "FAIL")])
    assert st == 500 and "FAIL" in body["error"]
    # classify
    st, body = cl.post_form("/v1/classify?return_logits=true", files=[("images", b) for b in IMAGES],
                            fields=[("prompts", "a"), ("prompts", "b"), ("prompts", "c")])
    probs, logits = stub.classify(IMAGES, ["a", "b", "c"], 729, True)
    assert st == 200 and np.array_equal(np.float32(body["scores"]), probs)
    assert np.array_equal(np.float32(body["logits"]), logits)
    st, body = cl.post_form("/v1/classify", files=[("images", IMAGES[0])], fields=[("prompts", "a")])
    assert st == 200 and "logits" not in body
    assert cl.post_form("/v1/classify", files=[("images", IMAGES[0])])[0] == 400
    # classify from embeddings (JSON)
    emb = stub.encode_images(IMAGES, "probe", 729)
    st, body = cl.req("POST", "/v1/classify_from_embeddings",
                      json.dumps({"image_embeddings": emb.tolist(), "prompts": ["p", "q"],
                                  "return_logits": True}).encode(), "application/json")
    probs, logits = stub.classify_from_embeddings(emb, ["p", "q"], True)
    assert st == 200 and np.array_equal(np.float32(body["scores"]), probs)
    assert np.array_equal(np.float32(body["logits"]), logits)
    bad_row = json.dumps({"image_embeddings": [[0.0] * 3], "prompts": ["p"]}).encode()
    assert cl.req("POST", "/v1/classify_from_embeddings", bad_row, "application/json")[0] == 400
    assert cl.req("POST", "/v1/classify_from_embeddings", b"{not json", "application/json")[0] == 400
    assert cl.req("POST", "/v1/classify_from_embeddings", b"{}", "application/json")[0] == 400
    assert cl.req("GET", "/v1/nothing")[0] == 404
    # a body-less POST (no Content-Length) unloads; the next request loads again
    st, body = cl.req("POST", "/unload")
    assert st == 200 and body["unloaded"] is True and body["model_loaded"] is False
    assert cl.req("GET", "/health")[1]["model_loaded"] is False
    st, body = cl.req("POST", "/v1/admin/load")
    assert st == 200 and body["loaded"] is True and body["model_loaded"] is True
    st, body = cl.req("POST", "/v1/admin/unload")
    assert st == 200 and body["source"] == "/v1/admin/unload" and body["unloaded"] is True
    st, body = cl.post_form("/v1/embeddings", files=[("images", IMAGES[1])])
    assert st == 200


def test_routes_in_process(serve):
    cl, svc = serve(worker_isolation=False)
    _check_routes(cl, StubEngine("m"), worker=False)


def test_routes_through_worker_processes(serve):
    cl, svc = serve(worker_isolation=True, worker_argv=[sys.executable, os.path.join(HERE, "serve_stub.py")])
    _check_routes(cl, StubEngine("m"), worker=True)
    # unload kills the worker; a crash mid-request is a 500 and the next request restarts it
    pid = cl.req("GET", "/health")[1]["worker_pid"]
    assert pid > 0
    cl.req("POST", "/v1/admin/unload")
    with pytest.raises(ProcessLookupError):
        os.kill(pid, 0)
    st, body = cl.post_form("/v1/text_embeddings", fields=[("prompts", "CRASH")])
    assert st == 500
    assert svc.worker.is_alive() is False
    st, body = cl.post_form("/v1/text_embeddings", fields=[("prompts", "fine")])
    assert st == 200 and np.array_equal(np.float32(body["embeddings"]), StubEngine("m").encode_texts(["fine"]))
    assert cl.req("GET", "/health")[1]["worker_pid"] not in (pid, -1)


@pytest.mark.parametrize("worker", [False, True])
def test_towers_left_out_and_load_failure(serve, worker):
    extra = {"worker_argv": [sys.executable, os.path.join(HERE, "serve_stub.py")]} if worker else {}
    cl, _ = serve(worker_isolation=worker, vision_only=True, model_path="m", **extra)
    assert cl.post_form("/v1/text_embeddings", fields=[("prompts", "x")])[0] == 503
    assert cl.post_form("/v1/classify", files=[("images", b"i")], fields=[("prompts", "x")])[0] == 503
    assert cl.post_form("/v1/embeddings", files=[("images", b"i")])[0] == 200
    cl, _ = serve(worker_isolation=worker, text_only=True, model_path="m", **extra)
    assert cl.post_form("/v1/embeddings", files=[("images", b"i")])[0] == 503
    assert cl.post_form("/v1/text_embeddings", fields=[("prompts", "x")])[0] == 200
    cl, _ = serve(worker_isolation=worker, model_path="fail", **extra)
    st, body = cl.post_form("/v1/embeddings", files=[("images", b"i")])
    assert st == 503 and "cannot load" in body["error"]
    st, body = cl.req("POST", "/v1/admin/load")
    assert st == 500 and "cannot load" in body["error"]


def test_idle_unload(serve):
    cl, svc = serve(worker_isolation=False, idle_unload_seconds=1, idle_poll_seconds=0.1)
    svc.start_idle_sweeper()
    assert cl.post_form("/v1/embeddings", files=[("images", b"i")])[0] == 200
    assert cl.req("GET", "/health")[1]["model_loaded"] is True
    t0 = time.monotonic()
    while cl.req("GET", "/health")[1]["model_loaded"] and time.monotonic() - t0 < 10:
        time.sleep(0.1)  # /health does not count as a request
    assert cl.req("GET", "/health")[1]["model_loaded"] is False
    assert time.monotonic() - t0 >= 0.5
