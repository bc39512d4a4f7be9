"""The GPU worker process: owns the engine (encoders, tokenizer, score
parameters) and serves the frames of s2x_serve.frames on an inherited
socket until SHUTDOWN or the parent closes it (the reference's
run_worker_loop, src/worker_session.cpp:998-1071).

    python -m s2x_serve.worker --fd N

Each request is answered with its reply frame or ERR {"error", "status"},
where status is the HTTP status the parent should give the failure.
"""
import argparse
import os
import socket
import sys
import time

from .frames import (Frame, FrameError, as_json, pack_floats, recv_frame, send_frame,
                     unpack_blobs, unpack_floats)


def _default_engine(**cfg):
    from .engine import Engine
    return Engine(**cfg)


def _error_status(e):
    return getattr(e, "status", 500)


def _scores_json(probs, logits):
    out = {"scores": probs.tolist()}
    if logits is not None:
        out["logits"] = logits.tolist()
    return out


def run_worker_loop(fd, engine_factory=None):
    """Serve frames on socket fd; 0 when the parent shuts the worker down."""
    make = engine_factory or _default_engine
    sock = socket.socket(fileno=fd)
    engine = None
    try:
        send_frame(sock, Frame.HELLO, 0, {"pid": os.getpid(), "role": "worker"})
        while True:
            try:
                ftype, rid, payload = recv_frame(sock)
            except FrameError as e:
                return 0 if e.kind == "eof" else 1
            try:
                if ftype == Frame.SHUTDOWN:
                    return 0
                if ftype == Frame.PING:
                    meta = as_json(payload)
                    send_frame(sock, Frame.PONG, rid,
                               {"t_send_ns": meta.get("t_send_ns", 0), "t_recv_ns": time.time_ns()})
                elif ftype == Frame.LOAD_REQ:
                    cfg = as_json(payload)
                    if engine is not None:
                        engine.close()
                        engine = None
                    try:
                        engine = make(**cfg)
                    except Exception as e:  # any load failure goes back as the reply
                        send_frame(sock, Frame.LOAD_RESP, rid, {"ok": False, "error": str(e)})
                        continue
                    send_frame(sock, Frame.LOAD_RESP, rid, {
                        "ok": True, "error": "", "hidden_size": engine.hidden_size,
                        "max_position_embeddings": engine.max_position_embeddings})
                elif engine is None:
                    send_frame(sock, Frame.ERR, rid, {"error": "model not loaded", "status": 503})
                elif ftype == Frame.ENCODE_IMAGES_REQ:
                    meta, blobs = unpack_blobs(payload)
                    embs = engine.encode_images(blobs, meta.get("pooling", "probe"),
                                                meta.get("max_num_patches"),
                                                bool(meta.get("return_last_hidden", False)))
                    send_frame(sock, Frame.ENCODE_IMAGES_RESP, rid,
                               pack_floats({"n": len(embs), "dim": int(embs.shape[1])}, embs))
                elif ftype == Frame.ENCODE_TEXT_REQ:
                    embs = engine.encode_texts(as_json(payload).get("prompts", []))
                    send_frame(sock, Frame.ENCODE_TEXT_RESP, rid,
                               pack_floats({"n": len(embs), "dim": int(embs.shape[1])}, embs))
                elif ftype == Frame.CLASSIFY_REQ:
                    meta, blobs = unpack_blobs(payload)
                    probs, logits = engine.classify(blobs, meta.get("prompts", []),
                                                    meta.get("max_num_patches"),
                                                    bool(meta.get("return_logits", False)))
                    send_frame(sock, Frame.CLASSIFY_RESP, rid, _scores_json(probs, logits))
                elif ftype == Frame.CLASSIFY_FROM_EMB_REQ:
                    meta, flat = unpack_floats(payload)
                    n, dim = int(meta.get("n", 0)), int(meta.get("dim", 0))
                    if n * dim != flat.size:
                        raise FrameError("protocol", "embedding count does not match n x dim")
                    probs, logits = engine.classify_from_embeddings(
                        flat.reshape(n, dim) if n else [], meta.get("prompts", []),
                        bool(meta.get("return_logits", False)))
                    send_frame(sock, Frame.CLASSIFY_FROM_EMB_RESP, rid, _scores_json(probs, logits))
                else:
                    send_frame(sock, Frame.ERR, rid, {"error": f"unknown frame type {ftype:#x}",
                                                     "status": 500})
            except FrameError as e:
                if e.kind in ("socket", "eof-mid-frame", "eof", "timeout"):
                    return 1
                send_frame(sock, Frame.ERR, rid, {"error": str(e), "status": 500})
            except Exception as e:  # a failed request must not end the worker
                send_frame(sock, Frame.ERR, rid, {"error": str(e), "status": _error_status(e)})
    finally:
        if engine is not None:
            engine.close()
        sock.close()


def main(argv=None):
    ap = argparse.ArgumentParser(prog="python -m s2x_serve.worker")
    ap.add_argument("--fd", type=int, required=True, help="inherited socket to the HTTP process")
    args, _ = ap.parse_known_args(argv)  # the server's own flags may follow
    return run_worker_loop(args.fd)


if __name__ == "__main__":
    sys.exit(main())
