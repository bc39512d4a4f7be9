"""The HTTP process's handle on its GPU worker (the reference's
WorkerSession, src/worker_session.h:33-108): start the worker over a
socketpair (it answers HELLO), send the load configuration, then pass
requests one at a time; shutdown() kills the worker (SIGKILL), which returns
every byte of device memory it held, and the next request starts a new one
with the last configuration.  A worker that died or stopped answering is
killed and restarted on the next request.

The worker is a separate program (python -m s2x_serve.worker) started by
fork + exec from this process, which loads no GPU library.
"""
import os
import signal
import socket
import subprocess
import sys
import threading

import numpy as np

from .frames import (Frame, FrameError, as_json, pack_blobs, pack_floats, recv_frame, send_frame,
                     unpack_floats)

PKG_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


class WorkerError(RuntimeError):
    def __init__(self, msg, status=500):
        super().__init__(msg)
        self.status = status


class WorkerSession:
    def __init__(self, argv=None, env=None, load_timeout=600.0, request_timeout=600.0):
        self.argv = list(argv) if argv else [sys.executable, "-m", "s2x_serve.worker"]
        self._env = dict(os.environ if env is None else env)
        pp = self._env.get("PYTHONPATH", "")
        self._env["PYTHONPATH"] = PKG_ROOT + (os.pathsep + pp if pp else "")
        self.load_timeout = load_timeout
        self.request_timeout = request_timeout
        self._lock = threading.Lock()
        self._proc = None
        self._sock = None
        self._cfg = None
        self._loaded = False
        self._next_id = 1
        self.hidden_size = 0
        self.max_position_embeddings = 0
        self.last_error = ""

    # -- state ---------------------------------------------------------------
    def _alive_locked(self):
        return self._proc is not None and self._proc.poll() is None and self._loaded

    def is_alive(self):
        with self._lock:
            return self._alive_locked()

    @property
    def pid(self):
        with self._lock:
            return self._proc.pid if self._alive_locked() else -1

    def _rid(self):
        rid = self._next_id
        self._next_id = self._next_id % 0xFFFFFFFF + 1
        return rid

    # -- lifecycle -----------------------------------------------------------
    def ensure_loaded(self, cfg):
        """Start + load the worker unless one with this configuration runs."""
        with self._lock:
            return self._ensure_locked(dict(cfg))

    def _ensure_locked(self, cfg):
        if self._alive_locked() and self._cfg == cfg:
            return True
        self._kill_locked()
        self._cfg = cfg  # kept for restarts after an unload
        try:
            self._spawn_locked()
            self._load_locked(cfg)
        except (FrameError, OSError, WorkerError) as e:
            self.last_error = str(e)
            self._kill_locked()
            return False
        return True

    def _spawn_locked(self):
        parent, child = socket.socketpair()
        try:
            self._proc = subprocess.Popen(self.argv + ["--fd", str(child.fileno())],
                                          pass_fds=[child.fileno()], env=self._env)
        finally:
            child.close()
        self._sock = parent
        parent.settimeout(self.load_timeout)
        ftype, _, _ = recv_frame(parent)
        if ftype != Frame.HELLO:
            raise WorkerError(f"worker began with frame {ftype:#x}, not HELLO")

    def _load_locked(self, cfg):
        rid = self._rid()
        send_frame(self._sock, Frame.LOAD_REQ, rid, cfg)
        ftype, _, payload = recv_frame(self._sock)
        meta = as_json(payload)
        if ftype != Frame.LOAD_RESP or not meta.get("ok"):
            raise WorkerError(meta.get("error") or "worker load failed", 503)
        self.hidden_size = int(meta.get("hidden_size", 0))
        self.max_position_embeddings = int(meta.get("max_position_embeddings", 0))
        self._loaded = True

    def shutdown(self):
        """Kill the worker (its device memory goes with it); idempotent."""
        with self._lock:
            self._kill_locked()

    def _kill_locked(self):
        proc, sock = self._proc, self._sock
        self._proc = self._sock = None
        self._loaded = False
        if proc is not None:
            if proc.poll() is None:
                try:
                    proc.send_signal(signal.SIGKILL)
                except ProcessLookupError:
                    pass
            try:
                proc.wait(timeout=60)
            except subprocess.TimeoutExpired:
                pass
        if sock is not None:
            sock.close()

    # -- requests ------------------------------------------------------------
    def _request(self, ftype, payload, expect):
        with self._lock:
            if not self._alive_locked():
                if self._cfg is None or not self._ensure_locked(self._cfg):
                    raise WorkerError(self.last_error or "worker not running", 503)
            rid = self._rid()
            try:
                self._sock.settimeout(self.request_timeout)
                send_frame(self._sock, ftype, rid, payload)
                while True:
                    rtype, rrid, data = recv_frame(self._sock)
                    if rrid == rid:
                        break  # (a reply to an abandoned request is dropped)
            except FrameError as e:
                self.last_error = f"worker: {e}"
                self._kill_locked()
                raise WorkerError(self.last_error, 500) from e
        if rtype == Frame.ERR:
            meta = as_json(data)
            self.last_error = meta.get("error", "worker error")
            raise WorkerError(self.last_error, int(meta.get("status", 500)))
        if rtype != expect:
            raise WorkerError(f"worker replied with frame {rtype:#x}", 500)
        return data

    def encode_images(self, blobs, pooling="probe", max_num_patches=None, return_last_hidden=False):
        data = self._request(Frame.ENCODE_IMAGES_REQ,
                             pack_blobs({"pooling": pooling, "max_num_patches": max_num_patches,
                                         "return_last_hidden": bool(return_last_hidden)}, blobs),
                             Frame.ENCODE_IMAGES_RESP)
        meta, flat = unpack_floats(data)
        return flat.reshape(int(meta["n"]), int(meta["dim"]))

    def encode_texts(self, prompts):
        data = self._request(Frame.ENCODE_TEXT_REQ, {"prompts": list(prompts)}, Frame.ENCODE_TEXT_RESP)
        meta, flat = unpack_floats(data)
        return flat.reshape(int(meta["n"]), int(meta["dim"]))

    def classify(self, blobs, prompts, max_num_patches=None, return_logits=False):
        data = self._request(Frame.CLASSIFY_REQ,
                             pack_blobs({"prompts": list(prompts), "max_num_patches": max_num_patches,
                                         "return_logits": bool(return_logits)}, blobs),
                             Frame.CLASSIFY_RESP)
        meta = as_json(data)
        return meta["scores"], meta.get("logits")

    def classify_from_embeddings(self, image_embeddings, prompts, return_logits=False):
        img = np.asarray(image_embeddings, np.float32)
        n = len(image_embeddings)
        dim = int(img.shape[1]) if n else 0
        data = self._request(Frame.CLASSIFY_FROM_EMB_REQ,
                             pack_floats({"prompts": list(prompts), "return_logits": bool(return_logits),
                                          "n": n, "dim": dim}, img.reshape(-1)),
                             Frame.CLASSIFY_FROM_EMB_RESP)
        meta = as_json(data)
        return meta["scores"], meta.get("logits")
