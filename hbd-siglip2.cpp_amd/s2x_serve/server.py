"""HTTP front end of the service (the reference's siglip2-server,
src/siglip2_server.cpp): configuration from flags and environment, the
routes, request parsing (query string, urlencoded and multipart forms,
JSON), model lifecycle (eager or lazy load, unload / load, idle unload) and
the choice between a GPU worker process (default) and in-process encoders
(SIGLIP2_WORKER_ISOLATION=0).  Python's threading HTTP/1.1 server: one
thread per connection, keep-alive, a 60 s socket timeout.

Status codes and error bodies ({"error": ...}) are the reference's: 400 for
a request without images / prompts, a bad pooling or a malformed JSON body,
501 for return_last_hidden, 503 when the model cannot be loaded or the
tower a route needs was left out (--vision-only / --text-only), 500 for a
failed encode.
"""
import email.parser
import email.policy
import json
import os
import sys
import threading
import time
import urllib.parse
from dataclasses import dataclass, field
from http.server import BaseHTTPRequestHandler, ThreadingHTTPServer

import numpy as np

from .session import WorkerSession

USAGE = """siglip2-server (libs2x on gfx950) -- the SigLIP2 embedding service

Usage: python -m s2x_serve --model <gguf> --tokenizer <spm.model> [--port 8890] [--lazy-load]
         [--host 0.0.0.0] [--default-max-num-patches 729] [--idle-unload-seconds 0]
         [--vision-only | --text-only]
Env: MODEL_PATH TOKENIZER_PATH HOST PORT DEFAULT_MAX_NUM_PATCHES
     IDLE_UNLOAD_SECONDS LAZY_LOAD VISION_ONLY TEXT_ONLY
     SIGLIP2_WORKER_ISOLATION=0  (encoders in this process instead of a worker)
"""


@dataclass
class Config:
    model_path: str = ""
    tokenizer_path: str = ""
    host: str = "0.0.0.0"
    port: int = 8890
    default_max_num_patches: int = 729
    idle_unload_seconds: int = 0  # 0 = never
    lazy_load: bool = False
    vision_only: bool = False
    text_only: bool = False
    worker_isolation: bool = True
    idle_poll_seconds: float = 10.0
    worker_argv: list = field(default=None)  # the worker program (default: python -m s2x_serve.worker)

    def worker_cfg(self):
        return {"model_path": self.model_path, "tokenizer_path": self.tokenizer_path,
                "default_max_num_patches": self.default_max_num_patches,
                "vision_only": self.vision_only, "text_only": self.text_only}


class UsageError(Exception):
    pass


class HelpRequested(Exception):
    pass


def parse_config(argv, environ=None):
    """Flags override the environment (src/siglip2_server.cpp:66-125)."""
    env = os.environ if environ is None else environ

    def flag(key):
        v = env.get(key, "")
        return v != "" and v != "0" and v != "false"

    def num(v, name):
        try:
            return int(v)
        except ValueError:
            raise UsageError(f"{name} must be an integer (got '{v}')") from None

    c = Config(model_path=env.get("MODEL_PATH", ""), tokenizer_path=env.get("TOKENIZER_PATH", ""),
               host=env.get("HOST", "0.0.0.0"), port=num(env.get("PORT", "8890"), "PORT"),
               default_max_num_patches=num(env.get("DEFAULT_MAX_NUM_PATCHES", "729"),
                                           "DEFAULT_MAX_NUM_PATCHES"),
               idle_unload_seconds=num(env.get("IDLE_UNLOAD_SECONDS", "0"), "IDLE_UNLOAD_SECONDS"),
               lazy_load=flag("LAZY_LOAD"), vision_only=flag("VISION_ONLY"), text_only=flag("TEXT_ONLY"))
    iso = env.get("SIGLIP2_WORKER_ISOLATION")
    if iso is not None:
        c.worker_isolation = iso != "" and iso[0] != "0"
    values = {"--model": "model_path", "--tokenizer": "tokenizer_path", "--host": "host"}
    ints = {"--port": "port", "--default-max-num-patches": "default_max_num_patches",
            "--idle-unload-seconds": "idle_unload_seconds"}
    switches = {"--lazy-load": "lazy_load", "--vision-only": "vision_only", "--text-only": "text_only"}
    i = 0
    while i < len(argv):
        a = argv[i]
        if a in ("-h", "--help"):
            raise HelpRequested()
        if a in values or a in ints:
            if i + 1 >= len(argv):
                raise UsageError(f"{a} needs a value")
            v = argv[i + 1]
            if a in values:
                setattr(c, values[a], v)
            else:
                setattr(c, ints[a], num(v, a))
            i += 2
        elif a in switches:
            setattr(c, switches[a], True)
            i += 1
        else:
            raise UsageError(f"Unknown arg: {a}")
    if c.vision_only and c.text_only:
        raise UsageError("--vision-only and --text-only are mutually exclusive")
    return c


class ServiceError(Exception):
    def __init__(self, status, msg):
        super().__init__(msg)
        self.status = status


class Service:
    """The model behind the routes: a WorkerSession, or an in-process engine
    built by engine_factory(**cfg) (s2x_serve.engine.Engine by default)."""

    def __init__(self, cfg, engine_factory=None):
        self.cfg = cfg
        self.worker = WorkerSession(argv=cfg.worker_argv) if cfg.worker_isolation else None
        self._make_engine = engine_factory
        self.engine = None
        self._lock = threading.Lock()  # in-process load / unload
        self.last_request = 0.0
        self._sweeper = None

    # -- lifecycle -----------------------------------------------------------
    def touch(self):
        self.last_request = time.monotonic()

    def loaded(self):
        return self.worker.is_alive() if self.worker else self.engine is not None

    def _load_in_process(self):
        with self._lock:
            if self.engine is None:
                make = self._make_engine
                if make is None:
                    from .engine import Engine as make
                try:
                    self.engine = make(**self.cfg.worker_cfg())
                except Exception as e:  # load failures become a 503 with the message
                    raise ServiceError(503, str(e)) from e

    def ensure(self):
        self.touch()
        if self.worker:
            if not self.worker.ensure_loaded(self.cfg.worker_cfg()):
                raise ServiceError(503, self.worker.last_error)
        else:
            self._load_in_process()

    def unload(self):
        was = self.loaded()
        if self.worker:
            self.worker.shutdown()
        else:
            with self._lock:
                if self.engine is not None:
                    self.engine.close()
                    self.engine = None
        return was, self.loaded()

    def load(self):
        was = self.loaded()
        self.ensure()
        return was, self.loaded()

    def start_idle_sweeper(self):
        """Unload after idle_unload_seconds without a request (/health does not
        count), checked every idle_poll_seconds (src/siglip2_server.cpp:1007-1031)."""
        if self.cfg.idle_unload_seconds <= 0 or self._sweeper is not None:
            return

        def sweep():
            while True:
                time.sleep(self.cfg.idle_poll_seconds)
                if not self.loaded() or self.last_request == 0.0:
                    continue
                idle = time.monotonic() - self.last_request
                if idle >= self.cfg.idle_unload_seconds:
                    print(f"[siglip2-server] idle-unload: {idle:.0f} s since last request "
                          f"(threshold {self.cfg.idle_unload_seconds} s)", file=sys.stderr, flush=True)
                    self.unload()

        self._sweeper = threading.Thread(target=sweep, name="s2x-idle-unload", daemon=True)
        self._sweeper.start()

    # -- towers --------------------------------------------------------------
    def _backend(self):
        return self.worker if self.worker else self.engine

    def require_vision(self):
        have = not self.cfg.text_only if self.worker else self.engine.has_vision
        if not have:
            raise ServiceError(503, "vision tower not loaded (server started with --text-only)")

    def require_text(self):
        have = not self.cfg.vision_only if self.worker else self.engine.has_text
        if not have:
            raise ServiceError(503, "text tower not loaded (server started with --vision-only)")

    def require_both(self, msg="classify requires both towers loaded"):
        both = (not self.cfg.text_only and not self.cfg.vision_only) if self.worker else (
            self.engine.has_vision and self.engine.has_text)
        if not both:
            raise ServiceError(503, msg)

    def hidden_size(self):
        return self.worker.hidden_size if self.worker else self.engine.hidden_size

    def call(self, name, *args):
        try:
            return getattr(self._backend(), name)(*args)
        except ServiceError:
            raise
        except Exception as e:  # engine / worker errors carry their HTTP status
            raise ServiceError(getattr(e, "status", 500), str(e)) from e


# -- request parsing ----------------------------------------------------------
class Request:
    """Form fields from the query string, an urlencoded or a multipart body
    (text fields in `fields`, every multipart part in `files`, as the
    reference's req.files / req.params), or a JSON body."""

    def __init__(self, path, headers, body):
        u = urllib.parse.urlsplit(path)
        self.path = u.path
        self.body = body
        self.fields = {}
        self.files = {}
        for k, v in urllib.parse.parse_qsl(u.query, keep_blank_values=True):
            self.fields.setdefault(k, []).append(v)
        ctype = headers.get("Content-Type", "") or ""
        if ctype.startswith("application/x-www-form-urlencoded"):
            for k, v in urllib.parse.parse_qsl(body.decode("utf-8", "replace"), keep_blank_values=True):
                self.fields.setdefault(k, []).append(v)
        elif ctype.startswith("multipart/form-data") and body:
            msg = email.parser.BytesParser(policy=email.policy.HTTP).parsebytes(
                b"Content-Type: " + ctype.encode("latin-1") + b"\r\n\r\n" + body)
            if not msg.is_multipart():
                raise ServiceError(400, "malformed multipart body")
            for part in msg.iter_parts():
                name = part.get_param("name", header="content-disposition")
                if name is None:
                    continue
                data = part.get_payload(decode=True) or b""
                self.files.setdefault(name, []).append(data)
                if part.get_filename() is None:
                    charset = part.get_content_charset() or "utf-8"
                    self.fields.setdefault(name, []).append(data.decode(charset, "replace"))

    def value(self, name, default=""):
        v = self.fields.get(name)
        return v[0] if v else default

    def has(self, name):
        return name in self.fields

    def texts(self, name):
        """Every value of a repeated form field (FastAPI's list[str] = Form(...))."""
        return list(self.fields.get(name, []))

    def file_values(self, name):
        return list(self.files.get(name, []))

    def json(self):
        try:
            return json.loads(self.body.decode("utf-8") or "null")
        except (UnicodeDecodeError, json.JSONDecodeError) as e:
            raise ServiceError(400, f"invalid JSON: {e}") from e


def _max_patches(req, svc):
    v = req.value("max_num_patches") if req.has("max_num_patches") else ""
    if not v:
        return svc.cfg.default_max_num_patches
    try:
        return int(v)
    except ValueError:
        raise ServiceError(400, f"max_num_patches must be an integer (got '{v}')") from None


def _rows(a):
    return a.tolist() if isinstance(a, np.ndarray) else a


# -- routes -------------------------------------------------------------------
def route_health(svc, req):
    body = {"status": "ok", "model": svc.cfg.model_path, "model_loaded": svc.loaded()}
    if svc.worker:
        body["worker_pid"] = svc.worker.pid
    return 200, body


def _unload(svc, req):
    was, now = svc.unload()
    out = {"unloaded": was, "model_loaded": now, "source": req.path}
    if svc.worker:
        out["mode"] = "worker-isolation"
    return 200, out


def route_admin_load(svc, req):
    try:
        was, now = svc.load()
    except ServiceError as e:
        return 500, {"error": str(e)}
    out = {"loaded": not was, "model_loaded": now}
    if svc.worker:
        out["mode"] = "worker-isolation"
    return 200, out


def route_embeddings(svc, req):
    svc.ensure()
    svc.require_vision()
    images = req.file_values("images")
    if not images:
        raise ServiceError(400, "No images provided")
    pooling = req.value("pooling")
    if pooling not in ("", "pooler", "probe", "mean"):
        raise ServiceError(400, f"pooling must be one of: pooler, probe, mean (got '{pooling}')")
    mnp = _max_patches(req, svc)
    if req.value("return_last_hidden") == "true":
        raise ServiceError(501, "return_last_hidden not implemented")
    embs = svc.call("encode_images", images, pooling or "probe", mnp, False)
    return 200, {"embeddings": _rows(embs)}


def route_text_embeddings(svc, req):
    svc.ensure()
    svc.require_text()
    prompts = req.texts("prompts")
    if not prompts:
        raise ServiceError(400, "No prompts provided")
    return 200, {"embeddings": _rows(svc.call("encode_texts", prompts))}


def route_classify(svc, req):
    svc.ensure()
    svc.require_both()
    images = req.file_values("images")
    prompts = req.texts("prompts")
    if not images:
        raise ServiceError(400, "No images provided")
    if not prompts:
        raise ServiceError(400, "No prompts provided")
    return_logits = req.value("return_logits") == "true"
    scores, logits = svc.call("classify", images, prompts, _max_patches(req, svc), return_logits)
    body = {"scores": _rows(scores)}
    if return_logits:
        body["logits"] = _rows(logits)
    return 200, body


def route_classify_from_embeddings(svc, req):
    svc.ensure()
    svc.require_text()
    svc.require_both("classify requires the model loaded with both towers")
    body = req.json()
    if not isinstance(body, dict) or "image_embeddings" not in body or "prompts" not in body:
        raise ServiceError(400, "JSON must contain image_embeddings and prompts")
    imgs, prompts = body["image_embeddings"], body["prompts"]
    if not isinstance(imgs, list) or not isinstance(prompts, list) or \
            not all(isinstance(p, str) for p in prompts):
        raise ServiceError(400, "image_embeddings must be a list of rows and prompts a list of strings")
    H = svc.hidden_size()
    rows = []
    for r in imgs:
        if not isinstance(r, list) or len(r) != H:
            raise ServiceError(400, "image_embedding row has wrong dim")
        try:
            rows.append([float(x) for x in r])
        except (TypeError, ValueError):
            raise ServiceError(400, "image_embedding values must be numbers") from None
    return_logits = bool(body.get("return_logits", False))
    scores, logits = svc.call("classify_from_embeddings", rows, prompts, return_logits)
    out = {"scores": _rows(scores)}
    if return_logits:
        out["logits"] = _rows(logits)
    return 200, out


GET_ROUTES = {"/health": route_health}
POST_ROUTES = {"/unload": _unload, "/v1/admin/unload": _unload, "/v1/admin/load": route_admin_load,
               "/v1/embeddings": route_embeddings, "/v1/text_embeddings": route_text_embeddings,
               "/v1/classify": route_classify,
               "/v1/classify_from_embeddings": route_classify_from_embeddings}


class Handler(BaseHTTPRequestHandler):
    protocol_version = "HTTP/1.1"
    server_version = "siglip2-server-s2x"
    timeout = 60  # socket read / write, as the reference's

    def log_message(self, fmt, *args):
        if os.environ.get("SIGLIP2_LOG_REQUESTS"):
            super().log_message(fmt, *args)

    def _read_body(self):
        if self.headers.get("Transfer-Encoding", "").lower() == "chunked":
            chunks = []
            while True:
                line = self.rfile.readline(65537)
                size = int(line.split(b";")[0].strip() or b"0", 16)
                if size == 0:
                    while self.rfile.readline(65537) not in (b"\r\n", b"\n", b""):
                        pass
                    return b"".join(chunks)
                chunks.append(self.rfile.read(size))
                self.rfile.readline(65537)
        n = int(self.headers.get("Content-Length") or 0)  # a body-less POST reads nothing
        return self.rfile.read(n) if n > 0 else b""

    def _send(self, status, body):
        data = json.dumps(body).encode()
        self.send_response(status)
        self.send_header("Content-Type", "application/json")
        self.send_header("Content-Length", str(len(data)))
        self.end_headers()
        self.wfile.write(data)

    def _dispatch(self, routes):
        try:
            body = self._read_body() if self.command == "POST" else b""
        except (ValueError, OSError):
            self._send(400, {"error": "malformed request body"})
            self.close_connection = True
            return
        try:
            req = Request(self.path, self.headers, body)
            route = routes.get(req.path)
            if route is None:
                self._send(404, {"error": f"no route for {self.command} {req.path}"})
                return
            status, out = route(self.server.service, req)
        except ServiceError as e:
            status, out = e.status, {"error": str(e)}
        except Exception as e:  # the service must answer, whatever failed
            status, out = 500, {"error": f"{type(e).__name__}: {e}"}
        self._send(status, out)

    def do_GET(self):
        self._dispatch(GET_ROUTES)

    def do_POST(self):
        self._dispatch(POST_ROUTES)


class Server(ThreadingHTTPServer):
    daemon_threads = True
    allow_reuse_address = True

    def __init__(self, service, address):
        self.service = service
        super().__init__(address, Handler)


def make_server(service, host=None, port=None):
    cfg = service.cfg
    return Server(service, (cfg.host if host is None else host, cfg.port if port is None else port))


def main(argv=None):
    try:
        cfg = parse_config(sys.argv[1:] if argv is None else argv)
    except HelpRequested:
        print(USAGE, file=sys.stderr)
        return 0
    except UsageError as e:
        print(e, file=sys.stderr)
        return 2
    if not cfg.model_path:
        print("--model (or MODEL_PATH env) is required.", file=sys.stderr)
        return 2
    if not cfg.vision_only and not cfg.tokenizer_path:
        print("--tokenizer (or TOKENIZER_PATH env) is required unless --vision-only.", file=sys.stderr)
        return 2
    svc = Service(cfg)
    mode = "ON (worker process owns the GPU)" if cfg.worker_isolation else "OFF (in-process)"
    print(f"[siglip2-server] worker-isolation: {mode}", file=sys.stderr, flush=True)
    if not cfg.lazy_load:
        try:
            svc.ensure()
        except ServiceError as e:
            print(f"load failed: {e}", file=sys.stderr)
            return 1
    svc.start_idle_sweeper()
    httpd = make_server(svc)
    host, port = httpd.server_address[:2]
    print(f"[siglip2-server] listening on {host}:{port} (model={cfg.model_path})", file=sys.stderr,
          flush=True)
    try:
        httpd.serve_forever()
    except KeyboardInterrupt:
        pass
    finally:
        httpd.server_close()
        svc.unload()
    return 0
