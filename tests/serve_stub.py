"""A CPU stand-in for s2x_serve.engine.Engine, for the service's tests
without a GPU: embeddings are derived from the request bytes (SHA-256),
scores come from s2x_serve.scoring.  Run as a program it is a worker
process (python tests/serve_stub.py --fd N).  Prompts "FAIL" and "CRASH"
make it fail a request and end its process."""
import hashlib
import os
import sys

import numpy as np

sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                                "hbd-siglip2.cpp_amd"))
from s2x_serve.engine import EngineError, parse_pooling  # noqa: E402  (no GPU import)
from s2x_serve.scoring import l2_normalize, score_image_text  # noqa: E402

DIM = 8


def _vec(data, salt):
    h = hashlib.sha256(salt + bytes(data)).digest()
    return np.frombuffer(h, np.uint8)[:DIM].astype(np.float32) - np.float32(127.5)


class StubEngine:
    hidden_size = DIM
    max_position_embeddings = 64

    def __init__(self, model_path, tokenizer_path="", default_max_num_patches=729,
                 vision_only=False, text_only=False, **_):
        if model_path == "fail":
            raise EngineError("stub: cannot load fail", 503)
        self.has_vision = not text_only
        self.has_text = not vision_only
        self.default = default_max_num_patches
        self.logit_scale, self.logit_bias = 2.0, -1.0

    def raw_images(self, blobs, pooling="probe", max_num_patches=None):
        p = parse_pooling(pooling)
        mnp = max_num_patches or self.default
        return np.stack([_vec(b, f"img:{p}:{mnp}:".encode()) for b in blobs])

    def raw_texts(self, prompts):
        for p in prompts:
            if p == "FAIL":
                raise EngineError("stub: FAIL prompt", 500)
            if p == "CRASH":
                os._exit(3)
        return np.stack([_vec(p.encode(), b"txt:") for p in prompts])

    def encode_images(self, blobs, pooling="probe", max_num_patches=None, return_last_hidden=False):
        if not self.has_vision:
            raise EngineError("vision tower not loaded (server started with --text-only)", 503)
        if return_last_hidden:
            raise EngineError("return_last_hidden not implemented", 501)
        return l2_normalize(self.raw_images(blobs, pooling, max_num_patches))

    def encode_texts(self, prompts):
        if not self.has_text:
            raise EngineError("text tower not loaded (server started with --vision-only)", 503)
        return l2_normalize(self.raw_texts(prompts))

    def classify(self, blobs, prompts, max_num_patches=None, return_logits=False):
        logits, probs = score_image_text(self.raw_images(blobs, "probe", max_num_patches),
                                         self.raw_texts(prompts), self.logit_scale, self.logit_bias)
        return probs, (logits if return_logits else None)

    def classify_from_embeddings(self, image_embeddings, prompts, return_logits=False):
        img = np.asarray(image_embeddings, np.float32).reshape(-1, DIM)
        logits, probs = score_image_text(img, self.raw_texts(prompts), self.logit_scale,
                                         self.logit_bias)
        return probs, (logits if return_logits else None)

    def close(self):
        pass


if __name__ == "__main__":
    from s2x_serve.worker import run_worker_loop
    fd = int(sys.argv[sys.argv.index("--fd") + 1])
    sys.exit(run_worker_loop(fd, StubEngine))
