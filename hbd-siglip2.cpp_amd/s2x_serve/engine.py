"""The service's GPU side: SigLIP2 towers from a GGUF file on libs2x, images
decoded on the host and preprocessed and encoded on the GPU, prompts
tokenized and encoded, image-text scores.  Used by the worker process (the
default) or in the HTTP process itself (SIGLIP2_WORKER_ISOLATION=0).

The vision and text encoders each run on a stream of their own, behind a
lock of their own, so that a classify call overlaps its text encode (on a
persistent helper thread) with its image encodes (on the calling thread),
as the reference's /v1/classify does (src/siglip2_server.cpp:790-832).
Embeddings are L2-normalized before they leave (src/siglip2_server.cpp:
706-708, 739); scores use the model's logit_scale / logit_bias.
"""
import ctypes
import io
import threading
from concurrent.futures import ThreadPoolExecutor

import numpy as np

from .scoring import l2_normalize, score_image_text
from .tokenizer import Tokenizer

POOL_MEAN, POOL_PROBE = 0, 1
# the NaFlex front end of the reference server: rescale 1/255, mean = std = 0.5
# (src/siglip2_server.cpp:354-359)
RESCALE = 1.0 / 255.0
MEAN = (0.5, 0.5, 0.5)
STD = (0.5, 0.5, 0.5)


class EngineError(RuntimeError):
    """A request the engine cannot serve; status is the HTTP status the
    reference gives it (400 bad request, 500 encode failure, 501 not
    implemented, 503 tower not loaded)."""

    def __init__(self, msg, status=500):
        super().__init__(msg)
        self.status = status


def parse_pooling(s):
    """The reference's parse_pooling (src/siglip2_server.cpp:528-533)."""
    if s in ("", None, "pooler", "probe"):
        return POOL_PROBE
    if s == "mean":
        return POOL_MEAN
    raise EngineError(f"pooling must be one of: pooler, probe, mean (got '{s}')", 400)


def decode_image(data):
    """Image file bytes (any format Pillow reads: JPEG, PNG, ...) -> h x w x 3
    u8 RGB, as the reference's stb_image decode with 3 channels requested."""
    from PIL import Image
    try:
        with Image.open(io.BytesIO(data)) as im:
            return np.array(im.convert("RGB"), np.uint8)  # (a writable copy)
    except Exception as e:  # Pillow raises several types for undecodable data
        raise EngineError(f"image decode failed: {e}", 500) from e


class Engine:
    def __init__(self, model_path, tokenizer_path="", default_max_num_patches=729,
                 vision_only=False, text_only=False, **_):
        import torch
        import s2x
        if vision_only and text_only:
            raise EngineError("vision_only and text_only are mutually exclusive", 400)
        if not model_path:
            raise EngineError("model path required", 503)
        if not vision_only and not tokenizer_path:
            raise EngineError("tokenizer path required (or pass --vision-only)", 503)
        self._s2x, self._torch = s2x, torch
        self.default_max_num_patches = int(default_max_num_patches)
        self.vision = self.text = None
        self.tokenizer = None
        self.hidden_size = 0
        self.max_position_embeddings = 0
        self.logit_scale = self.logit_bias = None
        self._vision_lock = threading.Lock()
        self._text_lock = threading.Lock()
        self._helper = None
        dev = torch.device("cuda", torch.cuda.current_device())
        g = ctypes.c_void_p()
        s2x.call("s2x_gguf_open", str(model_path).encode(), ctypes.byref(g))
        try:
            if not text_only:
                w = s2x.VisionWeights()
                s2x.call("s2x_gguf_vision_weights", g, ctypes.byref(w))
                h = ctypes.c_void_p()
                s2x.call("s2x_vision_create", ctypes.byref(w), ctypes.byref(h))
                self.vision = h
                self.hidden_size = w.hidden
                self._vstream = torch.cuda.Stream(device=dev)
                s2x.call("s2x_vision_set_stream", h, ctypes.c_void_p(self._vstream.cuda_stream))
            if not vision_only:
                t = s2x.TextWeights()
                s2x.call("s2x_gguf_text_weights", g, ctypes.byref(t))
                h = ctypes.c_void_p()
                s2x.call("s2x_text_create", ctypes.byref(t), ctypes.byref(h))
                self.text = h
                self.max_position_embeddings = t.max_pos
                self.text_dim = t.proj
                self.hidden_size = self.hidden_size or t.proj
                self._tstream = torch.cuda.Stream(device=dev)
                s2x.call("s2x_text_set_stream", h, ctypes.c_void_p(self._tstream.cuda_stream))
                self.tokenizer = Tokenizer(tokenizer_path)
            if self.vision is not None and self.text is not None:
                sc, bi = ctypes.c_float(), ctypes.c_float()
                s2x.call("s2x_gguf_score_params", g, ctypes.byref(sc), ctypes.byref(bi))
                self.logit_scale, self.logit_bias = sc.value, bi.value
                self._helper = ThreadPoolExecutor(max_workers=1, thread_name_prefix="s2x-text")
        except Exception:
            self.close()
            raise
        finally:
            s2x.lib.s2x_gguf_close(g)  # the encoders hold device copies

    @property
    def has_vision(self):
        return self.vision is not None

    @property
    def has_text(self):
        return self.text is not None

    def close(self):
        if self._helper is not None:
            self._helper.shutdown(wait=True)
            self._helper = None
        if self.vision is not None:
            self._s2x.lib.s2x_vision_destroy(self.vision)
            self.vision = None
        if self.text is not None:
            self._s2x.lib.s2x_text_destroy(self.text)
            self.text = None

    # -- vision -------------------------------------------------------------
    def _image_embeds(self, blobs, pooling, max_num_patches):
        """Raw (not normalized) embeddings [n, hidden] of image files."""
        if self.vision is None:
            raise EngineError("vision tower not loaded (server started with --text-only)", 503)
        if not blobs:
            raise EngineError("No images provided", 400)
        torch = self._torch
        mnp = int(max_num_patches) if max_num_patches else self.default_max_num_patches
        imgs = [decode_image(b) for b in blobs]
        hw = np.array([[im.shape[0], im.shape[1]] for im in imgs], np.int32)
        mean = (ctypes.c_float * 3)(*MEAN)
        std = (ctypes.c_float * 3)(*STD)
        with self._vision_lock, torch.cuda.stream(self._vstream):
            devs = [torch.from_numpy(im).to(self._vstream.device, non_blocking=False) for im in imgs]
            ptrs = (ctypes.c_void_p * len(devs))(*[d.data_ptr() for d in devs])
            out = torch.empty((len(imgs), self.hidden_size), dtype=torch.float32, device=self._vstream.device)
            try:
                self._s2x.call("s2x_vision_encode_rgb_batch_dev", self.vision, ptrs,
                               hw.ctypes.data, len(imgs), mnp, ctypes.c_float(RESCALE), mean, std,
                               pooling, ctypes.c_void_p(out.data_ptr()))
            except self._s2x.S2XError as e:
                raise EngineError(f"vision encode: {e}", 500) from e
            self._vstream.synchronize()
            return out.cpu().numpy()

    def encode_images(self, blobs, pooling="probe", max_num_patches=None, return_last_hidden=False):
        if return_last_hidden:
            raise EngineError("return_last_hidden not implemented", 501)
        return l2_normalize(self._image_embeds(blobs, parse_pooling(pooling), max_num_patches))

    # -- text ---------------------------------------------------------------
    def _text_embeds(self, prompts):
        if self.text is None:
            raise EngineError("text tower not loaded (server started with --vision-only)", 503)
        if not prompts:
            raise EngineError("No prompts provided", 400)
        n_tok = self.max_position_embeddings
        ids = np.empty((len(prompts), n_tok), np.int32)
        for i, p in enumerate(prompts):
            ids[i] = self.tokenizer.encode(p, n_tok)[0]
        if int(ids.max()) >= self.tokenizer.vocab_size or int(ids.min()) < 0:
            raise EngineError("tokenizer produced an id outside its vocabulary", 500)
        out = np.empty((len(prompts), self.text_dim), np.float32)
        with self._text_lock:
            try:
                self._s2x.call("s2x_text_encode_batch", self.text, ids.ctypes.data, n_tok,
                               len(prompts), out.ctypes.data)
            except self._s2x.S2XError as e:
                raise EngineError(f"text encode_batch: {e}", 500) from e
        return out

    def encode_texts(self, prompts):
        return l2_normalize(self._text_embeds(prompts))

    # -- scores -------------------------------------------------------------
    def _require_both(self):
        if self.vision is None or self.text is None:
            raise EngineError("classify requires both towers loaded", 503)

    def classify(self, blobs, prompts, max_num_patches=None, return_logits=False):
        """Sigmoid scores [n_img][n_txt] (and logits) of image files against
        prompts; the text encode runs beside the image encodes."""
        self._require_both()
        if not blobs:
            raise EngineError("No images provided", 400)
        if not prompts:
            raise EngineError("No prompts provided", 400)
        text_future = self._helper.submit(self._text_embeds, list(prompts))
        try:
            img = self._image_embeds(blobs, POOL_PROBE, max_num_patches)
        finally:
            txt = text_future.result()  # (re-raises the text side's error)
        return self._scores(img, txt, return_logits)

    def classify_from_embeddings(self, image_embeddings, prompts, return_logits=False):
        self._require_both()
        rows = list(image_embeddings)
        if any(len(r) != self.hidden_size for r in rows):
            raise EngineError("image_embedding row has wrong dim", 400)
        img = np.asarray(rows, np.float32).reshape(len(rows), self.hidden_size)
        txt = self._text_embeds(list(prompts))
        return self._scores(img, txt, return_logits)

    def _scores(self, img, txt, return_logits):
        logits, probs = score_image_text(img, txt, self.logit_scale, self.logit_bias)
        return probs, (logits if return_logits else None)
