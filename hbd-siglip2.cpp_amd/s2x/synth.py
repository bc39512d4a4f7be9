"""Seeded synthetic SigLIP2 weights and inputs (no checkpoint is available).

Linear weights ~ N(0, 0.02) quantized to Q8_0 (ggml's quantize_row_q8_0
rule: d = amax/127, q = roundf(x / d), fp16 d; K zero-padded to a multiple
of 32 as tools/siglip2-quantize/main.cpp:174-186 does for ffn_down),
biases ~ N(0, 0.02), LayerNorm gamma ~ 1 + N(0, 0.02), beta ~ N(0, 0.02),
position embeddings ~ N(0, 0.02), probe ~ N(0, 1).

Every tensor draws from its own numpy Generator seeded with (seed, index),
so a tensor's bytes do not depend on which other tensors were generated.
"""
import ctypes
import os
from concurrent.futures import ThreadPoolExecutor
from dataclasses import dataclass, field

import numpy as np

QK = 32


@dataclass
class VisionConfig:
    hidden: int = 1152
    inter: int = 4304
    n_head: int = 16
    n_layer: int = 27
    patch_dim: int = 768
    n_side: int = 16
    eps: float = 1e-6

    @property
    def inter_pad(self):
        return (self.inter + QK - 1) // QK * QK

    @property
    def d_head(self):
        return self.hidden // self.n_head


@dataclass
class TextConfig:
    hidden: int = 1152
    inter: int = 4304
    n_head: int = 16
    n_layer: int = 27
    vocab: int = 256000
    max_pos: int = 64
    proj: int = 1152
    eps: float = 1e-6

    @property
    def inter_pad(self):
        return (self.inter + QK - 1) // QK * QK


SO400M_VISION = VisionConfig()
SO400M_TEXT = TextConfig()


def _quantize_rows(w, k_pad):
    n, k = w.shape
    if k_pad != k:
        w = np.concatenate([w, np.zeros((n, k_pad - k), np.float32)], axis=1)
    b = w.reshape(n, k_pad // QK, QK)
    amax = np.abs(b).max(axis=2)
    d = (amax / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        idv = np.where(d != 0, np.float32(1.0) / d, np.float32(0.0)).astype(np.float32)
    v = b * idv[:, :, None]  # f32 products, as x * id in the C reference
    # roundf: half away from zero (v - trunc(v) is exact in f32)
    t = np.trunc(v)
    q = np.where(np.abs(v - t) >= np.float32(0.5), t + np.sign(v), t).astype(np.int8)
    out = np.empty((n, k_pad // QK, 34), np.uint8)
    out[:, :, 0:2] = d.astype(np.float16).view(np.uint8).reshape(n, k_pad // QK, 2)
    out[:, :, 2:] = q.view(np.uint8)
    return out.reshape(n, -1)


def quantize_q8_0(w, k_pad=None):
    """Rows of w (n, k) float32 -> raw Q8_0 bytes (n, k_pad/32 * 34), uint8.

    ggml quantize_row_q8_0_ref: amax over the block, d = amax/127 (f32),
    id = 1/d (0 if d == 0), q = roundf(x * id) (half away from zero),
    d stored as fp16 (round to nearest even).  Rows are done in chunks on a
    few threads (numpy releases the GIL in these loops)."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    n, k = w.shape
    k_pad = k if k_pad is None else k_pad
    assert k_pad % QK == 0 and k_pad >= k
    out = np.empty((n, k_pad // QK * 34), np.uint8)
    step = 4096

    def job(r0):
        out[r0:r0 + step] = _quantize_rows(w[r0:r0 + step], k_pad)

    if n <= step:
        job(0)
    else:
        with ThreadPoolExecutor(min(8, os.cpu_count() or 1)) as ex:
            list(ex.map(job, range(0, n, step)))
    return out


def _rng(seed, idx):
    return np.random.default_rng([seed, idx])


def _normal(seed, idx, shape, std=1.0, mean=0.0):
    x = _rng(seed, idx).standard_normal(shape, dtype=np.float32)
    if std != 1.0:
        x *= np.float32(std)
    if mean != 0.0:
        x += np.float32(mean)
    return x


@dataclass
class HostModel:
    """Host tensors of one tower plus the ctypes struct that points at them."""
    cfg: object
    tensors: dict = field(default_factory=dict)
    layers: list = field(default_factory=list)
    struct: object = None
    down_f16: bool = False  # ffn_down matrices as F16 rows
    _keep: list = field(default_factory=list)

    def ptr(self, a):
        a = np.ascontiguousarray(a)
        self._keep.append(a)
        return a.ctypes.data


def _linear(seed, idx, k, n, k_pad=None):
    w = _normal(seed, idx, (n, k), 0.02)
    return quantize_q8_0(w, k_pad)


LAYER_KEYS = ["ln1_w", "ln1_b", "qkv_w", "qkv_b", "o_w", "o_b", "ln2_w", "ln2_b",
              "up_w", "up_b", "down_w", "down_b"]


def _down(seed, idx, F, H, F_pad, f16):
    """ffn_down: Q8_0 with K padded to F_pad, or (f16) F16 rows of F halves
    from the same N(0, 0.02) draw (the reference converter's type for K % 32
    != 0)."""
    if f16:
        return _normal(seed, idx, (H, F), 0.02).astype(np.float16)
    return _linear(seed, idx, F, H, F_pad)


def _layer(seed, base, H, F, F_pad, f16=False):
    return {
        "ln1_w": _normal(seed, base + 0, (H,), 0.02, 1.0),
        "ln1_b": _normal(seed, base + 1, (H,), 0.02),
        "qkv_w": _linear(seed, base + 2, H, 3 * H),
        "qkv_b": _normal(seed, base + 3, (3 * H,), 0.02),
        "o_w": _linear(seed, base + 4, H, H),
        "o_b": _normal(seed, base + 5, (H,), 0.02),
        "ln2_w": _normal(seed, base + 6, (H,), 0.02, 1.0),
        "ln2_b": _normal(seed, base + 7, (H,), 0.02),
        "up_w": _linear(seed, base + 8, H, F),
        "up_b": _normal(seed, base + 9, (F,), 0.02),
        "down_w": _down(seed, base + 10, F, H, F_pad, f16),
        "down_b": _normal(seed, base + 11, (H,), 0.02),
    }


def _layers(seed, n_layer, H, F, F_pad, f16=False):
    """Every layer's tensors (each from its own seeded streams, so the
    values do not depend on the order the threads run in)."""
    with ThreadPoolExecutor(min(4, os.cpu_count() or 1)) as ex:
        return list(ex.map(lambda l: _layer(seed, 1000 + 100 * l, H, F, F_pad, f16), range(n_layer)))


def vision_model(cfg=SO400M_VISION, seed=0, down_f16=False):
    """Seeded vision tower weights; .struct is an s2x.VisionWeights.
    down_f16: ffn_down matrices (layers and MAP head) as F16."""
    from . import LayerWeights, VisionWeights
    H, F, Fp = cfg.hidden, cfg.inter, cfg.inter_pad
    m = HostModel(cfg)
    t = m.tensors
    t["patch_w"] = _linear(seed, 1, cfg.patch_dim, H)
    t["patch_b"] = _normal(seed, 2, (H,), 0.02)
    t["pos_embd"] = _normal(seed, 3, (cfg.n_side * cfg.n_side, H), 0.02)
    t["post_ln_w"] = _normal(seed, 4, (H,), 0.02, 1.0)
    t["post_ln_b"] = _normal(seed, 5, (H,), 0.02)
    t["probe"] = _normal(seed, 6, (H,), 1.0)
    t["hq_w"] = _linear(seed, 7, H, H)
    t["hk_w"] = _linear(seed, 8, H, H)
    t["hv_w"] = _linear(seed, 9, H, H)
    t["ho_w"] = _linear(seed, 10, H, H)
    t["hq_b"] = _normal(seed, 11, (H,), 0.02)
    t["hk_b"] = _normal(seed, 12, (H,), 0.02)
    t["hv_b"] = _normal(seed, 13, (H,), 0.02)
    t["ho_b"] = _normal(seed, 14, (H,), 0.02)
    t["hln_w"] = _normal(seed, 15, (H,), 0.02, 1.0)
    t["hln_b"] = _normal(seed, 16, (H,), 0.02)
    t["hup_w"] = _linear(seed, 17, H, F)
    t["hup_b"] = _normal(seed, 18, (F,), 0.02)
    t["hdown_w"] = _down(seed, 19, F, H, Fp, down_f16)
    t["hdown_b"] = _normal(seed, 20, (H,), 0.02)
    m.layers = _layers(seed, cfg.n_layer, H, F, Fp, down_f16)
    m.down_f16 = down_f16
    larr = (LayerWeights * max(1, cfg.n_layer))()
    for l, L in enumerate(m.layers):
        for k in LAYER_KEYS:
            setattr(larr[l], k, m.ptr(L[k]))
    m._keep.append(larr)
    s = VisionWeights()
    s.hidden, s.inter, s.inter_pad, s.n_head = H, F, Fp, cfg.n_head
    s.n_layer, s.patch_dim, s.n_side, s.eps = cfg.n_layer, cfg.patch_dim, cfg.n_side, cfg.eps
    for k, v in t.items():
        setattr(s, k, m.ptr(v))
    s.layers = ctypes.cast(larr, ctypes.POINTER(LayerWeights))
    s.down_f16 = int(down_f16)
    m.struct = s
    return m


def text_model(cfg=SO400M_TEXT, seed=0, down_f16=False):
    """Seeded text tower weights; .struct is an s2x.TextWeights.
    down_f16: ffn_down matrices as F16."""
    from . import LayerWeights, TextWeights
    H, F, Fp = cfg.hidden, cfg.inter, cfg.inter_pad
    m = HostModel(cfg)
    t = m.tensors
    t["tok_embd"] = _linear(seed, 1, H, cfg.vocab)
    t["pos_embd"] = _normal(seed, 2, (cfg.max_pos, H), 0.02)
    t["final_ln_w"] = _normal(seed, 3, (H,), 0.02, 1.0)
    t["final_ln_b"] = _normal(seed, 4, (H,), 0.02)
    t["head_w"] = _linear(seed, 5, H, cfg.proj)
    t["head_b"] = _normal(seed, 6, (cfg.proj,), 0.02)
    m.layers = _layers(seed, cfg.n_layer, H, F, Fp, down_f16)
    m.down_f16 = down_f16
    larr = (LayerWeights * max(1, cfg.n_layer))()
    for l, L in enumerate(m.layers):
        for k in LAYER_KEYS:
            setattr(larr[l], k, m.ptr(L[k]))
    m._keep.append(larr)
    s = TextWeights()
    s.hidden, s.inter, s.inter_pad, s.n_head = H, F, Fp, cfg.n_head
    s.n_layer, s.vocab, s.max_pos, s.proj, s.eps = (
        cfg.n_layer, cfg.vocab, cfg.max_pos, cfg.proj, cfg.eps)
    for k, v in t.items():
        setattr(s, k, m.ptr(v))
    s.layers = ctypes.cast(larr, ctypes.POINTER(LayerWeights))
    s.down_f16 = int(down_f16)
    m.struct = s
    return m


def pixels(n_img, n_pos, patch_dim=768, seed=1234):
    """Patch vectors uniform in [-1, 1], float32 [n_img * n_pos, patch_dim]."""
    r = np.random.default_rng([seed, n_img, n_pos])
    return r.uniform(-1.0, 1.0, size=(n_img * n_pos, patch_dim)).astype(np.float32)


def text_tokens(n_batch, n_tok=64, vocab=256000, eos=1, seed=4321):
    """Token ids uniform in [1, vocab) with an EOS-padded tail of random
    length: each prompt keeps 4..n_tok ids, the rest are `eos`."""
    r = np.random.default_rng([seed, n_batch, n_tok])
    ids = r.integers(1, vocab, size=(n_batch, n_tok), dtype=np.int32)
    lens = r.integers(4, n_tok + 1, size=n_batch)
    for b, L in enumerate(lens):
        ids[b, L:] = eos
    return ids, lens
