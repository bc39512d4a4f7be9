"""ctypes binding of the CPU oracle (oracle/_build/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's CPU-baseline leg, never by the product.  Build with `make -C oracle`.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "liboracle.so")

_lib = None
_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_f32 = ctypes.c_float


class OrcLayer(ctypes.Structure):
    _fields_ = [(n, _p) for n in (
        "ln1_w", "ln1_b", "qkv_w", "qkv_b", "o_w", "o_b", "ln2_w", "ln2_b",
        "up_w", "up_b", "down_w", "down_b")]


class OrcVision(ctypes.Structure):
    _fields_ = [
        ("hidden", _i32), ("inter", _i32), ("inter_pad", _i32), ("n_head", _i32),
        ("n_layer", _i32), ("patch_dim", _i32), ("n_side", _i32), ("eps", _f32),
        ("patch_w", _p), ("patch_b", _p), ("pos_embd", _p), ("post_ln_w", _p),
        ("post_ln_b", _p), ("probe", _p), ("hq_w", _p), ("hk_w", _p), ("hv_w", _p),
        ("ho_w", _p), ("hq_b", _p), ("hk_b", _p), ("hv_b", _p), ("ho_b", _p),
        ("hln_w", _p), ("hln_b", _p), ("hup_w", _p), ("hup_b", _p), ("hdown_w", _p),
        ("hdown_b", _p), ("layers", ctypes.POINTER(OrcLayer)), ("down_f16", _i32),
    ]


class OrcText(ctypes.Structure):
    _fields_ = [
        ("hidden", _i32), ("inter", _i32), ("inter_pad", _i32), ("n_head", _i32),
        ("n_layer", _i32), ("vocab", _i32), ("max_pos", _i32), ("proj", _i32),
        ("eps", _f32), ("tok_embd", _p), ("pos_embd", _p), ("final_ln_w", _p),
        ("final_ln_b", _p), ("head_w", _p), ("head_b", _p),
        ("layers", ctypes.POINTER(OrcLayer)), ("down_f16", _i32),
    ]


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} missing; run `make -C oracle`")
        L = ctypes.CDLL(LIB_PATH)
        sig = {
            "orc_fp32_to_fp16_n": ([_p, _p, _i64], None),
            "orc_fp16_to_fp32_n": ([_p, _p, _i64], None),
            "orc_quantize_q8_0_padded": ([_p, _i64, _i64, _i64, _p], None),
            "orc_dequantize_q8_0": ([_p, _i64, _i64, _p], None),
            "orc_quantize_q8_1": ([_p, _i64, _i64, _i64, _i64, _p, _p], None),
            "orc_block_dots": ([_p, _i64, _i64, _p, _i64, _p], None),
            "orc_mul_mat_q8_0_q8_1": ([_p, _i64, _i64, _p, _p, _i64, _p, ctypes.c_int], None),
            "orc_mul_mat_q8_0_f32": ([_p, _i64, _i64, _p, _i64, _i64, _i64, _p, ctypes.c_int], None),
            "orc_mul_mat_f16_f32": ([_p, _i64, _i64, _p, _i64, _i64, _p, ctypes.c_int], None),
            "orc_layernorm": ([_p, _i64, _i64, _i64, _p, _p, _f32, _p, _i64], None),
            "orc_gelu": ([_f32], _f32),
            "orc_gelu_tanhf": ([_f32], _f32),
            "orc_gelu_ggml": ([_f32], _f32),
            "orc_set_gelu_mode": ([ctypes.c_int], ctypes.c_int),
            "orc_gelu_array": ([ctypes.c_int, _p, _p, _i64], None),
            "orc_set_gemm_kernel": ([ctypes.c_int], ctypes.c_int),
            "orc_clear_gemm_cache": ([], None),
            "cq8_have_vnni": ([], ctypes.c_int),
            "orc_tanh_f32": ([_f32], _f32),
            "orc_attention": ([_p, _i64, _i64, _i64, _f32, _p, _p], None),
            "orc_attention_1q": ([_p, _p, _p, _i64, _i64, _i64, _i64, _f32, _p], None),
            "orc_resize_pos_embed": ([_p, _i64, _i64, _i64, _i64, _p], None),
            "orc_nf_target_size": ([_i32, _i32, _i32, _i32, _p, _p], None),
            "orc_nf_preprocess_rgb": ([_p, _i32, _i32, _i32, _i32, _f32, _p, _p, ctypes.c_int,
                                       _p, _i64, _p, _p], ctypes.c_int),
            "orc_vision_encode": ([ctypes.POINTER(OrcVision), _p, _i32, _i32, _i32, _p, _p,
                                   ctypes.c_int], None),
            "orc_text_encode": ([ctypes.POINTER(OrcText), _p, _i32, _p, _p, ctypes.c_int], None),
        }
        for name, (args, res) in sig.items():
            f = getattr(L, name)
            f.argtypes = args
            f.restype = res
        _lib = L
    return _lib


def _ptr(a):
    return a.ctypes.data if a is not None else None


def fp32_to_fp16(x):
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(x.shape, np.uint16)
    lib().orc_fp32_to_fp16_n(_ptr(x), _ptr(y), x.size)
    return y


def fp16_to_fp32(h):
    h = np.ascontiguousarray(h, np.uint16)
    y = np.empty(h.shape, np.float32)
    lib().orc_fp16_to_fp32_n(_ptr(h), _ptr(y), h.size)
    return y


def quantize_q8_0(w, k_pad=None):
    w = np.ascontiguousarray(w, np.float32)
    n, k = w.shape
    k_pad = k if k_pad is None else k_pad
    out = np.empty((n, k_pad // 32 * 34), np.uint8)
    lib().orc_quantize_q8_0_padded(_ptr(w), n, k, k_pad, _ptr(out))
    return out


def dequantize_q8_0(raw, n, k_pad):
    y = np.empty((n, k_pad), np.float32)
    lib().orc_dequantize_q8_0(_ptr(np.ascontiguousarray(raw)), n, k_pad, _ptr(y))
    return y


def quantize_q8_1(x, k_pad=None):
    """x (M, K) float32 -> qs (M, k_pad) int8, ds (M, k_pad/32, 2) uint16."""
    x = np.ascontiguousarray(x, np.float32)
    M, K = x.shape
    k_pad = K if k_pad is None else k_pad
    qs = np.empty((M, k_pad), np.int8)
    ds = np.empty((M, k_pad // 32, 2), np.uint16)
    lib().orc_quantize_q8_1(_ptr(x), M, K, K, k_pad, _ptr(qs), _ptr(ds))
    return qs, ds


def block_dots(w_raw, k_pad, n, qs, m):
    out = np.empty(k_pad // 32, np.int32)
    lib().orc_block_dots(_ptr(np.ascontiguousarray(w_raw)), k_pad, n,
                         _ptr(np.ascontiguousarray(qs)), m, _ptr(out))
    return out


def mul_mat_q8_0_q8_1(w_raw, k_pad, n, qs, ds, nthreads=0):
    M = qs.shape[0]
    y = np.empty((M, n), np.float32)
    lib().orc_mul_mat_q8_0_q8_1(_ptr(np.ascontiguousarray(w_raw)), k_pad, n,
                                _ptr(np.ascontiguousarray(qs)), _ptr(np.ascontiguousarray(ds)),
                                M, _ptr(y), nthreads)
    return y


def mul_mat_f16_f32(w16, x, nthreads=0):
    """w16 (N, K) float16 / uint16 bits, x (M, K) float32 -> (M, N) float32."""
    w16 = np.ascontiguousarray(w16).view(np.uint16)
    x = np.ascontiguousarray(x, np.float32)
    M, K = x.shape
    N = w16.shape[0]
    assert w16.shape == (N, K)
    y = np.empty((M, N), np.float32)
    lib().orc_mul_mat_f16_f32(_ptr(w16), K, N, _ptr(x), K, M, _ptr(y), nthreads)
    return y


def mul_mat_q8_0_f32(w_raw, k_pad, n, x, nthreads=0):
    x = np.ascontiguousarray(x, np.float32)
    M, K = x.shape
    y = np.empty((M, n), np.float32)
    lib().orc_mul_mat_q8_0_f32(_ptr(np.ascontiguousarray(w_raw)), k_pad, n, _ptr(x), K, K, M,
                               _ptr(y), nthreads)
    return y


def layernorm(x, w, b, eps=1e-6):
    x = np.ascontiguousarray(x, np.float32)
    M, H = x.shape
    y = np.empty_like(x)
    lib().orc_layernorm(_ptr(x), M, H, H, _ptr(w), _ptr(b), eps, _ptr(y), H)
    return y


def gelu(x):
    f = lib().orc_gelu
    return np.array([f(float(v)) for v in np.asarray(x, np.float32).ravel()],
                    np.float32).reshape(np.shape(x))


GELU_EXACT, GELU_TANHF, GELU_GGML = 0, 1, 2


def gelu_mode(mode, x):
    """GELU of an array in one of the oracle's modes: GELU_EXACT (the GPU's
    formulation), GELU_TANHF (the reference CUDA formula with libm tanhf),
    GELU_GGML (ggml-cpu's fp16 table)."""
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    lib().orc_gelu_array(mode, _ptr(x), _ptr(y), x.size)
    return y


def set_gemm_kernel(k):
    """The towers' GEMM kernel: 0 the scalar restatement (default), 1 the
    AVX-512 VNNI kernel of cpu_q8.c (same bits) where the CPU has it.
    Returns the previous kernel."""
    return lib().orc_set_gemm_kernel(k)


def have_vnni():
    return bool(lib().cq8_have_vnni())


def set_gelu_mode(mode):
    """The GELU the tower restatements use; returns the previous mode."""
    return lib().orc_set_gelu_mode(mode)


def tanh_f32(x):
    f = lib().orc_tanh_f32
    return np.array([f(float(v)) for v in np.asarray(x, np.float32).ravel()],
                    np.float32).reshape(np.shape(x))


def attention_1q(q, k, v, n_head, d_head, scale):
    """Single-query attention of q (H) over the rows of k and v ([n_pos, H])."""
    q = np.ascontiguousarray(q, np.float32)
    k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    out = np.empty(n_head * d_head, np.float32)
    lib().orc_attention_1q(_ptr(q), _ptr(k), _ptr(v), k.shape[1], k.shape[0], n_head, d_head,
                           scale, _ptr(out))
    return out


def attention(qkv, n_head, d_head, scale, key_valid=None):
    qkv = np.ascontiguousarray(qkv, np.float32)
    n_pos = qkv.shape[0]
    out = np.empty((n_pos, n_head * d_head), np.float32)
    kv = None if key_valid is None else np.ascontiguousarray(key_valid, np.uint8)
    lib().orc_attention(_ptr(qkv), n_pos, n_head, d_head, scale, _ptr(kv), _ptr(out))
    return out


def resize_pos_embed(pos, n_side, out_h, out_w):
    pos = np.ascontiguousarray(pos, np.float32)
    H = pos.shape[-1]
    out = np.empty((out_h * out_w, H), np.float32)
    lib().orc_resize_pos_embed(_ptr(pos), n_side, H, out_h, out_w, _ptr(out))
    return out


def nf_target_size(h, w, p, max_patches):
    th, tw = ctypes.c_int32(), ctypes.c_int32()
    lib().orc_nf_target_size(h, w, p, max_patches, ctypes.byref(th), ctypes.byref(tw))
    return th.value, tw.value


NF_MEAN = np.array([0.5, 0.5, 0.5], np.float32)
NF_STD = np.array([0.5, 0.5, 0.5], np.float32)


def _nf_call(fn, rgb, max_patches, p, rescale, mean, std, extra=()):
    rgb = np.ascontiguousarray(rgb, np.uint8)
    h, w = rgb.shape[:2]
    mean = np.ascontiguousarray(mean, np.float32)
    std = np.ascontiguousarray(std, np.float32)
    cap = max_patches * 3 * p * p
    out = np.empty(cap, np.float32)
    nh, nw = ctypes.c_int32(), ctypes.c_int32()
    st = fn(_ptr(rgb), h, w, max_patches, p, ctypes.c_float(rescale), _ptr(mean), _ptr(std), *extra,
            _ptr(out), cap, ctypes.byref(nh), ctypes.byref(nw))
    if st != 0:
        raise ValueError("preprocess failed")
    return out[: nh.value * nw.value * 3 * p * p].reshape(nh.value * nw.value, 3 * p * p), nh.value, nw.value


def nf_preprocess_rgb(rgb, max_patches, p=16, rescale=1.0 / 255.0, mean=NF_MEAN, std=NF_STD, fused=1):
    """NaFlex preprocessing of an (h, w, 3) uint8 image -> (patches, n_h, n_w)."""
    return _nf_call(lib().orc_nf_preprocess_rgb, rgb, max_patches, p, rescale, mean, std,
                    (ctypes.c_int(fused),))


REF_PREPROC_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_ref", "libref_preproc.so")
_ref = None


def ref_preprocess_lib():
    """The reference's own preprocessing (oracle/_ref, built by `make -C
    oracle ref` where the reference tree exists), or None."""
    global _ref
    if _ref is None and os.path.exists(REF_PREPROC_PATH):
        L = ctypes.CDLL(REF_PREPROC_PATH)
        L.ref_nf_preprocess_rgb.argtypes = [_p, _i32, _i32, _i32, _i32, _f32, _p, _p, _p, _i64, _p, _p]
        L.ref_nf_preprocess_rgb.restype = ctypes.c_int
        _ref = L
    return _ref


def ref_preprocess_rgb(rgb, max_patches, p=16, rescale=1.0 / 255.0, mean=NF_MEAN, std=NF_STD):
    return _nf_call(ref_preprocess_lib().ref_nf_preprocess_rgb, rgb, max_patches, p, rescale, mean, std)


LAYER_KEYS = [f[0] for f in OrcLayer._fields_]


class _Model:
    def __init__(self, struct, keep):
        self.struct = struct
        self._keep = keep


def vision_model(host):
    """Oracle view of an s2x.synth HostModel (vision): same host bytes."""
    cfg, t = host.cfg, host.tensors
    keep = []

    def P(a):
        a = np.ascontiguousarray(a)
        keep.append(a)
        return a.ctypes.data

    larr = (OrcLayer * max(1, cfg.n_layer))()
    for l, L in enumerate(host.layers):
        for k in LAYER_KEYS:
            setattr(larr[l], k, P(L[k]))
    keep.append(larr)
    s = OrcVision()
    s.hidden, s.inter, s.inter_pad, s.n_head = cfg.hidden, cfg.inter, cfg.inter_pad, cfg.n_head
    s.n_layer, s.patch_dim, s.n_side, s.eps = cfg.n_layer, cfg.patch_dim, cfg.n_side, cfg.eps
    for k, v in t.items():
        setattr(s, k, P(v))
    s.layers = ctypes.cast(larr, ctypes.POINTER(OrcLayer))
    s.down_f16 = int(getattr(host, "down_f16", False))
    return _Model(s, keep)


def text_model(host):
    cfg, t = host.cfg, host.tensors
    keep = []

    def P(a):
        a = np.ascontiguousarray(a)
        keep.append(a)
        return a.ctypes.data

    larr = (OrcLayer * max(1, cfg.n_layer))()
    for l, L in enumerate(host.layers):
        for k in LAYER_KEYS:
            setattr(larr[l], k, P(L[k]))
    keep.append(larr)
    s = OrcText()
    s.hidden, s.inter, s.inter_pad, s.n_head = cfg.hidden, cfg.inter, cfg.inter_pad, cfg.n_head
    s.n_layer, s.vocab, s.max_pos, s.proj, s.eps = (cfg.n_layer, cfg.vocab, cfg.max_pos,
                                                    cfg.proj, cfg.eps)
    for k, v in t.items():
        setattr(s, k, P(v))
    s.layers = ctypes.cast(larr, ctypes.POINTER(OrcLayer))
    s.down_f16 = int(getattr(host, "down_f16", False))
    return _Model(s, keep)


def vision_encode(model, pixels, n_h, n_w, pooling=1, nthreads=0, hidden=False):
    H = model.struct.hidden
    out = np.empty(H, np.float32)
    hid = np.empty((n_h * n_w, H), np.float32) if hidden else None
    px = np.ascontiguousarray(pixels, np.float32)
    lib().orc_vision_encode(ctypes.byref(model.struct), _ptr(px), n_h, n_w, pooling, _ptr(out),
                            _ptr(hid), nthreads)
    return (out, hid) if hidden else out


def text_encode(model, ids, mask=None, nthreads=0):
    ids = np.ascontiguousarray(ids, np.int32)
    out = np.empty(model.struct.proj, np.float32)
    m = None if mask is None else np.ascontiguousarray(mask, np.int32)
    lib().orc_text_encode(ctypes.byref(model.struct), _ptr(ids), ids.size, _ptr(m), _ptr(out),
                          nthreads)
    return out
