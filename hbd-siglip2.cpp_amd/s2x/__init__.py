"""Python bindings of libs2x.so, the gfx950 SigLIP2 Q8_0 hot path.

ctypes over the C-ABI declared in include/s2x.h.  Device memory is passed as
integer addresses (e.g. torch.Tensor.data_ptr()), streams as integer handles
(torch.cuda.current_stream().cuda_stream) or None for the null stream.

Importing this module loads the in-tree libs2x.so and fails loudly if it is
missing: there is no CPU fallback.
"""
import ctypes
import importlib.util
import os

__all__ = [
    "S2XError", "lib", "Epilogue", "LayerWeights", "VisionWeights", "TextWeights",
    "EPI_NONE", "EPI_BIAS", "EPI_BIAS_GELU", "EPI_BIAS_RESID", "EPI_GELU_Q81", "POOL_MEAN",
    "POOL_PROBE",
]

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(os.path.dirname(_HERE), "libs2x.so")

EPI_NONE, EPI_BIAS, EPI_BIAS_GELU, EPI_BIAS_RESID, EPI_GELU_Q81, EPI_GELU_F16 = 0, 1, 2, 3, 4, 5
POOL_MEAN, POOL_PROBE = 0, 1

if not os.path.exists(LIB_PATH):
    raise ImportError(
        f"libs2x.so not found at {LIB_PATH}; build it with "
        "`python hbd-siglip2.cpp_amd/build.py` (no CPU fallback exists)")



def _share_torch_hip_runtime():
    """Load PyTorch's bundled HIP runtime first, when PyTorch is installed.

    libs2x.so and PyTorch's ROCm build each bring a libamdhip64.so.7 (this
    image: /opt/rocm's and torch/lib's).  The soname is the same, so the
    process keeps whichever loads first for both; PyTorch fails to see any
    GPU on the /opt/rocm copy ("No HIP GPUs are available"), while libs2x.so
    runs on either.  Loading torch's copy (with RTLD_GLOBAL, without
    importing torch) before libs2x.so makes the import order irrelevant.
    """
    spec = importlib.util.find_spec("torch")
    if spec is None or not spec.origin:
        return
    hip = os.path.join(os.path.dirname(spec.origin), "lib", "libamdhip64.so")
    if os.path.exists(hip):
        ctypes.CDLL(hip, mode=ctypes.RTLD_GLOBAL)


_share_torch_hip_runtime()
lib = ctypes.CDLL(LIB_PATH)


class S2XError(RuntimeError):
    def __init__(self, status, msg):
        super().__init__(f"s2x status {status}: {msg}")
        self.status = status


_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_f32 = ctypes.c_float
_sz = ctypes.c_size_t
_fp = ctypes.POINTER(ctypes.c_float)


class Epilogue(ctypes.Structure):
    _fields_ = [("kind", _i32), ("bias", _p), ("resid", _p), ("ld_resid", _i64),
                ("resid_rows", _i64), ("q_out", _p), ("q_ds", _p), ("q_kpad", _i64)]


class LayerWeights(ctypes.Structure):
    _fields_ = [(n, _p) for n in (
        "ln1_w", "ln1_b", "qkv_w", "qkv_b", "o_w", "o_b", "ln2_w", "ln2_b",
        "up_w", "up_b", "down_w", "down_b")]


class VisionWeights(ctypes.Structure):
    _fields_ = [
        ("hidden", _i32), ("inter", _i32), ("inter_pad", _i32), ("n_head", _i32),
        ("n_layer", _i32), ("patch_dim", _i32), ("n_side", _i32), ("eps", _f32),
        ("patch_w", _p), ("patch_b", _p), ("pos_embd", _p), ("post_ln_w", _p),
        ("post_ln_b", _p), ("probe", _p), ("hq_w", _p), ("hk_w", _p), ("hv_w", _p),
        ("ho_w", _p), ("hq_b", _p), ("hk_b", _p), ("hv_b", _p), ("ho_b", _p),
        ("hln_w", _p), ("hln_b", _p), ("hup_w", _p), ("hup_b", _p), ("hdown_w", _p),
        ("hdown_b", _p), ("layers", ctypes.POINTER(LayerWeights)), ("down_f16", _i32),
    ]


class TextWeights(ctypes.Structure):
    _fields_ = [
        ("hidden", _i32), ("inter", _i32), ("inter_pad", _i32), ("n_head", _i32),
        ("n_layer", _i32), ("vocab", _i32), ("max_pos", _i32), ("proj", _i32),
        ("eps", _f32), ("tok_embd", _p), ("pos_embd", _p), ("final_ln_w", _p),
        ("final_ln_b", _p), ("head_w", _p), ("head_b", _p),
        ("layers", ctypes.POINTER(LayerWeights)), ("down_f16", _i32),
    ]


def _sig(name, argtypes, restype=ctypes.c_int):
    f = getattr(lib, name)
    f.argtypes = argtypes
    f.restype = restype
    return f


_sig("s2x_status_string", [ctypes.c_int], ctypes.c_char_p)
_sig("s2x_last_error", [], ctypes.c_char_p)
_sig("s2x_version", [], ctypes.c_char_p)
_sig("s2x_quantize_q8_1", [_p, _i64, _i64, _i64, _i64, _p, _p, _p])
_sig("s2x_weight_bytes", [_i64, _i64], _sz)
_sig("s2x_weight_create", [_p, ctypes.c_int, _i64, _i64, _p, ctypes.POINTER(_p)])
_sig("s2x_weight_create_in", [_p, _i64, _i64, _p, _p, ctypes.POINTER(_p)])
_sig("s2x_weight_destroy", [_p], None)
_sig("s2x_weight_k", [_p], _i64)
_sig("s2x_weight_n", [_p], _i64)
_sig("s2x_mul_mat_q8_0_q8_1", [_p, _p, _p, _i64, _p, _i64, ctypes.POINTER(Epilogue), _p])
_sig("s2x_mul_mat_q8_0_q8_1_split_k",
     [_p, _p, _p, _i64, _p, _i64, ctypes.POINTER(Epilogue), ctypes.c_int32, _p, _sz, _p])
_sig("s2x_mul_mat_workspace_size", [_i64, _i64, _i64], _sz)
_sig("s2x_mul_mat_q8_0_f32", [_p, _i64, _i64, _p, _i64, _i64, _i64, _p, _p, _sz, _p])
_sig("s2x_mul_mat_q8_0_f32_static", [_p, _i64, _i64, _p, _i64, _i64, _i64, _p, _p])
_sig("s2x_mul_mat_f16_workspace_size", [_i64, _i64, _i64], _sz)
_sig("s2x_mul_mat_f16_f32", [_p, _i64, _i64, _p, _i64, _i64, _p, _p, _sz, _p])
_sig("s2x_block_dots", [_p, _p, _i64, _i64, _p, _p])
_sig("s2x_mul_mat_qkv_attn_prep", [_p, _p, _p, _i64, _p, _p, _p, _i64, _i64, _i64, _i64, _p, _sz,
                                   _p])
_sig("s2x_layernorm", [_p, _i64, _i64, _i64, _p, _p, _f32, _p, _i64, _p])
_sig("s2x_layernorm_quantize_q8_1", [_p, _i64, _i64, _i64, _p, _p, _f32, _p, _p, _p, _i64, _p])
_sig("s2x_bias_residual", [_p, _p, _p, _p, _i64, _i64, _p])
_sig("s2x_bias_gelu", [_p, _p, _p, _i64, _i64, _p])
_sig("s2x_nf_target_size", [_i32, _i32, _i32, _i32, _p, _p])
_sig("s2x_nf_workspace_size", [_i32, _i32, _i32, _i32], _sz)
_sig("s2x_nf_preprocess_rgb_dev", [_p, _i32, _i32, _i32, _i32, _f32, _p, _p, _p, _i64, _p, _p, _p,
                                   _sz, _p])
_sig("s2x_nf_preprocess_rgb_batch_dev", [_p, _i32, _i32, _i32, _i32, _i32, _f32, _p, _p, _p, _i64,
                                         _p, _p, _p, _sz, _p])
_sig("s2x_attn_workspace_size", [_i64, _i64, _i64, _i64], _sz)
_sig("s2x_attn_prep", [_p, _i64, _p, _p, _p, _i64, _i64, _i64, _i64, _p, _sz, _p])
_sig("s2x_attn_run", [_p, _sz, _p, _p, _p, _i64, _i64, _i64, _i64, _f32, _p, _i64, _p])
_sig("s2x_attn_run_q8_1", [_p, _sz, _p, _p, _p, _i64, _i64, _i64, _i64, _f32, _i64, _p, _p, _i64,
                          _p, _i64, _p])
_sig("s2x_attn_fp64", [_p, _i64, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _f32, _p, _i64, _p])
_sig("s2x_attn_1q", [_p, _p, _p, _i64, _p, _p, _i64, _i64, _i64, _i64, _f32, _p, _p])
_sig("s2x_resize_pos_embed", [_p, _i64, _i64, _i64, _i64, _p, _p])
_sig("s2x_get_rows_q8_0", [_p, _i64, _i64, _p, _i64, _p, _i64, _p, _p])
_sig("s2x_vision_create", [ctypes.POINTER(VisionWeights), ctypes.POINTER(_p)])
_sig("s2x_vision_destroy", [_p], None)
_sig("s2x_vision_set_stream", [_p, _p])
_sig("s2x_vision_set_attention_fp64", [_p, ctypes.c_int])
_sig("s2x_vision_set_graphs", [_p, ctypes.c_int])
_sig("s2x_vision_set_split_k", [_p, ctypes.c_int])
_sig("s2x_vision_encode_rgb_batch_dev", [_p, _p, _p, _i32, _i32, _f32, _p, _p, _i32, _p])
_sig("s2x_text_set_attention_fp64", [_p, ctypes.c_int])
_sig("s2x_text_set_graphs", [_p, ctypes.c_int])
_sig("s2x_text_set_split_k", [_p, ctypes.c_int])
_sig("s2x_vision_encode", [_p, _p, _i32, _i32, _i32, _p])
_sig("s2x_vision_encode_batch_dev", [_p, _p, _i32, _i32, _i32, _i32, _p])
_sig("s2x_vision_encode_ragged_dev", [_p, _p, _p, _i32, _i32, _i32, _p])
_sig("s2x_vision_gemm_timing", [_p, ctypes.c_int])
_sig("s2x_vision_gemm_stats", [_p, ctypes.POINTER(ctypes.c_double),
                               ctypes.POINTER(ctypes.c_double), ctypes.POINTER(_i64), ctypes.c_int])
_sig("s2x_gguf_open", [ctypes.c_char_p, ctypes.POINTER(_p)])
_sig("s2x_gguf_close", [_p], None)
_sig("s2x_gguf_vision_weights", [_p, ctypes.POINTER(VisionWeights)])
_sig("s2x_gguf_text_weights", [_p, ctypes.POINTER(TextWeights)])
_sig("s2x_gguf_score_params", [_p, ctypes.POINTER(_f32), ctypes.POINTER(_f32)])
_sig("s2x_text_create", [ctypes.POINTER(TextWeights), ctypes.POINTER(_p)])
_sig("s2x_text_destroy", [_p], None)
_sig("s2x_text_set_stream", [_p, _p])
_sig("s2x_text_encode", [_p, _p, _i32, _p, _p])
_sig("s2x_text_encode_batch", [_p, _p, _i32, _i32, _p])


def check(status):
    """Raise S2XError unless status is S2X_OK."""
    if status != 0:
        raise S2XError(status, lib.s2x_last_error().decode())
    return status


def call(name, *args):
    """Call a status-returning C-ABI function by name and check the result."""
    return check(getattr(lib, name)(*args))


def version():
    return lib.s2x_version().decode()
