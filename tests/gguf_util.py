"""A small GGUF v3 writer for tests: synthetic towers written under the
siglip2 converter's tensor names (scripts/convert_siglip2_to_gguf.py:7-35)
and metadata keys (src/siglip2_vision.cpp:27-34, src/siglip2_text.cpp:27-34),
following the published GGUF layout (magic, version, counts, key/value
metadata, tensor directory, data aligned to general.alignment)."""
import struct

import numpy as np

GT_U32, GT_F32, GT_BOOL, GT_STRING, GT_ARRAY = 4, 6, 7, 8, 9
T_F32, T_F16, T_Q8_0 = 0, 1, 8
ALIGN = 32


def _str(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(t, v):
    if t == GT_U32:
        return struct.pack("<I", v)
    if t == GT_F32:
        return struct.pack("<f", v)
    if t == GT_BOOL:
        return struct.pack("<B", 1 if v else 0)
    if t == GT_STRING:
        return _str(v)
    if t == GT_ARRAY:  # v = (element type, list of values)
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(_value(et, x) for x in items)
    raise ValueError(t)


def write_gguf(path, kv, tensors, align=None):
    """kv: list of (key, gguf_type, value), an array value being (element
    type, items); tensors: list of (name, ggml_type, ne (innermost first),
    bytes).  align: data alignment, written as general.alignment (u32) when
    given (else the default 32, not written)."""
    if align is not None:
        kv = list(kv) + [("general.alignment", GT_U32, align)]
    A = align or ALIGN
    head = bytearray(b"GGUF")
    head += struct.pack("<IQQ", 3, len(tensors), len(kv))
    for key, t, v in kv:
        head += _str(key) + struct.pack("<I", t) + _value(t, v)
    offs, off = [], 0
    for name, t, ne, data in tensors:
        offs.append(off)
        off += len(data)
        off = (off + A - 1) // A * A
    for (name, t, ne, data), o in zip(tensors, offs):
        head += _str(name) + struct.pack("<I", len(ne))
        head += b"".join(struct.pack("<Q", e) for e in ne)
        head += struct.pack("<IQ", t, o)
    pad = (-len(head)) % A
    with open(path, "wb") as f:
        f.write(head)
        f.write(b"\0" * pad)
        pos = 0
        for (name, t, ne, data), o in zip(tensors, offs):
            f.write(b"\0" * (o - pos))
            f.write(data)
            pos = o + len(data)


def _q8(name, raw, k_pad, n):
    return (name, T_Q8_0, [k_pad, n], np.ascontiguousarray(raw).tobytes())


def _f32(name, a, ne):
    return (name, T_F32, ne, np.ascontiguousarray(a, np.float32).tobytes())


def _down(name, w, F, Fp, H):
    """ffn_down as the converter stores it: F16 rows of F halves (a float16
    array), else Q8_0 with K padded to Fp."""
    w = np.ascontiguousarray(w)
    if w.dtype == np.float16:
        return (name, T_F16, [F, H], w.tobytes())
    return _q8(name, w, Fp, H)


def _layer_tensors(tower, i, L, H, F, Fp):
    p = f"{tower}.blk.{i}."
    return [
        _f32(p + "ln1.weight", L["ln1_w"], [H]), _f32(p + "ln1.bias", L["ln1_b"], [H]),
        _q8(p + "attn_qkv.weight", L["qkv_w"], H, 3 * H), _f32(p + "attn_qkv.bias", L["qkv_b"], [3 * H]),
        _q8(p + "attn_o.weight", L["o_w"], H, H), _f32(p + "attn_o.bias", L["o_b"], [H]),
        _f32(p + "ln2.weight", L["ln2_w"], [H]), _f32(p + "ln2.bias", L["ln2_b"], [H]),
        _q8(p + "ffn_up.weight", L["up_w"], H, F), _f32(p + "ffn_up.bias", L["up_b"], [F]),
        _down(p + "ffn_down.weight", L["down_w"], F, Fp, H), _f32(p + "ffn_down.bias", L["down_b"], [H]),
    ]


def vision_tensors(hm):
    """(kv, tensors) of a synth.vision_model HostModel."""
    c, t = hm.cfg, hm.tensors
    H, F, Fp = c.hidden, c.inter, c.inter_pad
    kv = [("general.architecture", GT_STRING, "siglip2"),
          ("siglip2.vision.embedding_length", GT_U32, H),
          ("siglip2.vision.feed_forward_length", GT_U32, F),
          ("siglip2.vision.attention.head_count", GT_U32, c.n_head),
          ("siglip2.vision.block_count", GT_U32, c.n_layer),
          ("siglip2.vision.patch_size", GT_U32, 16),
          ("siglip2.vision.num_patches", GT_U32, c.n_side * c.n_side),
          ("siglip2.vision.num_channels", GT_U32, c.patch_dim // 256),
          ("siglip2.vision.layer_norm_eps", GT_F32, c.eps)]
    ts = [_q8("v.patch_embd.weight", t["patch_w"], c.patch_dim, H),
          _f32("v.patch_embd.bias", t["patch_b"], [H]),
          _f32("v.position_embd.weight", t["pos_embd"], [H, c.n_side * c.n_side]),
          _f32("v.post_ln.weight", t["post_ln_w"], [H]), _f32("v.post_ln.bias", t["post_ln_b"], [H]),
          _f32("v.head.probe", t["probe"], [H, 1, 1])]
    for s, w, b in (("q", "hq_w", "hq_b"), ("k", "hk_w", "hk_b"), ("v", "hv_w", "hv_b"),
                    ("o", "ho_w", "ho_b")):
        ts += [_q8(f"v.head.attn_{s}.weight", t[w], H, H), _f32(f"v.head.attn_{s}.bias", t[b], [H])]
    ts += [_f32("v.head.ln.weight", t["hln_w"], [H]), _f32("v.head.ln.bias", t["hln_b"], [H]),
           _q8("v.head.ffn_up.weight", t["hup_w"], H, F), _f32("v.head.ffn_up.bias", t["hup_b"], [F]),
           _down("v.head.ffn_down.weight", t["hdown_w"], F, Fp, H),
           _f32("v.head.ffn_down.bias", t["hdown_b"], [H])]
    for i, L in enumerate(hm.layers):
        ts += _layer_tensors("v", i, L, H, F, Fp)
    return kv, ts


def text_tensors(hm):
    c, t = hm.cfg, hm.tensors
    H, F, Fp = c.hidden, c.inter, c.inter_pad
    kv = [("siglip2.text.embedding_length", GT_U32, H),
          ("siglip2.text.feed_forward_length", GT_U32, F),
          ("siglip2.text.attention.head_count", GT_U32, c.n_head),
          ("siglip2.text.block_count", GT_U32, c.n_layer),
          ("siglip2.text.vocab_size", GT_U32, c.vocab),
          ("siglip2.text.max_position_embeddings", GT_U32, c.max_pos),
          ("siglip2.text.projection_size", GT_U32, c.proj),
          ("siglip2.text.layer_norm_eps", GT_F32, c.eps)]
    ts = [_q8("t.token_embd.weight", t["tok_embd"], H, c.vocab),
          _f32("t.position_embd.weight", t["pos_embd"], [H, c.max_pos]),
          _f32("t.final_ln.weight", t["final_ln_w"], [H]), _f32("t.final_ln.bias", t["final_ln_b"], [H]),
          _q8("t.head.weight", t["head_w"], H, c.proj), _f32("t.head.bias", t["head_b"], [c.proj])]
    for i, L in enumerate(hm.layers):
        ts += _layer_tensors("t", i, L, H, F, Fp)
    return kv, ts


def score_tensors(logit_scale, logit_bias):
    """The contrastive head's scalars as the converter writes them: F32 [1]."""
    return [_f32("mm.logit_scale", np.array([logit_scale], np.float32), [1]),
            _f32("mm.logit_bias", np.array([logit_bias], np.float32), [1])]
