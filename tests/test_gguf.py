"""GGUF reader (host only): a synthetic tower written to a GGUF v3 file under
the converter's names must come back as the same weight struct -- every
tensor byte for byte, F16 vectors widened exactly, F16 ffn_down kept as
F16, other F16 / F32 matrices quantized to Q8_0 by ggml's rule with K
zero-padded -- and malformed files
must be rejected with an error, never read past their end."""
import ctypes

import numpy as np
import pytest

import s2x
from s2x import synth
from gguf_util import GT_F32 as GT_F32_, GT_STRING as GT_STR_, GT_U32 as GT_U32_
from gguf_util import T_F16, T_F32 as T_F32_, text_tensors, vision_tensors, write_gguf

SMALL_V = synth.VisionConfig(hidden=288, inter=1076, n_head=4, n_layer=2)
SMALL_T = synth.TextConfig(hidden=288, inter=1076, n_head=4, n_layer=2, vocab=1000, max_pos=64,
                           proj=288)


def _open(path):
    g = ctypes.c_void_p()
    st = s2x.lib.s2x_gguf_open(str(path).encode(), ctypes.byref(g))
    return st, g


def _bytes(p, n):
    return ctypes.string_at(p, n)


def _q8_bytes(k_pad, n):
    return n * (k_pad // 32) * 34


def _check_layers(ws, hm, H, F, Fp):
    for i, L in enumerate(hm.layers):
        lw = ws.layers[i]
        for key, n in (("ln1_w", 4 * H), ("ln1_b", 4 * H), ("qkv_b", 12 * H), ("o_b", 4 * H),
                       ("ln2_w", 4 * H), ("ln2_b", 4 * H), ("up_b", 4 * F), ("down_b", 4 * H),
                       ("qkv_w", _q8_bytes(H, 3 * H)), ("o_w", _q8_bytes(H, H)),
                       ("up_w", _q8_bytes(H, F)), ("down_w", _q8_bytes(Fp, H))):
            assert _bytes(getattr(lw, key), n) == L[key].tobytes(), (i, key)


def test_gguf_vision_roundtrip(tmp_path):
    hm = synth.vision_model(SMALL_V, seed=31)
    kv, ts = vision_tensors(hm)
    path = tmp_path / "v.gguf"
    write_gguf(path, kv, ts)
    st, g = _open(path)
    assert st == 0, s2x.lib.s2x_last_error()
    try:
        w = s2x.VisionWeights()
        s2x.call("s2x_gguf_vision_weights", g, ctypes.byref(w))
        c = SMALL_V
        H, F, Fp = c.hidden, c.inter, c.inter_pad
        assert (w.hidden, w.inter, w.inter_pad, w.n_head, w.n_layer, w.patch_dim, w.n_side) == (
            H, F, Fp, c.n_head, c.n_layer, c.patch_dim, c.n_side)
        assert w.eps == np.float32(c.eps)
        t = hm.tensors
        for key, n in (("patch_w", _q8_bytes(c.patch_dim, H)), ("patch_b", 4 * H),
                       ("pos_embd", 4 * H * c.n_side ** 2), ("post_ln_w", 4 * H),
                       ("post_ln_b", 4 * H), ("probe", 4 * H), ("hq_w", _q8_bytes(H, H)),
                       ("hk_w", _q8_bytes(H, H)), ("hv_w", _q8_bytes(H, H)),
                       ("ho_w", _q8_bytes(H, H)), ("hq_b", 4 * H), ("hk_b", 4 * H),
                       ("hv_b", 4 * H), ("ho_b", 4 * H), ("hln_w", 4 * H), ("hln_b", 4 * H),
                       ("hup_w", _q8_bytes(H, F)), ("hup_b", 4 * F),
                       ("hdown_w", _q8_bytes(Fp, H)), ("hdown_b", 4 * H)):
            assert _bytes(getattr(w, key), n) == t[key].tobytes(), key
        _check_layers(w, hm, H, F, Fp)
    finally:
        s2x.lib.s2x_gguf_close(g)


def test_gguf_text_roundtrip(tmp_path):
    hm = synth.text_model(SMALL_T, seed=32)
    kv, ts = text_tensors(hm)
    path = tmp_path / "t.gguf"
    write_gguf(path, kv, ts)
    st, g = _open(path)
    assert st == 0, s2x.lib.s2x_last_error()
    try:
        w = s2x.TextWeights()
        s2x.call("s2x_gguf_text_weights", g, ctypes.byref(w))
        c = SMALL_T
        H = c.hidden
        assert (w.hidden, w.inter, w.inter_pad, w.n_head, w.n_layer, w.vocab, w.max_pos, w.proj) == (
            H, c.inter, c.inter_pad, c.n_head, c.n_layer, c.vocab, c.max_pos, c.proj)
        t = hm.tensors
        assert _bytes(w.tok_embd, _q8_bytes(H, c.vocab)) == t["tok_embd"].tobytes()
        assert _bytes(w.pos_embd, 4 * H * c.max_pos) == t["pos_embd"].tobytes()
        assert _bytes(w.head_w, _q8_bytes(H, c.proj)) == t["head_w"].tobytes()
        assert _bytes(w.head_b, 4 * c.proj) == t["head_b"].tobytes()
        _check_layers(w, hm, H, c.inter, c.inter_pad)
    finally:
        s2x.lib.s2x_gguf_close(g)


def test_gguf_f16_ffn_down_kept(tmp_path):
    """A converter-made q8_0 file stores every ffn_down (K = 4304 here F, not
    a multiple of 32) as F16: the reader binds those bytes as F16 rows and
    sets down_f16, as the reference's encoders keep the on-disk type; an F16
    LayerNorm weight is widened exactly."""
    hm = synth.vision_model(SMALL_V, seed=33, down_f16=True)
    kv, ts = vision_tensors(hm)
    c = SMALL_V
    H, F = c.hidden, c.inter
    ln16 = (1 + 0.02 * np.random.default_rng(5).standard_normal(H)).astype(np.float16)
    for i, (name, t, ne, data) in enumerate(ts):
        if name == "v.blk.1.ln1.weight":
            ts[i] = (name, T_F16, [H], ln16.tobytes())
    path = tmp_path / "v16.gguf"
    write_gguf(path, kv, ts)
    st, g = _open(path)
    assert st == 0, s2x.lib.s2x_last_error()
    try:
        w = s2x.VisionWeights()
        s2x.call("s2x_gguf_vision_weights", g, ctypes.byref(w))
        assert w.down_f16 == 1
        for l in range(c.n_layer):
            assert _bytes(w.layers[l].down_w, 2 * H * F) == hm.layers[l]["down_w"].tobytes()
        assert _bytes(w.hdown_w, 2 * H * F) == hm.tensors["hdown_w"].tobytes()
        got = np.frombuffer(_bytes(w.layers[1].ln1_w, 4 * H), np.float32)
        assert np.array_equal(got, ln16.astype(np.float32))
    finally:
        s2x.lib.s2x_gguf_close(g)


def test_gguf_mixed_ffn_down_rejected(tmp_path):
    # one F16 ffn_down among Q8_0 ones: no converter writes that
    hm = synth.vision_model(SMALL_V, seed=35)
    kv, ts = vision_tensors(hm)
    H, F = SMALL_V.hidden, SMALL_V.inter
    w16 = (np.random.default_rng(6).standard_normal((H, F)) * 0.02).astype(np.float16)
    ts = [(n, T_F16, [F, H], w16.tobytes()) if n == "v.blk.1.ffn_down.weight" else (n, t, ne, d)
          for n, t, ne, d in ts]
    path = tmp_path / "mixed.gguf"
    write_gguf(path, kv, ts)
    st, g = _open(path)
    assert st == 0
    try:
        w = s2x.VisionWeights()
        assert s2x.lib.s2x_gguf_vision_weights(g, ctypes.byref(w)) == 2  # S2X_ERR_UNSUPPORTED
        assert b"ffn_down types differ" in s2x.lib.s2x_last_error()
    finally:
        s2x.lib.s2x_gguf_close(g)


def test_gguf_f16_f32_other_matrices_quantized(tmp_path):
    """An F16 / F32 matrix other than ffn_down (a file converted to f16 or f32
    throughout) is quantized on load with ggml's Q8_0 rule."""
    hm = synth.vision_model(SMALL_V, seed=36)
    kv, ts = vision_tensors(hm)
    H = SMALL_V.hidden
    rng = np.random.default_rng(7)
    w16 = (rng.standard_normal((H, H)) * 0.02).astype(np.float16)
    w16[0, :32] = 0                      # an all-zero block: d = 0, q = 0
    w16[1, 5] = np.float16(65504.0)      # the largest fp16
    w32 = (rng.standard_normal((H, H)) * 0.02).astype(np.float32)
    for i, (name, t, ne, data) in enumerate(ts):
        if name == "v.blk.0.attn_o.weight":
            ts[i] = (name, T_F16, [H, H], w16.tobytes())
        if name == "v.head.attn_o.weight":
            ts[i] = (name, 0, [H, H], w32.tobytes())  # GGML_TYPE_F32
    path = tmp_path / "v16o.gguf"
    write_gguf(path, kv, ts)
    st, g = _open(path)
    assert st == 0, s2x.lib.s2x_last_error()
    try:
        w = s2x.VisionWeights()
        s2x.call("s2x_gguf_vision_weights", g, ctypes.byref(w))
        assert w.down_f16 == 0
        want = synth.quantize_q8_0(w16.astype(np.float32), H)
        assert _bytes(w.layers[0].o_w, want.nbytes) == want.tobytes()
        want = synth.quantize_q8_0(w32, H)
        assert _bytes(w.ho_w, want.nbytes) == want.tobytes()
    finally:
        s2x.lib.s2x_gguf_close(g)


def test_gguf_rejects_bad_files(tmp_path):
    hm = synth.vision_model(SMALL_V, seed=34)
    kv, ts = vision_tensors(hm)
    good = tmp_path / "good.gguf"
    write_gguf(good, kv, ts)
    raw = good.read_bytes()

    bad_magic = tmp_path / "magic.gguf"
    bad_magic.write_bytes(b"GGUX" + raw[4:])
    assert _open(bad_magic)[0] != 0

    truncated = tmp_path / "trunc.gguf"
    truncated.write_bytes(raw[: len(raw) // 2])  # tensor data past the end
    assert _open(truncated)[0] != 0
    assert b"past the end" in s2x.lib.s2x_last_error()

    missing = tmp_path / "missing.gguf"
    write_gguf(missing, kv, [t for t in ts if t[0] != "v.blk.1.attn_o.weight"])
    st, g = _open(missing)
    assert st == 0
    try:
        w = s2x.VisionWeights()
        assert s2x.lib.s2x_gguf_vision_weights(g, ctypes.byref(w)) != 0
        assert b"v.blk.1.attn_o.weight" in s2x.lib.s2x_last_error()
    finally:
        s2x.lib.s2x_gguf_close(g)

    assert _open(tmp_path / "does-not-exist.gguf")[0] != 0


def _converter_names():
    import json
    import os
    with open(os.path.join(os.path.dirname(__file__), "golden", "converter_names.json")) as f:
        return json.load(f)


def _keep_f32(name, rule):
    return (any(name.endswith(s) for s in rule["suffixes"]) or
            any(s in name for s in rule["substrings"]) or name in rule["names"])


def test_names_match_reference_converter():
    """The writer above and the reader are pinned to the names the
    reference's converter emits (tests/golden/converter_names.json, read from
    its source by tests/golden/make_converter_names.py): the same tensor set
    for a 2-layer tower, F32 exactly where the converter keeps F32, and the
    metadata keys with the converter's types."""
    import os
    import re
    ref = _converter_names()
    n_layer = 2
    gt = {GT_U32_: "uint32", GT_F32_: "float32", GT_STR_: "string"}
    for tower, hm, fn, own in (("v", synth.vision_model(SMALL_V, seed=3), vision_tensors, ref["vision_tensors"]),
                               ("t", synth.text_model(SMALL_T, seed=4), text_tensors, ref["text_tensors"])):
        kv, ts = fn(hm)
        want = set(own) | {f"{tower}.blk.{i}.{b}" for i in range(n_layer) for b in ref["block_tensors"]}
        names = [n for n, _, _, _ in ts]
        assert len(names) == len(set(names))
        assert set(names) == want, (set(names) ^ want)
        for n, t, _, _ in ts:
            # converter F32 tensors: F32 here; its matrices: Q8_0 (or F16 ffn_down)
            assert (t == T_F32_) == _keep_f32(n, ref["keep_f32"]), n
        for key, t, _ in kv:
            if key.startswith(ref["arch"] + "."):
                assert ref["metadata"].get(key) == gt[t], key
    # every name the reader binds is one the converter writes
    src = open(os.path.join(os.path.dirname(__file__), "..", "hbd-siglip2.cpp_amd", "csrc",
                            "s2x_gguf.cpp")).read()
    lit = set(re.findall(r'"((?:v|t)\.[\w.]+|siglip2\.[\w.]+)"', src))
    blk = set(re.findall(r'blk\(tower, i, "([\w.]+)"\)', src))
    assert lit and blk
    every = set(ref["vision_tensors"]) | set(ref["text_tensors"]) | set(ref["metadata"])
    assert lit <= every, lit - every
    assert blk == set(ref["block_tensors"])


def _converter_kv(vision_kv, text_kv, c_v, c_t):
    """Metadata as the reference converter writes it for a file holding both
    towers (scripts/convert_siglip2_to_gguf.py:306-353, keys and types from
    tests/golden/converter_names.json), plus gguf-py's general.* keys and a
    string array: bools, f32 arrays, strings and u32/f32 scalars."""
    import json
    import os
    from gguf_util import GT_ARRAY, GT_BOOL
    meta = json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                       "converter_names.json")))["metadata"]
    given = {k: (t, v) for k, t, v in list(vision_kv) + list(text_kv)}
    kv = [("general.architecture", GT_STR_, "siglip2"), ("general.name", GT_STR_,
          "siglip2-so400m-patch16-naflex"), ("general.type", GT_STR_, "model"),
          ("general.file_type", GT_U32_, 7), ("general.quantization_version", GT_U32_, 2)]
    extra = {"siglip2.has_vision": True, "siglip2.has_text": True,
             "siglip2.vision.hidden_act": "gelu_pytorch_tanh", "siglip2.text.hidden_act": "gelu_pytorch_tanh",
             "siglip2.preproc.default_max_num_patches": 256, "siglip2.preproc.rescale_factor": 1 / 255,
             "siglip2.preproc.image_mean": [0.5, 0.5, 0.5], "siglip2.preproc.image_std": [0.5, 0.5, 0.5]}
    code = {"bool": GT_BOOL, "uint32": GT_U32_, "float32": GT_F32_, "string": GT_STR_}
    for key, typ in sorted(meta.items()):
        if key in given:
            t, v = given[key]
            assert t == code[typ], key  # the writer's own keys carry the converter's types
        elif typ == "array":
            t, v = GT_ARRAY, (GT_F32_, extra[key])
        else:
            t, v = code[typ], extra[key]
        kv.append((key, t, v))
    kv.append(("tokenizer.ggml.tokens", GT_ARRAY, (GT_STR_, ["<pad>", "<eos>", "<bos>", "▁a"])))
    return kv


@pytest.mark.parametrize("align", [32, 64])
def test_gguf_converter_shaped_file(tmp_path, align):
    """A file shaped like the converter's output: both towers, every
    metadata key the converter writes with its type (bools, f32 arrays,
    strings), a string array, and general.alignment; both towers must come
    back byte for byte."""
    hv = synth.vision_model(SMALL_V, seed=41)
    ht = synth.text_model(SMALL_T, seed=42)
    kv_v, ts_v = vision_tensors(hv)
    kv_t, ts_t = text_tensors(ht)
    kv = _converter_kv(kv_v, kv_t, SMALL_V, SMALL_T)
    path = tmp_path / "both.gguf"
    write_gguf(path, kv, ts_v + ts_t, align=align)
    st, g = _open(path)
    assert st == 0, s2x.lib.s2x_last_error()
    try:
        w = s2x.VisionWeights()
        s2x.call("s2x_gguf_vision_weights", g, ctypes.byref(w))
        c = SMALL_V
        H, F, Fp = c.hidden, c.inter, c.inter_pad
        assert (w.hidden, w.n_layer, w.n_side) == (H, c.n_layer, c.n_side)
        assert _bytes(w.patch_w, _q8_bytes(c.patch_dim, H)) == hv.tensors["patch_w"].tobytes()
        assert _bytes(w.probe, 4 * H) == hv.tensors["probe"].tobytes()
        _check_layers(w, hv, H, F, Fp)
        tw = s2x.TextWeights()
        s2x.call("s2x_gguf_text_weights", g, ctypes.byref(tw))
        assert (tw.hidden, tw.n_layer, tw.vocab) == (SMALL_T.hidden, SMALL_T.n_layer, SMALL_T.vocab)
        _check_layers(tw, ht, SMALL_T.hidden, SMALL_T.inter, SMALL_T.inter_pad)
    finally:
        s2x.lib.s2x_gguf_close(g)


def test_gguf_rejects_non_power_of_two_alignment(tmp_path):
    hv = synth.vision_model(SMALL_V, seed=43)
    kv, ts = vision_tensors(hv)
    path = tmp_path / "bad_align.gguf"
    write_gguf(path, kv + [("general.alignment", GT_U32_, 48)], ts)
    st, g = _open(path)
    assert st != 0 and "alignment" in s2x.lib.s2x_last_error().decode()


def test_gguf_score_params(tmp_path):
    """mm.logit_scale / mm.logit_bias come back as written; a file without
    them is an error, not zeros."""
    from gguf_util import score_tensors
    hm = synth.text_model(SMALL_T, seed=3)
    kv, ts = text_tensors(hm)
    path = tmp_path / "s.gguf"
    write_gguf(path, kv, ts + score_tensors(2.302585, -10.25))
    st, g = _open(path)
    assert st == 0
    try:
        sc, bi = ctypes.c_float(), ctypes.c_float()
        assert s2x.lib.s2x_gguf_score_params(g, ctypes.byref(sc), ctypes.byref(bi)) == 0
        assert sc.value == np.float32(2.302585) and bi.value == np.float32(-10.25)
    finally:
        s2x.lib.s2x_gguf_close(g)
    path2 = tmp_path / "n.gguf"
    write_gguf(path2, kv, ts)
    st, g = _open(path2)
    try:
        sc, bi = ctypes.c_float(), ctypes.c_float()
        assert s2x.lib.s2x_gguf_score_params(g, ctypes.byref(sc), ctypes.byref(bi)) != 0
        assert b"mm.logit_scale" in s2x.lib.s2x_last_error()
    finally:
        s2x.lib.s2x_gguf_close(g)
