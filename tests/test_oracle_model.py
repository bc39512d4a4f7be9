"""Pins the oracle's position-embedding resize against PyTorch's
anti-aliased bilinear interpolation, and the oracle's whole tower graph
(patch/position embedding, pre-LN blocks, post-LN, MAP probe head, text
last-token pooling) against the HF transformers Siglip2 model run in fp32
with the same (dequantized) weights: its outputs are the fixture
tests/golden/hf_siglip2_small.npz, written by tests/golden/make_hf_fixtures.py
(transformers is not imported here).  CPU only."""
import hashlib
import os

import numpy as np
import pytest
import torch

from s2x import synth


@pytest.mark.parametrize("out_hw", [(16, 16), (27, 27), (8, 32), (24, 24), (18, 32), (32, 32),
                                    (16, 64), (5, 7), (3, 40)])
def test_resize_matches_torch_antialias(orc, out_hw):
    h, w = out_hw
    pos = np.random.default_rng(h * 100 + w).standard_normal((256, 48)).astype(np.float32)
    ours = orc.resize_pos_embed(pos, 16, h, w)
    t = torch.from_numpy(pos).reshape(16, 16, 48).permute(2, 0, 1).unsqueeze(0)
    ref = torch.nn.functional.interpolate(t, size=(h, w), mode="bilinear", align_corners=False,
                                          antialias=True)
    ref = ref.reshape(48, h * w).T.numpy()
    assert np.abs(ours - ref).max() < 2e-6


def test_resize_identity_at_native_grid(orc):
    pos = np.random.default_rng(0).standard_normal((256, 32)).astype(np.float32)
    assert np.array_equal(orc.resize_pos_embed(pos, 16, 16, 16), pos)


SMALL_V = synth.VisionConfig(hidden=288, inter=1076, n_head=4, n_layer=2)
SMALL_T = synth.TextConfig(hidden=288, inter=1076, n_head=4, n_layer=2, vocab=1000, max_pos=64,
                           proj=288)
FIXTURE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "hf_siglip2_small.npz")


def _sha(*arrays):
    h = hashlib.sha1()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def _cos(a, b):
    a, b = np.asarray(a, np.float64).ravel(), np.asarray(b, np.float64).ravel()
    return float(a @ b / np.linalg.norm(a) / np.linalg.norm(b))


@pytest.fixture(scope="module")
def hf():
    """HF transformers' Siglip2 outputs for the small towers below, written
    by tests/golden/make_hf_fixtures.py (fp32, same dequantized weights)."""
    return np.load(FIXTURE)


@pytest.mark.parametrize("grid", [(16, 16), (27, 27), (12, 20)])
def test_vision_graph_matches_hf_fp32(orc, hf, grid):
    host = synth.vision_model(SMALL_V, seed=3)
    assert _sha(host.tensors["patch_w"], host.tensors["probe"], host.layers[0]["qkv_w"]) == \
        str(hf["vision_weights_sha1"]), "synthetic weights changed: rerun make_hf_fixtures.py"
    om = orc.vision_model(host)
    h, w = grid
    k = f"v{h}x{w}"
    px = synth.pixels(1, h * w, seed=5)
    assert _sha(px) == str(hf[k + "_pixels_sha1"])
    ours, hid = orc.vision_encode(om, px, h, w, pooling=1, hidden=True)
    assert _cos(hid[::3], hf[k + "_hidden_rows3"].astype(np.float32)) > 0.9999
    assert _cos(ours, hf[k + "_pooled"]) > 0.999
    mean = orc.vision_encode(om, px, h, w, pooling=0)
    assert np.abs(mean - hid.astype(np.float64).mean(0)).max() < 1e-5
    assert _cos(mean, hf[k + "_hidden_mean"]) > 0.9999


def test_text_graph_matches_hf_fp32(orc, hf):
    host = synth.text_model(SMALL_T, seed=4)
    assert _sha(host.tensors["tok_embd"], host.tensors["head_w"], host.layers[0]["qkv_w"]) == \
        str(hf["text_weights_sha1"]), "synthetic weights changed: rerun make_hf_fixtures.py"
    om = orc.text_model(host)
    ids, lens = synth.text_tokens(3, 64, vocab=SMALL_T.vocab)
    assert np.array_equal(ids, hf["text_ids"])
    for b in range(3):
        assert _cos(orc.text_encode(om, ids[b]), hf[f"t{b}_pooled"]) > 0.999
    # key mask: HF drops masked keys the same way
    mask = hf["t0_mask"]
    assert int(mask.sum()) == int(lens[0])
    assert _cos(orc.text_encode(om, ids[0], mask), hf["t0_masked_pooled"]) > 0.999
