"""Writes tests/golden/hf_siglip2_small.npz: the outputs of HF transformers'
Siglip2VisionModel / Siglip2TextModel, run in fp32 on this container's CPU,
for the small synthetic towers the oracle tests use (the same seeded weights,
dequantized from Q8_0, and the same seeded inputs).  The oracle test
(tests/test_oracle_model.py) compares against the fixture; nothing imports
transformers at test time.

    python tests/golden/make_hf_fixtures.py

Stored per vision grid (16x16, 27x27, 12x20): every third row of
last_hidden_state (f16), its mean over all rows (f32) and pooler_output
(f32); per text prompt (3 prompts of 64 ids, and prompt 0 with a key mask):
pooler_output (f32).  Plus the sha1 of the synthetic inputs, so that a
change of the generators is caught instead of compared against."""
import hashlib
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "hbd-siglip2.cpp_amd"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
import pyoracle as orc  # noqa: E402  (dequantization of the Q8_0 weights)
from s2x import synth  # noqa: E402

SMALL_V = synth.VisionConfig(hidden=288, inter=1076, n_head=4, n_layer=2)
SMALL_T = synth.TextConfig(hidden=288, inter=1076, n_head=4, n_layer=2, vocab=1000, max_pos=64,
                           proj=288)
GRIDS = [(16, 16), (27, 27), (12, 20)]
OUT = os.path.join(HERE, "hf_siglip2_small.npz")


def sha(*arrays):
    h = hashlib.sha1()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def _deq(raw, n, k, k_pad):
    return torch.from_numpy(orc.dequantize_q8_0(raw, n, k_pad)[:, :k].copy())


def _load_layers(layers, hf_layers, cfg):
    H, F, Fp = cfg.hidden, cfg.inter, cfg.inter_pad
    for L, hl in zip(layers, hf_layers):
        qkv = _deq(L["qkv_w"], 3 * H, H, H)
        att = hl.self_attn
        with torch.no_grad():
            hl.layer_norm1.weight.copy_(torch.from_numpy(L["ln1_w"]))
            hl.layer_norm1.bias.copy_(torch.from_numpy(L["ln1_b"]))
            att.q_proj.weight.copy_(qkv[:H])
            att.k_proj.weight.copy_(qkv[H:2 * H])
            att.v_proj.weight.copy_(qkv[2 * H:])
            b = torch.from_numpy(L["qkv_b"])
            att.q_proj.bias.copy_(b[:H])
            att.k_proj.bias.copy_(b[H:2 * H])
            att.v_proj.bias.copy_(b[2 * H:])
            att.out_proj.weight.copy_(_deq(L["o_w"], H, H, H))
            att.out_proj.bias.copy_(torch.from_numpy(L["o_b"]))
            hl.layer_norm2.weight.copy_(torch.from_numpy(L["ln2_w"]))
            hl.layer_norm2.bias.copy_(torch.from_numpy(L["ln2_b"]))
            hl.mlp.fc1.weight.copy_(_deq(L["up_w"], F, H, H))
            hl.mlp.fc1.bias.copy_(torch.from_numpy(L["up_b"]))
            hl.mlp.fc2.weight.copy_(_deq(L["down_w"], H, F, Fp))
            hl.mlp.fc2.bias.copy_(torch.from_numpy(L["down_b"]))


def hf_vision(host):
    from transformers import Siglip2VisionConfig, Siglip2VisionModel
    c = host.cfg
    H, F, Fp = c.hidden, c.inter, c.inter_pad
    hc = Siglip2VisionConfig(hidden_size=H, intermediate_size=F, num_hidden_layers=c.n_layer,
                             num_attention_heads=c.n_head, num_channels=3, patch_size=16,
                             num_patches=c.n_side ** 2, hidden_act="gelu_pytorch_tanh",
                             layer_norm_eps=c.eps, attn_implementation="eager")
    m = Siglip2VisionModel(hc).eval()
    vm = getattr(m, "vision_model", m)
    t = host.tensors
    with torch.no_grad():
        vm.embeddings.patch_embedding.weight.copy_(_deq(t["patch_w"], H, c.patch_dim, c.patch_dim))
        vm.embeddings.patch_embedding.bias.copy_(torch.from_numpy(t["patch_b"]))
        vm.embeddings.position_embedding.weight.copy_(torch.from_numpy(t["pos_embd"]))
        vm.post_layernorm.weight.copy_(torch.from_numpy(t["post_ln_w"]))
        vm.post_layernorm.bias.copy_(torch.from_numpy(t["post_ln_b"]))
        hd = vm.head
        hd.probe.copy_(torch.from_numpy(t["probe"]).reshape(1, 1, H))
        hd.attention.in_proj_weight.copy_(torch.cat([_deq(t[k], H, H, H) for k in ("hq_w", "hk_w", "hv_w")]))
        hd.attention.in_proj_bias.copy_(torch.from_numpy(np.concatenate([t["hq_b"], t["hk_b"], t["hv_b"]])))
        hd.attention.out_proj.weight.copy_(_deq(t["ho_w"], H, H, H))
        hd.attention.out_proj.bias.copy_(torch.from_numpy(t["ho_b"]))
        hd.layernorm.weight.copy_(torch.from_numpy(t["hln_w"]))
        hd.layernorm.bias.copy_(torch.from_numpy(t["hln_b"]))
        hd.mlp.fc1.weight.copy_(_deq(t["hup_w"], F, H, H))
        hd.mlp.fc1.bias.copy_(torch.from_numpy(t["hup_b"]))
        hd.mlp.fc2.weight.copy_(_deq(t["hdown_w"], H, F, Fp))
        hd.mlp.fc2.bias.copy_(torch.from_numpy(t["hdown_b"]))
    _load_layers(host.layers, vm.encoder.layers, c)
    return m


def hf_text(host):
    from transformers import Siglip2TextConfig, Siglip2TextModel
    c = host.cfg
    H = c.hidden
    tc = Siglip2TextConfig(vocab_size=c.vocab, hidden_size=H, intermediate_size=c.inter,
                           num_hidden_layers=c.n_layer, num_attention_heads=c.n_head,
                           max_position_embeddings=c.max_pos, hidden_act="gelu_pytorch_tanh",
                           layer_norm_eps=c.eps, projection_size=c.proj, attn_implementation="eager")
    m = Siglip2TextModel(tc).eval()
    tm = getattr(m, "text_model", m)
    t = host.tensors
    with torch.no_grad():
        tm.embeddings.token_embedding.weight.copy_(_deq(t["tok_embd"], c.vocab, H, H))
        tm.embeddings.position_embedding.weight.copy_(torch.from_numpy(t["pos_embd"]))
        tm.final_layer_norm.weight.copy_(torch.from_numpy(t["final_ln_w"]))
        tm.final_layer_norm.bias.copy_(torch.from_numpy(t["final_ln_b"]))
        tm.head.weight.copy_(_deq(t["head_w"], c.proj, H, H))
        tm.head.bias.copy_(torch.from_numpy(t["head_b"]))
    _load_layers(host.layers, tm.encoder.layers, c)
    return m


def main():
    torch.manual_seed(0)
    out = {}
    vh = synth.vision_model(SMALL_V, seed=3)
    vm = hf_vision(vh)
    out["vision_weights_sha1"] = sha(vh.tensors["patch_w"], vh.tensors["probe"], vh.layers[0]["qkv_w"])
    for h, w in GRIDS:
        px = synth.pixels(1, h * w, seed=5)
        with torch.no_grad():
            r = vm(pixel_values=torch.from_numpy(px)[None],
                   pixel_attention_mask=torch.ones(1, h * w, dtype=torch.long),
                   spatial_shapes=torch.tensor([[h, w]]))
        hid = r.last_hidden_state[0].numpy()
        k = f"v{h}x{w}"
        out[k + "_pixels_sha1"] = sha(px)
        out[k + "_hidden_rows3"] = hid[::3].astype(np.float16)
        out[k + "_hidden_mean"] = hid.astype(np.float64).mean(0).astype(np.float32)
        out[k + "_pooled"] = r.pooler_output[0].numpy().astype(np.float32)
    th = synth.text_model(SMALL_T, seed=4)
    tm = hf_text(th)
    out["text_weights_sha1"] = sha(th.tensors["tok_embd"], th.tensors["head_w"], th.layers[0]["qkv_w"])
    ids, lens = synth.text_tokens(3, 64, vocab=SMALL_T.vocab)
    out["text_ids"] = ids.astype(np.int32)
    for b in range(3):
        with torch.no_grad():
            out[f"t{b}_pooled"] = tm(input_ids=torch.from_numpy(ids[b:b + 1]).long()).pooler_output[0].numpy()
    mask = np.zeros(64, np.int32)
    mask[:lens[0]] = 1
    out["t0_mask"] = mask
    with torch.no_grad():
        out["t0_masked_pooled"] = tm(input_ids=torch.from_numpy(ids[:1]).long(),
                                     attention_mask=torch.from_numpy(mask[None]).long()).pooler_output[0].numpy()
    np.savez_compressed(OUT, **{k: (np.asarray(v) if not isinstance(v, str) else np.asarray(v)) for k, v in out.items()})
    print(OUT, os.path.getsize(OUT), "bytes")


if __name__ == "__main__":
    main()
