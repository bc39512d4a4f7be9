"""Pins the oracle's position-embedding resize against PyTorch's
anti-aliased bilinear interpolation, and the oracle's whole tower graph
(patch/position embedding, pre-LN blocks, post-LN, MAP probe head, text
last-token pooling) against the HF transformers Siglip2 model run in fp32
with the same (dequantized) weights.  CPU only."""
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


def _deq(orc, raw, n, k, k_pad):
    return torch.from_numpy(orc.dequantize_q8_0(raw, n, k_pad)[:, :k].copy())


def _load_layers(orc, layers, hf_layers, cfg, attn_names):
    H, F, Fp = cfg.hidden, cfg.inter, cfg.inter_pad
    for L, hl in zip(layers, hf_layers):
        qkv = _deq(orc, L["qkv_w"], 3 * H, H, H)
        att = getattr(hl, attn_names)
        with torch.no_grad():
            hl.layer_norm1.weight.copy_(torch.from_numpy(L["ln1_w"]))
            hl.layer_norm1.bias.copy_(torch.from_numpy(L["ln1_b"]))
            att.q_proj.weight.copy_(qkv[:H]); att.k_proj.weight.copy_(qkv[H:2 * H])
            att.v_proj.weight.copy_(qkv[2 * H:])
            b = torch.from_numpy(L["qkv_b"])
            att.q_proj.bias.copy_(b[:H]); att.k_proj.bias.copy_(b[H:2 * H]); att.v_proj.bias.copy_(b[2 * H:])
            att.out_proj.weight.copy_(_deq(orc, L["o_w"], H, H, H))
            att.out_proj.bias.copy_(torch.from_numpy(L["o_b"]))
            hl.layer_norm2.weight.copy_(torch.from_numpy(L["ln2_w"]))
            hl.layer_norm2.bias.copy_(torch.from_numpy(L["ln2_b"]))
            hl.mlp.fc1.weight.copy_(_deq(orc, L["up_w"], F, H, H))
            hl.mlp.fc1.bias.copy_(torch.from_numpy(L["up_b"]))
            hl.mlp.fc2.weight.copy_(_deq(orc, L["down_w"], H, F, Fp))
            hl.mlp.fc2.bias.copy_(torch.from_numpy(L["down_b"]))


def _cos(a, b):
    a, b = np.asarray(a, np.float64).ravel(), np.asarray(b, np.float64).ravel()
    return float(a @ b / np.linalg.norm(a) / np.linalg.norm(b))


def _hf_vision(orc, host):
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
        vm.embeddings.patch_embedding.weight.copy_(_deq(orc, t["patch_w"], H, c.patch_dim, c.patch_dim))
        vm.embeddings.patch_embedding.bias.copy_(torch.from_numpy(t["patch_b"]))
        vm.embeddings.position_embedding.weight.copy_(torch.from_numpy(t["pos_embd"]))
        vm.post_layernorm.weight.copy_(torch.from_numpy(t["post_ln_w"]))
        vm.post_layernorm.bias.copy_(torch.from_numpy(t["post_ln_b"]))
        hd = vm.head
        hd.probe.copy_(torch.from_numpy(t["probe"]).reshape(1, 1, H))
        inw = torch.cat([_deq(orc, t[k], H, H, H) for k in ("hq_w", "hk_w", "hv_w")])
        hd.attention.in_proj_weight.copy_(inw)
        hd.attention.in_proj_bias.copy_(torch.from_numpy(np.concatenate([t["hq_b"], t["hk_b"], t["hv_b"]])))
        hd.attention.out_proj.weight.copy_(_deq(orc, t["ho_w"], H, H, H))
        hd.attention.out_proj.bias.copy_(torch.from_numpy(t["ho_b"]))
        hd.layernorm.weight.copy_(torch.from_numpy(t["hln_w"]))
        hd.layernorm.bias.copy_(torch.from_numpy(t["hln_b"]))
        hd.mlp.fc1.weight.copy_(_deq(orc, t["hup_w"], F, H, H))
        hd.mlp.fc1.bias.copy_(torch.from_numpy(t["hup_b"]))
        hd.mlp.fc2.weight.copy_(_deq(orc, t["hdown_w"], H, F, Fp))
        hd.mlp.fc2.bias.copy_(torch.from_numpy(t["hdown_b"]))
    _load_layers(orc, host.layers, vm.encoder.layers, c, "self_attn")
    return m


@pytest.mark.parametrize("grid", [(16, 16), (27, 27), (12, 20)])
def test_vision_graph_matches_hf_fp32(orc, grid):
    host = synth.vision_model(SMALL_V, seed=3)
    om = orc.vision_model(host)
    hf = _hf_vision(orc, host)
    h, w = grid
    px = synth.pixels(1, h * w, seed=5)
    with torch.no_grad():
        r = hf(pixel_values=torch.from_numpy(px)[None], pixel_attention_mask=torch.ones(1, h * w, dtype=torch.long),
               spatial_shapes=torch.tensor([[h, w]]))
    ours, hid = orc.vision_encode(om, px, h, w, pooling=1, hidden=True)
    assert _cos(hid, r.last_hidden_state[0].numpy()) > 0.9999
    assert _cos(ours, r.pooler_output[0].numpy()) > 0.999
    mean = orc.vision_encode(om, px, h, w, pooling=0)
    assert np.abs(mean - hid.astype(np.float64).mean(0)).max() < 1e-5
    assert _cos(mean, r.last_hidden_state[0].numpy().mean(0)) > 0.9999


def test_text_graph_matches_hf_fp32(orc):
    from transformers import Siglip2TextConfig, Siglip2TextModel
    host = synth.text_model(SMALL_T, seed=4)
    c = host.cfg
    H = c.hidden
    tc = Siglip2TextConfig(vocab_size=c.vocab, hidden_size=H, intermediate_size=c.inter,
                           num_hidden_layers=c.n_layer, num_attention_heads=c.n_head,
                           max_position_embeddings=c.max_pos, hidden_act="gelu_pytorch_tanh",
                           layer_norm_eps=c.eps, projection_size=c.proj,
                           attn_implementation="eager")
    m = Siglip2TextModel(tc).eval()
    tm = getattr(m, "text_model", m)
    t = host.tensors
    with torch.no_grad():
        tm.embeddings.token_embedding.weight.copy_(_deq(orc, t["tok_embd"], c.vocab, H, H))
        tm.embeddings.position_embedding.weight.copy_(torch.from_numpy(t["pos_embd"]))
        tm.final_layer_norm.weight.copy_(torch.from_numpy(t["final_ln_w"]))
        tm.final_layer_norm.bias.copy_(torch.from_numpy(t["final_ln_b"]))
        tm.head.weight.copy_(_deq(orc, t["head_w"], c.proj, H, H))
        tm.head.bias.copy_(torch.from_numpy(t["head_b"]))
    _load_layers(orc, host.layers, tm.encoder.layers, c, "self_attn")
    om = orc.text_model(host)
    ids, lens = synth.text_tokens(3, 64, vocab=c.vocab)
    for b in range(3):
        with torch.no_grad():
            ref = m(input_ids=torch.from_numpy(ids[b:b + 1]).long()).pooler_output[0].numpy()
        assert _cos(orc.text_encode(om, ids[b]), ref) > 0.999
    # key mask: HF drops masked keys the same way
    mask = np.zeros(64, np.int32)
    mask[:lens[0]] = 1
    with torch.no_grad():
        ref = m(input_ids=torch.from_numpy(ids[:1]).long(),
                attention_mask=torch.from_numpy(mask[None]).long()).pooler_output[0].numpy()
    assert _cos(orc.text_encode(om, ids[0], mask), ref) > 0.999
