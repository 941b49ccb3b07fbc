"""Pins for the prefix-LM prefill oracle (oracle/prefix_oracle.py).

The reference ships no golden vectors for the prefix path either, so every function is checked
against an independent formulation (torch's own GELU and scaled-dot-product attention, a textbook
RMSNorm), integer brute force (masks, positions) or an invariant a plausible mistake breaks
(padding invariance of the valid tokens' cache, the K/V-only last layer, zeroed projections
making a layer the identity).  Small CPU shapes only.
"""

import math

import pytest
import torch
import torch.nn.functional as F

from oracle import denoise_oracle as O
from oracle import prefix_oracle as P

G = P.PrefixGeometry(width=64, depth=3, num_heads=4, num_kv_heads=1, head_dim=16, mlp_dim=96)


def test_rms_norm_textbook():
    torch.manual_seed(0)
    x = O._bf(torch.randn(3, 7, 64))
    # w = 0: x / rms(x), rounded once
    y = P.rms_norm(x, torch.zeros(64), 1e-6)
    ref = x / torch.sqrt((x.double() ** 2).mean(-1, keepdim=True) + 1e-6).float()
    assert torch.allclose(y, O._bf(ref), atol=0, rtol=2 ** -7)
    # w = c: scaled by (1 + c), not by c (the Gemma convention)
    c = torch.full((64,), 0.5)
    y2 = P.rms_norm(x, c, 1e-6)
    assert torch.allclose(y2, O._bf(ref * 1.5), atol=0, rtol=2 ** -7)
    # scale invariance of the statistics
    assert torch.equal(P.rms_norm(x * 4, torch.zeros(64), 0.0), P.rms_norm(x, torch.zeros(64), 0.0))


def test_prefix_masks_brute_force():
    pad = torch.tensor([[1, 1, 1, 0, 0], [1, 0, 1, 1, 0]], dtype=torch.bool)
    pos, m = P.prefix_masks(pad)
    for b in range(2):
        c = -1
        for i in range(5):
            c += int(pad[b, i])
            assert pos[b, i].item() == c
            for j in range(5):
                allowed = bool(pad[b, i]) and bool(pad[b, j])
                assert m[b, 0, i, j].item() == (0.0 if allowed else torch.tensor(O.MASK_MIN).item())


def test_embed_tokens_scale():
    table = O._bf(torch.randn(11, 2048))
    table[3] = 1.0
    ids = torch.tensor([[3, 0, 10]])
    e = P.embed_tokens(ids, table, 2048)
    # bf16(sqrt(2048)) = 45.25 exactly (45.2548... rounds to 8 significant bits)
    assert torch.all(e[0, 0] == 45.25)
    assert torch.allclose(e[0, 2], table[10] * math.sqrt(2048), rtol=2 ** -8, atol=0)


def test_geglu_matches_torch_gelu():
    torch.manual_seed(1)
    g = O._bf(torch.randn(1000) * 3)
    u = O._bf(torch.randn(1000))
    act = O._bf(O.gelu_tanh(g) * u)
    ref = O._bf(F.gelu(g.double(), approximate="tanh").float() * u)
    assert (act - ref).abs().max().item() <= 2 ** -7 * ref.abs().max().item()


def test_attention_matches_sdpa_with_padding():
    torch.manual_seed(2)
    b, p, d = 2, 9, 16
    pad = torch.ones(b, p, dtype=torch.bool)
    pad[1, 6:] = False
    _, m = P.prefix_masks(pad)
    q = O._bf(torch.randn(b, 4, p, d))
    k = O._bf(torch.randn(b, 1, p, d))
    v = O._bf(torch.randn(b, 1, p, d))
    o = O.mqa_attention(q, k, v, m, d ** -0.5).view(b, p, 4, d)
    bool_mask = m[:, :, :, :] == 0
    ref = F.scaled_dot_product_attention(q.double(), k.double().expand(b, 4, p, d), v.double().expand(b, 4, p, d),
                                         attn_mask=bool_mask.expand(b, 4, p, p)).transpose(1, 2).float()
    valid = pad[:, :, None, None].expand_as(o)
    assert (o - ref)[valid].abs().max().item() < 0.03


def _cache(layers, embeds, pad, skip_last=True):
    return P.prefill(layers, G, embeds, pad, skip_last=skip_last)


def test_kv_only_last_layer_is_the_full_layers_cache():
    layers = P.random_layers(G, 3, seed=3)
    emb = O._bf(torch.randn(1, 12, 64))
    pad = torch.ones(1, 12, dtype=torch.bool)
    a = _cache(layers, emb, pad, skip_last=True)
    b = _cache(layers, emb, pad, skip_last=False)
    for (ka, va), (kb, vb) in zip(a, b):
        assert torch.equal(ka, kb) and torch.equal(va, vb)


def test_padding_does_not_touch_valid_tokens():
    layers = P.random_layers(G, 3, seed=4)
    emb = O._bf(torch.randn(1, 10, 64))
    pad = torch.ones(1, 10, dtype=torch.bool)
    base = _cache(layers, emb, pad)
    # six padded tokens of garbage appended: the ten valid tokens' cache must not move
    emb2 = torch.cat([emb, O._bf(torch.randn(1, 6, 64) * 50)], dim=1)
    pad2 = torch.cat([pad, torch.zeros(1, 6, dtype=torch.bool)], dim=1)
    ext = _cache(layers, emb2, pad2)
    for (k0, v0), (k1, v1) in zip(base, ext):
        assert torch.equal(k0, k1[:, :, :10]) and torch.equal(v0, v1[:, :, :10])


def test_zero_projections_make_identity_layers():
    # o_proj = 0 and down_proj = 0: every layer passes h through, so layer i's K/V are the first
    # layer's function of the embeddings with layer i's weights
    layers = P.random_layers(G, 3, seed=5)
    for w in layers:
        w["wo"] = torch.zeros_like(w["wo"])
        w["wd"] = torch.zeros_like(w["wd"])
    emb = O._bf(torch.randn(2, 8, 64))
    pad = torch.ones(2, 8, dtype=torch.bool)
    cache = _cache(layers, emb, pad)
    pos, m = P.prefix_masks(pad)
    cos, sin = O.rope_cos_sin(pos, G.head_dim, G.rope_theta)
    for i, w in enumerate(layers):
        _, k, v = P.prefix_layer(w, G, emb, cos, sin, m, kv_only=True)
        assert torch.equal(cache[i][0], k) and torch.equal(cache[i][1], v)


def test_rope_on_k_is_position_dependent_rotation():
    # K of a token at position 0 is the unrotated bf16 GEMM value; the rotation preserves norms
    layers = P.random_layers(G, 1, seed=6)
    emb = O._bf(torch.randn(1, 5, 64))
    pad = torch.ones(1, 5, dtype=torch.bool)
    (k, _), = _cache(layers, emb, pad)
    n = P.rms_norm(emb, layers[0]["ln1"], G.rms_eps)
    k_lin = O.linear_bf16(n, layers[0]["wk"])
    assert torch.equal(k[0, 0, 0], k_lin[0, 0])
    assert torch.allclose(k[0, 0].norm(dim=-1), k_lin[0].norm(dim=-1), rtol=2e-2)
