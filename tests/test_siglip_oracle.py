"""Pins for the SigLIP oracle (oracle/siglip_oracle.py).

The tower is third-party code (transformers' SigLIP, which the reference runs unmodified through
``get_image_features``).  The oracle's structure -- patch order, pre-norm residual layers,
multi-head attention, the tanh-GELU MLP, post_layernorm -- is pinned against the installed
transformers ``SiglipVisionModel`` in fp32 (an independent implementation of the same published
algorithm), on a small config with the oracle's own weights loaded into it.  The bf16 rounding
points are pinned separately: every oracle output is bf16-representable and within bf16 noise of
the fp32 result.
"""

import pytest
import torch

from oracle import denoise_oracle as O
from oracle import siglip_oracle as S

transformers = pytest.importorskip("transformers")

G = S.SiglipGeometry(width=64, depth=2, num_heads=4, mlp_dim=96, image=56, proj_dim=32)
ID = lambda x: x  # noqa: E731


def _hf_model(layers, heads):
    from transformers import SiglipVisionConfig, SiglipVisionModel

    cfg = SiglipVisionConfig(hidden_size=G.width, intermediate_size=G.mlp_dim, num_hidden_layers=G.depth,
                             num_attention_heads=G.num_heads, image_size=G.image, patch_size=G.patch,
                             hidden_act="gelu_pytorch_tanh", layer_norm_eps=G.ln_eps, vision_use_head=False)
    cfg._attn_implementation = "eager"
    m = SiglipVisionModel(cfg).float().eval()
    sd = {}
    strip = "paligemma_with_expert.paligemma.model.vision_tower."
    for i, w in enumerate(layers):
        for k, name in S.layer_names(i).items():
            sd[name[len(strip):]] = w[k]
    for k in ("patch_w", "patch_b", "pos", "post_w", "post_b"):
        sd[S.HEAD_NAMES[k][len(strip):]] = heads[k]
    # transformers 5.x flattens the vision model's keys; 4.x keeps a "vision_model." prefix
    if not any(k.startswith("vision_model.") for k in m.state_dict()):
        sd = {k[len("vision_model."):]: v for k, v in sd.items()}
    missing, unexpected = m.load_state_dict(sd, strict=False)
    assert not [u for u in unexpected], unexpected
    assert all("position_ids" in k for k in missing), missing
    return m


def test_tower_matches_transformers_fp32():
    layers, heads = S.random_weights(G, G.depth, seed=0, std=0.1)
    torch.manual_seed(0)
    px = torch.rand(3, 3, G.image, G.image) * 2 - 1
    ours = S.vision_tower(px, layers, heads, G, rnd=ID)
    with torch.no_grad():
        ref = _hf_model(layers, heads)(pixel_values=px).last_hidden_state
    assert ours.shape == ref.shape == (3, G.n_patches, G.width)
    assert torch.allclose(ours, ref, atol=2e-5, rtol=1e-4), (ours - ref).abs().max()


def test_patch_order_is_row_major_channel_first():
    px = torch.arange(2 * 3 * 56 * 56, dtype=torch.float32).reshape(2, 3, 56, 56)
    pt = S.patchify(px, G)
    # patch (py=1, px=2) of image 1 is row 1*4 + 2; its element (c=2, ky=3, kx=5) is column 2*196 + 3*14 + 5
    assert pt[1, 6, 2 * 196 + 3 * 14 + 5] == px[1, 2, 14 + 3, 28 + 5]


def test_bf16_rounding_points():
    layers, heads = S.random_weights(G, G.depth, seed=1)
    torch.manual_seed(1)
    px = torch.rand(2, 3, G.image, G.image) * 2 - 1
    f = S.image_features(px, layers, heads, G)
    assert torch.equal(f, O._bf(f))  # bf16-representable
    f32 = S.image_features(px, layers, heads, G, rnd=ID)
    cos = torch.nn.functional.cosine_similarity(f.flatten().double(), f32.flatten().double(), dim=0).item()
    assert cos > 0.9999
    half = S.image_features(px, layers, heads, G, out_scale=0.5)
    assert torch.equal(half, f * 0.5)  # scaling by a power of two is exact in bf16


def test_attention_flash_rounding_point():
    """p_bf16: P rounded to bf16 before P.V, normalised once.  Uniform scores make every
    unnormalised probability exactly 1, so both rounding points give the plain mean of V; for
    random scores the two differ by bf16 rounding of P only, and both match SDPA in fp32."""
    g = torch.Generator().manual_seed(3)
    n, h, s, d = 2, 3, 40, 72
    v = torch.randn(n, h, s, d, generator=g)
    q0 = torch.zeros(n, h, s, d)
    k = torch.randn(n, h, s, d, generator=g)
    ident = lambda t: t  # noqa: E731  (no output rounding: compare the raw products)
    a = S.attention(q0, k, v, ident, p_bf16=True)
    b = S.attention(q0, k, v, ident, p_bf16=False)
    mean_v = v.mean(dim=2, keepdim=True).expand(n, h, s, d).transpose(1, 2).reshape(n, s, h * d)
    torch.testing.assert_close(a, mean_v, rtol=0, atol=1e-6)
    torch.testing.assert_close(b, mean_v, rtol=0, atol=1e-6)
    q = torch.randn(n, h, s, d, generator=g)
    a = S.attention(q, k, v, ident, p_bf16=True)
    b = S.attention(q, k, v, ident, p_bf16=False)
    ref = torch.nn.functional.scaled_dot_product_attention(q, k, v).transpose(1, 2).reshape(n, s, h * d)
    torch.testing.assert_close(b, ref, rtol=0, atol=1e-5)
    err = (a - ref).abs().max().item()
    assert 0 < err < 2e-2  # bf16 rounding of P (8 significant bits) and nothing else
