"""CPU oracle of the pi0.5 prefix-LM prefill (PaliGemma's Gemma-2B language model over the prefix).

TEST INFRASTRUCTURE ONLY.  The checker for the prefill path: ``tests/`` and ``bench.py``'s
``cpu_baseline`` leg may import it; the product (``pi05-infer_amd/``) never does.

What it restates (paths relative to the pi05-infer repository):

* ``_build_prefix_cache`` (engine.py:770-794): the prefix's 2-D mask from ``make_att_2d_masks``
  with all-zero attention marks (every valid prefix token sees every valid prefix token,
  pi0_pytorch.py:236-250), positions ``cumsum(pad) - 1``, the additive fp32 4-D mask, and one
  ``GemmaModel.forward`` with ``use_cache=True`` whose per-layer K (after RoPE) and V form the
  ``DynamicCache`` the denoise loop consumes (gemma_pytorch.py:129-140;
  modeling_gemma.py:700-794).
* ``GemmaDecoderLayer.forward`` without adaRMS (modeling_gemma.py:460-517): regular
  ``GemmaRMSNorm`` ``bf16(x * rsqrt(mean(x^2) + eps) * (1 + w))`` with fp32 statistics and an
  fp32 weight (modeling_gemma.py:82-99; the norm weights stay fp32, gemma_pytorch.py:84-104),
  ``h = bf16(h + y)`` residuals (``_gated_residual`` with no gate, modeling_gemma.py:231-249),
  GeGLU MLP ``down(gelu_tanh(gate(x)) * up(x))`` (modeling_gemma.py:138-147).
* The last layer reduced to its K/V (patches/prefix_last_layer.py:84-112, on by default): the
  cache it writes is the full layer's.
* ``embed_language_tokens(ids) * sqrt(W)`` of ``embed_prefix`` (pi0_pytorch.py:225-228).

Rounding ledger: GEMM outputs bf16 (fp32 accumulation); RoPE in fp32 on the bf16 q/k values
and bf16 cos/sin, rounded once (what the compiled reference's fused pointwise kernel computes);
scores ``bf16(bf16(q.k) * 1/16)`` + fp32 mask, fp32 softmax, P bf16, O = bf16(P.V)
(modeling_gemma.py:252-275); GeGLU ``bf16(gelu_tanh(g) * u)`` in fp32 on the bf16 GEMM outputs,
rounded once (the compiled reference's fused GeGLU pointwise kernel; eager rounds gelu's output
first); residual adds bf16.  Pins: tests/test_prefix_oracle.py.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from .denoise_oracle import (
    F32,
    MASK_MIN,
    _bf,
    gelu_tanh,
    linear_bf16,
    make_att_2d_masks,
    mqa_attention,
    rope_apply,
    rope_cos_sin,
)


@dataclass(frozen=True)
class PrefixGeometry:
    """PaliGemma gemma_2b language model (gemma_pytorch.py:44-54)."""

    width: int = 2048
    depth: int = 18
    num_heads: int = 8
    num_kv_heads: int = 1
    head_dim: int = 256
    mlp_dim: int = 16384
    rms_eps: float = 1e-6
    rope_theta: float = 10000.0


def layer_names(i: int) -> dict[str, str]:
    """State-dict names of prefix-LM layer i (modeling_gemma.py:131-133, 291-302, 469-470)."""
    p = f"paligemma_with_expert.paligemma.model.language_model.layers.{i}."
    return {
        "wq": p + "self_attn.q_proj.weight",
        "wk": p + "self_attn.k_proj.weight",
        "wv": p + "self_attn.v_proj.weight",
        "wo": p + "self_attn.o_proj.weight",
        "wg": p + "mlp.gate_proj.weight",
        "wu": p + "mlp.up_proj.weight",
        "wd": p + "mlp.down_proj.weight",
        "ln1": p + "input_layernorm.weight",
        "ln2": p + "post_attention_layernorm.weight",
    }


def rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """Regular GemmaRMSNorm (modeling_gemma.py:82-99): ``x`` bf16 values, ``w`` fp32; fp32 math,
    bf16 output."""
    var = torch.mean(torch.square(x), dim=-1, keepdim=True)
    return _bf(x * torch.rsqrt(var + eps) * (1.0 + w))


def prefix_masks(pad: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Positions ``cumsum(pad) - 1`` int64 ``[B, P]`` and the additive fp32 mask ``[B, 1, P, P]``
    of the prefix (engine.py:773-777: all-zero attention marks, so pad alone decides)."""
    att = torch.zeros(pad.shape, dtype=F32)
    m2 = make_att_2d_masks(pad.bool(), att)
    pos = torch.cumsum(pad.to(torch.int64), dim=1) - 1
    return pos, torch.where(m2[:, None, :, :], 0.0, MASK_MIN)


def embed_tokens(ids: torch.Tensor, table: torch.Tensor, width: int) -> torch.Tensor:
    """``bf16(table[ids] * sqrt(width))`` (pi0_pytorch.py:225-228; the bf16 tensor times a Python
    float: fp32 math, one rounding)."""
    return _bf(table[ids] * math.sqrt(width))


def prefix_layer(w: dict, g: PrefixGeometry, h: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                 mask4d: torch.Tensor, kv_only: bool = False):
    """One decoder layer over the prefix (modeling_gemma.py:460-517, 408-457).  ``h`` ``[B, P, W]``
    bf16 values.  Returns (h_out or None, K ``[B, 1, P, D]``, V ``[B, 1, P, D]``)."""
    b, p, _ = h.shape
    n = rms_norm(h, w["ln1"], g.rms_eps)
    k = linear_bf16(n, w["wk"]).view(b, p, 1, g.head_dim)
    v = linear_bf16(n, w["wv"]).view(b, p, 1, g.head_dim)
    k = rope_apply(k, cos, sin)
    kc, vc = k.transpose(1, 2), v.transpose(1, 2)
    if kv_only:
        return None, kc, vc
    q = rope_apply(linear_bf16(n, w["wq"]).view(b, p, g.num_heads, g.head_dim), cos, sin)
    o = mqa_attention(q.transpose(1, 2), kc, vc, mask4d, g.head_dim ** -0.5)
    h = _bf(h + linear_bf16(o, w["wo"]))
    n2 = rms_norm(h, w["ln2"], g.rms_eps)
    act = _bf(gelu_tanh(linear_bf16(n2, w["wg"])) * linear_bf16(n2, w["wu"]))
    h = _bf(h + linear_bf16(act, w["wd"]))
    return h, kc, vc


def prefill(layers: list[dict], g: PrefixGeometry, embeds: torch.Tensor, pad: torch.Tensor,
            skip_last: bool = True) -> list[tuple[torch.Tensor, torch.Tensor]]:
    """The prefix KV cache: per layer (K, V) bf16 values ``[B, 1, P, D]`` (engine.py:770-794).
    ``embeds`` ``[B, P, W]`` (SigLIP image embeddings and scaled language embeddings), ``pad``
    ``[B, P]`` bool."""
    pos, mask4d = prefix_masks(pad)
    cos, sin = rope_cos_sin(pos, g.head_dim, g.rope_theta)
    h = _bf(embeds.float())
    cache = []
    for i, w in enumerate(layers):
        last = skip_last and i == len(layers) - 1
        h_next, k, v = prefix_layer(w, g, h, cos, sin, mask4d, kv_only=last)
        cache.append((k, v))
        if h_next is not None:
            h = h_next
    return cache


def random_layers(g: PrefixGeometry, depth: int, seed: int, std: float = 0.02) -> list[dict]:
    """bf16-valued random weights N(0, std) (norm weights N(0, 0.1), fp32) for ``depth`` layers."""
    gen = torch.Generator().manual_seed(seed)
    hd = g.num_heads * g.head_dim

    def n(*shape, s=std):
        return _bf(torch.randn(*shape, generator=gen) * s)

    out = []
    for _ in range(depth):
        out.append({
            "wq": n(hd, g.width), "wk": n(g.head_dim, g.width), "wv": n(g.head_dim, g.width),
            "wo": n(g.width, hd), "wg": n(g.mlp_dim, g.width), "wu": n(g.mlp_dim, g.width),
            "wd": n(g.width, g.mlp_dim),
            "ln1": torch.randn(g.width, generator=gen) * 0.1, "ln2": torch.randn(g.width, generator=gen) * 0.1,
        })
    return out
