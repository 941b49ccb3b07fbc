"""CPU oracle of the pi0.5 vision tower: SigLIP So400m/14 and PaliGemma's multi-modal projector.

TEST INFRASTRUCTURE ONLY: ``tests/`` and ``bench.py``'s ``cpu_baseline`` leg may import it; the
product never does.

The tower is third-party code the reference runs as-is: ``embed_image`` calls
``paligemma.model.get_image_features`` (gemma_pytorch.py:106-107; pi0_pytorch.py:200-220), i.e.
transformers' SigLIP vision model and PaliGemma projector, pinned by the reference at
transformers 4.53.2 with openpi's replacement files (neither is in the reference tree).  This
restates their published algorithm (the same in the installed transformers 5.15, against which
``tests/test_siglip_oracle.py`` pins this file in fp32):

* patch embedding: ``Conv2d(3, 1152, 14, stride 14)`` over each 224 x 224 image = a GEMM over the
  256 row-major patches, each flattened in (channel, ky, kx) order, in fp32 (the reference keeps
  ``patch_embedding`` and ``position_embedding`` in fp32, gemma_pytorch.py:93-97) plus the learned
  position embedding, rounded to bf16 where the bf16 encoder takes over;
* 27 pre-norm encoder layers: ``h += out_proj(attn(LN1(h)))``, ``h += fc2(gelu_tanh(fc1(LN2(h))))``,
  LayerNorm eps 1e-6, 16 heads of 72, every Linear with bias;
* ``post_layernorm``, then ``multi_modal_projector.linear`` (1152 -> 2048, bias), times
  ``out_scale`` (1.0: the image features enter the prefix unscaled, as the language embeddings
  are scaled explicitly by embed_prefix -- openpi's patched Gemma likewise drops the embedding
  normalizer, modeling_gemma.py:737-740, and the installed transformers 5.15 get_image_features
  applies no scale; transformers versions that divide the projector output by sqrt(2048)
  correspond to out_scale = 2048 ** -0.5 -- which one the pinned install with openpi's replacement
  files does is not verifiable here, so the scale is a parameter and that factor is parity
  unpinned).

Rounding ledger (``rnd`` = bf16 rounding; pass ``rnd=lambda x: x`` for the fp32 pin): Linear
outputs ``bf16(x.W^T + b)`` (bias in fp32 before the one rounding, as a GEMM epilogue adds it);
LayerNorm fp32 statistics, bf16 output; attention scores and softmax in fp32 (the reference runs
SDPA's flash kernel: no bf16 score rounding), O = bf16(P.V); GELU on the bf16 fc1 output, rounded;
residual adds bf16.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Callable

import torch

from .denoise_oracle import _bf, gelu_tanh

VT = "paligemma_with_expert.paligemma.model.vision_tower.vision_model."
PROJ = "paligemma_with_expert.paligemma.model.multi_modal_projector.linear."


@dataclass(frozen=True)
class SiglipGeometry:
    """PaliGemma's SigLIP vision config (gemma_pytorch.py:58-61 on transformers' defaults)."""

    width: int = 1152
    depth: int = 27
    num_heads: int = 16
    mlp_dim: int = 4304
    patch: int = 14
    image: int = 224
    channels: int = 3
    proj_dim: int = 2048
    ln_eps: float = 1e-6

    @property
    def head_dim(self) -> int:
        return self.width // self.num_heads

    @property
    def grid(self) -> int:
        return self.image // self.patch

    @property
    def n_patches(self) -> int:
        return self.grid * self.grid


def layer_names(i: int) -> dict[str, str]:
    p = f"{VT}encoder.layers.{i}."
    out = {}
    for n in ("q", "k", "v", "out"):
        out[f"w{n}"] = p + f"self_attn.{n}_proj.weight"
        out[f"b{n}"] = p + f"self_attn.{n}_proj.bias"
    out.update({"w1": p + "mlp.fc1.weight", "b1": p + "mlp.fc1.bias", "w2": p + "mlp.fc2.weight", "b2": p + "mlp.fc2.bias",
                "ln1w": p + "layer_norm1.weight", "ln1b": p + "layer_norm1.bias",
                "ln2w": p + "layer_norm2.weight", "ln2b": p + "layer_norm2.bias"})
    return out


HEAD_NAMES = {
    "patch_w": VT + "embeddings.patch_embedding.weight", "patch_b": VT + "embeddings.patch_embedding.bias",
    "pos": VT + "embeddings.position_embedding.weight", "post_w": VT + "post_layernorm.weight",
    "post_b": VT + "post_layernorm.bias", "proj_w": PROJ + "weight", "proj_b": PROJ + "bias",
}


def patchify(pixels: torch.Tensor, g: SiglipGeometry) -> torch.Tensor:
    """``[N, C, H, W]`` -> ``[N, grid*grid, C*p*p]``: patch (py, px) at row py*grid + px, flattened
    in (channel, ky, kx) order -- the row order of the conv output's flatten(2).transpose(1, 2)
    and the column order of the conv weight reshaped to ``[width, C*p*p]``."""
    n, c, _, _ = pixels.shape
    p, gr = g.patch, g.grid
    x = pixels.reshape(n, c, gr, p, gr, p).permute(0, 2, 4, 1, 3, 5)
    return x.reshape(n, gr * gr, c * p * p)


def embeddings(pixels: torch.Tensor, w: dict, g: SiglipGeometry, rnd: Callable = _bf) -> torch.Tensor:
    pw = w["patch_w"].reshape(g.width, -1)
    e = patchify(pixels.float(), g) @ pw.T + w["patch_b"] + w["pos"][: g.n_patches]
    return rnd(e)


def layer_norm(x: torch.Tensor, wt: torch.Tensor, b: torch.Tensor, eps: float, rnd: Callable = _bf) -> torch.Tensor:
    mean = x.mean(-1, keepdim=True)
    var = ((x - mean) ** 2).mean(-1, keepdim=True)
    return rnd((x - mean) / torch.sqrt(var + eps) * wt + b)


def linear_bias(x: torch.Tensor, wt: torch.Tensor, b: torch.Tensor, rnd: Callable = _bf, acc64: bool = False) -> torch.Tensor:
    """``rnd(x W^T + b)``; ``acc64`` accumulates in float64 instead of fp32 (the same rounding
    points, another summation precision: a measure of how far legitimate implementations of the
    same rounding ledger drift apart)."""
    if acc64:
        return rnd((x.double() @ wt.double().T + b.double()).float())
    return rnd(x @ wt.T + b)


def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, rnd: Callable = _bf, p_bf16: bool = False) -> torch.Tensor:
    """``[N, H, S, Dh]`` each; fp32 scores and softmax, O = rnd(P.V) -> ``[N, S, H*Dh]``.

    ``p_bf16``: flash attention's rounding point instead of the math path's: the unnormalised
    probabilities ``exp(s - max)`` are rounded to bf16 before ``P.V`` and the fp32 sum of the
    unrounded ones normalises the product once (what SDPA's flash / memory-efficient kernels
    compute; the reference leaves SigLIP's attention implementation unset, gemma_pytorch.py:45-61,
    so which one runs depends on the installed torch's dispatch).  The engine's kernel rounds here.
    """
    n, h, s, d = q.shape
    sc = (q @ k.transpose(-1, -2)) * (d ** -0.5)
    if p_bf16:
        e = torch.exp(sc - sc.amax(dim=-1, keepdim=True))
        o = (_bf(e) @ v) / e.sum(dim=-1, keepdim=True)
        return rnd(o).transpose(1, 2).reshape(n, s, h * d)
    p = torch.softmax(sc, dim=-1)
    return rnd(p @ v).transpose(1, 2).reshape(n, s, h * d)


def encoder_layer(w: dict, g: SiglipGeometry, h: torch.Tensor, rnd: Callable = _bf, p_bf16: bool = False,
                  acc64: bool = False) -> torch.Tensor:
    n, s, _ = h.shape
    lin = lambda x, wn, bn: linear_bias(x, w[wn], w[bn], rnd, acc64)  # noqa: E731
    x = layer_norm(h, w["ln1w"], w["ln1b"], g.ln_eps, rnd)
    heads = lambda t: t.view(n, s, g.num_heads, g.head_dim).transpose(1, 2)
    q = heads(lin(x, "wq", "bq"))
    k = heads(lin(x, "wk", "bk"))
    v = heads(lin(x, "wv", "bv"))
    h = rnd(h + lin(attention(q, k, v, rnd, p_bf16), "wout", "bout"))
    x = layer_norm(h, w["ln2w"], w["ln2b"], g.ln_eps, rnd)
    x = lin(rnd(gelu_tanh(lin(x, "w1", "b1"))), "w2", "b2")
    return rnd(h + x)


def vision_tower(pixels: torch.Tensor, layers: list[dict], heads: dict, g: SiglipGeometry, rnd: Callable = _bf,
                 p_bf16: bool = False, acc64: bool = False) -> torch.Tensor:
    """SigLIP last hidden state after post_layernorm ``[N, 256, width]``."""
    h = embeddings(pixels, heads, g, rnd)
    for w in layers:
        h = encoder_layer(w, g, h, rnd, p_bf16, acc64)
    return layer_norm(h, heads["post_w"], heads["post_b"], g.ln_eps, rnd)


def image_features(pixels: torch.Tensor, layers: list[dict], heads: dict, g: SiglipGeometry, out_scale: float = 1.0,
                   rnd: Callable = _bf, p_bf16: bool = False, acc64: bool = False) -> torch.Tensor:
    """``get_image_features``: projector(vision_tower(pixels)) * out_scale -> ``[N, 256, proj_dim]``."""
    f = linear_bias(vision_tower(pixels, layers, heads, g, rnd, p_bf16, acc64), heads["proj_w"], heads["proj_b"], rnd, acc64)
    return f if out_scale == 1.0 else rnd(f * out_scale)


def random_weights(g: SiglipGeometry, depth: int, seed: int, std: float = 0.02) -> tuple[list[dict], dict]:
    """bf16-valued encoder/projector weights (fp32 patch/position embeddings), N(0, std); LayerNorm
    weights 1 + N(0, 0.1), biases N(0, 0.02)."""
    gen = torch.Generator().manual_seed(seed)

    def n(*shape, s=std, bf=True):
        t = torch.randn(*shape, generator=gen) * s
        return _bf(t) if bf else t

    W, I = g.width, g.mlp_dim
    layers = []
    for _ in range(depth):
        w = {}
        for nm in ("q", "k", "v", "out"):
            w[f"w{nm}"] = n(W, W)
            w[f"b{nm}"] = n(W)
        w.update({"w1": n(I, W), "b1": n(I), "w2": n(W, I), "b2": n(W),
                  "ln1w": _bf(1 + n(W, s=0.1, bf=False)), "ln1b": n(W), "ln2w": _bf(1 + n(W, s=0.1, bf=False)), "ln2b": n(W)})
        layers.append(w)
    heads = {"patch_w": n(W, g.channels, g.patch, g.patch, bf=False), "patch_b": n(W, bf=False), "pos": n(g.n_patches, W, bf=False),
             "post_w": _bf(1 + n(W, s=0.1, bf=False)), "post_b": n(W), "proj_w": n(g.proj_dim, W), "proj_b": n(g.proj_dim)}
    return layers, heads
