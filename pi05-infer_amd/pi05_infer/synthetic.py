"""Seeded synthetic pi0.5 action-expert weights and denoise inputs.

There is no checkpoint or network here, so every benchmark and parity case runs on random-init
weights in the reference geometry (Gemma-300M expert: width 1024, depth 18, 8 query heads, 1 KV
head, head_dim 256, GeGLU mlp_dim 4096; action in/out 32 <-> 1024; pi0.5 time MLP 1024 -> 1024).

Draw recipe (fixed, so CPU oracle and GPU engine see identical values).  Every array is filled
from numpy PCG64 streams in chunks of 2**18 elements; chunk ``c`` of an array tagged ``tag`` uses
``SeedSequence([seed, tag, c])``, so the values do not depend on thread count, on the order in
which arrays are drawn, or (for weights, whose tag is the CRC32 of the parameter name) on the
model depth.

* weights: seed 0, every weight AND bias ~ N(0, 0.02) in fp32; the seven expert
  ``nn.Linear`` weights per layer are then rounded to bf16 (the reference's dtype policy,
  openpi_patched/gemma_pytorch.py:84-104: everything bf16 except ``input_layernorm``,
  ``post_attention_layernorm`` and ``model.norm``, whose adaRMS ``dense`` stays fp32; the action
  and time heads live outside the cast and stay fp32, pi0_pytorch.py:104-109);
* prefix KV: seed 1, K (tag 0) and V (tag 1) drawn as fp32 N(0, 1) of shape ``[B, L, P, D]``
  and rounded to bf16;
* noise x_1: sample ``b`` uses seed ``2 + b`` (tag 0), N(0, 1) fp32 ``[A, a]``.

The reference itself zero-initialises biases and adaRMS dense weights (modeling_gemma.py:77,
536-541), which makes every gate zero; that case is kept only as a special-case test
(:func:`zero_gate_weights`).
"""

from __future__ import annotations

import os
import zlib
from concurrent.futures import ThreadPoolExecutor
from dataclasses import dataclass

import numpy as np
import torch

_CHUNK = 1 << 18

EXPERT_PREFIX = "paligemma_with_expert.gemma_expert.model."


@dataclass(frozen=True)
class ExpertGeometry:
    """Geometry of the pi0.5 action expert (openpi ``gemma_300m``) and its denoise loop."""

    width: int = 1024
    depth: int = 18
    num_heads: int = 8
    num_kv_heads: int = 1
    head_dim: int = 256
    mlp_dim: int = 4096
    action_dim: int = 32
    action_horizon: int = 50
    rms_eps: float = 1e-6
    rope_theta: float = 10000.0
    time_min_period: float = 4e-3
    time_max_period: float = 4.0

    @property
    def num_norms(self) -> int:
        """adaRMS norms: two per layer plus the final norm (engine.py:580-586)."""
        return 2 * self.depth + 1


def layer_param_names(i: int) -> dict[str, str]:
    """Reference state-dict names of decoder layer ``i`` (modeling_gemma.py:291-302, 131-133, 469-470)."""
    p = f"{EXPERT_PREFIX}layers.{i}."
    return {
        "ln1_w": p + "input_layernorm.dense.weight",
        "ln1_b": p + "input_layernorm.dense.bias",
        "wq": p + "self_attn.q_proj.weight",
        "wk": p + "self_attn.k_proj.weight",
        "wv": p + "self_attn.v_proj.weight",
        "wo": p + "self_attn.o_proj.weight",
        "ln2_w": p + "post_attention_layernorm.dense.weight",
        "ln2_b": p + "post_attention_layernorm.dense.bias",
        "wgate": p + "mlp.gate_proj.weight",
        "wup": p + "mlp.up_proj.weight",
        "wdown": p + "mlp.down_proj.weight",
    }


HEAD_PARAM_NAMES = {
    "norm_w": EXPERT_PREFIX + "norm.dense.weight",
    "norm_b": EXPERT_PREFIX + "norm.dense.bias",
    "in_w": "action_in_proj.weight",
    "in_b": "action_in_proj.bias",
    "out_w": "action_out_proj.weight",
    "out_b": "action_out_proj.bias",
    "tin_w": "time_mlp_in.weight",
    "tin_b": "time_mlp_in.bias",
    "tout_w": "time_mlp_out.weight",
    "tout_b": "time_mlp_out.bias",
}

BF16_KEYS = ("wq", "wk", "wv", "wo", "wgate", "wup", "wdown")


def parameter_specs(g: ExpertGeometry) -> list[tuple[str, tuple[int, ...], bool]]:
    """(name, shape, is_bf16) of every parameter, in draw order."""
    W, H, D, I, a = g.width, g.num_heads, g.head_dim, g.mlp_dim, g.action_dim
    specs: list[tuple[str, tuple[int, ...], bool]] = [
        ("action_in_proj.weight", (W, a), False),
        ("action_in_proj.bias", (W,), False),
        ("action_out_proj.weight", (a, W), False),
        ("action_out_proj.bias", (a,), False),
        ("time_mlp_in.weight", (W, W), False),
        ("time_mlp_in.bias", (W,), False),
        ("time_mlp_out.weight", (W, W), False),
        ("time_mlp_out.bias", (W,), False),
    ]
    shapes = {
        "ln1_w": (3 * W, W),
        "ln1_b": (3 * W,),
        "wq": (H * D, W),
        "wk": (g.num_kv_heads * D, W),
        "wv": (g.num_kv_heads * D, W),
        "wo": (W, H * D),
        "ln2_w": (3 * W, W),
        "ln2_b": (3 * W,),
        "wgate": (I, W),
        "wup": (I, W),
        "wdown": (W, I),
    }
    for i in range(g.depth):
        for key, name in layer_param_names(i).items():
            specs.append((name, shapes[key], key in BF16_KEYS))
    specs.append((HEAD_PARAM_NAMES["norm_w"], (3 * W, W), False))
    specs.append((HEAD_PARAM_NAMES["norm_b"], (3 * W,), False))
    return specs


def seeded_normal(shape: tuple[int, ...], seed: int, tag: int, pool: ThreadPoolExecutor | None = None,
                  std: float = 1.0) -> np.ndarray:
    """N(0, std) fp32 array; chunk ``c`` is drawn from PCG64(SeedSequence([seed, tag, c])) as
    N(0, 1) and then multiplied by ``np.float32(std)``."""
    n = int(np.prod(shape))
    out = np.empty(n, dtype=np.float32)

    def fill(c: int) -> None:
        lo = c * _CHUNK
        hi = min(n, lo + _CHUNK)
        rng = np.random.Generator(np.random.PCG64(np.random.SeedSequence([seed, tag, c])))
        rng.standard_normal(hi - lo, dtype=np.float32, out=out[lo:hi])
        if std != 1.0:
            out[lo:hi] *= np.float32(std)

    chunks = range((n + _CHUNK - 1) // _CHUNK)
    if pool is None or len(chunks) == 1:
        for c in chunks:
            fill(c)
    else:
        list(pool.map(fill, chunks))
    return out.reshape(shape)


def _threads() -> int:
    return max(1, min(16, os.cpu_count() or 1))


def make_weights(g: ExpertGeometry = ExpertGeometry(), seed: int = 0, std: float = 0.02) -> dict[str, torch.Tensor]:
    """Seeded random-init expert + heads, CPU tensors, reference state-dict names."""
    out: dict[str, torch.Tensor] = {}
    with ThreadPoolExecutor(_threads()) as pool:
        for name, shape, is_bf16 in parameter_specs(g):
            t = torch.from_numpy(seeded_normal(shape, seed, zlib.crc32(name.encode()), pool, std))
            out[name] = t.to(torch.bfloat16) if is_bf16 else t
    return out


def zero_gate_weights(w: dict[str, torch.Tensor], g: ExpertGeometry) -> dict[str, torch.Tensor]:
    """Copy of ``w`` with every adaRMS gate row (dense rows [2W, 3W)) and gate bias zeroed.

    With gate = 0 every gated residual adds nothing (modeling_gemma.py:231-249), so each layer is
    the identity and the expert output is the final norm of bf16(action_in_proj(x)).
    """
    W = g.width
    out = dict(w)
    names = []
    for i in range(g.depth):
        n = layer_param_names(i)
        names += [(n["ln1_w"], n["ln1_b"]), (n["ln2_w"], n["ln2_b"])]
    for wn, bn in names:
        dw = out[wn].clone()
        db = out[bn].clone()
        dw[2 * W:] = 0
        db[2 * W:] = 0
        out[wn] = dw
        out[bn] = db
    return out


def make_prefix_kv(g: ExpertGeometry, prefix_len: int, batch: int = 1, seed: int = 1) -> tuple[torch.Tensor, torch.Tensor]:
    """Static prefix KV cache: K, V bf16 ``[B, L, P, D]`` from N(0, 1) (seed 1)."""
    shape = (batch, g.depth, prefix_len, g.head_dim)
    with ThreadPoolExecutor(_threads()) as pool:
        k = torch.from_numpy(seeded_normal(shape, seed, 0, pool)).to(torch.bfloat16)
        v = torch.from_numpy(seeded_normal(shape, seed, 1, pool)).to(torch.bfloat16)
    return k, v


def make_noise(g: ExpertGeometry, batch: int = 1, seed: int = 2) -> torch.Tensor:
    """Initial noise x_1 ``[B, A, a]`` fp32; sample ``b`` drawn from a generator seeded ``seed + b``."""
    rows = [torch.from_numpy(seeded_normal((g.action_horizon, g.action_dim), seed + b, 0)) for b in range(batch)]
    return torch.stack(rows)


def full_prefix_pad(prefix_len: int, batch: int = 1) -> torch.Tensor:
    """All-valid prefix pad mask ``[B, P]`` bool (the 'full-attention mask' of the benchmark)."""
    return torch.ones((batch, prefix_len), dtype=torch.bool)
