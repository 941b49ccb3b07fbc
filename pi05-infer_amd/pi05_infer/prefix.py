"""The prefix half of pi0.5 inference on the gfx950 prefill engine: PaliGemma's Gemma-2B language
model over the prefix embeddings, producing the KV cache the denoise loop consumes.

Mirrors the reference's ``_build_prefix_cache`` (engine.py:770-794) from the prefix embeddings on:
``embed_language_tokens`` + the ``sqrt(width)`` scaling of ``embed_prefix`` (pi0_pytorch.py:225-228)
and the prefill itself.  The image embeddings come from the vision tower (vision.py), assembled by
the engine's ``embed_prefix``; any ``[B, P, 2048]`` bf16 prefix embedding with its pad mask works.  Every computation
runs in ``libpi05_denoise.so`` (include/pi05_prefill.h); there is no fallback.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch

from . import _ext

PREFIX = "paligemma_with_expert.paligemma.model.language_model."


@dataclass(frozen=True)
class PrefixGeometry:
    """PaliGemma gemma_2b language model (gemma_pytorch.py:44-54)."""

    width: int = 2048
    depth: int = 18
    num_heads: int = 8
    num_kv_heads: int = 1
    head_dim: int = 256
    mlp_dim: int = 16384
    vocab_size: int = 257152
    rms_eps: float = 1e-6
    rope_theta: float = 10000.0


def layer_param_names(i: int) -> dict[str, str]:
    """State-dict names of layer i (modeling_gemma.py:131-133, 291-302, 469-470)."""
    p = f"{PREFIX}layers.{i}."
    return {
        "wq": p + "self_attn.q_proj.weight", "wk": p + "self_attn.k_proj.weight", "wv": p + "self_attn.v_proj.weight",
        "wo": p + "self_attn.o_proj.weight", "wg": p + "mlp.gate_proj.weight", "wu": p + "mlp.up_proj.weight",
        "wd": p + "mlp.down_proj.weight", "ln1": p + "input_layernorm.weight", "ln2": p + "post_attention_layernorm.weight",
    }


EMBED_NAME = PREFIX + "embed_tokens.weight"


def parameter_specs(g: PrefixGeometry, with_embedding: bool = True) -> list[tuple[str, tuple[int, ...], torch.dtype]]:
    """(name, shape, dtype) of every prefix-LM tensor: projections bf16, norm weights fp32 (the
    reference keeps ``*layernorm*`` in fp32, gemma_pytorch.py:84-104)."""
    hd = g.num_heads * g.head_dim
    specs = []
    for i in range(g.depth):
        n = layer_param_names(i)
        specs += [(n["wq"], (hd, g.width), torch.bfloat16), (n["wk"], (g.head_dim, g.width), torch.bfloat16),
                  (n["wv"], (g.head_dim, g.width), torch.bfloat16), (n["wo"], (g.width, hd), torch.bfloat16),
                  (n["wg"], (g.mlp_dim, g.width), torch.bfloat16), (n["wu"], (g.mlp_dim, g.width), torch.bfloat16),
                  (n["wd"], (g.width, g.mlp_dim), torch.bfloat16), (n["ln1"], (g.width,), torch.float32),
                  (n["ln2"], (g.width,), torch.float32)]
    if with_embedding:
        specs.append((EMBED_NAME, (g.vocab_size, g.width), torch.bfloat16))
    return specs


def make_weights(g: PrefixGeometry, seed: int = 0, device="cuda", std: float = 0.02,
                 with_embedding: bool = True) -> dict[str, torch.Tensor]:
    """Seeded random init generated on ``device``: projections N(0, std) bf16, norm weights
    N(0, 0.1) fp32, embedding N(0, 1) bf16 (no checkpoint download here)."""
    gen = torch.Generator(device=device).manual_seed(seed)
    out = {}
    for name, shape, dtype in parameter_specs(g, with_embedding):
        s = 1.0 if name == EMBED_NAME else (0.1 if dtype == torch.float32 else std)
        out[name] = (torch.randn(*shape, generator=gen, device=device) * s).to(dtype)
    return out


class PrefixLM:
    """Gemma-2B prefix prefill with the reference's entry points: ``embed_language_tokens`` and
    ``build_prefix_cache`` (engine.py:770-794).  One engine context per (batch, prefix_len)."""

    def __init__(self, geometry: PrefixGeometry = PrefixGeometry(), skip_last_layer: bool = True):
        self.geometry = geometry
        self.skip_last_layer = skip_last_layer
        self.params: dict[str, torch.Tensor] = {}
        self.device = torch.device("cpu")
        self._contexts: dict[tuple[int, int], _ext.PrefixContext] = {}
        self._stale: set = set()

    def load_state_dict(self, state_dict: dict, strict: bool = False):
        specs = parameter_specs(self.geometry)
        names = {n for n, _, _ in specs}
        missing = [n for n in names if n not in state_dict]
        unexpected = [n for n in state_dict if n.startswith(PREFIX) and n not in names]
        if strict and (missing or unexpected):
            raise KeyError(f"missing={missing[:5]} unexpected={unexpected[:5]}")
        for name, shape, dtype in specs:
            if name not in state_dict:
                continue
            t = state_dict[name]
            if tuple(t.shape) != tuple(shape):
                raise ValueError(f"{name}: shape {tuple(t.shape)} != {shape}")
            t = t.to(device=self.device, dtype=dtype).contiguous()
            if name in self.params:
                self.params[name].copy_(t)
            else:
                self.params[name] = t
        self._stale = set(self._contexts)
        return missing, unexpected

    def to(self, device):
        device = torch.device(device)
        if device.type == "cuda" and device.index is None:
            device = torch.device("cuda", torch.cuda.current_device())
        self.params = {k: v.to(device).contiguous() for k, v in self.params.items()}
        self.device = device
        self.close()
        return self

    def _context(self, batch: int, prefix_len: int) -> _ext.PrefixContext:
        if self.device.type != "cuda":
            raise RuntimeError("the prefill engine runs on a gfx950 GPU; call .to('cuda') first")
        key = (batch, prefix_len)
        ctx = self._contexts.get(key)
        if ctx is None:
            g = self.geometry
            d = _ext.prefix_default_dims()
            d.depth, d.batch, d.prefix_len = g.depth, batch, prefix_len
            d.rms_eps, d.rope_theta, d.skip_last_layer = g.rms_eps, g.rope_theta, int(self.skip_last_layer)
            ctx = _ext.PrefixContext(d, self.device)
            for i in range(g.depth):
                n = layer_param_names(i)
                try:
                    ctx.bind_layer(i, *(self.params[n[k]] for k in ("wq", "wk", "wv", "wo", "wg", "wu", "wd", "ln1", "ln2")))
                except KeyError as e:
                    ctx.close()
                    raise RuntimeError(f"prefix-LM weights not loaded: {e}") from None
            ctx.refresh_weights()
            self._contexts[key] = ctx
        elif key in self._stale:
            ctx.refresh_weights()
            self._stale.discard(key)
        return ctx

    @torch.no_grad()
    def embed_language_tokens(self, tokens: torch.Tensor, prefix_len: Optional[int] = None) -> torch.Tensor:
        """``embed_tokens(tokens) * sqrt(width)`` in bf16 (gemma_pytorch.py:109-110 with
        pi0_pytorch.py:225-228's scaling).  ``prefix_len``: the length of the prefix these tokens
        end, so the context the prefill will use serves the lookup too."""
        if EMBED_NAME not in self.params:
            raise RuntimeError("embed_tokens weight not loaded")
        if prefix_len is not None:
            ctx = self._context(tokens.shape[0], prefix_len)
        else:
            ctx = next(iter(self._contexts.values()), None) or self._context(1, 1)
        return ctx.embed_tokens(tokens, self.params[EMBED_NAME])

    @torch.no_grad()
    def build_prefix_cache(self, prefix_embs: torch.Tensor, prefix_pad_masks: torch.Tensor):
        """``(prefix_output, prefix_pad_masks, past_key_values)`` as ``_build_prefix_cache``
        returns them (engine.py:770-794): ``past_key_values`` is a list of per-layer (K, V) bf16
        ``[B, 1, P, D]``; ``prefix_output`` is None (the last layer computes only its K/V, as with
        the reference's default prefix_last_layer patch)."""
        b, p, w = prefix_embs.shape
        if w != self.geometry.width:
            raise ValueError(f"prefix_embs width {w} != {self.geometry.width}")
        ctx = self._context(b, p)
        g = self.geometry
        kv = torch.empty((2, g.depth, b, 1, p, g.head_dim), dtype=torch.bfloat16, device=self.device)
        ks = [kv[0, i] for i in range(g.depth)]
        vs = [kv[1, i] for i in range(g.depth)]
        ctx.forward(prefix_embs.to(device=self.device, dtype=torch.bfloat16).contiguous(), prefix_pad_masks.to(self.device),
                    ks, vs)
        return None, prefix_pad_masks, list(zip(ks, vs))

    def close(self) -> None:
        for c in self._contexts.values():
            c.close()
        self._contexts.clear()
        self._stale.clear()
