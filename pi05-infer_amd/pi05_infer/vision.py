"""The pi0.5 vision tower on the gfx950 engine: SigLIP So400m/14 and PaliGemma's multi-modal
projector, i.e. ``embed_image`` -> ``get_image_features`` (gemma_pytorch.py:106-107), producing the
image part of the prefix embeddings (pi0_pytorch.py:190-255).  Every computation runs in
``libpi05_denoise.so`` (include/pi05_siglip.h); there is no fallback.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _ext

VT = "paligemma_with_expert.paligemma.model.vision_tower.vision_model."
PROJ = "paligemma_with_expert.paligemma.model.multi_modal_projector.linear."


@dataclass(frozen=True)
class VisionGeometry:
    """PaliGemma's SigLIP config (gemma_pytorch.py:58-61 on transformers' SiglipVisionConfig
    defaults); ``out_scale`` multiplies the projector output (1: the image features enter the
    prefix as the projector returns them)."""

    width: int = 1152
    depth: int = 27
    num_heads: int = 16
    mlp_dim: int = 4304
    patch: int = 14
    image: int = 224
    channels: int = 3
    proj_dim: int = 2048
    ln_eps: float = 1e-6
    out_scale: float = 1.0

    @property
    def n_patches(self) -> int:
        return (self.image // self.patch) ** 2


LAYER_KEYS = ("wq", "bq", "wk", "bk", "wv", "bv", "wo", "bo", "w1", "b1", "w2", "b2", "ln1_w", "ln1_b", "ln2_w", "ln2_b")


def layer_param_names(i: int) -> dict[str, str]:
    """State-dict names of encoder layer i (transformers' SiglipEncoderLayer)."""
    p = f"{VT}encoder.layers.{i}."
    a = p + "self_attn."
    return {
        "wq": a + "q_proj.weight", "bq": a + "q_proj.bias", "wk": a + "k_proj.weight", "bk": a + "k_proj.bias",
        "wv": a + "v_proj.weight", "bv": a + "v_proj.bias", "wo": a + "out_proj.weight", "bo": a + "out_proj.bias",
        "w1": p + "mlp.fc1.weight", "b1": p + "mlp.fc1.bias", "w2": p + "mlp.fc2.weight", "b2": p + "mlp.fc2.bias",
        "ln1_w": p + "layer_norm1.weight", "ln1_b": p + "layer_norm1.bias", "ln2_w": p + "layer_norm2.weight",
        "ln2_b": p + "layer_norm2.bias",
    }


HEAD_PARAM_NAMES = {
    "patch_w": VT + "embeddings.patch_embedding.weight", "patch_b": VT + "embeddings.patch_embedding.bias",
    "pos": VT + "embeddings.position_embedding.weight", "post_w": VT + "post_layernorm.weight",
    "post_b": VT + "post_layernorm.bias", "proj_w": PROJ + "weight", "proj_b": PROJ + "bias",
}
HEAD_KEYS = ("patch_w", "patch_b", "pos", "post_w", "post_b", "proj_w", "proj_b")
FP32_HEADS = ("patch_w", "patch_b", "pos")  # kept fp32 by gemma_pytorch.py:93-97


def parameter_specs(g: VisionGeometry) -> list[tuple[str, tuple[int, ...], torch.dtype]]:
    """(name, shape, dtype) of every vision-tower tensor."""
    W, I, bf = g.width, g.mlp_dim, torch.bfloat16
    shapes = {"wq": (W, W), "wk": (W, W), "wv": (W, W), "wo": (W, W), "w1": (I, W), "b1": (I,), "w2": (W, I)}
    specs = []
    for i in range(g.depth):
        n = layer_param_names(i)
        specs += [(n[k], shapes.get(k, (W,)), bf) for k in LAYER_KEYS]
    hs = {"patch_w": (W, g.channels, g.patch, g.patch), "patch_b": (W,), "pos": (g.n_patches, W), "post_w": (W,),
          "post_b": (W,), "proj_w": (g.proj_dim, W), "proj_b": (g.proj_dim,)}
    specs += [(HEAD_PARAM_NAMES[k], hs[k], torch.float32 if k in FP32_HEADS else bf) for k in HEAD_KEYS]
    return specs


def make_weights(g: VisionGeometry, seed: int = 0, device="cuda", std: float = 0.02) -> dict[str, torch.Tensor]:
    """Seeded random init on ``device``: matrices and biases N(0, std), LayerNorm weights
    1 + N(0, 0.1) (no checkpoint download here)."""
    gen = torch.Generator(device=device).manual_seed(seed)
    out = {}
    for name, shape, dtype in parameter_specs(g):
        t = torch.randn(*shape, generator=gen, device=device)
        is_ln_w = name.endswith(("layer_norm1.weight", "layer_norm2.weight", "post_layernorm.weight"))
        out[name] = (1 + 0.1 * t if is_ln_w else t * std).to(dtype)
    return out


class VisionTower:
    """SigLIP + projector with the reference's entry point ``embed_image`` (gemma_pytorch.py:106-107).
    One engine context per image count (batch x camera views)."""

    def __init__(self, geometry: VisionGeometry = VisionGeometry()):
        self.geometry = geometry
        self.params: dict[str, torch.Tensor] = {}
        self.device = torch.device("cpu")
        self._contexts: dict[int, _ext.VisionContext] = {}
        self._stale: set = set()

    def load_state_dict(self, state_dict: dict, strict: bool = False):
        specs = parameter_specs(self.geometry)
        names = {n for n, _, _ in specs}
        missing = [n for n in names if n not in state_dict]
        unexpected = [n for n in state_dict if (n.startswith(VT) or n.startswith(PROJ)) and n not in names]
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

    def _context(self, n_images: int) -> _ext.VisionContext:
        if self.device.type != "cuda":
            raise RuntimeError("the vision tower runs on a gfx950 GPU; call .to('cuda') first")
        ctx = self._contexts.get(n_images)
        if ctx is None:
            g = self.geometry
            d = _ext.vision_default_dims()
            d.depth, d.n_images, d.ln_eps, d.out_scale = g.depth, n_images, g.ln_eps, g.out_scale
            ctx = _ext.VisionContext(d, self.device)
            try:
                for i in range(g.depth):
                    n = layer_param_names(i)
                    ctx.bind_layer(i, *(self.params[n[k]] for k in LAYER_KEYS))
                ctx.bind_heads(*(self.params[HEAD_PARAM_NAMES[k]] for k in HEAD_KEYS))
            except KeyError as e:
                ctx.close()
                raise RuntimeError(f"vision-tower weights not loaded: {e}") from None
            ctx.refresh_weights()
            self._contexts[n_images] = ctx
        elif n_images in self._stale:
            ctx.refresh_weights()
            self._stale.discard(n_images)
        return ctx

    @torch.no_grad()
    def embed_image(self, image: torch.Tensor) -> torch.Tensor:
        """``get_image_features``: images ``[N, 3, 224, 224]`` in [-1, 1] -> ``[N, 256, 2048]`` bf16."""
        g = self.geometry
        if image.dim() != 4 or tuple(image.shape[1:]) != (g.channels, g.image, g.image):
            raise ValueError(f"image must be [N, {g.channels}, {g.image}, {g.image}], got {tuple(image.shape)}")
        ctx = self._context(image.shape[0])
        return ctx.forward(image.to(device=self.device, dtype=torch.float32).contiguous())

    def close(self) -> None:
        for c in self._contexts.values():
            c.close()
        self._contexts.clear()
        self._stale.clear()
