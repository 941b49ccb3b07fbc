"""pi0.5 inference engine whose denoise loop runs on hand-written gfx950 kernels.

Drop-in for the reference's ``pi05_infer.engine`` on the denoise path: ``OpenPi0Inference``
keeps ``sample_actions(observation, noise=None) -> {"actions"}`` (engine.py:344-406),
``capture_cuda_graph`` / ``is_cuda_graph_enabled`` / ``release_cuda_graph`` (engine.py:831-860,
_vendored/base_policy.py:96-107), ``enable_torch_compile`` (a no-op here: there is nothing to
compile, engine.py:1003-1059), ``invalidate_weight_derived_caches`` (engine.py:526-554) and
``predict_action_batch`` (engine.py:321-342).

Every denoise computation happens in ``libpi05_denoise.so``; PyTorch only provides device
memory, streams and the random noise draw.  An observation carries either the prefix KV cache and
pad mask that ``_build_prefix_cache`` produces (the reference's frozen-prefix mode,
tools/bitexact_compiled_toggles.py:354-376), or the prefix embeddings and pad mask, in which case
the attached ``PrefixLM`` (prefix.py) runs the Gemma-2B prefill on the GPU first, or the camera
images and tokenized prompt, in which case ``embed_prefix`` (pi0_pytorch.py:190-255) runs the
attached ``VisionTower`` (vision.py, SigLIP + projector) and the token embedding before the
prefill.  Image preprocessing (resize, augmentation, HWC -> CHW) happens before the observation
reaches the engine: images arrive as ``[B, 3, 224, 224]`` in [-1, 1].
"""

from __future__ import annotations

import logging
from dataclasses import dataclass, field
from typing import Any, Optional, Sequence

import torch

from . import _ext
from . import transforms as _transforms
from .synthetic import BF16_KEYS, HEAD_PARAM_NAMES, ExpertGeometry, layer_param_names

logger = logging.getLogger(__name__)


@dataclass(frozen=True)
class OpenPi0InferConfig:
    """Inference config: the pi0.5 fields of openpi's ``Pi0Config`` that the denoise path reads
    plus the reference's inference extras (engine.py:120-140)."""

    config_name: str = "pi05_libero"
    pi05: bool = True
    action_dim: int = 32
    action_horizon: int = 50
    max_token_len: int = 200
    dtype: str = "bfloat16"
    paligemma_variant: str = "gemma_2b"
    action_expert_variant: str = "gemma_300m"
    num_images_in_input: int = 2
    noise_method: str = "flow_sde"
    noise_level: float = 0.5
    action_chunk: int = 5
    action_env_dim: int = 7
    num_steps: int = 10
    train_expert_only: bool = False


@dataclass
class Observation:
    """What ``sample_actions`` consumes, one of three prefix forms: the prefix KV cache of
    ``_build_prefix_cache`` (per layer K and V bf16 ``[B, 1, P, D]``, or stacked ``[B, L, P, D]``)
    with its pad mask ``[B, P]``; the prefix embeddings ``[B, P, 2048]`` (``embed_prefix``'s
    output, pi0_pytorch.py:190-255) with the pad mask; or the camera views (``images``: per view
    ``[B, 3, 224, 224]`` in [-1, 1], ``image_masks``: per view ``[B]`` bool) and the tokenized
    prompt ``[B, T]`` with its mask, as ``_preprocess_observation`` returns them
    (pi0_pytorch.py:165-174).  The robot state is unused by pi0.5's suffix (pi0_pytorch.py:269-287)."""

    prefix_k: Any
    prefix_v: Any
    prefix_pad_masks: Optional[torch.Tensor]
    state: Optional[torch.Tensor] = None
    extra: dict = field(default_factory=dict)
    prefix_embs: Optional[torch.Tensor] = None
    images: Optional[list] = None
    image_masks: Optional[list] = None
    tokenized_prompt: Optional[torch.Tensor] = None
    tokenized_prompt_mask: Optional[torch.Tensor] = None

    @classmethod
    def from_dict(cls, d: dict) -> "Observation":
        if "images" in d:
            imgs, masks = d["images"], d["image_masks"]
            imgs = list(imgs.values()) if isinstance(imgs, dict) else list(imgs)
            masks = list(masks.values()) if isinstance(masks, dict) else list(masks)
            return cls(None, None, None, d.get("state"), images=imgs, image_masks=masks,
                       tokenized_prompt=d["tokenized_prompt"], tokenized_prompt_mask=d["tokenized_prompt_mask"])
        if "prefix_embs" in d:
            return cls(None, None, d["prefix_pad_masks"], d.get("state"), prefix_embs=d["prefix_embs"])
        if "past_key_values" in d:
            kv = d["past_key_values"]
            ks = [p[0] for p in kv]
            vs = [p[1] for p in kv]
        else:
            ks, vs = d["prefix_k"], d["prefix_v"]
        return cls(ks, vs, d["prefix_pad_masks"], d.get("state"))


def _split_layers(t: Any, depth: int) -> list[torch.Tensor]:
    if isinstance(t, torch.Tensor):
        if t.dim() != 4:
            raise ValueError("stacked prefix K/V must be [B, L, P, D]")
        return [t[:, i : i + 1] for i in range(depth)]
    return list(t)


class OpenPi0Inference:
    """pi0.5 action prediction with the gfx950 denoise engine."""

    def __init__(self, config: OpenPi0InferConfig, geometry: ExpertGeometry = ExpertGeometry()):
        if not config.pi05:
            raise NotImplementedError("only pi0.5 (adaRMS action expert) is implemented")
        if config.action_horizon != geometry.action_horizon or config.action_dim != geometry.action_dim:
            raise ValueError("config action_horizon/action_dim must match the expert geometry")
        self.config = config
        self.geometry = geometry
        self.params: dict[str, torch.Tensor] = {}
        self.device = torch.device("cpu")
        self.logger = logger
        self._contexts: dict[tuple, _ext.DenoiseContext] = {}
        self._stale_contexts: set = set()
        self.cuda_graph_manager = None
        self.torch_compile_enabled = False
        self._torch_compile_mode = None
        self.training = False
        self.schedule: Optional[str] = None  # None: the library's default for the device
        self._pending_ctx: Optional[_ext.DenoiseContext] = None  # context of the last predict, until its status is read
        self.prefix_lm = None  # optional PrefixLM (prefix.py): prefix embeddings -> KV cache
        self.vision_tower = None  # optional VisionTower (vision.py): camera images -> image embeddings
        # until setup_wrappers installs the checkpoint's transforms: the policy's Outputs slice only
        # (no norm stats), so env-facing actions never carry the model's padding dims
        self.setup_wrappers(output_transforms=_transforms.output_transforms_for(config.config_name, None))

    # ------------------------------------------------------------------ parameters
    def expected_parameters(self) -> dict[str, tuple[tuple[int, ...], torch.dtype]]:
        from .synthetic import parameter_specs

        return {n: (s, torch.bfloat16 if bf else torch.float32) for n, s, bf in parameter_specs(self.geometry)}

    def load_state_dict(self, state_dict: dict, strict: bool = False):
        """Copy matching tensors in (dtype policy of gemma_pytorch.py:84-104 applied); returns
        (missing, unexpected) like ``nn.Module.load_state_dict``."""
        spec = self.expected_parameters()
        missing = [n for n in spec if n not in state_dict]
        unexpected = [n for n in state_dict if n not in spec]
        if strict and (missing or unexpected):
            raise KeyError(f"missing={missing[:5]} unexpected={unexpected[:5]}")
        for name, (shape, dtype) in spec.items():
            if name not in state_dict:
                continue
            t = state_dict[name]
            if tuple(t.shape) != tuple(shape):
                raise ValueError(f"{name}: shape {tuple(t.shape)} != {shape}")
            t = t.to(device=self.device, dtype=dtype).contiguous()
            if name in self.params:
                self.params[name].copy_(t)  # in place: keeps addresses for bound contexts
            else:
                self.params[name] = t
        self._mark_weights_changed()
        return missing, unexpected

    def state_dict(self) -> dict[str, torch.Tensor]:
        return dict(self.params)

    def parameters(self):
        return iter(self.params.values())

    def to(self, device=None, dtype=None):
        if dtype is not None:
            raise ValueError("the engine keeps the reference dtype policy; dtype cannot be changed")
        if device is not None:
            device = torch.device(device)
            if device.type == "cuda" and device.index is None:
                device = torch.device("cuda", torch.cuda.current_device())
            self.params = {k: v.to(device).contiguous() for k, v in self.params.items()}
            self.device = device
            self._drop_contexts()
            if self.prefix_lm is not None:
                self.prefix_lm.to(device)
            if self.vision_tower is not None:
                self.vision_tower.to(device)
        return self

    def attach_prefix_lm(self, prefix_lm) -> None:
        """Run the Gemma-2B prefill (prefix.PrefixLM) for observations that carry prefix
        embeddings instead of a KV cache; its depth must equal the expert's."""
        if prefix_lm.geometry.depth != self.geometry.depth:
            raise ValueError("prefix LM and action expert must have the same depth (one KV layer per expert layer)")
        prefix_lm.to(self.device)
        self.prefix_lm = prefix_lm

    def attach_vision_tower(self, vision_tower) -> None:
        """Run SigLIP + the projector (vision.VisionTower) for observations that carry camera
        images; the projector's width must equal the prefix LM's."""
        vision_tower.to(self.device)
        self.vision_tower = vision_tower

    @torch.no_grad()
    def embed_prefix(self, images, img_masks, lang_tokens, lang_masks):
        """``(prefix_embs, prefix_pad_masks, prefix_att_masks)`` as pi0_pytorch.py:190-255 builds
        them: one vision-tower call over all views stacked on the batch dim, each view's 256 image
        embeddings padded by its image mask, then the scaled token embeddings padded by the prompt
        mask; the attention mask is all zeros (full attention over the prefix)."""
        if self.vision_tower is None or self.prefix_lm is None:
            raise ValueError("embed_prefix needs an attached VisionTower and PrefixLM")
        bsize = images[0].shape[0]
        all_embs = self.vision_tower.embed_image(torch.cat(list(images), dim=0) if len(images) > 1 else images[0])
        n_img = all_embs.shape[1]
        embs, pads = [], []
        for v, m in enumerate(img_masks):
            embs.append(all_embs[v * bsize : (v + 1) * bsize])
            pads.append(m.to(device=all_embs.device, dtype=torch.bool)[:, None].expand(bsize, n_img))
        embs.append(self.prefix_lm.embed_language_tokens(lang_tokens, prefix_len=len(images) * n_img + lang_tokens.shape[1]))
        pads.append(lang_masks.to(device=all_embs.device, dtype=torch.bool))
        embs = torch.cat(embs, dim=1)
        pads = torch.cat(pads, dim=1)
        return embs, pads, torch.zeros_like(pads)

    def _build_prefix_cache(self, images, img_masks, lang_tokens, lang_masks):
        """``(prefix_output, prefix_pad_masks, past_key_values)`` from camera images and prompt
        (engine.py:770-794): ``embed_prefix`` then the prefill."""
        embs, pads, _ = self.embed_prefix(images, img_masks, lang_tokens, lang_masks)
        return self.prefix_lm.build_prefix_cache(embs, pads)

    def eval(self):
        self.training = False
        return self

    def train(self, mode: bool = True):
        if mode:
            raise NotImplementedError("inference-only engine")
        return self

    # ------------------------------------------------------------------ engine contexts
    def _drop_contexts(self) -> None:
        self._pending_ctx = None
        for c in self._contexts.values():
            c.close()
        self._contexts.clear()
        self._stale_contexts.clear()

    def _mark_weights_changed(self) -> None:
        self._stale_contexts = set(self._contexts)

    def _bind(self, ctx: _ext.DenoiseContext) -> None:
        p = self.params
        for i in range(self.geometry.depth):
            n = layer_param_names(i)
            ctx.bind_layer(i, *(p[n[k]] for k in ("wq", "wk", "wv", "wo", "wgate", "wup", "wdown",
                                                    "ln1_w", "ln1_b", "ln2_w", "ln2_b")))
        h = HEAD_PARAM_NAMES
        ctx.bind_heads(*(p[h[k]] for k in ("norm_w", "norm_b", "in_w", "in_b", "out_w", "out_b",
                                            "tin_w", "tin_b", "tout_w", "tout_b")))

    def _context(self, batch: int, prefix_len: int, num_steps: int) -> _ext.DenoiseContext:
        if self.device.type != "cuda":
            raise RuntimeError("the denoise engine runs on a gfx950 GPU; call .to('cuda') first")
        key = (batch, prefix_len, num_steps)
        ctx = self._contexts.get(key)
        if ctx is None:
            missing = [n for n in self.expected_parameters() if n not in self.params]
            if missing:
                raise RuntimeError(f"weights not loaded: {missing[:3]} ...")
            ctx = _ext.DenoiseContext(self.geometry, batch, prefix_len, num_steps, self.device)
            if self.schedule is not None:
                ctx.set_schedule(self.schedule)
            self._bind(ctx)
            ctx.refresh_weights()
            self._contexts[key] = ctx
        elif key in self._stale_contexts:
            ctx.refresh_weights()
            self._stale_contexts.discard(key)
        return ctx

    # ------------------------------------------------------------------ reference API
    def sample_noise(self, shape, device):
        """pi0_pytorch.py:176-183."""
        return torch.normal(mean=0.0, std=1.0, size=shape, dtype=torch.float32, device=device)

    @torch.no_grad()
    def sample_actions(self, observation, noise: Optional[torch.Tensor] = None) -> dict:
        """Prefix KV + ``num_steps`` flow_ode Euler steps (engine.py:344-406) -> ``{"actions"}``.

        Random draws match the reference's: the initial noise when none is passed, then one
        ``sample_noise`` of the action shape per Euler step (its flow_ode update adds
        ``sample_noise * std`` with std = 0, and the graph path draws the same tensor "so RNG
        consumption matches the eager path", engine.py:389-405), so a generator seeded once gives
        the reference's noise on every later predict too.  Like the reference's, the call only
        enqueues GPU work; ``output_transform`` (or ``predict_action_batch``) waits for it and
        raises ``Pi05Error`` if the launch failed."""
        actions, _ = self._run(observation, noise, trace=False)
        return {"actions": actions}

    @torch.no_grad()
    def sample_actions_with_velocities(self, observation, noise: Optional[torch.Tensor] = None):
        """Like ``sample_actions`` but also returns every step's velocity ``[steps, B, A, a]``
        (the reference's per-step ``v_t``, engine.py:659-661); for parity checks."""
        return self._run(observation, noise, trace=True)

    def _run(self, observation, noise, trace: bool):
        obs = Observation.from_dict(observation) if isinstance(observation, dict) else observation
        pad = obs.prefix_pad_masks
        if obs.prefix_k is None and obs.prefix_embs is None and obs.images is not None:
            _, pad, kv = self._build_prefix_cache(obs.images, obs.image_masks, obs.tokenized_prompt,
                                                  obs.tokenized_prompt_mask)
            ks = [k for k, _ in kv]
            vs = [v for _, v in kv]
        elif obs.prefix_k is None:
            if obs.prefix_embs is None or self.prefix_lm is None:
                raise ValueError("the observation has no prefix KV cache; prefix embeddings need an attached PrefixLM")
            _, pad, kv = self.prefix_lm.build_prefix_cache(obs.prefix_embs, pad)
            ks = [k for k, _ in kv]
            vs = [v for _, v in kv]
        else:
            ks = _split_layers(obs.prefix_k, self.geometry.depth)
            vs = _split_layers(obs.prefix_v, self.geometry.depth)
        bsize, plen = pad.shape
        device = self.device
        cfg = self.config
        if noise is None:
            noise = self.sample_noise((bsize, cfg.action_horizon, cfg.action_dim), device)
        x = noise.to(device=device, dtype=torch.float32).clone().contiguous()
        ctx = self._context(bsize, plen, cfg.num_steps)
        ctx.prime_prefix(ks, vs, pad.to(device))
        tr = None
        if trace:
            tr = torch.empty((cfg.num_steps, bsize, cfg.action_horizon, cfg.action_dim), dtype=torch.float32, device=device)
        ctx.denoise(x, tr)
        self._pending_ctx = ctx
        # the reference's per-step draws (engine.py:391-397, 399-403): discarded, generator only
        for _ in range(cfg.num_steps):
            self.sample_noise(x.shape, device)
        return x, tr

    def _raise_pending_error(self) -> None:
        """Raise ``Pi05Error`` (PI05_E_HIP) if the last predict's launch failed; the caller has just
        waited for the GPU (a device-to-host copy), so the status read adds no wait."""
        ctx, self._pending_ctx = self._pending_ctx, None
        if ctx is not None and ctx.handle is not None:
            ctx.status()

    def set_schedule(self, name: Optional[str]) -> None:
        """Execution schedule of the denoise loop: ``"persistent"`` (the whole loop is one
        cooperative kernel) or ``"graph"`` (one hipGraph of per-layer kernels); None restores the
        library default.  Applies to existing contexts too (each predict primes its prefix)."""
        if name is not None and name not in _ext.SCHEDULES:
            raise ValueError(f"schedule must be one of {sorted(_ext.SCHEDULES)} or None, got {name!r}")
        self.schedule = name
        if name is not None:
            for c in self._contexts.values():
                c.set_schedule(name)

    def capture_cuda_graph(self, train_batch_size: int, eval_batch_size: int):
        """Request graph execution (engine.py:831-860).  The engine already runs its whole Euler
        loop as one launch: one cooperative kernel (the persistent schedule), or, in the graph
        schedule, a hipGraph of per-layer kernels captured lazily per (B, P, num_steps) signature.
        A caller may also capture ``sample_actions`` itself (``torch.cuda.graph``) in the
        persistent schedule and replay it: the launch carries no per-call state.  The graph
        schedule refuses capture (``Pi05Error`` PI05_E_STATE), its loop being a hipGraph already."""
        self.cuda_graph_manager = {"eval_batch_size": eval_batch_size}

    def is_cuda_graph_enabled(self) -> bool:
        return self.cuda_graph_manager is not None

    def release_cuda_graph(self):
        for c in self._contexts.values():
            c.release_graph()
        self.cuda_graph_manager = None

    def enable_torch_compile(self, mode: str = "max-autotune"):
        """Compatibility shim: the denoise path is hand-written HIP, so there is nothing to compile."""
        self.torch_compile_enabled = True
        self._torch_compile_mode = mode

    def invalidate_weight_derived_caches(self):
        """Re-pack weights and rebuild the adaRMS table in place after an in-place weight update
        (engine.py:526-554); device addresses stay stable, so captured graphs stay valid."""
        for key, ctx in self._contexts.items():
            ctx.refresh_weights()
        self._stale_contexts.clear()

    def setup_wrappers(self, transforms: Sequence = (), output_transforms: Sequence = ()) -> None:
        """Install the per-sample input and output transforms (engine.py:217-223).  The output
        transforms run in ``output_transform``; the input transforms (openpi's image and prompt
        preprocessing) are kept for the caller but not applied here: observations reach this engine
        already preprocessed."""
        self._input_transforms = list(transforms)
        self._output_transform = _transforms.compose(output_transforms)

    def output_transform(self, outputs: dict) -> dict:
        """Model-space outputs -> env-space outputs (engine.py:269-283): the installed output
        transforms (Unnormalize with the checkpoint's norm stats, the policy's Outputs slice to the
        env action dims), applied on the host like the reference, then the first ``action_chunk``
        actions."""
        host = {k: (v.detach().cpu() if isinstance(v, torch.Tensor) else v) for k, v in outputs.items()}
        self._raise_pending_error()
        out = self._output_transform(host)
        out["actions"] = out["actions"][:, : self.config.action_chunk]
        return out

    def predict_action_batch(self, env_obs, **kwargs) -> torch.Tensor:
        """Observation -> env-space actions ``[B, action_chunk, env action dims]`` (engine.py:321-342).

        The reference first turns raw environment observations into the model's ``Observation``
        (openpi image transforms and prompt tokenisation, engine.py:225-268, 284-319); here the
        observation arrives in that preprocessed form (prefix cache, prefix embeddings, or images
        and tokenized prompt), and the rest is the reference's: ``sample_actions``, then
        ``output_transform({"actions", "state"})``."""
        obs = Observation.from_dict(env_obs) if isinstance(env_obs, dict) else env_obs
        outputs = self.sample_actions(obs, kwargs.get("noise"))
        return self.output_transform({"actions": outputs["actions"], "state": obs.state})["actions"]

    def close(self) -> None:
        self._pending_ctx = None
        self._drop_contexts()
        if self.prefix_lm is not None:
            self.prefix_lm.close()
        if self.vision_tower is not None:
            self.vision_tower.close()


Engine = OpenPi0Inference
EngineConfig = OpenPi0InferConfig

__all__ = ["Engine", "EngineConfig", "Observation", "OpenPi0Inference", "OpenPi0InferConfig"]
