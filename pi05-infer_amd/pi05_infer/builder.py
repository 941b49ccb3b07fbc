"""Model construction with the reference's signatures (builder.py:34-151).

``build_model(model_path, config_name, *, data_kwargs=None, **config_overrides)`` returns an
``OpenPi0Inference`` on CPU; the caller moves it with ``.to("cuda")``.  ``model_path`` is either
a checkpoint directory (``*.safetensors``, or ``model_state_dict/full_weights.pt`` /
``actor/model_state_dict/full_weights.pt`` loaded with ``weights_only=True``), or
``"random"`` / ``"random:<seed>"`` / ``None`` for the seeded random-init expert used by the
benchmark (there is no checkpoint download here).  A checkpoint that also holds PaliGemma's
language model and vision tower gets them as an attached ``PrefixLM`` and ``VisionTower``, so
``sample_actions`` runs from camera images and a tokenized prompt, as the reference's model does;
``prefix_towers=True`` forces that (random-init towers for ``"random"``), ``False`` skips it.
"""

from __future__ import annotations

import glob
import os
from typing import Any, Optional

import torch

from . import transforms
from .engine import OpenPi0InferConfig, OpenPi0Inference
from .synthetic import ExpertGeometry, make_weights

# pi0.5 TrainConfigs the reference ships (dataconfig/__init__.py:43-94); pi0_libero is a pi0 model.
_PI05_CONFIGS = {"pi05_libero", "pi05_turtle"}
_PI0_CONFIGS = {"pi0_libero"}


def _parse_random(model_path: Optional[str]) -> Optional[int]:
    if model_path is None or model_path == "random":
        return 0
    if isinstance(model_path, str) and model_path.startswith("random:"):
        return int(model_path.split(":", 1)[1])
    return None


def _load_checkpoint(checkpoint_dir: str) -> dict[str, torch.Tensor]:
    full = os.path.join(checkpoint_dir, "model_state_dict", "full_weights.pt")
    actor_full = os.path.join(checkpoint_dir, "actor", "model_state_dict", "full_weights.pt")
    for path in (full, actor_full):
        if os.path.exists(path):
            return torch.load(path, map_location="cpu", weights_only=True)
    import safetensors.torch

    paths = sorted(glob.glob(os.path.join(checkpoint_dir, "*.safetensors")))
    if not paths:
        raise FileNotFoundError(f"no safetensors or full_weights.pt under {checkpoint_dir}")
    sd: dict[str, torch.Tensor] = {}
    for p in paths:
        sd.update(safetensors.torch.load_file(p, device="cpu"))
    return sd


def _output_transforms(config_name: str, checkpoint_dir: Optional[str], data_kwargs: Optional[dict]) -> list:
    """Unnormalize with the checkpoint's norm stats (``<checkpoint>/<asset_id>/norm_stats.json``,
    builder.py:118-121) and the policy's Outputs (builder.py:130-135).  ``data_kwargs`` may name
    ``norm_stats_path`` (a JSON file or asset directory), ``asset_id``, ``use_quantile_norm`` and
    ``extra_delta_transform``."""
    kw = dict(data_kwargs or {})
    path = kw.get("norm_stats_path")
    if path is None and checkpoint_dir is not None:
        path = transforms.find_norm_stats(checkpoint_dir, kw.get("asset_id", transforms.DEFAULT_ASSET_ID))
    stats = transforms.load_norm_stats(path) if path is not None else None
    return transforms.output_transforms_for(config_name, stats, use_quantiles=bool(kw.get("use_quantile_norm", True)),
                                            extra_delta_transform=bool(kw.get("extra_delta_transform", False)))


def build_model(
    model_path: Optional[str],
    config_name: str,
    *,
    data_kwargs: Optional[dict] = None,
    geometry: ExpertGeometry = ExpertGeometry(),
    prefix_towers: Optional[bool] = None,
    prefix_geometry=None,
    vision_geometry=None,
    **config_overrides: Any,
) -> OpenPi0Inference:
    """Construct a ready-to-run inference engine (builder.py:34-138).  ``prefix_geometry`` /
    ``vision_geometry`` default to Gemma-2B and SigLIP So400m/14."""
    if config_name in _PI0_CONFIGS:
        raise NotImplementedError(f"{config_name} is a pi0 config; this engine implements pi0.5 only")
    if config_name not in _PI05_CONFIGS:
        raise ValueError(f"unknown config_name {config_name!r}; expected one of {sorted(_PI05_CONFIGS)}")
    fields = {f for f in OpenPi0InferConfig.__dataclass_fields__}
    unknown = set(config_overrides) - fields
    if unknown:
        raise TypeError(f"unknown config overrides: {sorted(unknown)}")
    config = OpenPi0InferConfig(config_name=config_name, **config_overrides)
    model = OpenPi0Inference(config, geometry)
    seed = _parse_random(model_path)
    state = make_weights(geometry, seed=seed) if seed is not None else _load_checkpoint(str(model_path))
    missing, _ = model.load_state_dict(state, strict=False)
    if missing:
        raise KeyError(f"checkpoint lacks {len(missing)} expert tensors, e.g. {missing[:3]}")
    model.setup_wrappers(output_transforms=_output_transforms(config_name, None if seed is not None else str(model_path), data_kwargs))
    from . import prefix, vision

    if prefix_towers is None:
        prefix_towers = seed is None and any(k.startswith(prefix.PREFIX) for k in state)
    if prefix_towers:
        pg = prefix_geometry or prefix.PrefixGeometry(depth=geometry.depth)
        vg = vision_geometry or vision.VisionGeometry()
        plm, vt = prefix.PrefixLM(pg), vision.VisionTower(vg)
        if seed is not None:
            tower_state = {**prefix.make_weights(pg, seed=seed + 1, device="cpu"), **vision.make_weights(vg, seed=seed + 2, device="cpu")}
        else:
            tower_state = state
        for name, module in (("prefix LM", plm), ("vision tower", vt)):
            tmissing, _ = module.load_state_dict(tower_state, strict=False)
            if tmissing:
                raise KeyError(f"checkpoint lacks {len(tmissing)} {name} tensors, e.g. {tmissing[:3]}")
        model.attach_prefix_lm(plm)
        model.attach_vision_tower(vt)
    return model


def get_model(cfg, torch_dtype=None) -> OpenPi0Inference:
    """omegaconf-shaped shim with the reference's signature (builder.py:141-151)."""
    openpi_cfg = dict(cfg.openpi) if getattr(cfg, "openpi", None) is not None else {}
    config_name = openpi_cfg.pop("config_name", None)
    data_kwargs = getattr(cfg, "openpi_data", None)
    return build_model(model_path=cfg.model_path, config_name=config_name, data_kwargs=data_kwargs, **openpi_cfg)
