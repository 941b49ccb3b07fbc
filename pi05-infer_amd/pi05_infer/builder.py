"""Model construction with the reference's signatures (builder.py:34-151).

``build_model(model_path, config_name, *, data_kwargs=None, **config_overrides)`` returns an
``OpenPi0Inference`` on CPU; the caller moves it with ``.to("cuda")``.  ``model_path`` is either
a checkpoint directory (``*.safetensors``, or ``model_state_dict/full_weights.pt`` /
``actor/model_state_dict/full_weights.pt`` loaded with ``weights_only=True``), or
``"random"`` / ``"random:<seed>"`` / ``None`` for the seeded random-init expert used by the
benchmark (there is no checkpoint download here).  Only the action-expert, time-MLP and action
projection tensors are read; the prefix towers are not part of this engine.
"""

from __future__ import annotations

import glob
import os
from typing import Any, Optional

import torch

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


def build_model(
    model_path: Optional[str],
    config_name: str,
    *,
    data_kwargs: Optional[dict] = None,
    geometry: ExpertGeometry = ExpertGeometry(),
    **config_overrides: Any,
) -> OpenPi0Inference:
    """Construct a ready-to-run inference engine (builder.py:34-138)."""
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
    return model


def get_model(cfg, torch_dtype=None) -> OpenPi0Inference:
    """omegaconf-shaped shim with the reference's signature (builder.py:141-151)."""
    openpi_cfg = dict(cfg.openpi) if getattr(cfg, "openpi", None) is not None else {}
    config_name = openpi_cfg.pop("config_name", None)
    data_kwargs = getattr(cfg, "openpi_data", None)
    return build_model(model_path=cfg.model_path, config_name=config_name, data_kwargs=data_kwargs, **openpi_cfg)
