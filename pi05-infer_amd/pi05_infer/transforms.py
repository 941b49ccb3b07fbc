"""Output transforms of ``predict_action_batch``: model-space actions -> env-space actions.

The reference composes, per sample and on the host (builder.py:118-136, engine.py:269-283):

* the model transforms' outputs (empty for pi0.5);
* openpi's ``Unnormalize(norm_stats, use_quantiles)`` with the checkpoint's norm stats
  (``<checkpoint>/<asset_id>/norm_stats.json``, builder.py:118-121);
* the policy's data-transform outputs: ``AbsoluteActions`` when the data config sets
  ``extra_delta_transform`` (dataconfig/libero_dataconfig.py:85-90), then ``LiberoOutputs``
  (the first 7 action dims, dataconfig/policies/libero_policy.py:105-120) or ``TurtleOutputs``
  (the first 6, dataconfig/policies/turtle_policy.py:21, 89-93);

and the engine then keeps the first ``action_chunk`` actions (engine.py:282).

``Unnormalize``, ``Normalize`` and ``AbsoluteActions`` live in openpi (``openpi.transforms``), which
is not part of the reference tree; they are restated here from openpi's published code.  Their
parity is unpinned: nothing in the reference holds their outputs.  What the tests pin is that
``Unnormalize`` inverts ``Normalize`` (closed form), the padding rules, and the slices the
reference tree itself defines.

Each transform maps a dict of batched tensors ``{"actions": [B, H, a], "state": [B, s]}`` to a
dict; every operation is per sample, so applying it to the batch equals the reference's per-sample
loop.  Norm statistics are float64 (openpi parses the JSON into float64 numpy arrays), so an
unnormalized action tensor is float64, as the reference's ``np.asarray`` recombination returns it.
"""

from __future__ import annotations

import dataclasses
import json
import os
from typing import Callable, Iterable, Optional, Sequence

import torch

Transform = Callable[[dict], dict]

# action dims the policies' Outputs keep (libero_policy.py:120, turtle_policy.py:21)
LIBERO_ACTION_DIM = 7
TURTLE_ACTION_DIM = 6
# asset id of the norm stats the reference's pi0.5 configs load (dataconfig/__init__.py:60-85;
# README.md:83-86: ckpt/physical-intelligence/libero/norm_stats.json)
DEFAULT_ASSET_ID = "physical-intelligence/libero"
NORM_EPS = 1e-6  # openpi's normalisation epsilon


@dataclasses.dataclass(frozen=True)
class NormStats:
    """Per-key statistics of openpi's ``normalize.NormStats``: mean/std and the 1 % / 99 % quantiles."""

    mean: torch.Tensor
    std: torch.Tensor
    q01: Optional[torch.Tensor] = None
    q99: Optional[torch.Tensor] = None


def _f64(v) -> Optional[torch.Tensor]:
    return None if v is None else torch.as_tensor(v, dtype=torch.float64)


def load_norm_stats(path: str) -> dict[str, NormStats]:
    """Read openpi's ``norm_stats.json`` (``{"norm_stats": {key: {"mean", "std", "q01", "q99"}}}``).
    ``path`` is the JSON file or the asset directory holding it."""
    if os.path.isdir(path):
        path = os.path.join(path, "norm_stats.json")
    with open(path) as f:
        raw = json.load(f)
    stats = raw.get("norm_stats", raw)
    return {k: NormStats(_f64(v["mean"]), _f64(v["std"]), _f64(v.get("q01")), _f64(v.get("q99"))) for k, v in stats.items()}


def find_norm_stats(checkpoint_dir: str, asset_id: str = DEFAULT_ASSET_ID) -> Optional[str]:
    """``<checkpoint_dir>/<asset_id>/norm_stats.json`` if it exists (openpi's load_norm_stats layout)."""
    p = os.path.join(checkpoint_dir, asset_id, "norm_stats.json")
    return p if os.path.exists(p) else None


def _pad_last(x: torch.Tensor, n: int, value: float) -> torch.Tensor:
    if x.shape[-1] >= n:
        return x
    return torch.cat([x, torch.full((*x.shape[:-1], n - x.shape[-1]), value, dtype=x.dtype, device=x.device)], dim=-1)


def _apply(data: dict, stats: dict[str, NormStats], fn) -> dict:
    out = dict(data)
    for key, st in stats.items():
        if key in out and out[key] is not None:
            out[key] = fn(out[key], st)
    return out


@dataclasses.dataclass(frozen=True)
class Normalize:
    """openpi ``transforms.Normalize`` (the input-side inverse; used here to pin ``Unnormalize``)."""

    norm_stats: Optional[dict]
    use_quantiles: bool = False

    def __call__(self, data: dict) -> dict:
        if self.norm_stats is None:
            return data
        return _apply(data, self.norm_stats, self._quantile if self.use_quantiles else self._zscore)

    @staticmethod
    def _zscore(x: torch.Tensor, st: NormStats) -> torch.Tensor:
        # statistics wider than x are cut to its width; narrower ones are padded as Unnormalize
        # pads them (mean 0, std 1), so the two are exact inverses
        n = x.shape[-1]
        mean = _pad_last(st.mean.to(x.device), n, 0.0)[..., :n]
        std = _pad_last(st.std.to(x.device), n, 1.0)[..., :n]
        return (x.to(torch.float64) - mean) / (std + NORM_EPS)

    @staticmethod
    def _quantile(x: torch.Tensor, st: NormStats) -> torch.Tensor:
        d = st.q01.shape[-1]
        x = x.to(torch.float64)
        q01, q99 = st.q01.to(x.device), st.q99.to(x.device)
        return torch.cat([(x[..., :d] - q01) / (q99 - q01 + NORM_EPS) * 2.0 - 1.0, x[..., d:]], dim=-1)


@dataclasses.dataclass(frozen=True)
class Unnormalize:
    """openpi ``transforms.Unnormalize``: ``x * (std + 1e-6) + mean`` with mean padded by 0 and std
    by 1 to the action width, or with quantiles ``(x + 1) / 2 * (q99 - q01 + 1e-6) + q01`` on the
    first ``len(q01)`` dims (the rest pass through).  Parity unpinned (openpi is not in the tree)."""

    norm_stats: Optional[dict]
    use_quantiles: bool = False

    def __call__(self, data: dict) -> dict:
        if self.norm_stats is None:
            return data
        return _apply(data, self.norm_stats, self._quantile if self.use_quantiles else self._zscore)

    @staticmethod
    def _zscore(x: torch.Tensor, st: NormStats) -> torch.Tensor:
        n = x.shape[-1]
        mean = _pad_last(st.mean.to(x.device), n, 0.0)
        std = _pad_last(st.std.to(x.device), n, 1.0)
        return x.to(torch.float64) * (std + NORM_EPS) + mean

    @staticmethod
    def _quantile(x: torch.Tensor, st: NormStats) -> torch.Tensor:
        if st.q01 is None or st.q99 is None:
            raise ValueError("quantile unnormalisation needs q01 and q99 in the norm stats")
        d = st.q01.shape[-1]
        x = x.to(torch.float64)
        q01, q99 = st.q01.to(x.device), st.q99.to(x.device)
        if d < x.shape[-1]:
            return torch.cat([(x[..., :d] + 1.0) / 2.0 * (q99 - q01 + NORM_EPS) + q01, x[..., d:]], dim=-1)
        return (x + 1.0) / 2.0 * (q99 - q01 + NORM_EPS) + q01


@dataclasses.dataclass(frozen=True)
class AbsoluteActions:
    """openpi ``transforms.AbsoluteActions``: add the state to the action dims ``mask`` selects
    (delta -> absolute); the reference enables it through ``extra_delta_transform`` with
    ``make_bool_mask(6, -1)`` (libero_dataconfig.py:85-90)."""

    mask: Sequence[bool]

    def __call__(self, data: dict) -> dict:
        if "actions" not in data or data.get("state") is None:
            return data
        out = dict(data)
        actions = data["actions"]
        state = data["state"].to(actions.dtype).to(actions.device)
        m = torch.as_tensor(list(self.mask), dtype=torch.bool, device=actions.device)
        d = m.shape[0]
        add = torch.where(m, state[..., :d], torch.zeros((), dtype=actions.dtype, device=actions.device))
        out["actions"] = torch.cat([actions[..., :d] + add[..., None, :], actions[..., d:]], dim=-1)
        return out


def make_bool_mask(*dims: int) -> tuple[bool, ...]:
    """openpi ``transforms.make_bool_mask``: positive n -> n Trues, negative n -> |n| Falses."""
    out: list[bool] = []
    for d in dims:
        out.extend([d > 0] * abs(d))
    return tuple(out)


@dataclasses.dataclass(frozen=True)
class PolicyOutputs:
    """``LiberoOutputs`` / ``TurtleOutputs``: keep only ``actions[..., :action_dim]`` (the rest of the
    model's 32 dims is padding) and drop every other key (libero_policy.py:120, turtle_policy.py:93)."""

    action_dim: int

    def __call__(self, data: dict) -> dict:
        return {"actions": data["actions"][..., : self.action_dim]}


def compose(transforms: Iterable[Transform]) -> Transform:
    fns = list(transforms)

    def run(data: dict) -> dict:
        for fn in fns:
            data = fn(data)
        return data

    return run


def policy_output_dim(config_name: str) -> int:
    """Action dims the config's policy returns to the environment."""
    if config_name.endswith("turtle"):
        return TURTLE_ACTION_DIM
    return LIBERO_ACTION_DIM


def output_transforms_for(config_name: str, norm_stats: Optional[dict], use_quantiles: bool = True,
                          extra_delta_transform: bool = False) -> list[Transform]:
    """The output transform list ``build_model`` hands to ``setup_wrappers`` (builder.py:130-135):
    Unnormalize, then the data transforms' outputs.  pi0.5 configs normalise with quantiles (openpi
    sets ``use_quantile_norm`` for every model type except pi0; parity unpinned)."""
    fns: list[Transform] = []
    if norm_stats is not None:
        fns.append(Unnormalize(norm_stats, use_quantiles=use_quantiles))
    if extra_delta_transform:
        fns.append(AbsoluteActions(make_bool_mask(6, -1)))
    fns.append(PolicyOutputs(policy_output_dim(config_name)))
    return fns
