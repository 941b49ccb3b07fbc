"""Output transforms of predict_action_batch (pi05_infer/transforms.py), on the CPU.

The policy Outputs slices are the reference's own (libero_policy.py:105-120,
turtle_policy.py:21, 89-93).  Unnormalize / Normalize / AbsoluteActions restate openpi, which the
reference tree does not contain: their parity is unpinned; these tests pin that Unnormalize is the
exact inverse of Normalize (closed form), the padding rules, and the composition order of
builder.py:130-135.
"""

import json

import pytest
import torch

from pi05_infer import transforms as T
from pi05_infer.engine import OpenPi0InferConfig, OpenPi0Inference


def _stats(d=7, seed=0):
    g = torch.Generator().manual_seed(seed)
    mean = torch.randn(d, generator=g, dtype=torch.float64)
    std = torch.rand(d, generator=g, dtype=torch.float64) + 0.1
    q01 = mean - 2 * std
    q99 = mean + 2 * std
    return {"actions": T.NormStats(mean, std, q01, q99), "state": T.NormStats(mean[:8] if d >= 8 else mean, std[:8] if d >= 8 else std, q01, q99)}


def _write(tmp_path, stats, asset="physical-intelligence/libero"):
    d = tmp_path / asset
    d.mkdir(parents=True)
    raw = {"norm_stats": {k: {"mean": v.mean.tolist(), "std": v.std.tolist(), "q01": v.q01.tolist(), "q99": v.q99.tolist()}
                          for k, v in stats.items()}}
    (d / "norm_stats.json").write_text(json.dumps(raw))
    return d


def test_load_norm_stats_roundtrip(tmp_path):
    st = _stats()
    d = _write(tmp_path, st)
    got = T.load_norm_stats(str(d))
    assert set(got) == {"actions", "state"}
    for k in got:
        for f in ("mean", "std", "q01", "q99"):
            assert getattr(got[k], f).dtype == torch.float64
            assert torch.equal(getattr(got[k], f), getattr(st[k], f))
    assert T.find_norm_stats(str(tmp_path)) == str(d / "norm_stats.json")
    assert T.find_norm_stats(str(tmp_path), "other/asset") is None


@pytest.mark.parametrize("quantiles", [False, True])
def test_unnormalize_inverts_normalize(quantiles):
    st = _stats(7)
    x = torch.randn(3, 50, 32, dtype=torch.float32)
    data = {"actions": x.clone(), "state": torch.randn(3, 8)}
    norm = T.Normalize({"actions": st["actions"]}, use_quantiles=quantiles)
    unnorm = T.Unnormalize({"actions": st["actions"]}, use_quantiles=quantiles)
    back = unnorm(norm(data))["actions"]
    assert back.dtype == torch.float64
    torch.testing.assert_close(back, x.double(), rtol=0, atol=1e-9)


def test_unnormalize_closed_forms_and_padding():
    st = _stats(7)["actions"]
    x = torch.linspace(-1.5, 1.5, 2 * 5 * 32, dtype=torch.float32).reshape(2, 5, 32)
    # quantiles: only the first len(q01) dims are mapped, [-1, 1] -> [q01, q99]
    q = T.Unnormalize({"actions": st}, use_quantiles=True)({"actions": x})["actions"]
    ref = (x[..., :7].double() + 1) / 2 * (st.q99 - st.q01 + 1e-6) + st.q01
    torch.testing.assert_close(q[..., :7], ref, rtol=0, atol=0)
    assert torch.equal(q[..., 7:], x[..., 7:].double())
    lo = T.Unnormalize({"actions": st}, use_quantiles=True)({"actions": -torch.ones(1, 1, 7)})["actions"][0, 0]
    torch.testing.assert_close(lo, st.q01, rtol=0, atol=1e-12)
    # mean/std: mean padded with 0 and std with 1 past the stats' width
    z = T.Unnormalize({"actions": st}, use_quantiles=False)({"actions": x})["actions"]
    torch.testing.assert_close(z[..., :7], x[..., :7].double() * (st.std + 1e-6) + st.mean, rtol=0, atol=0)
    torch.testing.assert_close(z[..., 7:], x[..., 7:].double() * (1 + 1e-6), rtol=0, atol=0)
    # no stats: identity
    assert T.Unnormalize(None)({"actions": x})["actions"] is x


def test_absolute_actions_adds_state_to_masked_dims():
    mask = T.make_bool_mask(6, -1)
    assert mask == (True,) * 6 + (False,)
    actions = torch.randn(2, 5, 32, dtype=torch.float64)
    state = torch.randn(2, 8, dtype=torch.float64)
    out = T.AbsoluteActions(mask)({"actions": actions, "state": state})["actions"]
    torch.testing.assert_close(out[..., :6], actions[..., :6] + state[:, None, :6], rtol=0, atol=0)
    assert torch.equal(out[..., 6:], actions[..., 6:])


@pytest.mark.parametrize("config_name,dim", [("pi05_libero", 7), ("pi05_turtle", 6)])
def test_policy_outputs_slice_and_composition_order(config_name, dim):
    st = _stats(7)
    fns = T.output_transforms_for(config_name, st, use_quantiles=True)
    assert isinstance(fns[0], T.Unnormalize) and isinstance(fns[-1], T.PolicyOutputs)
    x = torch.rand(4, 50, 32) * 2 - 1
    out = T.compose(fns)({"actions": x, "state": torch.zeros(4, 8)})
    assert set(out) == {"actions"} and out["actions"].shape == (4, 50, dim)
    # Unnormalize first, then the slice: the kept dims are the unnormalized ones
    ref = (x[..., :dim].double() + 1) / 2 * (st["actions"].q99[:dim] - st["actions"].q01[:dim] + 1e-6) + st["actions"].q01[:dim]
    torch.testing.assert_close(out["actions"], ref, rtol=0, atol=0)


def test_engine_output_transform_env_space_and_chunk(tmp_path):
    cfg = OpenPi0InferConfig(config_name="pi05_libero", action_chunk=5)
    model = OpenPi0Inference(cfg)
    x = torch.rand(3, 50, 32) * 2 - 1
    # default (no norm stats installed): the policy slice and the chunk
    out = model.output_transform({"actions": x, "state": None})["actions"]
    assert out.shape == (3, 5, 7) and torch.equal(out, x[:, :5, :7])
    # with the checkpoint's norm stats, as build_model installs them
    st = _stats(7)
    model.setup_wrappers(output_transforms=T.output_transforms_for("pi05_libero", st))
    out = model.output_transform({"actions": x, "state": torch.zeros(3, 8)})["actions"]
    assert out.shape == (3, 5, 7) and out.dtype == torch.float64
    ref = (x[:, :5, :7].double() + 1) / 2 * (st["actions"].q99 - st["actions"].q01 + 1e-6) + st["actions"].q01
    torch.testing.assert_close(out, ref, rtol=0, atol=0)


def test_builder_installs_norm_stats_from_data_kwargs(tmp_path):
    from pi05_infer import builder

    st = _stats(7)
    d = _write(tmp_path, st)
    fns = builder._output_transforms("pi05_turtle", None, {"norm_stats_path": str(d)})
    assert isinstance(fns[0], T.Unnormalize) and fns[0].use_quantiles
    assert torch.equal(fns[0].norm_stats["actions"].q99, st["actions"].q99)
    assert fns[-1].action_dim == 6
    # checkpoint layout <ckpt>/<asset_id>/norm_stats.json
    fns = builder._output_transforms("pi05_libero", str(tmp_path), None)
    assert isinstance(fns[0], T.Unnormalize) and fns[-1].action_dim == 7
    # random init: no stats, slice only
    fns = builder._output_transforms("pi05_libero", None, None)
    assert len(fns) == 1 and fns[0].action_dim == 7
