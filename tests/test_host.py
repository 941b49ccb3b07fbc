"""Host-side logic that runs without a GPU: the builder, the engine's Python surface, the dtype
policy and the synthetic-input recipe."""

from dataclasses import replace

import pytest
import torch

from pi05_infer import synthetic as S
from pi05_infer.builder import build_model, get_model
from pi05_infer.engine import Observation, OpenPi0InferConfig, OpenPi0Inference

SMALL = replace(S.ExpertGeometry(), width=64, depth=2, head_dim=16, mlp_dim=128)


def test_build_model_random_init_and_dtype_policy():
    m = build_model("random:0", "pi05_libero", geometry=SMALL, num_steps=4)
    assert m.config.num_steps == 4 and m.config.config_name == "pi05_libero"
    for name, t in m.state_dict().items():
        is_expert_linear = any(k in name for k in ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj"))
        assert t.dtype == (torch.bfloat16 if is_expert_linear else torch.float32), name
    assert len(m.state_dict()) == len(S.parameter_specs(SMALL))


@pytest.mark.parametrize(
    "args,exc",
    [
        (("random", "pi0_libero"), NotImplementedError),
        (("random", "no_such_config"), ValueError),
    ],
)
def test_build_model_rejects_unsupported_configs(args, exc):
    with pytest.raises(exc):
        build_model(*args, geometry=SMALL)


def test_build_model_rejects_unknown_overrides():
    with pytest.raises(TypeError):
        build_model("random", "pi05_libero", geometry=SMALL, no_such_field=1)


def test_get_model_shim():
    class Cfg:
        model_path = "random:3"
        openpi = {"config_name": "pi05_turtle", "num_steps": 5}
        openpi_data = None

    m = get_model(Cfg())
    assert m.config.config_name == "pi05_turtle" and m.config.num_steps == 5


def test_checkpoint_roundtrip_safetensors(tmp_path):
    import safetensors.torch

    w = S.make_weights(SMALL, seed=5)
    safetensors.torch.save_file({k: v.contiguous() for k, v in w.items()}, str(tmp_path / "model.safetensors"))
    m = build_model(str(tmp_path), "pi05_libero", geometry=SMALL)
    for k, v in w.items():
        assert torch.equal(m.state_dict()[k], v)


def test_checkpoint_full_weights_pt(tmp_path):
    w = S.make_weights(SMALL, seed=6)
    d = tmp_path / "model_state_dict"
    d.mkdir()
    torch.save(w, str(d / "full_weights.pt"))
    m = build_model(str(tmp_path), "pi05_libero", geometry=SMALL)
    assert torch.equal(m.state_dict()["action_in_proj.weight"], w["action_in_proj.weight"])


def test_load_state_dict_checks_shapes_and_reports_missing():
    m = OpenPi0Inference(OpenPi0InferConfig(), SMALL)
    w = S.make_weights(SMALL)
    bad = dict(w)
    bad["action_in_proj.weight"] = torch.zeros(3, 3)
    with pytest.raises(ValueError):
        m.load_state_dict(bad)
    part = {k: v for k, v in w.items() if "layers.1." not in k}
    missing, unexpected = m.load_state_dict({**part, "extra.tensor": torch.zeros(1)})
    assert missing and all("layers.1." in n for n in missing) and unexpected == ["extra.tensor"]
    with pytest.raises(KeyError):
        m.load_state_dict(part, strict=True)


def test_engine_requires_gpu_and_pi05():
    with pytest.raises(NotImplementedError):
        OpenPi0Inference(OpenPi0InferConfig(pi05=False), SMALL)
    m = build_model("random", "pi05_libero", geometry=SMALL)
    k, v = S.make_prefix_kv(SMALL, 8)
    obs = Observation(k, v, S.full_prefix_pad(8))
    with pytest.raises(RuntimeError, match="gfx950"):
        m.sample_actions(obs, S.make_noise(SMALL))


def test_sample_actions_draws_noise_like_the_reference(monkeypatch):
    """The reference draws the initial noise when none is passed (engine.py:350-354) and then one
    sample_noise of the action shape per Euler step, on the eager and the graph path alike
    (engine.py:391-397, 399-403).  With the GPU context stubbed out, the denoise input must be the
    first draw of a seeded generator and the next predict's the (2 + num_steps)-th: 1 + num_steps
    draws per predict without noise, num_steps with it."""
    steps = 4
    m = build_model("random:0", "pi05_libero", geometry=SMALL, num_steps=steps)
    seen = []

    class FakeContext:
        def prime_prefix(self, ks, vs, pad):
            pass

        def denoise(self, x, trace):
            seen.append(x.clone())

    monkeypatch.setattr(m, "_context", lambda *args: FakeContext())
    calls = []
    draw = m.sample_noise
    monkeypatch.setattr(m, "sample_noise", lambda shape, device: calls.append(tuple(shape)) or draw(shape, device))
    k, v = S.make_prefix_kv(SMALL, 8)
    obs = Observation(k, v, S.full_prefix_pad(8))
    shape = (1, SMALL.action_horizon, SMALL.action_dim)
    torch.manual_seed(7)
    m.sample_actions(obs)
    m.sample_actions(obs)
    assert calls == [shape] * (2 * (1 + steps))
    torch.manual_seed(7)
    stream = [torch.normal(0.0, 1.0, size=shape) for _ in range(2 * (1 + steps))]
    assert torch.equal(seen[0], stream[0]) and torch.equal(seen[1], stream[1 + steps])
    calls.clear()
    m.sample_actions(obs, stream[0])
    assert calls == [shape] * steps


def test_observation_from_dynamic_cache_dict():
    k, v = S.make_prefix_kv(SMALL, 8)
    kv = [(k[:, i : i + 1], v[:, i : i + 1]) for i in range(SMALL.depth)]
    obs = Observation.from_dict({"past_key_values": kv, "prefix_pad_masks": S.full_prefix_pad(8)})
    assert len(obs.prefix_k) == SMALL.depth and torch.equal(obs.prefix_v[1], v[:, 1:2])


def test_observation_from_preprocessed_images_dict():
    """openpi's preprocessed observation: per-view images and masks keep their order."""
    imgs = {"base_0_rgb": torch.zeros(1, 3, 224, 224), "left_wrist_0_rgb": torch.ones(1, 3, 224, 224)}
    masks = {"base_0_rgb": torch.tensor([True]), "left_wrist_0_rgb": torch.tensor([False])}
    obs = Observation.from_dict({"images": imgs, "image_masks": masks, "tokenized_prompt": torch.zeros(1, 4, dtype=torch.long),
                                 "tokenized_prompt_mask": torch.ones(1, 4, dtype=torch.bool)})
    assert obs.prefix_k is None and obs.prefix_embs is None and obs.prefix_pad_masks is None
    assert [float(t.mean()) for t in obs.images] == [0.0, 1.0]
    assert [bool(m[0]) for m in obs.image_masks] == [True, False]


def test_embed_prefix_needs_vision_tower_and_prefix_lm():
    m = build_model("random", "pi05_libero", geometry=SMALL)
    with pytest.raises(ValueError, match="VisionTower and PrefixLM"):
        m.embed_prefix([torch.zeros(1, 3, 224, 224)], [torch.tensor([True])], torch.zeros(1, 4, dtype=torch.long),
                       torch.ones(1, 4, dtype=torch.bool))


def test_vision_tower_weights_and_device_checks():
    from pi05_infer.vision import VisionGeometry, VisionTower, parameter_specs

    g = VisionGeometry(depth=2)
    specs = parameter_specs(g)
    assert len(specs) == 2 * 16 + 7
    fp32 = [n for n, _, dt in specs if dt == torch.float32]
    assert all("embeddings" in n for n in fp32) and len(fp32) == 3  # patch weight/bias, position embedding
    vt = VisionTower(g)
    missing, _ = vt.load_state_dict({})
    assert len(missing) == len(specs)
    with pytest.raises(RuntimeError, match="gfx950"):
        vt.embed_image(torch.zeros(1, 3, 224, 224))
    with pytest.raises(ValueError, match="image must be"):
        vt.embed_image(torch.zeros(1, 3, 112, 112))


def test_build_model_attaches_prefix_towers_from_a_full_checkpoint(tmp_path):
    """A checkpoint with the language model and vision tower comes back with both attached (tiny
    tower geometries; the C ABIs check geometry only when a GPU context is made)."""
    import safetensors.torch

    from pi05_infer import prefix, vision

    pg = prefix.PrefixGeometry(width=32, depth=SMALL.depth, num_heads=2, head_dim=16, mlp_dim=64, vocab_size=50)
    vg = vision.VisionGeometry(width=32, depth=1, num_heads=2, mlp_dim=48, image=28, proj_dim=32)
    sd = {**S.make_weights(SMALL, seed=3), **prefix.make_weights(pg, seed=4, device="cpu"), **vision.make_weights(vg, seed=5, device="cpu")}
    safetensors.torch.save_file({k: v.contiguous() for k, v in sd.items()}, str(tmp_path / "model.safetensors"))
    m = build_model(str(tmp_path), "pi05_libero", geometry=SMALL, prefix_geometry=pg, vision_geometry=vg)
    assert m.prefix_lm is not None and m.vision_tower is not None
    name = prefix.layer_param_names(1)["wq"]
    assert torch.equal(m.prefix_lm.params[name], sd[name].to(torch.bfloat16))
    pw = vision.HEAD_PARAM_NAMES["patch_w"]
    assert m.vision_tower.params[pw].dtype == torch.float32 and torch.equal(m.vision_tower.params[pw], sd[pw])
    expert_only = build_model(str(tmp_path), "pi05_libero", geometry=SMALL, prefix_towers=False)
    assert expert_only.prefix_lm is None and expert_only.vision_tower is None
    assert build_model("random", "pi05_libero", geometry=SMALL).prefix_lm is None


def test_compat_shims():
    m = build_model("random", "pi05_libero", geometry=SMALL)
    assert not m.is_cuda_graph_enabled()
    m.capture_cuda_graph(train_batch_size=1, eval_batch_size=1)
    assert m.is_cuda_graph_enabled()
    m.release_cuda_graph()
    assert not m.is_cuda_graph_enabled()
    m.enable_torch_compile("max-autotune")
    assert m.torch_compile_enabled
    out = m.output_transform({"actions": torch.zeros(2, 50, 32)})
    # the policy's Outputs slice (LiberoOutputs: 7 env action dims) and the action chunk
    assert out["actions"].shape == (2, m.config.action_chunk, 7)


def test_synthetic_recipe_is_deterministic_and_depth_independent():
    a = S.make_weights(SMALL, seed=0)
    b = S.make_weights(replace(SMALL, depth=1), seed=0)
    n0 = S.layer_param_names(0)["wq"]
    assert torch.equal(a[n0], b[n0])
    assert torch.equal(a["action_in_proj.weight"], b["action_in_proj.weight"])
    c = S.make_weights(SMALL, seed=1)
    assert not torch.equal(a[n0], c[n0])
    x = S.make_noise(SMALL, batch=3)
    assert torch.equal(x[1], S.make_noise(SMALL, batch=1, seed=3)[0])
    k1, _ = S.make_prefix_kv(SMALL, 16, batch=2)
    assert k1.dtype == torch.bfloat16 and k1.shape == (2, SMALL.depth, 16, SMALL.head_dim)
    std = a[n0].float().std().item()
    assert 0.018 < std < 0.022
