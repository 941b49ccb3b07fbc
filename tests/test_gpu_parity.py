"""GPU parity of the gfx950 denoise engine against the CPU oracle, through the C ABI.

Tolerance (the path is bf16 on the GPU, fp32 with bf16 rounding points in the oracle): for every
per-step velocity and for the final actions, cosine similarity >= 0.9999 and max-abs error
<= 2e-2 of the oracle's range of that tensor.  Integer work (RoPE positions, key masks) is read
back through pi05_get_step_invariants and compared bit-exactly with the oracle's
position_ids / attention_mask_4d (test_step_invariants_bit_exact).
"""

from dataclasses import replace

import pytest
import torch

from oracle import denoise_oracle as O
from pi05_infer import synthetic as S
from pi05_infer.engine import Observation, OpenPi0InferConfig, OpenPi0Inference, _split_layers

pytestmark = pytest.mark.gpu

COS_MIN = 0.9999
REL_MAXABS = 2e-2


def _close(ref: torch.Tensor, got: torch.Tensor, what: str) -> None:
    ref = ref.double().flatten().cpu()
    got = got.double().flatten().cpu()
    assert torch.isfinite(got).all(), f"{what}: non-finite values"
    cos = torch.nn.functional.cosine_similarity(ref, got, dim=0).item()
    maxabs = (ref - got).abs().max().item()
    rng = (ref.max() - ref.min()).item()
    print(f"{what}: cos={cos:.7f} maxabs={maxabs:.3e} range={rng:.3f}", flush=True)
    assert cos >= COS_MIN, f"{what}: cosine {cos} < {COS_MIN}"
    assert maxabs <= REL_MAXABS * rng, f"{what}: max-abs {maxabs} > {REL_MAXABS} * range {rng}"


@pytest.fixture(scope="module")
def full_weights():
    return S.make_weights(S.ExpertGeometry())


SCHEDULES = ("persistent", "graph")


def _run_case(weights, depth=18, P=968, B=1, steps=10, pad_fn=None, zero_gate=False, schedules=SCHEDULES):
    """Oracle once, then the engine under each schedule; returns results per schedule."""
    g = replace(S.ExpertGeometry(), depth=depth)
    w = {k: v for k, v in weights.items() if ".layers." not in k or int(k.split(".layers.")[1].split(".")[0]) < depth}
    if zero_gate:
        w = S.zero_gate_weights(w, g)
    k, v = S.make_prefix_kv(g, P, B)
    x1 = S.make_noise(g, B)
    pad = S.full_prefix_pad(P, B)
    if pad_fn is not None:
        pad_fn(pad)
    og = O.geometry_from(g)
    table = O.adarms_table(w, og, steps)
    act_ref, vs_ref = O.sample_actions(w, og, k, v, pad, x1, steps, table)
    model = OpenPi0Inference(OpenPi0InferConfig(num_steps=steps), g)
    model.load_state_dict(w)
    model.to("cuda")
    obs = Observation(k.cuda(), v.cuda(), pad.cuda())
    got = {}
    for sched in schedules:
        print(f"  schedule {sched}", flush=True)
        model.set_schedule(sched)
        act, vs = model.sample_actions_with_velocities(obs, x1.cuda())
        torch.cuda.synchronize()
        got[sched] = (act, vs)
    return model, obs, x1, table, (act_ref, vs_ref), got


def _check(name, ref, got, steps):
    act_ref, vs_ref = ref
    for sched, (act, vs) in got.items():
        for s in range(steps):
            _close(vs_ref[s], vs[s], f"{name} [{sched}] step {s} velocity")
        _close(act_ref, act, f"{name} [{sched}] actions")


def test_c1_full_parity_and_table(full_weights):
    print("case C1: depth 18, B=1, P=968, 10 steps", flush=True)
    model, obs, x1, table, ref, got = _run_case(full_weights)
    _check("C1", ref, got, 10)
    ctx = next(iter(model._contexts.values()))
    tab = ctx.adarms_table().cpu()
    torch.testing.assert_close(tab, table, rtol=1e-5, atol=1e-5)
    # every schedule is deterministic and does not drift between predicts; a predict with other
    # noise in between must not leave anything behind that a later predict reads
    for sched in SCHEDULES:
        model.set_schedule(sched)
        first = model.sample_actions(obs, x1.cuda())["actions"].clone()
        assert torch.equal(first, got[sched][0]), sched
        other = model.sample_actions(obs, (x1 * -0.5).cuda())["actions"].clone()
        assert not torch.equal(other, first)
        again = model.sample_actions(obs, x1.cuda())["actions"]
        assert torch.equal(again, first), sched
    model.close()


def test_c2_short_prefix(full_weights):
    print("case C2: depth 18, B=1, P=456", flush=True)
    model, _, _, _, ref, got = _run_case(full_weights, P=456)
    _check("C2", ref, got, 10)
    model.close()


def test_c4_long_prefix(full_weights):
    print("case C4: depth 18, B=1, P=3272", flush=True)
    model, _, _, _, ref, got = _run_case(full_weights, P=3272)
    _check("C4", ref, got, 10)
    model.close()


def test_c3_batch8(full_weights):
    print("case C3: depth 18, B=8, P=968 (M = 400 rows per GEMM)", flush=True)
    model, _, _, _, ref, got = _run_case(full_weights, B=8)
    _check("C3", ref, got, 10)
    model.close()


def test_batch2_pair_items(full_weights):
    """B=2: the two-sample kernel instance -- one 32-key block per wave in the attention splits and
    the qkv / gate_up / down_proj pair items over sample halves of 1 (gate_up's K split over the four
    waves)."""
    print("case B=2: depth 3, B=2, P=200, 2 steps", flush=True)
    model, _, _, _, ref, got = _run_case(full_weights, depth=3, P=200, B=2, steps=2)
    _check("B=2", ref, got, 2)
    model.close()


def test_batch5_batch_paths(full_weights):
    """B=5: the batched kernel at an odd batch -- grouped attention items (4 row blocks of a sample
    sharing each K/V block; 7 key splits), gate_up split by rows (waves 0..3 take samples 0..3, wave
    0 also sample 4) and the qkv / down_proj pair items over sample halves of 3 and 2."""
    print("case B=5: depth 4, B=5, P=968, 3 steps", flush=True)
    model, _, _, _, ref, got = _run_case(full_weights, depth=4, B=5, steps=3)
    _check("B=5", ref, got, 3)
    model.close()


def test_batch16_multi_pass_items(full_weights):
    """B=16: the GEMM phases' per-workgroup loops run more than once -- gate_up rows four samples
    per wave, qkv thirds of six samples (two per wave for two waves), down_proj halves of eight (two
    per wave), o_proj's wave pairs eight iterations -- with a ragged prefix.  The grouped attention
    has two key splits here, 224 items that fill the grid once (test_batch40_grouped_items_wrap
    covers items that wrap around it)."""
    print("case B=16: depth 2, B=16, P=100, 2 steps", flush=True)

    def pad_fn(pad):
        pad[3, 90:] = False
        pad[11, 0:7] = False

    model, _, _, _, ref, got = _run_case(full_weights, depth=2, P=100, B=16, steps=2, pad_fn=pad_fn, schedules=("persistent",))
    _check("B=16", ref, got, 2)
    model.close()


def test_batch40_grouped_items_wrap(full_weights):
    """B=40: 7 x 40 = 280 grouped attention items (one key split) on 256 workgroups, so workgroups
    0..23 take a second item and restage their LDS K/V ring for it; every other per-workgroup loop
    also runs many passes."""
    print("case B=40: depth 2, B=40, P=64, 2 steps", flush=True)

    def pad_fn(pad):
        pad[7, 50:] = False
        pad[33, 0:5] = False

    model, _, _, _, ref, got = _run_case(full_weights, depth=2, P=64, B=40, steps=2, pad_fn=pad_fn, schedules=("persistent",))
    _check("B=40", ref, got, 2)
    model.close()


def test_ragged_prefix_padding(full_weights):
    """B=3: the grouped attention items (12 key splits at this prefix) with the row-split gate_up
    (three waves one sample each, the fourth idle) and o_proj (one sample per item)."""
    print("case ragged: depth 4, B=3, P=300, padded tails", flush=True)

    def pad_fn(pad):
        pad[0, 280:] = False
        pad[1, 100:] = False
        pad[2, 5:17] = False

    model, _, _, _, ref, got = _run_case(full_weights, depth=4, P=300, B=3, steps=3, pad_fn=pad_fn)
    _check("ragged", ref, got, 3)
    model.close()


def test_ragged_grouped_attention(full_weights):
    """B=4 (grouped attention: each 32-key block and its key-valid bytes staged through LDS) with
    padded tails, an interior hole and a sample whose valid keys end inside a block."""
    print("case ragged grouped: depth 3, B=4, P=300, padded tails and a hole", flush=True)

    def pad_fn(pad):
        pad[0, 281:] = False
        pad[1, 40:77] = False
        pad[2, 130:] = False
        pad[3, 0:3] = False

    model, _, _, _, ref, got = _run_case(full_weights, depth=3, P=300, B=4, steps=2, pad_fn=pad_fn)
    _check("ragged grouped", ref, got, 2)
    model.close()


def test_tiny_prefix_and_odd_steps(full_weights):
    print("case tiny: depth 2, B=1, P=1, 7 steps", flush=True)
    model, _, _, _, ref, got = _run_case(full_weights, depth=2, P=1, steps=7)
    _check("tiny", ref, got, 7)
    model.close()


def test_zero_gates_identity_layers(full_weights):
    print("case zero-gate: depth 3, P=64", flush=True)
    model, _, _, _, ref, got = _run_case(full_weights, depth=3, P=64, steps=2, zero_gate=True)
    _check("zero-gate", ref, got, 2)
    model.close()


def test_weight_refresh_in_place(full_weights):
    print("case refresh: depth 2, P=128, weights updated in place", flush=True)
    g = replace(S.ExpertGeometry(), depth=2)
    w = {k: v for k, v in full_weights.items() if ".layers." not in k or int(k.split(".layers.")[1].split(".")[0]) < 2}
    k, v = S.make_prefix_kv(g, 128)
    x1 = S.make_noise(g)
    pad = S.full_prefix_pad(128)
    model = OpenPi0Inference(OpenPi0InferConfig(num_steps=3), g)
    model.load_state_dict(w)
    model.to("cuda")
    obs = Observation(k.cuda(), v.cuda(), pad.cuda())
    first = model.sample_actions(obs, x1.cuda())["actions"].clone()
    # RL-style weight sync: scale one layer's down_proj and the time MLP in place
    name = S.layer_param_names(1)["wdown"]
    model.params[name].mul_(1.5)
    model.params["time_mlp_out.weight"].mul_(0.5)
    model.invalidate_weight_derived_caches()
    w2 = dict(w)
    w2[name] = (w[name].float() * 1.5).to(torch.bfloat16)
    w2["time_mlp_out.weight"] = w["time_mlp_out.weight"] * 0.5
    og = O.geometry_from(g)
    ref, _ = O.sample_actions(w2, og, k, v, pad, x1, 3)
    for sched in SCHEDULES:
        model.set_schedule(sched)
        second = model.sample_actions(obs, x1.cuda())["actions"]
        assert not torch.equal(first, second)
        _close(ref, second, f"refresh actions [{sched}]")
    model.close()


def test_bad_prefix_shapes_rejected(full_weights):
    from pi05_infer import _ext

    g = replace(S.ExpertGeometry(), depth=2)
    w = {k: v for k, v in full_weights.items() if ".layers." not in k or int(k.split(".layers.")[1].split(".")[0]) < 2}
    model = OpenPi0Inference(OpenPi0InferConfig(num_steps=2), g)
    model.load_state_dict(w)
    model.to("cuda")
    k, v = S.make_prefix_kv(g, 32)
    pad = S.full_prefix_pad(32).cuda()
    ctx = model._context(1, 32, 2)
    with pytest.raises(ValueError):
        ctx.prime_prefix([k[:, i : i + 1, :16].cuda() for i in range(2)], [v[:, i : i + 1].cuda() for i in range(2)], pad)
    with pytest.raises(ValueError):
        ctx.prime_prefix([k[:, i : i + 1].cuda() for i in range(1)], [v[:, i : i + 1].cuda() for i in range(1)], pad)
    with pytest.raises(ValueError):
        ctx.denoise(torch.zeros(1, 50, 16, device="cuda"))
    bad = _ext.make_dims(g, 1, 32, 2)
    bad.head_dim = 128
    with pytest.raises(_ext.Pi05Error):
        _ext.check_dims(bad)
    with pytest.raises(_ext.Pi05Error):
        ctx._call(ctx.lib.pi05_set_schedule(ctx.handle, 7))
    # switching schedule drops the primed prefix: denoise must refuse until primed again
    other = "graph" if ctx.schedule == "persistent" else "persistent"
    ctx.set_schedule(other)
    assert ctx.schedule == other
    with pytest.raises(_ext.Pi05Error, match="PI05_E_STATE"):
        ctx.denoise(torch.zeros(1, 50, 32, device="cuda"))
    model.close()


def test_persistent_is_default_and_single_launch(full_weights):
    g = replace(S.ExpertGeometry(), depth=2)
    w = {k: v for k, v in full_weights.items() if ".layers." not in k or int(k.split(".layers.")[1].split(".")[0]) < 2}
    model = OpenPi0Inference(OpenPi0InferConfig(num_steps=2), g)
    model.load_state_dict(w)
    model.to("cuda")
    ctx = model._context(1, 32, 2)
    assert ctx.schedule == "persistent"
    assert ctx.launches_per_step() == 0
    ctx.set_schedule("graph")
    assert ctx.launches_per_step() in (1 + 2 * 5, 1 + 2 * 6)
    model.close()


INVARIANT_CASES = {
    # name: (B, P, pad_fn)
    "full_c1": (1, 968, None),
    "ragged_tails": (3, 300, lambda p: (p[0, 280:].zero_(), p[1, 100:].zero_())),
    "interior_holes": (3, 77, lambda p: (p[0, 5:17].zero_(), p[1, ::3].zero_(), p[2, 40:41].zero_())),
    "padded_head": (2, 64, lambda p: (p[0, :10].zero_(), p[1, 1:].zero_())),
    "single_key": (1, 1, None),
    "odd_length": (3, 33, lambda p: p[1, 32:].zero_()),
}


@pytest.mark.parametrize("case", sorted(INVARIANT_CASES))
def test_step_invariants_bit_exact(full_weights, case):
    """RoPE positions and key masks are integer work: the context's copies must equal the oracle's
    position_ids and the zero entries of attention_mask_4d exactly (engine.py:471-478;
    pi0_pytorch.py:56-85, 160-163), under both schedules, before and after a predict."""
    B, P, pad_fn = INVARIANT_CASES[case]
    print(f"case invariants/{case}: B={B}, P={P}", flush=True)
    g = replace(S.ExpertGeometry(), depth=1)
    w = {k: v for k, v in full_weights.items() if ".layers." not in k or int(k.split(".layers.")[1].split(".")[0]) < 1}
    pad = S.full_prefix_pad(P, B)
    if pad_fn is not None:
        pad_fn(pad)
    pos_ref = O.position_ids(pad, g.action_horizon)
    allowed_ref = (O.attention_mask_4d(pad, g.action_horizon) == 0.0).to(torch.uint8)  # [B, 1, A, P + A]
    # every query row sees the same keys: the table is per key
    assert torch.equal(allowed_ref, allowed_ref[:, :, :1].expand_as(allowed_ref))
    k, v = S.make_prefix_kv(g, P, B)
    model = OpenPi0Inference(OpenPi0InferConfig(num_steps=2), g)
    model.load_state_dict(w)
    model.to("cuda")
    obs = Observation(k.cuda(), v.cuda(), pad.cuda())
    x1 = S.make_noise(g, B).cuda()
    for sched in SCHEDULES:
        model.set_schedule(sched)
        model.sample_actions(obs, x1)
        ctx = model._context(B, P, 2)
        for when in ("after predict", "after re-prime"):
            if when == "after re-prime":
                ctx.prime_prefix(_split_layers(obs.prefix_k, g.depth), _split_layers(obs.prefix_v, g.depth), obs.prefix_pad_masks)
            pos, valid, stray = ctx.step_invariants()
            torch.cuda.synchronize()
            assert torch.equal(pos.cpu(), pos_ref), f"{case} [{sched}] positions {when}"
            assert torch.equal(valid.cpu(), allowed_ref[:, 0, 0]), f"{case} [{sched}] key mask {when}"
            assert stray.item() == 0, f"{case} [{sched}] {stray.item()} padding slots marked valid {when}"
    model.close()


def test_timeout_is_reported_and_the_next_predict_recovers(full_weights):
    """The persistent kernel's waits are bounded.  With the spin limit cut to a few polls some wait
    gives up; every workgroup still leaves normally, the launch is reported as PI05_E_HIP (once),
    and the next predict with the default limit is exact again."""
    from pi05_infer import _ext

    g = replace(S.ExpertGeometry(), depth=2)
    w = {k: v for k, v in full_weights.items() if ".layers." not in k or int(k.split(".layers.")[1].split(".")[0]) < 2}
    model = OpenPi0Inference(OpenPi0InferConfig(num_steps=3), g)
    model.load_state_dict(w)
    model.to("cuda")
    k, v = S.make_prefix_kv(g, 64)
    obs = Observation(k.cuda(), v.cuda(), S.full_prefix_pad(64).cuda())
    x1 = S.make_noise(g).cuda()
    good = model.sample_actions(obs, x1)["actions"].clone()
    ctx = model._context(1, 64, 3)
    assert ctx.schedule == "persistent"
    ctx.status()  # nothing pending
    print("forcing a timed-out wait (spin limit 1)", flush=True)
    ctx.set_spin_limit(1)
    model.sample_actions(obs, x1)
    with pytest.raises(_ext.Pi05Error, match="PI05_E_HIP"):
        ctx.status()
    ctx.status()  # reported once
    # reported by the next denoise when nobody asked for the status
    model.sample_actions(obs, x1)
    torch.cuda.synchronize()
    with pytest.raises(_ext.Pi05Error, match="PI05_E_HIP"):
        model.sample_actions(obs, x1)
    # predict_action_batch waits for its actions (the host copy of output_transform) and raises
    # for the timed-out launch itself, as the reference's synchronising copy would
    with pytest.raises(_ext.Pi05Error, match="PI05_E_HIP"):
        model.predict_action_batch(obs, noise=x1)
    ctx.set_spin_limit(0)
    again = model.sample_actions(obs, x1)["actions"]
    ctx.status()
    assert torch.equal(again, good)
    assert torch.equal(model.predict_action_batch(obs, noise=x1), good.cpu()[:, :5, :7])
    model.close()


def test_placement_check_reports_a_misplaced_launch(full_weights):
    """Every persistent launch checks that workgroups w and w + 8 ran on one XCD (its intra-XCD
    hand-offs need it).  With the check's offset skewed for the odd workgroups (the placement and
    the work stay as they are) the launch is reported as PI05_E_HIP, once; with the skew removed
    the next predicts are exact and report nothing.  Run at B = 1 and B = 3 (kernel instances 0
    and 2, which share the check)."""
    from pi05_infer import _ext

    for B in (1, 3):
        g, model = _small_model(full_weights)
        k, v = S.make_prefix_kv(g, 64, B)
        obs = Observation(k.cuda(), v.cuda(), S.full_prefix_pad(64, B).cuda())
        x1 = S.make_noise(g, B).cuda()
        good = model.sample_actions(obs, x1)["actions"].clone()
        ctx = model._context(B, 64, 3)
        ctx.status()  # the real placement passes the check
        print(f"skewing the placement check (B={B})", flush=True)
        ctx.skew_placement_check(3)
        got = model.sample_actions(obs, x1)["actions"]
        with pytest.raises(_ext.Pi05Error, match="XCD"):
            ctx.status()
        ctx.status()  # reported once
        assert torch.equal(got, good)  # the work itself ran as usual
        ctx.skew_placement_check(0)
        again = model.sample_actions(obs, x1)["actions"]
        ctx.status()
        assert torch.equal(again, good)
        model.close()


def _small_model(full_weights, depth=2, steps=3):
    g = replace(S.ExpertGeometry(), depth=depth)
    w = {k: v for k, v in full_weights.items() if ".layers." not in k or int(k.split(".layers.")[1].split(".")[0]) < depth}
    model = OpenPi0Inference(OpenPi0InferConfig(num_steps=steps), g)
    model.load_state_dict(w)
    model.to("cuda")
    return g, model


def test_seeded_predicts_draw_noise_like_the_reference(full_weights):
    """Seeded once, two predicts without noise equal predicts fed the noises the reference would
    draw from that generator: x1, then num_steps discarded draws (one per Euler step,
    engine.py:391-403), then the next predict's x1."""
    steps = 3
    g, model = _small_model(full_weights, steps=steps)
    k, v = S.make_prefix_kv(g, 64)
    obs = Observation(k.cuda(), v.cuda(), S.full_prefix_pad(64).cuda())
    torch.manual_seed(1234)
    a1 = model.sample_actions(obs)["actions"].clone()
    a2 = model.sample_actions(obs)["actions"].clone()
    torch.manual_seed(1234)
    shape = (1, g.action_horizon, g.action_dim)
    draws = [torch.normal(0.0, 1.0, size=shape, device="cuda") for _ in range(2 + steps)]
    b1 = model.sample_actions(obs, draws[0])["actions"]
    b2 = model.sample_actions(obs, draws[1 + steps])["actions"]
    torch.cuda.synchronize()
    assert torch.equal(a1, b1) and torch.equal(a2, b2) and not torch.equal(a1, a2)
    model.close()


def test_captured_predict_replays_match_uncaptured(full_weights):
    """sample_actions captured with torch.cuda.graph (persistent schedule) and replayed: each
    replay, with eager predicts and host synchronisations between the replays, equals the
    uncaptured predict of the same noise bit for bit (the kernel takes its flag epoch from device
    memory, so a replay never meets flags of its own epoch).  The graph schedule refuses capture."""
    from pi05_infer import _ext

    g, model = _small_model(full_weights, depth=2, steps=3)
    k, v = S.make_prefix_kv(g, 64)
    obs = Observation(k.cuda(), v.cuda(), S.full_prefix_pad(64).cuda())
    xs = [S.make_noise(g, seed=sd).cuda() for sd in (2, 3)]
    refs = [model.sample_actions(obs, x)["actions"].clone() for x in xs]
    torch.cuda.synchronize()
    x_static = xs[0].clone()
    graph = torch.cuda.CUDAGraph()
    print("capturing sample_actions (persistent schedule)", flush=True)
    with torch.cuda.graph(graph):
        out = model.sample_actions(obs, x_static)["actions"]
    torch.cuda.synchronize()
    for i in (0, 1, 0, 1):
        x_static.copy_(xs[i])
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, refs[i]), f"replay of noise {i}"
        eager = model.sample_actions(obs, xs[1 - i])["actions"]
        torch.cuda.synchronize()
        assert torch.equal(eager, refs[1 - i])
    model._context(1, 64, 3).status()
    del graph
    model.set_schedule("graph")
    model.sample_actions(obs, xs[0])  # builds the schedule's own graph outside any capture
    torch.cuda.synchronize()
    g2 = torch.cuda.CUDAGraph()
    with pytest.raises(_ext.Pi05Error, match="PI05_E_STATE"):
        with torch.cuda.graph(g2):
            model.sample_actions(obs, x_static)
    model.close()


def test_epoch_wraparound_keeps_predicts_exact(full_weights):
    """The launch whose epoch reaches 2^31 zeroes the flags and the next runs as epoch 1: the
    predicts on either side of the wrap equal the first one bit for bit."""
    g, model = _small_model(full_weights, depth=2, steps=3)
    k, v = S.make_prefix_kv(g, 96)
    obs = Observation(k.cuda(), v.cuda(), S.full_prefix_pad(96).cuda())
    x1 = S.make_noise(g).cuda()
    good = model.sample_actions(obs, x1)["actions"].clone()
    ctx = model._context(1, 96, 3)
    ctx.set_epoch(2**31 - 2)
    for i in range(4):  # epochs 2^31 - 1, 2^31 (zeroes the flags), 1, 2
        got = model.sample_actions(obs, x1)["actions"]
        torch.cuda.synchronize()
        assert torch.equal(got, good), f"predict {i} after the epoch was set"
    ctx.status()
    model.close()


def test_back_to_back_predicts_without_host_sync(full_weights):
    """pi05_denoise only enqueues: predicts queued back to back with no host synchronisation in
    between give the same actions as one predict at a time."""
    g = replace(S.ExpertGeometry(), depth=3)
    w = {k: v for k, v in full_weights.items() if ".layers." not in k or int(k.split(".layers.")[1].split(".")[0]) < 3}
    model = OpenPi0Inference(OpenPi0InferConfig(num_steps=4), g)
    model.load_state_dict(w)
    model.to("cuda")
    k, v = S.make_prefix_kv(g, 200)
    obs = Observation(k.cuda(), v.cuda(), S.full_prefix_pad(200).cuda())
    noises = [S.make_noise(g).cuda() * s for s in (1.0, -0.5, 2.0)]
    single = []
    for n in noises:
        single.append(model.sample_actions(obs, n)["actions"].clone())
        torch.cuda.synchronize()
    queued = [model.sample_actions(obs, n)["actions"] for n in noises]
    torch.cuda.synchronize()
    for a, b in zip(single, queued):
        assert torch.equal(a, b)
    model.close()


def test_predict_action_batch_returns_env_space_actions(full_weights):
    """predict_action_batch = sample_actions, then the output transforms (engine.py:321-342):
    Unnormalize with the installed norm stats and the policy's Outputs slice, then the chunk."""
    from pi05_infer import transforms as T

    g = replace(S.ExpertGeometry(), depth=2)
    w = {k: v for k, v in full_weights.items() if ".layers." not in k or int(k.split(".layers.")[1].split(".")[0]) < 2}
    model = OpenPi0Inference(OpenPi0InferConfig(config_name="pi05_turtle", num_steps=3, action_chunk=5), g)
    model.load_state_dict(w)
    model.to("cuda")
    k, v = S.make_prefix_kv(g, 40)
    obs = Observation(k.cuda(), v.cuda(), S.full_prefix_pad(40).cuda(), state=torch.zeros(1, 8, device="cuda"))
    x1 = S.make_noise(g).cuda()
    raw = model.sample_actions(obs, x1)["actions"].cpu()
    got = model.predict_action_batch(obs, noise=x1)
    assert got.shape == (1, 5, 6) and torch.equal(got, raw[:, :5, :6])
    q01 = torch.linspace(-2, 0, 6, dtype=torch.float64)
    stats = {"actions": T.NormStats(torch.zeros(6, dtype=torch.float64), torch.ones(6, dtype=torch.float64), q01, q01 + 3)}
    model.setup_wrappers(output_transforms=T.output_transforms_for("pi05_turtle", stats))
    got = model.predict_action_batch(obs, noise=x1)
    ref = (raw[:, :5, :6].double() + 1) / 2 * (3 + 1e-6) + q01
    torch.testing.assert_close(got, ref, rtol=0, atol=0)
    model.close()
