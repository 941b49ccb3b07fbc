"""GPU parity of the prefix-LM prefill (Gemma-2B over the prefix) against the CPU oracle, through
the C ABI (include/pi05_prefill.h).

Tolerance, as for the denoise path (bf16 on the GPU, fp32 with bf16 rounding points in the
oracle): per layer, the K and V of the valid prefix tokens have cosine similarity >= 0.9999 with
the oracle's and max-abs error <= 2e-2 of the oracle tensor's range.  The token embedding is
exact (one fp32 product rounded to bf16).  Padded tokens' K/V are don't-care (no valid query ever
attends to them) and are only required to be finite.
"""

from dataclasses import replace

import pytest
import torch

from oracle import denoise_oracle as O
from oracle import prefix_oracle as PO
from pi05_infer import _ext
from pi05_infer import synthetic as S

pytestmark = pytest.mark.gpu

COS_MIN = 0.9999
REL_MAXABS = 2e-2
G = PO.PrefixGeometry()


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


def _context(depth: int, batch: int, plen: int, layers, skip_last: int = 1) -> tuple:
    d = _ext.prefix_default_dims()
    d.depth, d.batch, d.prefix_len, d.skip_last_layer = depth, batch, plen, skip_last
    ctx = _ext.PrefixContext(d, torch.device("cuda"))
    keep = []
    for i, w in enumerate(layers):
        t = {k: (v.to(torch.bfloat16) if k not in ("ln1", "ln2") else v.float()).cuda().contiguous() for k, v in w.items()}
        keep.append(t)
        ctx.bind_layer(i, t["wq"], t["wk"], t["wv"], t["wo"], t["wg"], t["wu"], t["wd"], t["ln1"], t["ln2"])
    ctx.refresh_weights()
    torch.cuda.synchronize()
    return ctx, keep


def _run(ctx, embeds: torch.Tensor, pad: torch.Tensor, depth: int):
    b, p, _ = embeds.shape
    ks = [torch.full((b, 1, p, G.head_dim), float("nan"), dtype=torch.bfloat16, device="cuda") for _ in range(depth)]
    vs = [torch.full((b, 1, p, G.head_dim), float("nan"), dtype=torch.bfloat16, device="cuda") for _ in range(depth)]
    ctx.forward(embeds.to(torch.bfloat16).cuda().contiguous(), pad.cuda(), ks, vs)
    torch.cuda.synchronize()
    return ks, vs


def _compare(ref_cache, ks, vs, pad, name):
    for l, (kr, vr) in enumerate(ref_cache):
        for b in range(pad.shape[0]):
            valid = pad[b].bool()
            for what, r, g in (("K", kr, ks[l]), ("V", vr, vs[l])):
                gb = g[b, 0].float().cpu()
                assert torch.isfinite(gb).all(), f"{name} layer {l} {what}[{b}]: non-finite (padded rows included)"
                _close(r[b, 0][valid], gb[valid], f"{name} layer {l} {what}[{b}]")


@pytest.fixture(scope="module")
def layers3():
    return PO.random_layers(G, 3, seed=11)


def test_prefill_parity_single_sample(layers3):
    print("case prefill: depth 3, B=1, P=96, all valid", flush=True)
    torch.manual_seed(0)
    emb = O._bf(torch.randn(1, 96, G.width))
    pad = torch.ones(1, 96, dtype=torch.bool)
    ref = PO.prefill(layers3, G, emb, pad)
    ctx, _keep = _context(3, 1, 96, layers3)
    ks, vs = _run(ctx, emb, pad, 3)
    _compare(ref, ks, vs, pad, "B1P96")


def test_prefill_parity_ragged_batch(layers3):
    print("case prefill: depth 3, B=2, P=77 (odd, not a multiple of 32), sample 1 padded from 57", flush=True)
    torch.manual_seed(1)
    emb = O._bf(torch.randn(2, 77, G.width))
    pad = torch.ones(2, 77, dtype=torch.bool)
    pad[1, 57:] = False
    ref = PO.prefill(layers3, G, emb, pad)
    ctx, _keep = _context(3, 2, 77, layers3)
    ks, vs = _run(ctx, emb, pad, 3)
    _compare(ref, ks, vs, pad, "B2P77")


def test_kv_only_last_layer_matches_full_layer(layers3):
    print("case prefill: last layer K/V only vs full", flush=True)
    torch.manual_seed(2)
    emb = O._bf(torch.randn(1, 40, G.width))
    pad = torch.ones(1, 40, dtype=torch.bool)
    ctx1, k1 = _context(3, 1, 40, layers3, skip_last=1)
    a = _run(ctx1, emb, pad, 3)
    ctx0, k0 = _context(3, 1, 40, layers3, skip_last=0)
    b = _run(ctx0, emb, pad, 3)
    # each context tunes its own GEMM algorithms (and the K/V-only layer runs an N=512 GEMM), so
    # accumulation orders may differ: equal up to bf16 rounding of the GEMM outputs
    for l in range(3):
        _close(b[0][l].float(), a[0][l].float(), f"K/V-only vs full: layer {l} K")
        _close(b[1][l].float(), a[1][l].float(), f"K/V-only vs full: layer {l} V")


def test_embed_tokens_exact_and_rejects_bad_ids():
    print("case prefill: language-token embedding", flush=True)
    torch.manual_seed(3)
    d = _ext.prefix_default_dims()
    d.depth, d.prefix_len = 1, 8
    ctx = _ext.PrefixContext(d, torch.device("cuda"))
    table = O._bf(torch.randn(1000, G.width))
    ids = torch.randint(0, 1000, (2, 13))
    got = ctx.embed_tokens(ids.cuda(), table.to(torch.bfloat16).cuda())
    ref = PO.embed_tokens(ids, table, G.width)
    assert torch.equal(got.float().cpu(), ref)
    bad = ids.clone()
    bad[1, 4] = 1000
    tb = table.to(torch.bfloat16).cuda()
    # host ids are checked before the copy
    with pytest.raises(_ext.Pi05Error):
        ctx.embed_tokens(bad, tb)
    # device ids: the call only enqueues; the bad row is zero and status() reports it, once
    out = ctx.embed_tokens(bad.cuda(), tb)
    with pytest.raises(_ext.Pi05Error):
        ctx.status()
    ctx.status()
    assert torch.equal(out[1, 4].float().cpu(), torch.zeros(G.width))
    keep = torch.ones(2, 13, dtype=torch.bool)
    keep[1, 4] = False
    assert torch.equal(out.float().cpu()[keep], ref[keep])
    # or the next call reports it (and enqueues nothing); the call after that runs
    ctx.embed_tokens(bad.cuda(), tb)
    torch.cuda.synchronize()
    with pytest.raises(_ext.Pi05Error):
        ctx.embed_tokens(ids.cuda(), tb)
    got = ctx.embed_tokens(ids.cuda(), tb)
    ctx.status()
    assert torch.equal(got.float().cpu(), ref)


def test_prefill_then_denoise_matches_oracle_chain(layers3):
    """The prefill's cache fed to the denoise engine (pi05_prime_prefix) against the oracle chain:
    oracle prefill -> oracle denoise."""
    print("case prefill -> denoise: depth 3, B=1, P=64 (10 padded), 4 steps", flush=True)
    from pi05_infer.engine import Observation, OpenPi0InferConfig, OpenPi0Inference

    torch.manual_seed(4)
    P, steps = 64, 4
    emb = O._bf(torch.randn(1, P, G.width))
    pad = torch.ones(1, P, dtype=torch.bool)
    pad[0, 54:] = False
    ref_cache = PO.prefill(layers3, G, emb, pad)
    k_ref = torch.cat([k for k, _ in ref_cache], dim=1)  # [B, L, P, D]
    v_ref = torch.cat([v for _, v in ref_cache], dim=1)
    eg = replace(S.ExpertGeometry(), depth=3)
    w = S.make_weights(eg)
    x1 = S.make_noise(eg, 1)
    og = O.geometry_from(eg)
    table = O.adarms_table(w, og, steps)
    act_ref, _ = O.sample_actions(w, og, k_ref, v_ref, pad, x1, steps, table)
    # through the Python API: the observation carries prefix embeddings, the attached PrefixLM
    # builds the cache (build_prefix_cache), the expert denoises on it
    from pi05_infer.prefix import PrefixGeometry, PrefixLM, layer_param_names

    plm = PrefixLM(PrefixGeometry(depth=3))
    sd = {}
    for i, lw in enumerate(layers3):
        n = layer_param_names(i)
        for k in ("wq", "wk", "wv", "wo", "wg", "wu", "wd", "ln1", "ln2"):
            sd[n[k]] = lw[k]
    missing, _ = plm.load_state_dict(sd)
    assert missing == [PO.layer_names(0)["wq"].split("layers.")[0] + "embed_tokens.weight"]
    model = OpenPi0Inference(OpenPi0InferConfig(num_steps=steps), eg)
    model.load_state_dict(w)
    model.to("cuda")
    model.attach_prefix_lm(plm)
    obs = Observation(None, None, pad.cuda(), prefix_embs=emb.to(torch.bfloat16).cuda())
    act, _ = model.sample_actions_with_velocities(obs, x1.cuda())
    torch.cuda.synchronize()
    _close(act_ref, act, "prefill->denoise actions")


def test_full_depth_prefill_then_denoise_c5_geometry():
    """All 18 Gemma-2B layers (17 full + the K/V-only last) into the 18-layer expert: the cache's
    rounding noise grows with depth, so the parity bar (cos >= 0.9999, max-abs <= 2e-2 of the
    range) is applied to the denoise output (actions and every step's velocity), with the per-layer
    K/V cosine reported."""
    print("case prefill -> denoise: depth 18, B=1, P=96 (16 padded), 10 steps", flush=True)
    from pi05_infer.engine import Observation, OpenPi0InferConfig, OpenPi0Inference
    from pi05_infer.prefix import PrefixGeometry, PrefixLM, layer_param_names

    torch.manual_seed(5)
    P, steps = 96, 10
    layers = PO.random_layers(G, 18, seed=21)
    print("  weights generated", flush=True)
    emb = O._bf(torch.randn(1, P, G.width))
    pad = torch.ones(1, P, dtype=torch.bool)
    pad[0, 80:] = False
    ref_cache = PO.prefill(layers, G, emb, pad)
    print("  oracle prefill done", flush=True)
    plm = PrefixLM(PrefixGeometry())
    plm.load_state_dict({layer_param_names(i)[k]: lw[k] for i, lw in enumerate(layers) for k in lw})
    del layers
    eg = S.ExpertGeometry()
    w = S.make_weights(eg)
    x1 = S.make_noise(eg, 1)
    og = O.geometry_from(eg)
    table = O.adarms_table(w, og, steps)
    k_ref = torch.cat([k for k, _ in ref_cache], dim=1)
    v_ref = torch.cat([v for _, v in ref_cache], dim=1)
    act_ref, vs_ref = O.sample_actions(w, og, k_ref, v_ref, pad, x1, steps, table)
    print("  oracle denoise done", flush=True)
    model = OpenPi0Inference(OpenPi0InferConfig(num_steps=steps), eg)
    model.load_state_dict(w)
    model.to("cuda")
    model.attach_prefix_lm(plm)
    _, _, kv = plm.build_prefix_cache(emb.to(torch.bfloat16).cuda(), pad.cuda())
    valid = pad[0]
    for l in (0, 5, 11, 17):
        for what, r, g in (("K", ref_cache[l][0], kv[l][0]), ("V", ref_cache[l][1], kv[l][1])):
            rr, gg = r[0, 0][valid].double().flatten(), g[0, 0].float().cpu()[valid].double().flatten()
            print(f"  layer {l} {what}: cos={torch.nn.functional.cosine_similarity(rr, gg, dim=0).item():.7f}", flush=True)
    obs = Observation(None, None, pad.cuda(), prefix_embs=emb.to(torch.bfloat16).cuda())
    act, vs = model.sample_actions_with_velocities(obs, x1.cuda())
    torch.cuda.synchronize()
    for s in range(steps):
        _close(vs_ref[s], vs[s], f"depth-18 prefill->denoise step {s} velocity")
    _close(act_ref, act, "depth-18 prefill->denoise actions")
    model.close()


def test_full_vocabulary_prompt_embed_prefill_denoise():
    """Token ids across Gemma's whole vocabulary (0 .. 257151, both ends included) through
    embed_tokens with a 257,152-row table, the prefill (depth 2) and the denoise (depth 2, 3 steps):
    the embeddings equal the oracle's bit for bit, and the actions meet the parity bar against the
    oracle chain on the same embeddings."""
    print("case full vocabulary: 257152-row table, 40 tokens (5 padded), prefill depth 2 -> denoise depth 2", flush=True)
    from pi05_infer.engine import Observation, OpenPi0InferConfig, OpenPi0Inference
    from pi05_infer.prefix import EMBED_NAME, PrefixGeometry, PrefixLM, layer_param_names

    vocab, T, steps = 257152, 40, 3
    gen = torch.Generator().manual_seed(12)
    table = torch.randn(vocab, G.width, generator=gen).to(torch.bfloat16)
    ids = torch.randint(0, vocab, (1, T), generator=gen)
    ids[0, :6] = torch.tensor([0, 1, vocab - 1, vocab - 2, 131072, 65535])
    pad = torch.ones(1, T, dtype=torch.bool)
    pad[0, 35:] = False
    layers = PO.random_layers(G, 2, seed=13)
    plm = PrefixLM(PrefixGeometry(depth=2))
    sd = {layer_param_names(i)[k]: lw[k] for i, lw in enumerate(layers) for k in lw}
    sd[EMBED_NAME] = table
    plm.load_state_dict(sd, strict=True)
    plm.to("cuda")
    got = plm.embed_language_tokens(ids.cuda(), prefix_len=T)
    torch.cuda.synchronize()
    ref = PO.embed_tokens(ids, table.float(), G.width)
    assert torch.equal(got.float().cpu(), ref), "token embeddings differ from the oracle's"
    print("  embeddings equal the oracle's", flush=True)
    ref_cache = PO.prefill(layers, G, ref, pad)
    k_ref = torch.cat([k for k, _ in ref_cache], dim=1)
    v_ref = torch.cat([v for _, v in ref_cache], dim=1)
    eg = replace(S.ExpertGeometry(), depth=2)
    w = S.make_weights(eg)
    x1 = S.make_noise(eg, 1)
    og = O.geometry_from(eg)
    act_ref, vs_ref = O.sample_actions(w, og, k_ref, v_ref, pad, x1, steps, O.adarms_table(w, og, steps))
    model = OpenPi0Inference(OpenPi0InferConfig(num_steps=steps), eg)
    model.load_state_dict(w)
    model.to("cuda")
    model.attach_prefix_lm(plm)
    obs = Observation(None, None, pad.cuda(), prefix_embs=got)
    act, vs = model.sample_actions_with_velocities(obs, x1.cuda())
    torch.cuda.synchronize()
    for s in range(steps):
        _close(vs_ref[s], vs[s], f"full-vocabulary chain step {s} velocity")
    _close(act_ref, act, "full-vocabulary chain actions")
    model.close()
