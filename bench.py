#!/usr/bin/env python3
"""Benchmark of the pi0.5 action-expert denoise loop on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c1|c2|c3|c4]
                    [--schedule persistent|graph] [--no-cpu-baseline]
    python bench.py --workload prefill [--steps K] [--warmup W] [--no-cpu-baseline]
    python bench.py --workload vision [--steps K] [--warmup W] [--no-cpu-baseline]
    python bench.py --workload e2e [--steps K] [--warmup W]

One bench "step" is one predict's denoise: the 10-step flow-matching Euler loop of the 18-layer
expert over a static prefix KV cache, with weights, KV and noise already resident in HBM.  In the
default (persistent) schedule that is ONE launch of the cooperative denoise kernel; in the graph
schedule one hipGraph replay.  Random-init weights (seed 0), N(0,1) bf16 prefix KV (seed 1),
N(0,1) noise (seed 2): synthetic data, no checkpoint.  Prints ONE JSON line.

``--workload prefill`` measures the prefix-LM prefill instead (Gemma-2B over a 968-token prefix,
bs=1, 17 full layers + the last layer's K/V): one step is one prefill, MFMA-bound, reported
against the bf16 dense MFMA peak.  ``--workload vision`` measures the vision tower (SigLIP
So400m/14 + projector over 3 camera views of 224 x 224, M = 768 patches) the same way, and
``--workload e2e`` a whole ``sample_actions`` from 3 camera images and a 200-token prompt (vision
tower, token embedding, 968-token prefill, 10-step denoise) through the Python API.
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "pi05-infer_amd"))
sys.path.insert(0, ROOT)

CONFIGS = {
    "c1": dict(batch=1, prefix_len=968),
    "c2": dict(batch=1, prefix_len=456),
    "c3": dict(batch=8, prefix_len=968),
    "c4": dict(batch=1, prefix_len=3272),
}
METRIC = "denoise ms/predict (10 steps, bs=1, 968 prefix) + % peak HBM GB/s"
HBM_PEAK_GBS = 8000.0  # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
PREFILL_METRIC = "prefix prefill ms (Gemma-2B, bs=1, 968 tokens) + % peak bf16 MFMA"
VISION_METRIC = "vision tower ms (SigLIP So400m/14 + projector, 3 views of 224x224) + % peak bf16 MFMA"


E2E_METRIC = "end-to-end sample_actions ms/predict (3 images 224x224 + 200 tokens -> 968-token prefix, 10 steps, bs=1)"


def bench_e2e(args) -> int:
    import torch

    from pi05_infer import synthetic as S
    from pi05_infer.builder import build_model
    from pi05_infer.engine import Observation
    from pi05_infer.prefix import PrefixGeometry, PrefixLM
    from pi05_infer.prefix import make_weights as prefix_weights
    from pi05_infer.vision import VisionGeometry, VisionTower
    from pi05_infer.vision import make_weights as vision_weights

    dev = torch.device("cuda", torch.cuda.current_device())
    steps, B, views, T = 10, 1, 3, 200
    model = build_model("random:0", "pi05_libero", num_steps=steps)
    model.to(dev)
    plm = PrefixLM(PrefixGeometry())
    plm.to(dev)
    plm.load_state_dict(prefix_weights(PrefixGeometry(), seed=1, device=dev))
    vt = VisionTower(VisionGeometry())
    vt.to(dev)
    vt.load_state_dict(vision_weights(VisionGeometry(), seed=2, device=dev))
    model.attach_prefix_lm(plm)
    model.attach_vision_tower(vt)
    gen = torch.Generator(device=dev).manual_seed(3)
    images = {f"view{i}": torch.rand(B, 3, 224, 224, generator=gen, device=dev) * 2 - 1 for i in range(views)}
    masks = {k: torch.ones(B, dtype=torch.bool, device=dev) for k in images}
    tokens = torch.randint(0, PrefixGeometry().vocab_size, (B, T), generator=gen, device=dev)
    obs = Observation.from_dict({"images": images, "image_masks": masks, "tokenized_prompt": tokens,
                                 "tokenized_prompt_mask": torch.ones(B, T, dtype=torch.bool, device=dev)})
    x1 = S.make_noise(S.ExpertGeometry(), B).to(dev)
    for _ in range(args.warmup):
        model.sample_actions(obs, x1)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        out = model.sample_actions(obs, x1)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    assert out["actions"].shape == (B, 50, 32) and bool(torch.isfinite(out["actions"]).all())
    # host time to enqueue one predict (the call returns before the GPU is done): where it nears
    # the GPU time, the host's kernel submissions are what paces back-to-back predicts
    issue = []
    for _ in range(5):
        t = time.perf_counter()
        model.sample_actions(obs, x1)
        issue.append((time.perf_counter() - t) * 1e3)
        torch.cuda.synchronize()
    issue_ms = statistics.median(issue)

    # the same predict phase by phase (each phase timed alone, same clock, same inputs)
    imgs, img_masks = list(images.values()), list(masks.values())

    def timed(fn, reps=args.steps):
        fn()
        torch.cuda.synchronize()
        t = time.perf_counter()
        for _ in range(reps):
            r = fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t) * 1e3 / reps, r

    vis_ms, _ = timed(lambda: vt.embed_image(torch.cat(imgs, dim=0)))
    emb_ms, (embs, pads, _) = timed(lambda: model.embed_prefix(imgs, img_masks, tokens, obs.tokenized_prompt_mask))
    pre_ms, (_, _, kv) = timed(lambda: plm.build_prefix_cache(embs, pads))
    kv_obs = Observation([k for k, _ in kv], [v for _, v in kv], pads)
    den_ms, _ = timed(lambda: model.sample_actions(kv_obs, x1))
    phases = {"vision_ms": round(vis_ms, 3), "embed_prefix_ms (vision + token embedding + concat)": round(emb_ms, 3),
              "prefill_ms": round(pre_ms, 3), "denoise_ms (prime + 10 steps)": round(den_ms, 3),
              "host_issue_ms (one predict enqueued, GPU idle before)": round(issue_ms, 3)}

    cpu = None
    if not args.no_cpu_baseline:
        from oracle import denoise_oracle as O
        from oracle import prefix_oracle as PO
        from oracle import siglip_oracle as SO
        from pi05_infer.prefix import layer_param_names as pnames
        from pi05_infer.vision import HEAD_KEYS, HEAD_PARAM_NAMES, LAYER_KEYS
        from pi05_infer.vision import layer_param_names as vnames

        threads = host_threads()
        torch.set_num_threads(threads)
        # one SigLIP layer, one Gemma-2B layer and one expert predict of the fp32 oracle, scaled
        okeys = dict(zip(LAYER_KEYS, ("wq", "bq", "wk", "bk", "wv", "bv", "wout", "bout", "w1", "b1", "w2", "b2", "ln1w",
                                      "ln1b", "ln2w", "ln2b")))
        v0 = {okeys[k]: vt.params[vnames(0)[k]].float().cpu() for k in LAYER_KEYS}
        vh = {k: vt.params[HEAD_PARAM_NAMES[k]].float().cpu() for k in HEAD_KEYS}
        t = time.perf_counter()
        h = SO.embeddings(torch.cat(imgs).cpu(), vh, SO.SiglipGeometry())
        SO.encoder_layer(v0, SO.SiglipGeometry(), h)
        v_layer = time.perf_counter() - t
        p0 = {k: plm.params[pnames(0)[k]].float().cpu() for k in ("wq", "wk", "wv", "wo", "wg", "wu", "wd", "ln1", "ln2")}
        g = PO.PrefixGeometry()
        pos, mask4d = PO.prefix_masks(pads.cpu())
        cos, sin = O.rope_cos_sin(pos, g.head_dim, g.rope_theta)
        t = time.perf_counter()
        PO.prefix_layer(p0, g, embs.float().cpu(), cos, sin, mask4d)
        p_layer = time.perf_counter() - t
        w = {n: t_.cpu() for n, t_ in model.params.items()}
        og = O.geometry_from(S.ExpertGeometry())
        k_ref = torch.cat([k.cpu() for k, _ in kv], dim=1)
        v_ref = torch.cat([v.cpu() for _, v in kv], dim=1)
        t = time.perf_counter()
        O.sample_actions(w, og, k_ref, v_ref, pads.cpu(), x1.cpu(), steps, O.adarms_table(w, og, steps))
        d_pred = time.perf_counter() - t
        cpu = {
            "value": round((v_layer * 27 + p_layer * 18 + d_pred) * 1e3, 1),
            "unit": "ms/predict",
            "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": "one SigLIP layer (x27) + one Gemma-2B layer (x18) + one full expert predict of the fp32 CPU "
                      f"oracle on the same inputs; host {cpu_model()}",
        }
    line = {
        "metric": E2E_METRIC,
        "value": round(ms, 3),
        "unit": "ms/predict",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 3),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random-init expert / Gemma-2B / SigLIP weights seeds 0-2, uniform [-1, 1] images, random token "
                "ids in [0, 257152), N(0,1) noise)",
        "config": {"workload": f"sample_actions: SigLIP over {views} views of 224x224 + {T}-token prompt -> "
                               f"{views * 256 + T}-token Gemma-2B prefill -> {steps}-step denoise, bs={B}",
                   "batch": B, "prefix_len": views * 256 + T, "num_steps": steps,
                   "timing": "host wall clock around K back-to-back predicts, synchronized at both ends"},
        "phases": phases,
        "roofline": None,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    model.close()
    torch.cuda.synchronize()
    return 0


def vision_flops(depth: int, n_images: int) -> int:
    """FLOPs of one vision-tower call: per layer q, k, v, out (1152 x 1152), fc1, fc2 (1152 x 4304)
    and the attention's Q.K^T and P.V over 16 heads of 72; the patch convolution (588 -> 1152) and
    the projector (1152 -> 2048) once."""
    W, I, S, H, D = 1152, 4304, 256, 16, 72
    M = n_images * S
    layer = 2 * M * W * (4 * W + 2 * I) + 2 * 2 * n_images * H * S * S * D
    return depth * layer + 2 * M * 588 * W + 2 * M * W * 2048


def bench_vision(args) -> int:
    import torch

    from pi05_infer import _ext
    from pi05_infer.vision import HEAD_KEYS, HEAD_PARAM_NAMES, LAYER_KEYS, VisionGeometry, layer_param_names, make_weights

    d = _ext.vision_default_dims()
    N, L = d.n_images, d.depth
    dev = torch.device("cuda", torch.cuda.current_device())
    g = VisionGeometry()
    w = make_weights(g, seed=0, device=dev, std=0.02)
    ctx = _ext.VisionContext(d, dev)
    for i in range(L):
        n = layer_param_names(i)
        ctx.bind_layer(i, *(w[n[k]] for k in LAYER_KEYS))
    ctx.bind_heads(*(w[HEAD_PARAM_NAMES[k]] for k in HEAD_KEYS))
    ctx.refresh_weights()
    gen = torch.Generator(device=dev).manual_seed(1)
    px = torch.rand(N, 3, 224, 224, generator=gen, device=dev) * 2 - 1
    out = torch.empty(N, 256, 2048, dtype=torch.bfloat16, device=dev)
    stream = torch.cuda.current_stream()
    for _ in range(args.warmup):
        ctx.forward(px, out, stream=stream)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(args.steps):
        ctx.forward(px, out, stream=stream)
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    flops = vision_flops(L, N)
    tflops = flops / (ms * 1e-3) / 1e12

    cpu = None
    if not args.no_cpu_baseline:
        from oracle import siglip_oracle as SO

        threads = host_threads()
        torch.set_num_threads(threads)
        og = SO.SiglipGeometry()
        n0 = layer_param_names(0)
        okeys = dict(zip(LAYER_KEYS, ("wq", "bq", "wk", "bk", "wv", "bv", "wout", "bout", "w1", "b1", "w2", "b2", "ln1w",
                                      "ln1b", "ln2w", "ln2b")))
        w0 = {okeys[k]: w[n0[k]].float().cpu() for k in LAYER_KEYS}
        heads = {k: w[HEAD_PARAM_NAMES[k]].float().cpu() for k in HEAD_KEYS}
        pxc = px.cpu()
        t0 = time.perf_counter()
        h = SO.embeddings(pxc, heads, og)
        x = SO.layer_norm(h, heads["post_w"], heads["post_b"], og.ln_eps)
        SO.linear_bias(x, heads["proj_w"], heads["proj_b"])
        heads_ms = (time.perf_counter() - t0) * 1e3
        times = []
        for _ in range(2):
            t0 = time.perf_counter()
            SO.encoder_layer(w0, og, h)
            times.append(time.perf_counter() - t0)
        layer_ms = statistics.median(times) * 1e3
        cpu = {
            "value": round(layer_ms * L + heads_ms, 1),
            "unit": "ms/call",
            "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"one encoder layer of the fp32 CPU oracle over {N} images (median of 2) scaled to {L} layers, "
                      f"plus the embeddings, post-norm and projector once; host {cpu_model()}",
        }
    out_line = {
        "metric": VISION_METRIC,
        "value": round(ms, 4),
        "unit": "ms/call",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random-init SigLIP/projector weights N(0, 0.02), uniform [-1, 1] pixels, seeds 0/1)",
        "config": {"workload": f"SigLIP So400m/14 depth {L} + projector, {N} images of 224x224 (M = {N * 256})",
                   "n_images": N},
        "roofline": {"kernel": "whole tower (hipBLASLt GEMMs + HIP kernels)", "bound": "mfma",
                     "achieved": round(tflops, 1), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tflops / BF16_PEAK_TFLOPS, 4), "traffic": None, "flops_per_call": flops},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out_line), flush=True)
    ctx.close()
    torch.cuda.synchronize()
    return 0


def prefill_flops(depth: int, batch: int, prefix_len: int, skip_last: bool = True) -> int:
    """FLOPs of one prefill: per full layer the q|k|v, o_proj, gate|up and down_proj GEMMs and the
    attention's Q.K^T and P.V over every (query, key) pair; the last layer's K/V projection only."""
    W, H, D, I = 2048, 8, 256, 16384
    M = batch * prefix_len
    gemm = 2 * M * W * ((H + 2) * D + H * D + 2 * I) + 2 * M * I * W
    attn = 2 * 2 * batch * prefix_len * prefix_len * D * H
    full = depth - 1 if skip_last else depth
    return full * (gemm + attn) + (2 * M * W * 2 * D if skip_last else 0)


def bench_prefill(args) -> int:
    import torch

    from pi05_infer import _ext

    d = _ext.prefix_default_dims()
    B, P, L = d.batch, d.prefix_len, d.depth
    dev = torch.device("cuda", torch.cuda.current_device())
    ctx = _ext.PrefixContext(d, dev)
    gen = torch.Generator(device=dev).manual_seed(0)

    def rnd(*shape, std=0.02, dtype=torch.bfloat16):
        return (torch.randn(*shape, generator=gen, device=dev) * std).to(dtype)

    layers = []
    for i in range(L):
        w = dict(wq=rnd(2048, 2048), wk=rnd(256, 2048), wv=rnd(256, 2048), wo=rnd(2048, 2048), wg=rnd(16384, 2048),
                 wu=rnd(16384, 2048), wd=rnd(2048, 16384), ln1=rnd(2048, std=0.1, dtype=torch.float32),
                 ln2=rnd(2048, std=0.1, dtype=torch.float32))
        ctx.bind_layer(i, w["wq"], w["wk"], w["wv"], w["wo"], w["wg"], w["wu"], w["wd"], w["ln1"], w["ln2"])
        layers.append(w)
    ctx.refresh_weights()
    emb = torch.randn(B, P, 2048, generator=gen, device=dev).to(torch.bfloat16)
    pad = torch.ones(B, P, dtype=torch.bool, device=dev)
    ks = [torch.empty(B, 1, P, 256, dtype=torch.bfloat16, device=dev) for _ in range(L)]
    vs = [torch.empty(B, 1, P, 256, dtype=torch.bfloat16, device=dev) for _ in range(L)]
    stream = torch.cuda.current_stream()
    for _ in range(args.warmup):
        ctx.forward(emb, pad, ks, vs, stream=stream)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(args.steps):
        ctx.forward(emb, pad, ks, vs, stream=stream)
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    flops = prefill_flops(L, B, P)
    tflops = flops / (ms * 1e-3) / 1e12

    cpu = None
    if not args.no_cpu_baseline:
        from oracle import prefix_oracle as PO

        threads = host_threads()
        torch.set_num_threads(threads)
        g = PO.PrefixGeometry()
        w0 = {k: v.float().cpu() for k, v in layers[0].items()}
        h = emb.float().cpu()
        pos, mask4d = PO.prefix_masks(pad.cpu())
        from oracle import denoise_oracle as O

        cos, sin = O.rope_cos_sin(pos, g.head_dim, g.rope_theta)
        times = []
        for _ in range(2):
            t0 = time.perf_counter()
            PO.prefix_layer(w0, g, h, cos, sin, mask4d)
            times.append(time.perf_counter() - t0)
        layer_ms = statistics.median(times) * 1e3
        cpu = {
            "value": round(layer_ms * (L - 1) + layer_ms * 512 / (2560 + 2048 + 32768 + 16384), 1),
            "unit": "ms/prefill",
            "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"one full decoder layer of the fp32 CPU oracle at B={B}, P={P} (median of 2), scaled to "
                      f"{L - 1} full layers + the K/V-only last layer; host {cpu_model()}",
        }
    out = {
        "metric": PREFILL_METRIC,
        "value": round(ms, 4),
        "unit": "ms/prefill",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random-init Gemma-2B weights N(0, 0.02), N(0,1) bf16 prefix embeddings, seed 0)",
        "config": {"workload": f"Gemma-2B prefix prefill, depth {L} (last layer K/V only), bs={B}, {P} tokens",
                   "batch": B, "prefix_len": P},
        "roofline": {"kernel": "whole prefill (hipBLASLt GEMMs + HIP kernels)", "bound": "mfma",
                     "achieved": round(tflops, 1), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tflops / BF16_PEAK_TFLOPS, 4), "traffic": None, "flops_per_prefill": flops},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    ctx.close()
    torch.cuda.synchronize()
    return 0


def algorithmic_bytes_per_predict(depth: int, batch: int, prefix_len: int, steps: int) -> int:
    """Compulsory HBM bytes of one predict: per step the bf16 expert weights, the KV cache of
    prefix + suffix keys, one modulation-table slice, the fp32 action in/out weights and x in/out."""
    W, H, D, I, A, a = 1024, 8, 256, 4096, 50, 32
    weights = depth * ((H + 2) * D * W + W * H * D + 2 * I * W + W * I) * 2
    kv = depth * batch * (prefix_len + A) * D * 2 * 2
    mod = (2 * depth + 1) * 3 * W * 4
    heads = (W * a * 2 + W + a) * 4
    x = batch * A * a * 4 * 2
    return steps * (weights + kv + mod + heads + x)


def algorithmic_flops_per_predict(depth: int, batch: int, prefix_len: int, steps: int) -> int:
    """FLOPs of one predict: per step the expert GEMMs over the 50 action rows of each sample, the
    MQA attention (8 heads of 256 over prefix + action keys: Q.K^T and P.V) and the fp32 action
    in/out projections."""
    W, H, D, I, A, a = 1024, 8, 256, 4096, 50, 32
    rows = A * batch
    per_layer = (H + 2) * D * W + W * H * D + 2 * I * W + W * I
    gemm = 2 * rows * per_layer * depth
    attn = 4 * H * rows * D * (prefix_len + A) * depth
    heads = 2 * rows * a * W * 2
    return steps * (gemm + attn + heads)


def roofline_entry(schedule, mfma_bound, gbs, nbytes, tflops, flops, launch_us, traffic) -> dict:
    """The bench line's roofline: HBM at B = 1 (60-81 FLOP/B), MFMA where the arithmetic intensity
    passes the ridge (B = 8: 400 FLOP/B); the other side is reported beside it."""
    hbm = {"achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
           "algorithmic_bytes_per_launch": nbytes}
    mfma = {"achieved": round(tflops, 1), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(tflops / BF16_PEAK_TFLOPS, 4), "flops_per_launch": flops}
    main, other = (mfma, ("hbm", hbm)) if mfma_bound else (hbm, ("mfma", mfma))
    out = {"kernel": "denoise_loop_kernel (whole predict, one launch)" if schedule == "persistent"
           else "whole predict (one hipGraph replay)", "bound": "mfma" if mfma_bound else "hbm"}
    out.update(main)
    out.update({"traffic": traffic, "avg_launch_us": round(launch_us, 2), other[0]: other[1]})
    return out


def host_threads() -> int:
    """CPU threads for the CPU baseline: the cores this process may run on (its affinity set, which
    is the host's CPU share where the scheduler restricts it), capped by OMP_NUM_THREADS when set."""
    try:
        n = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        n = os.cpu_count() or 1
    omp = os.environ.get("OMP_NUM_THREADS")
    if omp and omp.isdigit() and int(omp) > 0:
        n = min(n, int(omp))
    return max(1, n)


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor()


class GpuState:
    """Graphics / memory clock (MHz), socket power (W) and temperatures (C) of the benchmark's GPU
    from amdsmi, as the reference's bench records SM clock, memory clock, power and temperature
    with every run (bench/standalone_infer_bench.py:281-316).  The firmware refreshes the metrics
    table about once a second (its system_clock_counter changes then), so a sample counts only if
    the table was refreshed after the GPU started on the predicts: ``fresh()`` says how many such
    refreshes have been seen.  amdsmi enumerates every GPU of the host whatever
    HIP_VISIBLE_DEVICES says, so the handle is resolved by the device's PCI address; on a
    multi-GPU host where that fails nothing is reported rather than another card's state."""

    def __init__(self, device_index: int):
        self.samples: list[dict] = []
        self.error = None
        self.handle = None
        self.start_counter = None
        try:
            import amdsmi
            import torch

            self.smi = amdsmi
            amdsmi.amdsmi_init()
            props = torch.cuda.get_device_properties(device_index)
            bdf = f"{props.pci_domain_id:04x}:{props.pci_bus_id:02x}:{props.pci_device_id:02x}"
            handles = amdsmi.amdsmi_get_processor_handles()
            for h in handles:
                if str(amdsmi.amdsmi_get_gpu_device_bdf(h)).lower().startswith(bdf):
                    self.handle = h
                    break
            if self.handle is None and len(handles) == 1:
                self.handle = handles[0]
            if self.handle is None:
                self.error = f"no amdsmi GPU at PCI address {bdf} among {len(handles)}"
        except Exception as exc:  # diagnostics only
            self.error = repr(exc)

    def _metrics(self):
        return self.smi.amdsmi_get_gpu_metrics_info(self.handle)

    def mark_start(self) -> None:
        """The table's refresh counter now, before the predicts start: samples with it are stale."""
        if self.handle is None:
            return
        try:
            self.start_counter = self._metrics().get("system_clock_counter")
        except Exception as exc:
            self.error = repr(exc)
            self.handle = None

    def sample(self) -> None:
        if self.handle is None:
            return
        try:
            m = self._metrics()
            cnt = m.get("system_clock_counter")
            if cnt == self.start_counter or any(x["counter"] == cnt for x in self.samples):
                return  # not refreshed since the predicts started, or already recorded
            pw = m.get("current_socket_power", "N/A")
            if not isinstance(pw, (int, float)):
                pw = m.get("average_socket_power", "N/A")
            xcd = [c for c in (m.get("current_gfxclks") or []) if isinstance(c, (int, float)) and c < 0xFFFF]
            self.samples.append({"counter": cnt, "gfx_clk_mhz": m.get("current_gfxclk", "N/A"),
                                 "gfx_clk_xcd_min_mhz": min(xcd) if xcd else "N/A", "mem_clk_mhz": m.get("current_uclk", "N/A"),
                                 "power_w": pw, "hotspot_c": m.get("temperature_hotspot", "N/A"),
                                 "mem_temp_c": m.get("temperature_mem", "N/A")})
        except Exception as exc:
            self.error = repr(exc)
            self.handle = None

    def fresh(self) -> int:
        return len(self.samples)

    def summary(self, window: str) -> dict:
        out = {"source": "amdsmi gpu_metrics refreshed while predicts ran (the firmware refreshes it about once a second)",
               "window": window, "samples": len(self.samples)}
        if self.error:
            out["error"] = self.error
        for key in ("gfx_clk_mhz", "gfx_clk_xcd_min_mhz", "mem_clk_mhz", "power_w", "hotspot_c", "mem_temp_c"):
            vals = [x[key] for x in self.samples if isinstance(x[key], (int, float)) and x[key] < 0xFFFF]
            if vals:
                out[key] = {"median": statistics.median(vals), "min": min(vals), "max": max(vals)}
        return out


def run_sampling(gpu: GpuState, done) -> None:
    """Sample the GPU state every ~20 ms until done() (the last event of the queued predicts) holds."""
    while not done():
        gpu.sample()
        time.sleep(0.02)


def clock_window(gpu: GpuState, run_batch, min_fresh: int = 2, max_s: float = 4.0) -> str:
    """Keep the GPU on untimed predicts until the metrics table has been refreshed min_fresh times
    since the predicts started (or max_s passed): the timed region alone is often shorter than
    the firmware's refresh period.  Returns a description of the window for the bench line."""
    import torch

    t0 = time.perf_counter()
    batches = 0
    while gpu.handle is not None and gpu.fresh() < min_fresh and time.perf_counter() - t0 < max_s:
        ev = run_batch()
        run_sampling(gpu, ev.query)
        torch.cuda.synchronize()
        batches += 1
    return f"the timed region, then {batches} batch(es) of untimed predicts of the same workload ({time.perf_counter() - t0:.2f} s)"


def read_traffic(name: str):
    """HBM bytes per launch measured with rocprofv3 FETCH_SIZE/WRITE_SIZE (profiles/)."""
    path = os.path.join(ROOT, "profiles", name)
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(float(line.split(":", 1)[1]))
    except OSError:
        return None
    return None


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="c1", choices=sorted(CONFIGS))
    ap.add_argument("--schedule", default=None, choices=["persistent", "graph"],
                    help="execution schedule (default: the library's choice, persistent on MI355X)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-predicts", type=int, default=8, help="predicts in the CPU-baseline sample")
    ap.add_argument("--workload", default="denoise", choices=["denoise", "prefill", "vision", "e2e"])
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this engine runs the denoise loop on one GPU; runs with --gpus > 1 are not "
              "supported (data-parallel sharding over samples needs no communication).",
              file=sys.stderr)
        return 2
    if args.workload == "prefill":
        return bench_prefill(args)
    if args.workload == "vision":
        return bench_vision(args)
    if args.workload == "e2e":
        return bench_e2e(args)

    import torch

    from pi05_infer import synthetic as S
    from pi05_infer.builder import build_model
    from pi05_infer.engine import Observation

    cfg = CONFIGS[args.config]
    B, P, steps = cfg["batch"], cfg["prefix_len"], 10
    g = S.ExpertGeometry()
    model = build_model("random:0", "pi05_libero", num_steps=steps)
    model.to("cuda")
    k, v = S.make_prefix_kv(g, P, B)
    x1 = S.make_noise(g, B).cuda()
    obs = Observation(k.cuda(), v.cuda(), S.full_prefix_pad(P, B).cuda())
    if args.schedule is not None:
        model.set_schedule(args.schedule)
    model.sample_actions(obs, x1)  # builds the context, primes the prefix (and captures the graph)
    ctx = model._context(B, P, steps)
    schedule = ctx.schedule
    stream = torch.cuda.current_stream()
    xs = [x1.clone() for _ in range(args.warmup + args.steps)]

    for i in range(args.warmup):
        ctx.denoise(xs[i], stream=stream)
    torch.cuda.synchronize()
    ctx.status()
    # timed region: K predicts back to back on `stream`, the stream every launch goes to, with an
    # event between consecutive predicts (K + 1 events: per-predict times and their distribution)
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
    gpu = GpuState(torch.cuda.current_device())
    gpu.mark_start()
    torch.cuda.synchronize()
    evs[0].record(stream)
    for i in range(args.steps):
        ctx.denoise(xs[args.warmup + i], stream=stream)
        evs[i + 1].record(stream)
    # the launches are queued: sample clocks, power and temperatures until the last one ends
    run_sampling(gpu, evs[-1].query)
    torch.cuda.synchronize()
    ctx.status()  # no launch of the timed region timed out

    def soak():  # 50 more predicts (not timed) for the clock window
        for _ in range(50):
            ctx.denoise(xs[0].clone(), stream=stream)
        ev = torch.cuda.Event()
        ev.record(stream)
        return ev

    window = clock_window(gpu, soak)
    ctx.status()
    ms_per_predict = evs[0].elapsed_time(evs[-1]) / args.steps
    per = sorted(evs[i].elapsed_time(evs[i + 1]) for i in range(args.steps))

    def pct(q):
        return per[min(len(per) - 1, int(round(q * (len(per) - 1))))]

    timing = {"mean": round(ms_per_predict, 4), "p50": round(pct(0.5), 4), "p90": round(pct(0.9), 4),
              "min": round(per[0], 4), "max": round(per[-1], 4), "unit": "ms/predict", "n": args.steps}

    # dominant kernel: in the persistent schedule the whole predict is one launch of
    # denoise_loop_kernel, so its average launch duration is the timed region / K (back-to-back
    # launches on one stream; the gap between two launches is included)
    pred_bytes = algorithmic_bytes_per_predict(g.depth, B, P, steps)
    launch_us = ms_per_predict * 1e3
    pred_gbs = pred_bytes / (launch_us * 1e-6) / 1e9
    # the MFMA side of the roofline (the bound at B = 8: 400 FLOP/B against a ridge of ~315)
    pred_flops = algorithmic_flops_per_predict(g.depth, B, P, steps)
    pred_tflops = pred_flops / (launch_us * 1e-6) / 1e12
    mfma_bound = pred_flops / pred_bytes > BF16_PEAK_TFLOPS / HBM_PEAK_GBS * 1e3

    cpu = None
    if not args.no_cpu_baseline:
        from oracle import denoise_oracle as O

        threads = host_threads()
        torch.set_num_threads(threads)
        w = {n: t.cpu() for n, t in model.params.items()}
        og = O.geometry_from(g)
        table = O.adarms_table(w, og, steps)
        pad = S.full_prefix_pad(P, B)
        times = []
        for _ in range(args.cpu_predicts):
            t0 = time.perf_counter()
            O.sample_actions(w, og, k, v, pad, x1.cpu(), steps, table)
            times.append((time.perf_counter() - t0) * 1e3)
        cpu = {
            "value": round(statistics.median(times), 3),
            "unit": "ms/predict",
            "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"{args.cpu_predicts} full predicts ({steps} steps, B={B}, P={P}) of the fp32 CPU oracle, median; "
                      f"host {cpu_model()}, os.cpu_count()={os.cpu_count()}, affinity/OMP threads used={threads}",
        }

    traffic = read_traffic(f"denoise_loop_{args.config}_traffic.txt") if schedule == "persistent" else None
    out = {
        "metric": METRIC,
        "value": round(ms_per_predict, 4),
        "unit": "ms/predict",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_predict, 4),
        "step": f"one predict ({steps} Euler steps)",
        "ms_per_euler_step": round(ms_per_predict / steps, 4),
        "timing": timing,
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random-init weights seed 0, N(0,1) bf16 prefix KV seed 1, N(0,1) noise seed 2)",
        "config": {
            "workload": f"pi0.5 action-expert {steps}-step flow-matching denoise, depth 18, bs={B}, {P}-token prefix KV",
            "batch": B,
            "prefix_len": P,
            "num_steps": steps,
            "schedule": schedule,
            "launches_per_step": ctx.launches_per_step(),
        },
        "roofline": roofline_entry(schedule, mfma_bound, pred_gbs, pred_bytes, pred_tflops, pred_flops, launch_us, traffic),
        "cpu_baseline": cpu,
        "gpu_state": gpu.summary(window),
    }
    print(json.dumps(out), flush=True)
    # release the context (device memory, pinned error word) before interpreter teardown
    model.close()
    torch.cuda.synchronize()
    return 0


if __name__ == "__main__":
    sys.exit(main())
