"""Per-phase timeline of one decoder layer inside the persistent denoise kernel.

Loads the profiling build of the denoise library (``python pi05-infer_amd/build_lib.py --stamps``,
compiled with -DPI05_PHASE_TIMESTAMPS: thread 0 of every workgroup records s_memrealtime, a
100 MHz counter common to the whole device, at fixed points of every phase of Euler step 1,
layers 0..3), runs whole predicts of the chosen workload and prints, for one layer, each recorded
event's time after the previous layer's last down_proj publish: median / max / min over the
workgroups that record it, averaged over the predicts.

Events (qkv and gate_up at B = 1): 0 phase entry, 1 before the flag wait, 2 wait done, 4 MFMAs
done (gate_up: wave 0, which only polls, passes it right after the wait), 3 after the barrier that
follows the MFMAs, 7 cross-wave reduction done, 5 before the publish, 6 after it.  Attention splits: 4/7/8/9 waves 0/1/2/3 done attending, 3 the
waves' partials exchanged, 5 stores issued, 6 published.  Merges: 1, 2, 6.  o_proj: 2 wait done,
4 MFMAs done, 5/6 publish.  down_proj: 2 wait done, 4 MFMAs done, 8/9 publish (the batch
instances, which split K: 5 quarter partial stored, 7 finisher's wait done, 8/9 finisher publish).

    python pi05-infer_amd/phase_stamps.py [--batch B] [--prefix P] [--layer L] [--reps K]
"""

from __future__ import annotations

import argparse
import ctypes
import os
import statistics
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
for _p in (ROOT, HERE):
    if _p not in sys.path:
        sys.path.insert(0, _p)

PHASES = ["io", "qkv", "split", "merge", "o_proj", "gate_up", "down"]
N_WG, N_LAYERS, N_PH, N_EV = 256, 4, 7, 16  # pi05_phase_ts[workgroup][layer * 7 + phase][event]


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--prefix", type=int, default=968)
    ap.add_argument("--layer", type=int, default=2, help="layer of Euler step 1 to show (1..3)")
    ap.add_argument("--reps", type=int, default=5)
    args = ap.parse_args()
    if not 1 <= args.layer < N_LAYERS:
        raise SystemExit("--layer must be 1, 2 or 3 (the previous layer's publish is the origin)")
    from pi05_infer import _ext

    path = os.path.join(HERE, "pi05_infer", "stamps", _ext.LIB_NAME)
    lib = _ext.load_library(path)
    lib.pi05_debug_phase_timestamps.restype = ctypes.c_int
    lib.pi05_debug_phase_timestamps.argtypes = [ctypes.c_void_p]
    lib.pi05_debug_phase_timestamps_clear.restype = ctypes.c_int
    import torch

    from pi05_infer import synthetic as S
    from pi05_infer.builder import build_model
    from pi05_infer.engine import Observation

    B, P, steps = args.batch, args.prefix, 10
    g = S.ExpertGeometry()
    model = build_model("random:0", "pi05_libero", num_steps=steps)
    model.to("cuda")
    k, v = S.make_prefix_kv(g, P, B)
    x1 = S.make_noise(g, B).cuda()
    model.sample_actions(Observation(k.cuda(), v.cuda(), S.full_prefix_pad(P, B).cuda()), x1)
    ctx = model._context(B, P, steps)
    st = torch.cuda.current_stream()
    for _ in range(5):
        ctx.denoise(x1.clone(), stream=st)
    torch.cuda.synchronize()
    n = N_WG * N_LAYERS * N_PH * N_EV
    L = args.layer
    per_event: dict = {}
    for rep in range(args.reps):
        if lib.pi05_debug_phase_timestamps_clear() != 0:
            raise RuntimeError("clearing the stamps failed")
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(st)
        ctx.denoise(x1.clone(), stream=st)
        e1.record(st)
        torch.cuda.synchronize()
        ctx.status()
        buf = (ctypes.c_ulonglong * n)()
        if lib.pi05_debug_phase_timestamps(ctypes.addressof(buf)) != 0:
            raise RuntimeError("reading the stamps failed")
        ts = np.frombuffer(buf, dtype=np.uint64).reshape(N_WG, N_LAYERS, N_PH, N_EV).astype(np.int64)
        print(f"predict {rep}: {e0.elapsed_time(e1):.3f} ms (profiling build)", flush=True)
        prev = ts[:, L - 1, 6, 9]
        t0 = prev[prev > 0].max()
        for ph in range(1, N_PH):
            for ev in range(N_EV):
                col = ts[:, L, ph, ev]
                m = col > 0
                if m.any():
                    us = (col[m] - t0) / 100.0
                    per_event.setdefault((ph, ev), []).append((np.median(us), us.max(), us.min(), int(m.sum())))
    print(f"B={B}, P={P}: layer {L} of Euler step 1, us after layer {L - 1}'s last down_proj publish; "
          f"median / max / min over the workgroups, mean over {args.reps} predicts")
    for (ph, ev), rows in sorted(per_event.items()):
        med, mx, mn = (statistics.mean(r[i] for r in rows) for i in range(3))
        print(f"{PHASES[ph]:8s} ev{ev:2d}: median {med:7.2f}  max {mx:7.2f}  min {mn:7.2f}  workgroups {rows[0][3]}")
    model.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
