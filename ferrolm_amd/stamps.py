"""In-kernel timeline of one speculative step, as the step graphs replay it.

    python -m ferrolm_amd.build --stamps        # libferro_gpu_stamps.so (-DFERRO_STAMPS)
    python -m ferrolm_amd.stamps [--config 2] [--warmup 8] [--steps 3]

Runs the configuration's greedy decode (graphs on, as bench.py times it) on the
library built with stamps: every GEMV, attention, merge and split
output-projection launch takes a slot in launch order, and thread 0 of each of
its workgroups records s_memrealtime (100 MHz) at entry and at exit. After the
warmup it clears the slots, runs one step, and prints each launch in order: its
first entry relative to the step's first entry, its span (first entry to last
exit), the median workgroup's own time, and the gap from its last exit to the
next launch's first entry (a graph node boundary, plus any launch without a
slot: the embedding, the argmax and the accept kernels). Then one line per
kernel label. Repeated over --steps steps, the spans and gaps are medians.
Measurement aid only: the product library is built without stamps.
"""
from __future__ import annotations

import argparse
import os
import sys
from collections import defaultdict

import numpy as np

TICK_US = 0.01  # s_memrealtime counts at 100 MHz


def timeline(ticks: np.ndarray, labels: list) -> list:
    """Per labelled slot with records: (label, workgroups, first entry, last exit,
    median workgroup ticks), ordered by first entry."""
    out = []
    for s, lab in enumerate(labels):
        t = ticks[s].astype(np.int64)
        live = t[:, 0] > 0
        if not live.any():
            continue
        t = t[live]
        out.append((lab, int(live.sum()), int(t[:, 0].min()), int(t[:, 1].max()), float(np.median(t[:, 1] - t[:, 0]))))
    return sorted(out, key=lambda x: x[2])


def main() -> int:
    # the binding picks its library when it is first imported: the stamps build
    os.environ["FERRO_STAMPS"] = "1"
    from . import gpu, spec, synth
    if not gpu.LIB_PATH.name.endswith("_stamps.so"):
        raise SystemExit("ferrolm_amd.gpu was imported before the stamps library was selected")
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--config", type=int, default=2)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--seed", type=int, default=2024)
    a = ap.parse_args()
    wl = synth.build(a.config, seed=a.seed)
    ctx = gpu.Context(0)
    target = gpu.Model(ctx, wl.target)
    draft = gpu.Model(ctx, wl.draft) if wl.draft is not None else target.truncated(wl.draft_layers)
    prompt = synth.prompt_ids(wl.prompt_len, wl.target.cfg.vocab, a.seed)
    r = spec.Runner(ctx, target, draft, prompt, wl.k,
                    kv_blocks=(wl.prompt_len + (a.warmup + a.steps + 2) * (wl.k + 1) + 64) // 16 + 1)
    r.prefill()
    for _ in range(a.warmup):
        r.step()
    runs, step_us = [], []
    for _ in range(a.steps):
        gpu.stamps_reset(ctx)
        r.step()
        ticks, labels = gpu.stamps_read(ctx)
        runs.append(timeline(ticks, labels))
        step_us.append(gpu.last_step_times(ctx))
    n = min(len(x) for x in runs)
    rows = []
    for i in range(n):
        lab = runs[0][i][0]
        t0s = [x[0][2] for x in runs]
        start = np.median([x[i][2] - t0 for x, t0 in zip(runs, t0s)]) * TICK_US
        span = np.median([x[i][3] - x[i][2] for x in runs]) * TICK_US
        wg = np.median([x[i][4] for x in runs]) * TICK_US
        gap = np.median([x[i + 1][2] - x[i][3] for x in runs]) * TICK_US if i + 1 < n else float("nan")
        rows.append((lab, runs[0][i][1], start, span, wg, gap))
    st = np.median(np.array(step_us), axis=0)
    print(f"# In-kernel timeline, {wl.name}, one speculative step (graphs), median of {a.steps} steps\n")
    print(f"Device times (HIP events): draft {st[0]:.1f} us, verify {st[1]:.1f} us, step {st[2]:.1f} us. "
          f"Launches with a slot: {n}; first entry to last exit: {(runs[0][n - 1][3] - runs[0][0][2]) * TICK_US:.1f} us "
          f"(first step).\n")
    print("| # | kernel | workgroups | start us | span us | median workgroup us | gap to next us |")
    print("|---|---|---|---|---|---|---|")
    for i, (lab, w, start, span, wg, gap) in enumerate(rows):
        print(f"| {i} | {lab} | {w} | {start:.2f} | {span:.2f} | {wg:.2f} | {gap:.2f} |")
    agg = defaultdict(list)
    for i, (lab, w, start, span, wg, gap) in enumerate(rows):
        agg[lab].append((span, gap, wg))
    print("\n| kernel | launches | mean span us | mean gap to next us | mean median workgroup us | total span + gap us |")
    print("|---|---|---|---|---|---|")
    tot_s = tot_g = 0.0
    for lab, v in sorted(agg.items(), key=lambda kv: -sum(x[0] + (0 if np.isnan(x[1]) else x[1]) for x in kv[1])):
        sp = np.array([x[0] for x in v])
        gp = np.array([x[1] for x in v if not np.isnan(x[1])])
        tot_s += sp.sum()
        tot_g += gp.sum()
        print(f"| {lab} | {len(v)} | {sp.mean():.2f} | {gp.mean() if len(gp) else float('nan'):.2f} | "
              f"{np.mean([x[2] for x in v]):.2f} | {sp.sum() + gp.sum():.1f} |")
    print(f"\nSum of spans {tot_s:.1f} us, sum of gaps {tot_g:.1f} us.")
    return 0


if __name__ == "__main__":
    sys.exit(main())
