#!/usr/bin/env python3
"""Benchmark of the greedy speculative-decoding verify path on one MI355X.

Metric: accepted tok/s and verify-step microseconds for the
SmolLM2-1.7B-shape int4-AWQ target with a SmolLM2-135M-shape bf16 draft,
k=3, batch 1 (configuration 2: prompt of 1024 random ids). A "step" is one
speculative step of the reference engine (src/engine.rs:499-717): k draft
rounds, the target's verify pass over k+1 rows, greedy accept, rollback.

Flow: build the synthetic models (random weights, seeded), upload them,
prefill the prompt (untimed), run W warmup steps, then time exactly K steps
(the API synchronises at every step, so the wall clock brackets finished
device work). `value` = tokens emitted in the timed steps / their wall time
(the reference's `generate` rate, src/main.rs:321-327). verify_step_us is
the device time of the verify pass (HIP events, mean over the timed steps).

roofline: GEMV launches are bracketed with HIP events (fg_profile) during
a second pass over K steps from the same state; the target's int4 GEMV
class gives achieved = algorithmic bytes per launch / mean launch time
(no roofline when no target GEMV was recorded).
cpu_baseline: the C oracle (the reference's CPU algorithm restated) resumes
from a copy of the GPU's KV state before the timed steps and runs as many
spec steps as fit in --cpu-seconds on the host cores; its emitted tokens are
compared with the GPU's from the same state. It runs the oracle's fast path
where the CPU has AVX-512: the reference's register tiles, eight-wide
attention scores and spinning thread pool, bit-identical to the portable
loops. The record names the CPU model, the path and the threads.
batched: the batched verify configurations on the same box, after the
headline (unless --no-batched): cfg3 at 32 sequences and cfg4 at 16, each
its emitted tok/s over all sequences, verify and draft step times and the
verify GEMMs' MFMA roofline (see measure_batched).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "accepted tok/s + verify-step µs, 1.7B int4-AWQ target + 135M draft, k=3, bs=1"
HBM_PEAK_GBS = 8000.0
# L2-to-memory bytes per launch of the target int4 decode GEMVs (class mean), counted by
# request size with rocprofv3 --pmc (TCC_EA0_RDREQ_{32,64,128}B, TCC_EA0_WRREQ_64B; a
# plain copy of known size reads back exactly); profiles/gemv_int4_cfg2_pmc.md has the
# commands and the per-GEMV figures, taken at commit 5450b44. A measurement of the
# current kernels, re-taken whenever they change.
MEASURED_TRAFFIC = {"int4": 11_382_519}


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), or the platform's processor string."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or "unknown"


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--config", type=int, default=2)
    ap.add_argument("--seed", type=int, default=2024)
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-profile", action="store_true")
    ap.add_argument("--no-batched", action="store_true",
                    help="skip the batched verify sub-records (cfg3 B=32, cfg4 B=16) of the headline run")
    ap.add_argument("--batched-steps", type=int, default=12)
    ap.add_argument("--batch", type=int, default=0, help="sequences for configs 3/4 (default: the config's own)")
    ap.add_argument("--serve", action="store_true",
                    help="serve 32 requests with a shared prefix through the engine (continuous batching) instead")
    ap.add_argument("--awq", action="store_true",
                    help="time the AWQ alpha search (fg_awq_search) of one 1.7B-shape layer instead")
    ap.add_argument("--prefill", action="store_true",
                    help="only time the warm prefill of the config's prompt through the target and the draft")
    ap.add_argument("--copy-calib", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB and exit (calibrates rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path (--gpus {a.gpus} requested)",
              file=sys.stderr)
        return 2
    if a.copy_calib > 0:
        # one elementwise kernel that reads and writes exactly copy_calib MiB each
        import torch
        src = torch.ones(a.copy_calib << 18, dtype=torch.float32, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.neg(src, out=dst)
        torch.cuda.synchronize()
        log(f"copy calibration: 3 x torch.neg over {a.copy_calib} MiB")
        return 0

    if a.awq:
        return run_awq(a)
    if a.serve:
        return run_serve(a)

    from ferrolm_amd import gpu, spec, synth
    from ferrolm_amd.weights import KIND_NAMES

    t0 = time.time()
    wl = synth.build(a.config, seed=a.seed)
    log(f"built {wl.name} models in {time.time() - t0:.1f}s")
    ctx = gpu.Context(0)
    target = gpu.Model(ctx, wl.target)
    draft = gpu.Model(ctx, wl.draft) if wl.draft is not None else target.truncated(wl.draft_layers)
    log(f"uploaded: target {target.weight_bytes() / 1e9:.3f} GB, draft {draft.weight_bytes() / 1e9:.3f} GB")
    if a.batch > 1 or wl.batch > 1:
        return run_batched(a, wl, ctx, target, draft)
    cfg = wl.target.cfg
    prompt = synth.prompt_ids(wl.prompt_len, cfg.vocab, a.seed)
    if a.prefill:
        print(json.dumps({"workload": wl.name, "prefill": measure_prefill(ctx, target, draft, prompt, None)}),
              flush=True)
        return 0
    k = wl.k
    total_steps = a.warmup + 2 * a.steps
    kv_blocks = (wl.prompt_len + total_steps * (k + 1) + 64) // 16 + 1
    r = spec.Runner(ctx, target, draft, prompt, k, kv_blocks=kv_blocks)
    t1 = time.time()
    first = r.prefill()
    log(f"prefill of {wl.prompt_len} tokens: {time.time() - t1:.2f}s, first token {first}")
    for _ in range(a.warmup):
        r.step()
    log(f"warmup {a.warmup} steps done; context {len(r.tokens)}")

    # Snapshot for the CPU baseline and the full-size parity check.
    snap = None
    if not a.no_cpu:
        snap = dict(tokens=list(r.tokens), computed=r.computed, dcomp=r.dcomp, tb=list(r.tb), db=list(r.db),
                    tkv=[r.tkv.layer(i) for i in range(cfg.layers)],
                    dkv=[r.dkv.layer(i) for i in range(draft.cfg.layers)])
    ctx_start = len(r.tokens)

    # Timed region: exactly K steps.
    st0 = len(r.stats.verify_us)
    emitted = []
    ctx.sync()
    tt = time.perf_counter()
    for _ in range(a.steps):
        emitted.append(r.step())
    ctx.sync()
    elapsed = time.perf_counter() - tt
    n_tok = sum(len(e) for e in emitted)
    value = n_tok / elapsed
    verify_us = float(np.mean(r.stats.verify_us[st0:]))
    draft_us = float(np.mean(r.stats.draft_us[st0:]))
    acc = r.stats.accepted_per_step[st0:]
    acceptance = float(np.sum(acc)) / (k * len(acc)) if acc else 0.0
    log(f"timed {a.steps} steps: {elapsed * 1e3:.1f} ms, {n_tok} tokens, {value:.1f} tok/s, "
        f"verify {verify_us:.1f} us, draft {draft_us:.1f} us, acceptance {acceptance:.3f}")

    roofline = None
    if not a.no_profile:
        gpu.profile(ctx, True)
        gpu.profile_read(ctx, reset=True)
        tp = time.perf_counter()
        for _ in range(a.steps):
            r.step()
        ctx.sync()
        prof_elapsed = time.perf_counter() - tp
        recs = gpu.profile_read(ctx, reset=True)
        gpu.profile(ctx, False)
        for rec in recs:
            what = "gemm" if rec["gemm"] else f"gemv passes<={rec['passes']}"
            log(f"{what} {rec['kind']}: {rec['launches']} launches, "
                f"{rec['us'] / rec['launches']:.2f} us avg, {rec['bytes'] / rec['us'] / 1e3:.0f} GB/s")
        log(f"profiled pass: {prof_elapsed * 1e3:.1f} ms for {a.steps} steps "
            f"(unprofiled {elapsed * 1e3:.1f} ms)")
        tkind = KIND_NAMES[wl.target_kind]
        dom = [x for x in recs if x["kind"] == tkind and not x["gemm"]]
        if dom:
            dom = max(dom, key=lambda x: x["us"])
            ach = dom["bytes"] / dom["us"] / 1e3
            roofline = {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": round(ach / HBM_PEAK_GBS, 4),
                        "traffic": MEASURED_TRAFFIC.get(dom["kind"]) if a.config == 2 else None,
                        "kernel": f"k_gemv {dom['kind']} (target projections, m={k + 1})",
                        "bytes_per_launch": round(dom["bytes"] / dom["launches"]),
                        "us_per_launch": round(dom["us"] / dom["launches"], 3), "launches": dom["launches"]}

    prefill = measure_prefill(ctx, target, draft, prompt, first[0])

    cpu = None
    parity = None
    if snap is not None:
        import oracle
        ncores = len(os.sched_getaffinity(0))
        threads = int(os.environ.get("OMP_NUM_THREADS", ncores))
        oracle.threads(threads)
        fast = oracle.fast(True, threads)
        ot = oracle.Model(wl.target)
        od = oracle.Model(wl.draft) if wl.draft is not None else ot.truncated(wl.draft_layers)
        okv = ot.kv(kv_blocks)
        odkv = od.kv(kv_blocks + 64)
        for i, (kk, vv) in enumerate(snap["tkv"]):
            okv.set_layer(i, kk, vv)
        for i, (kk, vv) in enumerate(snap["dkv"]):
            odkv.set_layer(i, kk, vv)
        tokens = list(snap["tokens"])
        comp, dcomp = snap["computed"], snap["dcomp"]
        tb, db = list(snap["tb"]), list(snap["db"])
        pool_t, pool_d = max(tb) + 1, max(db) + 1
        cpu_emitted = []
        tc = time.perf_counter()
        while (time.perf_counter() - tc < a.cpu_seconds or len(cpu_emitted) < 2) and len(cpu_emitted) < a.steps:
            while len(tb) * 16 < comp + k + 1:
                tb.append(pool_t)
                pool_t += 1
            while len(db) * 16 < len(tokens) + k - 1:
                db.append(pool_d)
                pool_d += 1
            out, _, comp, dcomp = oracle.spec_step(ot, okv, od, odkv, tokens, comp, dcomp, tb, db, k)
            cpu_emitted.append([int(x) for x in out])
            tokens.extend(int(x) for x in out)
        cpu_elapsed = time.perf_counter() - tc
        n_cpu = sum(len(e) for e in cpu_emitted)
        oracle.fast(False)
        path = ("the reference's AVX-512 register tiles and spinning pool" if fast
                else "portable loops (no AVX-512 on this CPU)")
        cpu = {"value": round(n_cpu / cpu_elapsed, 3), "unit": "tok/s", "cores": threads, "kind": "port",
               "sample": f"{len(cpu_emitted)} spec steps of {wl.name} from the GPU's KV state at context "
                         f"{ctx_start} ({n_cpu} tokens, {cpu_elapsed:.1f}s), C oracle, {path}, {threads} threads",
               "ms_per_step": round(cpu_elapsed / len(cpu_emitted) * 1e3, 2), "cpu_model": cpu_model(),
               "path": "avx512" if fast else "portable"}
        gpu_first = emitted[:len(cpu_emitted)]
        same = sum(1 for x, y in zip(gpu_first, cpu_emitted) if x == y)
        parity = {"steps_compared": len(cpu_emitted), "steps_identical": same}
        log(f"cpu baseline: {cpu['value']} tok/s ({cpu['ms_per_step']} ms/step); parity {same}/{len(cpu_emitted)}")

    batched = None
    if a.config == 2 and not a.no_batched:
        # the headline's models and caches are not needed any more
        del r
        target.close()
        draft.close()
        batched = []
        for c, B in ((3, 32), (4, 16)):
            bwl = synth.build(c, seed=a.seed)
            bt, bd = gpu.Model(ctx, bwl.target), gpu.Model(ctx, bwl.draft)
            batched.append(measure_batched(a, bwl, ctx, bt, bd, B, a.batched_steps, 3))
            bt.close()
            bd.close()

    line = {
        "metric": METRIC, "value": round(value, 2), "unit": "tok/s", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": round(elapsed / a.steps * 1e3, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": KIND_NAMES[wl.target_kind], "data": "synthetic",
        "config": {"workload": f"{wl.name}: {'SmolLM2-1.7B' if a.config == 2 else cfg.hidden}-shape "
                               f"{KIND_NAMES[wl.target_kind]} target + draft, k={k}, batch {wl.batch}, "
                               f"prompt {wl.prompt_len} random ids",
                   "target_layers": cfg.layers, "hidden": cfg.hidden, "k": k, "batch": wl.batch,
                   "prompt": wl.prompt_len, "context_at_timed_start": ctx_start},
        "verify_step_us": round(verify_us, 2), "draft_us": round(draft_us, 2), "acceptance": round(acceptance, 4),
        "roofline": roofline, "cpu_baseline": cpu, "parity": parity, "prefill": prefill, "batched": batched,
    }
    print(json.dumps(line), flush=True)
    return 0


def measure_prefill(ctx, target, draft, prompt, first_token, reps=5):
    """Time to first token of the prompt: one forward of the whole prompt
    through each model (the target's gives the first token; the draft's runs in
    the first speculative step), warm, into caches of their own so the
    speculative state is untouched (first_token, when given, is checked against
    the target's). Wall time per forward, host planning and
    launches included. `tflops` is the target's algorithmic rate: 2 flops per
    weight per token, the lm_head for the last row only, and causal attention
    (QK and PV, 4·hd flops per query head and visible position)."""
    from ferrolm_amd import gpu
    n = len(prompt)
    nb = (n + 15) // 16
    ch = [(prompt, 0, list(range(nb)), gpu.LOGITS_LAST)]
    out = {"tokens": n, "reps": reps}
    for name, m in (("target", target), ("draft", draft)):
        kv = gpu.KvCache(ctx, m.cfg, nb)
        o = gpu.forward(ctx, m, kv, ch, logits=False)
        if name == "target" and first_token is not None and int(o.argmax[0]) != first_token:
            raise RuntimeError("a second prefill of the prompt gave another first token")
        ctx.sync()
        t0 = time.perf_counter()
        for _ in range(reps):
            gpu.forward(ctx, m, kv, ch, logits=False)
        ctx.sync()
        out[f"{name}_ms"] = round((time.perf_counter() - t0) / reps * 1e3, 3)
        del kv
    c = target.cfg
    qd, kvd = c.heads * c.head_dim, c.kv_heads * c.head_dim
    layer_params = c.hidden * (qd + 2 * kvd) + qd * c.hidden + 3 * c.intermediate * c.hidden
    flops = (2.0 * n * layer_params * c.layers + 2.0 * c.vocab * c.hidden
             + 4.0 * c.head_dim * c.heads * (n * (n + 1) / 2) * c.layers)
    out["target_tok_per_s"] = round(n / out["target_ms"] * 1e3, 1)
    out["target_tflops"] = round(flops / (out["target_ms"] * 1e-3) / 1e12, 1)
    log(f"prefill of {n} tokens (warm, {reps} reps): target {out['target_ms']:.2f} ms "
        f"({out['target_tok_per_s']:.0f} tok/s, {out['target_tflops']:.0f} TFLOP/s), draft {out['draft_ms']:.2f} ms")
    return out


def measure_batched(a, wl, ctx, target, draft, B: int, steps: int, warmup: int) -> dict:
    """Batched verify (configs 3 and 4): B sequences with context lengths drawn
    uniformly (cfg3 128-2048, cfg4 512-4096), block tables from a shuffled pool,
    every step one device speculative step over all of them (Engine::execute
    over decoding sequences, src/engine.rs:499-654). Returns emitted tok/s over
    all sequences, the verify and draft device times per step, and the MFMA
    roofline of the target's verify GEMMs: the dominant weight kind's GEMM
    launches (events around each, in a second pass of `steps` steps), the
    algorithmic 2*rows*n*k over their summed time against the dense bf16 peak.
    No CPU baseline here: the oracle would need a host copy of the whole cache;
    every sequence's step is checked against the oracle by a GPU test."""
    from ferrolm_amd import gpu, spec, synth
    from ferrolm_amd.weights import KIND_NAMES
    k = wl.k
    cfg = wl.target.cfg
    lo, hi = (512, 4096) if wl.name == "cfg4" else (128, 2048)
    rng = np.random.default_rng(a.seed)
    lens = [int(x) for x in rng.integers(lo, hi + 1, B)]
    prompts = [[int(t) for t in synth.prompt_ids(n, cfg.vocab, a.seed + 1 + i)] for i, n in enumerate(lens)]
    total = warmup + 2 * steps
    blocks = sum((n + total * (k + 1) + 32) // 16 + 2 for n in lens)
    b = spec.Batch(ctx, target, draft, prompts, k, kv_blocks=blocks, seed=a.seed)
    t1 = time.time()
    b.prefill(max_tokens=2048)
    log(f"{wl.name} B={B}: prefill of {B} prompts ({sum(lens)} tokens, {min(lens)}..{max(lens)}): "
        f"{time.time() - t1:.2f}s")
    for _ in range(warmup):
        b.step()
    st0 = len(b.stats.verify_us)
    ctx.sync()
    tt = time.perf_counter()
    n_tok = 0
    for _ in range(steps):
        n_tok += sum(len(e) for e in b.step())
    ctx.sync()
    elapsed = time.perf_counter() - tt
    value = n_tok / elapsed
    verify_us = float(np.mean(b.stats.verify_us[st0:]))
    draft_us = float(np.mean(b.stats.draft_us[st0:]))
    acceptance = b.stats.accepted / max(1, b.stats.proposed)
    log(f"{wl.name} B={B}: timed {steps} steps: {elapsed * 1e3:.1f} ms, {n_tok} tokens, {value:.1f} tok/s, "
        f"verify {verify_us:.1f} us, draft {draft_us:.1f} us")
    roofline = None
    if not a.no_profile:
        gpu.profile(ctx, True)
        gpu.profile_read(ctx, reset=True)
        for _ in range(steps):
            b.step()
        ctx.sync()
        recs = gpu.profile_read(ctx, reset=True)
        gpu.profile(ctx, False)
        for rec in recs:
            what = "gemm" if rec["gemm"] else f"gemv passes<={rec['passes']}"
            log(f"{wl.name} {what} {rec['kind']}: {rec['launches']} launches, "
                f"{rec['us'] / rec['launches']:.2f} us avg, {rec['bytes'] / rec['us'] / 1e3:.0f} GB/s, "
                f"{rec['flops'] / rec['us'] / 1e6:.1f} TFLOP/s")
        tkind = KIND_NAMES[wl.target_kind]
        dom = [x for x in recs if x["kind"] == tkind and x["gemm"]]
        if dom:
            dom = max(dom, key=lambda x: x["us"])
            ach = dom["flops"] / dom["us"] / 1e6
            # the GEMM runs bf16 MFMA on two activation pieces (hi + lo): it issues
            # twice the algorithmic flops; both rates are priced against the dense
            # bf16 peak
            roofline = {"bound": "mfma", "achieved": round(ach, 2), "peak": 2500.0, "unit": "TFLOP/s",
                        "frac": round(ach / 2500.0, 5), "mfma_issue_frac": round(2 * ach / 2500.0, 5),
                        "traffic": None,
                        "kernel": f"k_gemm {dom['kind']} weights, bf16 MFMA (target verify GEMMs, {B * (k + 1)} rows)",
                        "flops_per_launch": round(dom["flops"] / dom["launches"]),
                        "us_per_launch": round(dom["us"] / dom["launches"], 3), "launches": dom["launches"]}
    rec = {"workload": f"{wl.name}: {KIND_NAMES[wl.target_kind]} target ({cfg.layers} layers, hidden {cfg.hidden}) "
                       f"+ bf16 draft, k={k}, {B} sequences, contexts {lo}-{hi}, shuffled 16-token blocks",
           "value": round(value, 2), "unit": "tok/s", "batch": B, "k": k, "steps": steps, "warmup": warmup,
           "ms_per_step": round(elapsed / steps * 1e3, 4), "verify_step_us": round(verify_us, 2),
           "draft_us": round(draft_us, 2), "acceptance": round(acceptance, 4), "roofline": roofline}
    del b
    return rec


def run_batched(a, wl, ctx, target, draft) -> int:
    """--config 3 / 4: the batched verify (measure_batched) as the line."""
    from ferrolm_amd.weights import KIND_NAMES
    B = a.batch if a.batch > 1 else wl.batch
    cfg = wl.target.cfg
    r = measure_batched(a, wl, ctx, target, draft, B, a.steps, a.warmup)
    metric = (f"accepted tok/s + verify-step µs, {cfg.hidden}-hidden {KIND_NAMES[wl.target_kind]} target + draft, "
              f"k={wl.k}, bs={B}")
    line = {
        "metric": metric, "value": r["value"], "unit": "tok/s", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": r["ms_per_step"], "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": KIND_NAMES[wl.target_kind], "data": "synthetic",
        "config": {"workload": r["workload"], "batch": B, "k": wl.k},
        "verify_step_us": r["verify_step_us"], "draft_us": r["draft_us"], "acceptance": r["acceptance"],
        "roofline": r["roofline"], "cpu_baseline": None, "parity": None,
    }
    print(json.dumps(line), flush=True)
    return 0


def run_serve(a) -> int:
    """--serve: the serving engine (ferrolm_amd.engine: continuous batching,
    chunked prefill, prefix cache, speculation) on configuration 3's models
    (1.7B-shape int8 target, 135M-shape bf16 draft, k=4): 32 greedy requests,
    each a shared 512-token system prompt plus 128 tokens of its own, 64 new
    tokens each, submitted at once; a 2048-token step budget. value = tokens
    generated / wall time from the first submission to the last finish
    (prefill included). No CPU baseline: the oracle has no multi-request
    engine, and serving 32 1.7B requests on the host would take hours."""
    from ferrolm_amd import gpu, synth
    from ferrolm_amd.engine import Engine, EngineConfig, Params

    t0 = time.time()
    wl = synth.build(3, seed=a.seed)
    log(f"built {wl.name} models in {time.time() - t0:.1f}s")
    ctx = gpu.Context(0)
    target = gpu.Model(ctx, wl.target)
    draft = gpu.Model(ctx, wl.draft)
    cfg = wl.target.cfg
    system = [int(t) for t in synth.prompt_ids(512, cfg.vocab, a.seed)]
    reqs = [system + [int(t) for t in synth.prompt_ids(128, cfg.vocab, a.seed + 1 + i)] for i in range(32)]
    ecfg = EngineConfig(kv_blocks=32 * 48, max_batch_tokens=2048, max_seqs=32, spec_k=wl.k)

    def serve(n_reqs):
        e = Engine(ctx, target, draft, ecfg)
        out = [e.submit(p, Params(max_tokens=64, ignore_eos=True)) for p in reqs[:n_reqs]]
        t = time.perf_counter()
        e.run_until_idle()
        return out, e.stats, time.perf_counter() - t

    serve(2)  # warm the graphs and allocations
    out, st, el = serve(len(reqs))
    gen = sum(len(r.tokens) for r in out)
    log(f"served {len(out)} requests: {gen} tokens in {el:.2f}s, {st.steps} steps, cached {st.cached_tokens}")
    line = {
        "metric": "serving throughput: generated tok/s, 32 requests with a shared 512-token prefix",
        "value": round(gen / el, 2), "unit": "tok/s", "n_gpus": 1, "steps": st.steps, "warmup": 1,
        "ms_per_step": round(el / max(st.steps, 1) * 1e3, 3), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8", "data": "synthetic",
        "config": {"workload": "serve: cfg3 models (1.7B int8 + 135M bf16 draft, k=4), 32 requests x (512 shared + "
                               "128 own) prompt tokens, 64 new each, budget 2048", "requests": len(out)},
        "generated_tokens": gen, "prompt_tokens": st.prompt_tokens, "cached_tokens": st.cached_tokens,
        "computed_tokens": st.computed_tokens, "preemptions": st.preemptions, "peak_running": st.peak_running,
        "spec_proposed": st.spec_proposed, "spec_accepted": st.spec_accepted,
        "roofline": None, "cpu_baseline": None, "parity": None,
    }
    print(json.dumps(line), flush=True)
    return 0


def run_awq(a) -> int:
    """--awq: the AWQ alpha search with its final quantization (fg_awq_search,
    src/awq.rs:152-217) over the four projections of one layer of the
    SmolLM2-1.7B shape (q/k/v 6144x2048, o 2048x2048, gate/up 16384x2048,
    down 2048x8192), int4, 256 calibration rows per projection (N(0, 1), 1% of
    the channels x 20; the reference's calibrate keeps 256 rows in its test).
    value = layers per second, wall time of the four calls, host-device copies
    included. cpu_baseline: the C oracle's search over the same four
    projections on the host cores, whose alphas, errors, codes and scales
    must equal the device's (parity)."""
    from ferrolm_amd import gpu, host
    from ferrolm_amd.weights import INT4, bf16_to_f32, shape

    cfg = shape("smollm2-1.7b")
    H, inter = cfg.hidden, cfg.intermediate
    projs = [("qkv", (cfg.heads + 2 * cfg.kv_heads) * cfg.head_dim, H), ("o", H, cfg.heads * cfg.head_dim),
             ("gate_up", 2 * inter, H), ("down", H, inter)]
    m = 256
    rng = np.random.default_rng(a.seed)
    mats = []
    for i, (name, rows, kdim) in enumerate(projs):
        w = bf16_to_f32(host.random_bf16(a.seed, 900 + i, rows, kdim, 0.02))
        x = rng.standard_normal((m, kdim)).astype(np.float32)
        x[:, rng.choice(kdim, kdim // 100, replace=False)] *= 20.0
        mats.append((name, w, x))
    ctx = gpu.Context(0)
    gpu.awq_search(ctx, INT4, mats[1][1][:64, :256].copy(), mats[1][2][:16, :256].copy())  # warm the path
    per, res = {}, {}
    t_all = time.perf_counter()
    for name, w, x in mats:
        t = time.perf_counter()
        res[name] = gpu.awq_search(ctx, INT4, w, x)
        per[name] = time.perf_counter() - t
        log(f"device awq search {name} {w.shape[0]}x{w.shape[1]}: {per[name] * 1e3:.1f} ms, alpha {res[name][1]:.1f}")
    dev = time.perf_counter() - t_all
    t = time.perf_counter()
    gpu.quantize(ctx, INT4, mats[2][1])
    tq = time.perf_counter() - t
    cpu, parity = None, None
    if not a.no_cpu:
        import oracle
        threads = int(os.environ.get("OMP_NUM_THREADS", len(os.sched_getaffinity(0))))
        oracle.threads(threads)
        same = 0
        tc = time.perf_counter()
        for name, w, x in mats:
            o = oracle.awq_search(INT4, w, x)
            d = res[name]
            same += int(d[1] == o[1] and d[2] == o[2] and d[3] == o[3] and np.array_equal(d[0], o[0])
                        and np.array_equal(d[4].q, o[4].q) and np.array_equal(d[4].s, o[4].s))
        ce = time.perf_counter() - tc
        cpu = {"value": round(1.0 / ce, 4), "unit": "layers/s", "cores": threads, "kind": "port",
               "sample": f"the same four projections, C oracle, {threads} threads, {ce:.1f}s"}
        parity = {"projections_compared": len(mats), "projections_identical": same}
        log(f"cpu baseline: {ce:.1f} s per layer; parity {same}/{len(mats)}")
    flops = sum(2.0 * m * w.shape[0] * w.shape[1] * 12 for _, w, _ in mats)
    line = {
        "metric": "AWQ alpha search + quantization, one SmolLM2-1.7B-shape layer, int4, 256 calibration rows",
        "value": round(1.0 / dev, 3), "unit": "layers/s", "n_gpus": 1, "steps": 1, "warmup": 1,
        "ms_per_step": round(dev * 1e3, 2), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic",
        "config": {"workload": "awq: 4 projections of one 1.7B-shape layer, int4, m=256", "calibration_rows": m},
        "per_projection_ms": {k: round(v * 1e3, 1) for k, v in per.items()},
        "alphas": {k: r[1] for k, r in res.items()},
        "quantize_gate_up_ms": round(tq * 1e3, 2),
        "matmul_fma_tflops": round(flops / dev / 1e12, 2),
        "roofline": None, "cpu_baseline": cpu, "parity": parity,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
