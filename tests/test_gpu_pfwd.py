"""The persistent forward: a greedy draft round, or the target's verify pass
with its accept, of one sequence as one launch (Engine::propose and
Engine::execute, src/engine.rs:563-717; each is Model::forward,
src/model.rs:269-362, then sampler::argmax, src/sampler.rs:42-51).

- A target drafting for itself accepts every proposal and emits its own
  greedy tokens (tests/engine.rs:134-160), for GQA groups of 1, 3 and 4, a
  qkv bias, tied embeddings and padded k-blocks; the acceptance count is
  the check that every draft argmax is right.
- With a one-layer draft, every step (emitted ids, accepted count, the
  draft's progress) equals oracle.spec_step from the device's own state,
  and the caches equal the oracle's after the steps: bf16, int8 and int4
  weights (the draft is the target's first layer, so both launches take
  the same weight kind).
- Tails of 3 and 4 rows (a draft that lags the target), across a 64-position
  span boundary: the same, from the same state.
- The same generation with and without the persistent path (FERRO_PFWD=1 at
  context creation turns it on) emits the same ids with the same
  acceptance; the caches agree to 1e-5 of their largest entry and are not
  bit-identical (the persistent path really ran).
- A wait limit of one poll (FERRO_PFWD_SPIN=1) makes the launch time out:
  the step reports an error instead of results, and the next context works.

The persistent path is opt-in: every context here that should take it is
made with FERRO_PFWD=1.
"""
import os

import numpy as np
import pytest

import oracle
from ferrolm_amd import gpu, spec
from ferrolm_amd.synth import quantize_model, random_model
from ferrolm_amd.weights import BF16, INT4, INT8, Config

pytestmark = pytest.mark.gpu

CFGS = {
    # hidden 352: 11 k-blocks padded to 12
    "gqa3": Config(vocab=2048, hidden=352, intermediate=704, layers=3, heads=6, kv_heads=2, head_dim=64,
                   rms_eps=1e-5, max_position=512),
    "gqa4-bias-tied": Config(vocab=1024, hidden=256, intermediate=512, layers=2, heads=8, kv_heads=2, head_dim=64,
                             rms_eps=1e-6, max_position=512, qkv_bias=True, tie_embeddings=True),
    "gqa1": Config(vocab=1536, hidden=256, intermediate=768, layers=2, heads=4, kv_heads=4, head_dim=64,
                   rms_eps=1e-5, max_position=512),
}
K = 3


def log(msg):
    print(f"[pfwd] {msg}", flush=True)


def prompt_for(cfg, n, seed):
    return [int(x) for x in np.random.default_rng(seed).integers(3, cfg.vocab, n)]


def context(**env):
    """A context created with the given environment switches."""
    old = {k: os.environ.get(k) for k in env}
    os.environ.update(env)
    try:
        return gpu.Context(0)
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


@pytest.fixture(scope="module")
def pctx():
    c = context(FERRO_PFWD="1")
    yield c
    c.close()


def copy_kv(gkv, okv, layers):
    for i in range(layers):
        okv.set_layer(i, *gkv.layer(i))


def kv_close(gkv, okv, layers, tol=1e-4):
    for i in range(layers):
        for g, o in zip(gkv.layer(i), okv.layer(i)):
            assert np.abs(g - o).max() <= tol * max(1e-30, np.abs(o).max()), i


@pytest.mark.parametrize("name,kind", [(n, BF16) for n in CFGS] + [("gqa3", INT8), ("gqa3", INT4)],
                         ids=[*CFGS, "gqa3-int8", "gqa3-int4"])
def test_self_draft_accepts_every_proposal(pctx, name, kind):
    ctx = pctx
    cfg = CFGS[name]
    hm = random_model(cfg, seed=11, std=0.05)
    if kind != BF16:
        hm = quantize_model(hm, kind)
    om = oracle.Model(hm)
    prompt = prompt_for(cfg, 50, 3)
    want, _, _ = oracle.generate(om, None, prompt, 60, 0, kv_blocks=64)
    tm = gpu.Model(ctx, hm)
    st = spec.GenStats()
    got = spec.generate(ctx, tm, tm.truncated(cfg.layers), prompt, 60, K, kv_blocks=64, stats=st)
    log(f"{name}: {st.spec_steps} steps, {st.accepted}/{st.proposed} accepted")
    assert np.array_equal(got, want)
    assert st.spec_steps > 0 and st.accepted == st.proposed


@pytest.mark.parametrize("kind", [BF16, INT8, INT4], ids=["bf16", "int8", "int4"])
def test_one_layer_draft_steps_match_oracle(pctx, kind):
    ctx = pctx
    cfg = CFGS["gqa3"]
    hm = random_model(cfg, seed=5, std=0.05)
    if kind != BF16:
        hm = quantize_model(hm, kind)
    tm = gpu.Model(ctx, hm)
    dm = tm.truncated(1)
    r = spec.Runner(ctx, tm, dm, prompt_for(cfg, 40, 9), K, kv_blocks=64)
    r.prefill()
    r.step()  # the draft's prefill of the prompt
    ot = oracle.Model(hm)
    od = ot.truncated(1)
    okv, odkv = ot.kv(64), od.kv(64 + 64)  # the runner's draft cache: kv_blocks + max_seqs
    copy_kv(r.tkv, okv, cfg.layers)
    copy_kv(r.dkv, odkv, 1)
    accepted = 0
    for step in range(24):
        # the tables the device step is about to use, grown first so both see them
        assert r.tpool.grow(r.tb, r.computed + K + 1) and r.dpool.grow(r.db, len(r.tokens) + K - 1)
        em, acc, comp, dcomp = oracle.spec_step(ot, okv, od, odkv, r.tokens, r.computed, r.dcomp, r.tb, r.db, K)
        got = r.step()
        assert got == [int(x) for x in em], step
        assert r.stats.accepted_per_step[-1] == acc, step
        assert (r.computed, r.dcomp) == (comp, dcomp), step
        accepted += acc
    log(f"one-layer draft, kind {kind}: {accepted} of {24 * K} accepted, context {r.computed}")
    assert accepted < 24 * K  # proposals rejected (acceptance: the self-draft tests)
    kv_close(r.dkv, odkv, 1)
    kv_close(r.tkv, okv, cfg.layers)


@pytest.mark.parametrize("rows", [3, 4])
def test_lagging_draft_tail(pctx, rows):
    ctx = pctx
    """The draft's first round over `rows` rows whose positions cross 64."""
    cfg = CFGS["gqa4-bias-tied"]
    hm = random_model(cfg, seed=21, std=0.05)
    tm = gpu.Model(ctx, hm)
    dm = tm.truncated(1)
    r = spec.Runner(ctx, tm, dm, prompt_for(cfg, 61, 4), K, kv_blocks=64)
    r.prefill()
    r.step()  # computed: 62 .. 65
    r.dcomp = r.computed - (rows - 1)  # the tail: tokens[dcomp:], `rows` long
    assert len(r.tokens) - r.dcomp == rows and r.dcomp < 64 <= r.computed + K
    ot = oracle.Model(hm)
    od = ot.truncated(1)
    okv, odkv = ot.kv(64), od.kv(64 + 64)  # the runner's draft cache: kv_blocks + max_seqs
    copy_kv(r.tkv, okv, cfg.layers)
    copy_kv(r.dkv, odkv, 1)
    assert r.tpool.grow(r.tb, r.computed + K + 1) and r.dpool.grow(r.db, len(r.tokens) + K - 1)
    em, acc, comp, dcomp = oracle.spec_step(ot, okv, od, odkv, r.tokens, r.computed, r.dcomp, r.tb, r.db, K)
    got = r.step()
    log(f"tail of {rows}: emitted {got}, accepted {r.stats.accepted_per_step[-1]}")
    assert got == [int(x) for x in em]
    assert r.stats.accepted_per_step[-1] == acc
    assert (r.computed, r.dcomp) == (comp, dcomp)
    kv_close(r.dkv, odkv, 1)


def test_matches_kernel_path():
    cfg = CFGS["gqa3"]
    hm = random_model(cfg, seed=8, std=0.05)
    prompt = prompt_for(cfg, 45, 6)
    runs = []
    for env in ({"FERRO_PFWD": "1"}, {}):
        c = context(**env)
        try:
            tm = gpu.Model(c, hm)
            r = spec.Runner(c, tm, tm.truncated(2), prompt, K, kv_blocks=64)
            while len(r.generated) < 40:
                r.step()
            runs.append((list(r.generated), list(r.stats.accepted_per_step),
                         [r.dkv.layer(i) for i in range(2)] + [r.tkv.layer(i) for i in range(cfg.layers)]))
        finally:
            c.close()
    (g1, a1, kv1), (g2, a2, kv2) = runs
    assert g1 == g2 and a1 == a2
    same = True
    for l1, l2 in zip(kv1, kv2):
        for x, y in zip(l1, l2):
            assert np.abs(x - y).max() <= 1e-5 * np.abs(y).max()
            same &= np.array_equal(x, y)
    log(f"persistent vs kernel path: {sum(a1)} accepted in {len(a1)} steps")
    assert not same


def test_wait_timeout_is_reported():
    cfg = CFGS["gqa1"]
    hm = random_model(cfg, seed=2, std=0.05)
    c = context(FERRO_PFWD="1", FERRO_PFWD_SPIN="1")
    try:
        tm = gpu.Model(c, hm)
        r = spec.Runner(c, tm, tm.truncated(1), prompt_for(cfg, 20, 1), K, kv_blocks=16)
        r.prefill()
        with pytest.raises(gpu.FgError, match="timed out"):
            r.step()
    finally:
        c.close()
    c = context(FERRO_PFWD="1")
    try:
        tm = gpu.Model(c, hm)
        got = spec.generate(c, tm, tm.truncated(1), prompt_for(cfg, 20, 1), 8, K, kv_blocks=16)
        assert len(got) == 8
    finally:
        c.close()
