"""Sampling on the device (fg_forward_sampled, fg_spec_step_sampled) against
the oracle's restatement of sampler::distribution / draw / sample and of the
engine's sampling branch (src/sampler.rs:52-111, src/engine.rs:575-610,
658-717), and against the exact two-token distribution by the reference's
chi-square test (tests/engine.rs:196-243).

Draws compare token for token: given the same logits, the device computes
the reference's arithmetic (its exp is the correctly rounded one; glibc's
expf, which the oracle calls, differs from it in the last bit in rare cases,
which could only move a draw whose uniform falls within ~1e-7 of a bucket
boundary).
"""
import numpy as np
import pytest

import oracle
from ferrolm_amd import gpu
from ferrolm_amd.gpu import SamplingParams
from ferrolm_amd.spec import Batch, generate
from ferrolm_amd.weights import load_model

from conftest import GOLDEN, chi_square, exact_two_token_distribution, reference_prompts

pytestmark = pytest.mark.gpu

PARAMS = [SamplingParams(1.0, 1.0, 4), SamplingParams(0.7, 0.9, 50), SamplingParams(1.3, 0.5, 1024),
          SamplingParams(2.0, 1.0, 1), SamplingParams(0.8, 0.95, 300), SamplingParams(0.0, 1.0, 0),
          # wide rows: no top-k limit (the reference's default), and a limit above 1024
          SamplingParams(1.0, 1.0, 0), SamplingParams(0.9, 0.9, 0), SamplingParams(1.1, 0.97, 3000)]


def _tied_model():
    """A random model with a 8192-token tied vocabulary whose embedding
    repeats rows 0..99 at 100..199, so the logits hold exact ties."""
    from ferrolm_amd.synth import random_model
    from ferrolm_amd.weights import Config
    cfg = Config(vocab=8192, hidden=128, intermediate=256, layers=2, heads=4, kv_heads=2, head_dim=32,
                 rms_eps=1e-5, max_position=1024, tie_embeddings=True)
    hm = random_model(cfg, seed=41, std=0.05)
    hm.embed[100:200] = hm.embed[0:100]
    return hm


def test_forward_sampled_matches_the_oracle_on_device_logits(ctx):
    """Each selected row's token and the advanced generator state equal
    oracle.sample on the device's own logits of that row, over temperatures,
    top-k 1..1024, 0 (no limit) and above 1024, top-p cuts, ties, several seeds, one row and several rows
    in one call (each row its own parameters and generator)."""
    hm = _tied_model()
    m = gpu.Model(ctx, hm)
    rng = np.random.default_rng(42)
    prompts = [[int(x) for x in rng.integers(3, 8000, n)] for n in (37, 5, 90)]
    tables = [list(range(8 * i, 8 * i + 8)) for i in range(3)]
    kv = gpu.KvCache(ctx, hm.cfg, 24)
    chunks = [(p, 0, t, gpu.LOGITS_LAST) for p, t in zip(prompts, tables)]
    lg = gpu.forward(ctx, m, kv, chunks).logits
    ties = [np.sum(row[:100] == row[100:200]) for row in lg]
    assert min(ties) == 100
    for seed in range(1, 5):
        for p in PARAMS:
            # one row
            kv1 = gpu.KvCache(ctx, hm.cfg, 8)
            st = np.array([gpu.rng_init(seed)], np.uint64)
            tok = gpu.forward_sampled(ctx, m, kv1, [(prompts[0], 0, tables[0][:8], gpu.LOGITS_LAST)],
                                      [p], st)
            r = oracle.Rng(seed)
            assert int(tok[0]) == oracle.sample(lg[0], (p.temperature, p.top_p, p.top_k), r), (seed, p)
            assert int(st[0]) == r.state
        # three rows, each with other parameters and its own generator
        ps = [PARAMS[(seed + j) % len(PARAMS)] for j in range(3)]
        kv3 = gpu.KvCache(ctx, hm.cfg, 24)
        st = np.array([gpu.rng_init(seed * 10 + j) for j in range(3)], np.uint64)
        tok = gpu.forward_sampled(ctx, m, kv3, chunks, ps, st)
        for j in range(3):
            r = oracle.Rng(seed * 10 + j)
            p = ps[j]
            assert int(tok[j]) == oracle.sample(lg[j], (p.temperature, p.top_p, p.top_k), r), (seed, j, p)
            assert int(st[j]) == r.state


def test_device_rejects_negative_top_k(ctx):
    hm = _tied_model()
    m = gpu.Model(ctx, hm)
    kv = gpu.KvCache(ctx, hm.cfg, 8)
    st = np.array([gpu.rng_init(1)], np.uint64)
    with pytest.raises(gpu.FgError, match="top_k"):
        gpu.forward_sampled(ctx, m, kv, [([5, 6, 7], 0, list(range(8)), gpu.LOGITS_LAST)],
                            [SamplingParams(1.0, 0.9, -1)], st)


@pytest.mark.parametrize("params", [SamplingParams(1.0, 1.0, 4), SamplingParams(0.8, 0.9, 64),
                                    SamplingParams(1.0, 1.0, 0), SamplingParams(0.9, 0.85, 0)],
                         ids=["t1-k4", "t0.8-p0.9-k64", "t1-nolimit", "t0.9-p0.85-nolimit"])
def test_spec_sampling_matches_the_oracle_engine(ctx, params):
    """Sampled speculative generation (one-layer draft, k=3) emits the
    oracle engine's tokens for the same seeds: the same draft draws,
    acceptances, residual and bonus draws from the same generator."""
    hm = load_model(GOLDEN / "llama-gqa")
    om = oracle.Model(hm)
    tm = gpu.Model(ctx, hm)
    dm, od = tm.truncated(1), om.truncated(1)
    p = (params.temperature, params.top_p, params.top_k)
    total = [0, 0]
    for i, prompt in enumerate(reference_prompts(4, 7)):
        want, (prop, acc, _) = oracle.generate_sampled(om, od, prompt, 24, 3, p, seed=100 + i, kv_blocks=200)
        sp = SamplingParams(params.temperature, params.top_p, params.top_k, seed=100 + i)
        got = generate(ctx, tm, dm, prompt, 24, 3, kv_blocks=200, params=sp)
        assert np.array_equal(got, want), (i, got.tolist(), want.tolist())
        total[0] += prop
        total[1] += acc
    assert 0 < total[1] < total[0]  # proposals both accepted and rejected


def test_device_speculative_sampling_keeps_the_target_distribution(ctx):
    """tests/engine.rs:196-243 on the device: the first two sampled tokens
    after a fixed prompt over 4000 requests (seeds 1..4000), without a draft
    (both tokens by fg_forward_sampled) and with a one-layer draft (the
    second token from a speculative step, k=3), against the exact
    distribution: chi-square below the 0.1% critical value 37.7 (15 degrees
    of freedom)."""
    hm = load_model(GOLDEN / "llama-gqa")
    m = oracle.Model(hm)
    prompt = reference_prompts(1, 5)[0]
    exact = exact_two_token_distribution(m, prompt, (1.0, 1.0, 4))
    assert len(exact) == 16
    tm = gpu.Model(ctx, hm)
    dm = tm.truncated(1)
    n, per = 4000, 250
    plain, spec = {}, {}
    proposed = accepted = 0
    bpr = (len(prompt) + 2 + 15) // 16
    for b0 in range(0, n, per):
        ps = [SamplingParams(1.0, 1.0, 4, seed=b0 + i + 1) for i in range(per)]
        # without a draft: the prompt's token, then the next one
        kv = gpu.KvCache(ctx, hm.cfg, per * bpr)
        tables = [list(range(i * bpr, (i + 1) * bpr)) for i in range(per)]
        st = np.array([gpu.rng_init(p.seed) for p in ps], np.uint64)
        t1 = gpu.forward_sampled(ctx, tm, kv, [(prompt, 0, t, gpu.LOGITS_LAST) for t in tables], ps, st)
        t2 = gpu.forward_sampled(ctx, tm, kv, [([int(a)], len(prompt), t, gpu.LOGITS_LAST)
                                                for a, t in zip(t1, tables)], ps, st)
        for a, b in zip(t1, t2):
            plain[(int(a), int(b))] = plain.get((int(a), int(b)), 0) + 1
        # with the draft: prefill, then one speculative step
        bt = Batch(ctx, tm, dm, [prompt] * per, 3, kv_blocks=per * (bpr + 1), seed=b0, params=ps)
        first = bt.prefill()
        out = bt.step()
        for a, e in zip(first, out):
            spec[(int(a), int(e[0]))] = spec.get((int(a), int(e[0])), 0) + 1
        proposed += bt.stats.proposed
        accepted += bt.stats.accepted
    c_plain, c_spec = chi_square(plain, exact, n), chi_square(spec, exact, n)
    print(f"chi-square vs exact: plain {c_plain:.1f}, speculative {c_spec:.1f} (df 15); "
          f"{accepted}/{proposed} proposals accepted")
    assert 0 < accepted < proposed
    assert c_plain < 37.7, c_plain
    assert c_spec < 37.7, c_spec


def test_no_limit_sampling_at_the_full_vocabulary(ctx):
    """top_k 0 over a 49152-token vocabulary (the SmolLM2 one): the sort, the
    sequential sums and the top-p prefix of the whole distribution give the
    oracle's tokens and generator states, several rows in one call."""
    from ferrolm_amd.synth import random_model
    from ferrolm_amd.weights import Config
    cfg = Config(vocab=49152, hidden=64, intermediate=128, layers=1, heads=2, kv_heads=1, head_dim=32,
                 rms_eps=1e-5, max_position=256, tie_embeddings=True)
    hm = random_model(cfg, seed=3, std=0.3)
    m = gpu.Model(ctx, hm)
    rng = np.random.default_rng(5)
    prompts = [[int(x) for x in rng.integers(3, 49000, n)] for n in (9, 21, 4)]
    tables = [list(range(2 * i, 2 * i + 2)) for i in range(3)]
    chunks = [(p, 0, t, gpu.LOGITS_LAST) for p, t in zip(prompts, tables)]
    lg = gpu.forward(ctx, m, gpu.KvCache(ctx, cfg, 6), chunks).logits
    ps = [SamplingParams(1.0, 1.0, 0), SamplingParams(0.7, 0.9, 0), SamplingParams(1.2, 0.5, 5000)]
    for seed in (1, 2):
        st = np.array([gpu.rng_init(seed * 10 + j) for j in range(3)], np.uint64)
        tok = gpu.forward_sampled(ctx, m, gpu.KvCache(ctx, cfg, 6), chunks, ps, st)
        for j in range(3):
            r = oracle.Rng(seed * 10 + j)
            p = ps[j]
            assert int(tok[j]) == oracle.sample(lg[j], (p.temperature, p.top_p, p.top_k), r), (seed, j)
            assert int(st[j]) == r.state
