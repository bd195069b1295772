"""The serving engine (ferrolm_amd.engine): the reference's BlockManager unit
tests (src/kv.rs:215-270) on the CPU, and its engine tests
(tests/engine.rs:65-290) on the device: under greedy decoding a request's
tokens do not depend on batching, prompt chunking, prefix-cache hits,
preemption with recompute, reservation or speculation."""
import ctypes

import pytest

from ferrolm_amd.engine import (CANCELLED, LENGTH, REJECTED, ROOT, BlockManager, Engine, EngineConfig, Params,
                                chain)

from conftest import GOLDEN, reference_prompts


# ---- BlockManager (CPU) -------------------------------------------------------

def test_allocates_until_full_then_evicts_idle_cached_blocks_lru():
    m = BlockManager(3, 2, True)
    a, b, c = m.allocate(), m.allocate(), m.allocate()
    assert m.allocate() is None
    ka = m.publish(a, ROOT, [1, 2])
    m.publish(b, ka, [3, 4])
    m.release(b)
    m.release(a)
    m.release(c)
    assert m.available() == 3
    # a sequence with the same first block shares it
    assert m.lookup(ROOT, [1, 2]) == a
    assert m.lookup(ROOT, [9, 9]) is None
    # the uncached free block goes first, then the least recently released
    # cached one (b); a is in use
    assert m.allocate() == c
    assert m.allocate() == b
    assert m.stats.evicted == 1
    assert m.lookup(ka, [3, 4]) is None, "evicted block must be forgotten"
    assert m.allocate() is None
    m.release(a)
    assert m.lookup(ROOT, [1, 2]) == a, "idle block stays cached"
    assert m.refs(a) == 1


def test_keys_depend_on_the_whole_prefix():
    k1 = chain(chain(ROOT, [1, 2]), [3, 4])
    k2 = chain(chain(ROOT, [5, 6]), [3, 4])
    assert k1 != k2
    m = BlockManager(2, 2, False)
    a = m.allocate()
    m.publish(a, ROOT, [1, 2])
    m.release(a)
    assert m.lookup(ROOT, [1, 2]) is None, "prefix caching disabled"


def test_a_key_collision_is_a_miss_not_a_wrong_block():
    m = BlockManager(2, 2, True)
    a = m.allocate()
    k = m.publish(a, ROOT, [1, 2])
    m.tokens[a] = (7, 7)  # as if another block's tokens hashed to the same key
    assert m.by_key[k] == a
    assert m.lookup(ROOT, [1, 2]) is None


def test_releasing_a_free_block_is_an_error():
    m = BlockManager(1, 16, True)
    b = m.allocate()
    m.release(b)
    with pytest.raises(AssertionError):
        m.release(b)


# ---- the engine on the device ---------------------------------------------------

def _rng_ids(n, seed):
    import oracle
    rng = ctypes.c_uint64(oracle.lib().or_rng_new(seed))
    return [3 + oracle.lib().or_rng_next(ctypes.byref(rng)) % 509 for _ in range(n)]


@pytest.fixture(scope="module")
def models(ctx):
    from ferrolm_amd import gpu
    from ferrolm_amd.weights import load_model
    hm = load_model(GOLDEN / "llama-gqa")
    return gpu.Model(ctx, hm)


def greedy(max_tokens):
    return Params(max_tokens=max_tokens, ignore_eos=True)


def serve(ctx, model, cfg, reqs, draft=None):
    e = Engine(ctx, model, draft, cfg)
    out = [e.submit(p, s) for p, s in reqs]
    e.run_until_idle()
    return [(r.tokens, r.finish) for r in out], e.stats


def alone(ctx, model, reqs):
    return [serve(ctx, model, EngineConfig(max_seqs=1, prefix_cache=False), [r])[0][0][0] for r in reqs]


@pytest.mark.gpu
def test_batching_and_chunked_prefill_do_not_change_outputs(ctx, models):
    import oracle
    from ferrolm_amd.weights import load_model
    reqs = [(p, greedy(24)) for p in reference_prompts(24, 1)]
    want = alone(ctx, models, reqs)
    # alone, each request is the reference engine's greedy generation (the oracle's)
    om = oracle.Model(load_model(GOLDEN / "llama-gqa"))
    for i, (p, _) in enumerate(reqs):
        assert want[i] == [int(t) for t in oracle.generate(om, None, p, 24, 0)[0]], i
    for budget, admission in [(37, "continuous"), (512, "continuous"), (64, "static")]:
        cfg = EngineConfig(max_batch_tokens=budget, admission=admission, prefix_cache=False)
        got, st = serve(ctx, models, cfg, reqs)
        for i, (g, f) in enumerate(got):
            assert f == LENGTH
            assert g == want[i], (i, budget, admission)
        assert st.peak_running > 1, "requests never overlapped"


@pytest.mark.gpu
def test_prefix_cache_hits_do_not_change_outputs(ctx, models):
    system = _rng_ids(100, 9)
    reqs = [(system + p, greedy(16)) for p in reference_prompts(16, 2)]
    want = alone(ctx, models, reqs)
    got, st = serve(ctx, models, EngineConfig(max_seqs=4), reqs)
    for i, (g, _) in enumerate(got):
        assert g == want[i], i
    # the first four are admitted together, before the shared prefix is
    # cached; each later one reuses its 6 full blocks
    assert st.cached_tokens >= 12 * 96, st.cached_tokens


@pytest.mark.gpu
def test_preemption_and_recompute_do_not_change_outputs(ctx, models):
    reqs = [(p, greedy(40)) for p in reference_prompts(20, 3)]
    want = alone(ctx, models, reqs)
    # 40 blocks of 16 tokens cannot hold 20 growing sequences
    got, st = serve(ctx, models, EngineConfig(kv_blocks=40, max_batch_tokens=128), reqs)
    for i, (g, _) in enumerate(got):
        assert g == want[i], i
    assert st.preemptions > 0, "the test never preempted"


@pytest.mark.gpu
def test_speculative_greedy_decoding_matches_the_target_exactly(ctx, models):
    reqs = [(p, greedy(30)) for p in reference_prompts(12, 4)]
    want = alone(ctx, models, reqs)
    # a related draft (the target's first layer) and a perfect one (the target itself)
    for layers, k in [(1, 4), (3, 3), (1, 1)]:
        got, st = serve(ctx, models, EngineConfig(spec_k=k, kv_blocks=200), reqs, draft=models.truncated(layers))
        for i, (g, _) in enumerate(got):
            assert g == want[i], (i, layers, k)
        print(f"draft layers {layers}, k={k}: {100 * st.spec_accepted / st.spec_proposed:.0f}% accepted")
        assert st.spec_proposed > 0
        if layers == 3:
            assert st.spec_accepted == st.spec_proposed, "the target as its own draft"
    # a small token budget: prompts are prefilled in chunks while earlier
    # requests speculate, and those steps run one target forward
    # (fg_spec_step_mixed: the chunks ride in the verify pass)
    got, st = serve(ctx, models, EngineConfig(spec_k=3, kv_blocks=200, max_batch_tokens=40), reqs,
                    draft=models.truncated(1))
    for i, (g, _) in enumerate(got):
        assert g == want[i], (i, "mixed")
    assert st.mixed_steps > 0, "no step carried chunks in its verify pass"


@pytest.mark.gpu
def test_reserving_whole_sequences_admits_fewer_at_once(ctx, models):
    reqs = [(p, greedy(8)) for p in reference_prompts(16, 6)]
    a, sa = serve(ctx, models, EngineConfig(kv_blocks=100), reqs)
    b, sb = serve(ctx, models, EngineConfig(kv_blocks=100, reserve_tokens=512), reqs)
    assert a == b
    # 100 blocks reserve three 512-token sequences; paging fits many more
    assert sb.peak_running == 3
    assert sa.peak_running > 6, sa.peak_running


@pytest.mark.gpu
def test_rejects_what_cannot_be_served_and_honours_cancellation(ctx, models):
    e = Engine(ctx, models, None, EngineConfig(kv_blocks=8))
    too_long = e.submit([5] * 200, greedy(4))
    empty = e.submit([], greedy(4))
    bad = e.submit([600], greedy(4))
    cancelled = e.submit([5] * 10, greedy(1000))
    cancelled.cancel()
    ok = e.submit([5] * 10, greedy(1000))
    e.run_until_idle()
    assert too_long.finish == REJECTED and empty.finish == REJECTED and bad.finish == REJECTED
    assert cancelled.finish == CANCELLED
    # the context is full at 8 blocks of 16 tokens
    assert (len(ok.tokens), ok.finish) == (118, LENGTH)


@pytest.mark.gpu
def test_sampled_requests_are_reproducible_and_mix_with_greedy_ones(ctx, models):
    """Sampling through the engine: the same seeds give the same tokens
    whether the requests run alone or batched with greedy ones, with and
    without a draft (per-request generators, src/engine.rs:292-299)."""
    ps = reference_prompts(6, 7)
    reqs = [(p, Params(temperature=0.8, top_p=0.9, top_k=(40 if i % 4 == 0 else 0), seed=100 + i, max_tokens=20,
                       ignore_eos=True) if i % 2 == 0 else greedy(20)) for i, p in enumerate(ps)]
    want = alone(ctx, models, reqs)
    got, _ = serve(ctx, models, EngineConfig(max_batch_tokens=64), reqs)
    assert [g for g, _ in got] == want
    # with a draft, the sampled requests follow the speculative sampling rule:
    # reproducible for the same seeds, greedy ones unchanged
    d1, _ = serve(ctx, models, EngineConfig(spec_k=3, kv_blocks=200), reqs, draft=models.truncated(1))
    d2, _ = serve(ctx, models, EngineConfig(spec_k=3, kv_blocks=200, max_batch_tokens=64), reqs,
                  draft=models.truncated(1))
    assert d1 == d2
    for i in range(1, len(reqs), 2):
        assert d1[i][0] == want[i]
