"""The C ABI's refusal paths on the device: each bad input comes back as an
FgError with its message (the reference's shape assert!s and bounds checks,
src/model.rs:284-287, src/kv.rs:48-56, src/engine.rs:512-520), and nothing
is launched: the GEMV profiler records no launch and the cache is unchanged.
A valid call on the same objects then still works."""
import numpy as np
import pytest

from ferrolm_amd import gpu
from ferrolm_amd.weights import load_model

from conftest import GOLDEN

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def setup(ctx):
    hm = load_model(GOLDEN / "llama-gqa")
    m = gpu.Model(ctx, hm)
    kv = gpu.KvCache(ctx, hm.cfg, 8)
    return hm, m, kv


def refused(ctx, kv, call, match):
    """call() raises FgError matching `match`; no GEMV was launched and layer
    0 of the cache holds the same bits as before."""
    k0, v0 = kv.layer(0)
    gpu.profile_read(ctx, reset=True)
    gpu.profile(ctx, True)
    try:
        with pytest.raises(gpu.FgError, match=match):
            call()
    finally:
        gpu.profile(ctx, False)
    assert sum(r["launches"] for r in gpu.profile_read(ctx, reset=True)) == 0
    k1, v1 = kv.layer(0)
    assert np.array_equal(k0, k1) and np.array_equal(v0, v1)


def test_forward_refusals(ctx, setup):
    hm, m, kv = setup
    V = hm.cfg.vocab
    ok = [3, 4, 5]
    # block id beyond the cache (src/kv.rs:48-56 indexes the cache with it)
    refused(ctx, kv, lambda: gpu.forward(ctx, m, kv, [(ok, 0, [8], gpu.LOGITS_LAST)]), "block id beyond the cache")
    # token outside the vocabulary (the embedding gather, src/model.rs:296-298)
    refused(ctx, kv, lambda: gpu.forward(ctx, m, kv, [([3, V, 5], 0, [0], gpu.LOGITS_LAST)]),
            "token outside the vocabulary")
    # a chunk longer than its block table covers (src/model.rs:284-291)
    refused(ctx, kv, lambda: gpu.forward(ctx, m, kv, [(list(range(3, 20)), 0, [0], gpu.LOGITS_LAST)]),
            "chunk overruns its cache blocks")
    # a position at or past max_position
    mp = hm.cfg.max_position
    refused(ctx, kv, lambda: gpu.forward(ctx, m, kv, [(ok, mp - 1, list(range(8)) * (mp // 128 + 1),
                                                      gpu.LOGITS_LAST)]),
            "max_position|overruns")
    # the same objects still run a valid chunk
    out = gpu.forward(ctx, m, kv, [(ok, 0, [1], gpu.LOGITS_LAST)])
    assert out.argmax.shape == (1,) and int(out.argmax[0]) < V


def test_spec_step_refusals(ctx, setup):
    hm, m, kv = setup
    draft = m.truncated(1)
    dkv = gpu.KvCache(ctx, hm.cfg, 8)
    prompt = [3, 9, 27, 81, 243]
    gpu.forward(ctx, m, kv, [(prompt, 0, [0], gpu.LOGITS_LAST)])
    pos = len(prompt) - 1
    # tail must end at the last token (draft_pos + n_tail == pos + 1, src/engine.rs:667-669)
    bad = gpu.SpecSeq(tail=np.array([243], np.uint32), draft_pos=0, pos=pos, blocks=np.array([0], np.uint32),
                      draft_blocks=np.array([0], np.uint32))
    refused(ctx, kv, lambda: gpu.spec_step(ctx, m, kv, draft, dkv, [bad], 3), "tail must end at the last token")
    # a verify row past the target's block table
    short = gpu.SpecSeq(tail=np.array(prompt, np.uint32), draft_pos=0, pos=14, blocks=np.array([0], np.uint32),
                        draft_blocks=np.array([0, 1], np.uint32))
    refused(ctx, kv, lambda: gpu.spec_step(ctx, m, kv, draft, dkv,
                                           [gpu.SpecSeq(tail=np.arange(3, 18, dtype=np.uint32), draft_pos=0,
                                                        pos=14, blocks=short.blocks,
                                                        draft_blocks=short.draft_blocks)], 3),
            "chunk overruns its cache blocks")
    # k must be positive
    good = gpu.SpecSeq(tail=np.array(prompt, np.uint32), draft_pos=0, pos=pos, blocks=np.array([0], np.uint32),
                       draft_blocks=np.array([0], np.uint32))
    refused(ctx, kv, lambda: gpu.spec_step(ctx, m, kv, draft, dkv, [good], 0), "bad argument")
    # chunks riding in the verify pass (fg_spec_step_mixed): no FG_LOGITS_ALL,
    # tokens inside the vocabulary
    V = hm.cfg.vocab
    refused(ctx, kv, lambda: gpu.spec_step_mixed(ctx, m, kv, draft, dkv, [good], 3,
                                                 [([5, 6, 7], 0, [2], gpu.LOGITS_ALL)]),
            "chunks take FG_LOGITS_NONE or FG_LOGITS_LAST")
    refused(ctx, kv, lambda: gpu.spec_step_mixed(ctx, m, kv, draft, dkv, [good], 3,
                                                 [([5, V, 7], 0, [2], gpu.LOGITS_LAST)]),
            "token outside the vocabulary")
    # a valid mixed step: the chunk's greedy token equals a plain forward's
    toks, acc, am = gpu.spec_step_mixed(ctx, m, kv, draft, dkv, [good], 3, [([5, 6, 7], 0, [2], gpu.LOGITS_LAST),
                                                                            ([8, 9], 0, [3], gpu.LOGITS_NONE)])
    assert 1 <= len(toks[0]) <= 4 and 0 <= int(acc[0]) <= 3 and am.shape == (1,)
    kv2 = gpu.KvCache(ctx, hm.cfg, 8)
    assert int(am[0]) == int(gpu.forward(ctx, m, kv2, [([5, 6, 7], 0, [2], gpu.LOGITS_LAST)]).argmax[0])
    # and a valid step runs
    toks, acc = gpu.spec_step(ctx, m, kv, draft, dkv, [good], 3)
    assert 1 <= len(toks[0]) <= 4 and 0 <= int(acc[0]) <= 3


def test_cache_and_model_shape_refusals(ctx, setup):
    hm, m, kv = setup
    from dataclasses import replace
    with pytest.raises(gpu.FgError, match="head_dim 96"):
        gpu.KvCache(ctx, replace(hm.cfg, head_dim=96), 4)
    with pytest.raises(gpu.FgError, match="block_size must be 16"):
        gpu.KvCache(ctx, hm.cfg, 4, block_size=32)
    # a cache whose head count does not match the model
    other = gpu.KvCache(ctx, replace(hm.cfg, kv_heads=hm.cfg.kv_heads * 2), 8)
    with pytest.raises(gpu.FgError, match="cache does not match the model"):
        gpu.forward(ctx, m, other, [([3, 4], 0, [0], gpu.LOGITS_LAST)])
