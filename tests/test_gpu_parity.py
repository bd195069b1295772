"""Parity of the HIP path (through the C ABI) with the CPU oracle and the
reference's transformers fixtures.

Tolerances: the device GEMV sums in a different order from the reference's
FMA chains (MFMA over exact operand pieces, f32 accumulation), so products
agree to f32 rounding, checked as |gpu - oracle| <= 2e-5 * sum|x||w|.
Logits follow the reference test's bar (1e-3 of the largest logit,
tests/reference.rs:53-91) and the north star's 1e-2 relative; per-layer
hidden states its 2e-2 relative. Token ids must be identical.
"""
import json

import numpy as np
import pytest

import oracle
from ferrolm_amd import gpu
from ferrolm_amd.spec import Batch, generate
from ferrolm_amd.weights import BF16, INT4, INT8, Matrix, bf16_to_f32, f32_to_bf16, load_model

from conftest import FIXTURES, GOLDEN, assert_argmax_parity

pytestmark = pytest.mark.gpu


def rand_matrix(kind, n, k, seed):
    rng = np.random.default_rng(seed)
    wb = f32_to_bf16(rng.standard_normal((n, k)).astype(np.float32))
    if kind == BF16:
        return Matrix(BF16, n, k, bf16=wb)
    return oracle.quantize(kind, bf16_to_f32(wb).reshape(n, k))


@pytest.mark.parametrize("kind", [BF16, INT8, INT4])
@pytest.mark.parametrize("n,k", [(32, 32), (96, 544), (64, 2048), (2048, 576), (160, 8192)])
def test_matmul_matches_oracle(ctx, kind, n, k):
    w = rand_matrix(kind, n, k, seed=n * 7 + k)
    dm = gpu.Mat(ctx, w)
    deq = w.to_f32().astype(np.float64)
    rng = np.random.default_rng(k)
    for m in [1, 2, 3, 4, 5, 8, 13, 17, 40, 70, 100, 160]:  # past 16 rows: the GEMM (split K for the small n)
        x = rng.standard_normal((m, k)).astype(np.float32)
        x[:, ::7] *= 20.0  # a few large channels, as activations have
        y = dm.matmul(x)
        ref = oracle.matmul(w, x)
        scale = np.abs(x).astype(np.float64) @ np.abs(deq).T
        exact = x.astype(np.float64) @ deq.T
        assert np.all(np.abs(y - ref) <= 2e-5 * scale + 1e-30), (kind, n, k, m)
        assert np.all(np.abs(y - exact) <= 2e-5 * scale + 1e-30), (kind, n, k, m)


def test_matmul_bias_and_batch_invariance(ctx):
    w = rand_matrix(BF16, 64, 256, seed=3)
    dm = gpu.Mat(ctx, w)
    x = np.random.default_rng(1).standard_normal((13, 256)).astype(np.float32)
    b = np.linspace(-1, 1, 64).astype(np.float32)
    y = dm.matmul(x, b)
    y0 = dm.matmul(x)
    assert np.array_equal(y, y0 + b)
    # each row alone gives the same bits as inside the batch (same kernel plan per row group)
    for i in [0, 5, 12]:
        yi = dm.matmul(x[i:i + 1])
        assert np.allclose(yi[0], y0[i], rtol=0, atol=2e-5 * np.abs(y0[i]).max())


def scattered_table(tokens, bs=16):
    blocks = (tokens + bs - 1) // bs
    return [(i * 7) % blocks for i in range(blocks)], blocks


@pytest.mark.parametrize("name", FIXTURES)
def test_fixture_forward_matches_transformers_and_oracle(ctx, name):
    d = GOLDEN / name
    hm = load_model(d)
    ref = json.loads((d / "reference.json").read_text())
    prompt, greedy = ref["prompt"], ref["greedy"]
    table, blocks = scattered_table(len(prompt) + len(greedy) + 1)
    m = gpu.Model(ctx, hm)
    kv = gpu.KvCache(ctx, hm.cfg, blocks)
    out = gpu.forward(ctx, m, kv, [(prompt, 0, table, gpu.LOGITS_ALL)], hidden=True)
    worst, scale = 0.0, 1.0
    for row, e in zip(ref["logits_rows"], ref["logits"]):
        e = np.array(e)
        worst = max(worst, float(np.abs(out.logits[row] - e).max()))
        scale = max(scale, float(np.abs(e).max()))
    assert worst < 1e-3 * scale, f"{name}: logits differ from transformers by {worst}"
    om = oracle.Model(hm)
    okv = om.kv(blocks)
    ol, oh = om.forward(okv, [(prompt, 0, table, 2)], hidden=True)
    assert np.abs(out.logits - ol).max() < 1e-4 * np.abs(ol).max()
    rel = np.linalg.norm(out.hidden - oh, axis=-1) / np.linalg.norm(oh, axis=-1)
    assert rel.max() < 1e-4, rel.max()  # the north star's bar is 2e-2
    assert_argmax_parity(out.argmax, ol)  # every row's greedy token, near-ties excused
    # KV slots: every written position holds the oracle's keys/values
    for li in range(hm.cfg.layers):
        gk, gv = kv.layer(li)
        ok, ov = okv.layer(li)
        assert np.array_equal(gk != 0, ok != 0)
        assert np.abs(gk - ok).max() <= 1e-4 * np.abs(ok).max()
        assert np.abs(gv - ov).max() <= 1e-4 * np.abs(ov).max()
    # greedy continuation, one token per step, as tests/reference.rs:93-113
    nxt = int(out.argmax[len(prompt) - 1])
    toks = [nxt]
    pos = len(prompt)
    while len(toks) < len(greedy):
        o = gpu.forward(ctx, m, kv, [([nxt], pos, table, gpu.LOGITS_LAST)], logits=False)
        nxt = int(o.argmax[0])
        toks.append(nxt)
        pos += 1
    assert toks == greedy, f"{name}: greedy continuation differs from transformers"


def rng_prompts(n, seed, lo=3, hi=511, max_len=150):
    st = oracle.lib().or_rng_new(seed)
    import ctypes
    s = ctypes.c_uint64(st)
    out = []
    for _ in range(n):
        ln = 1 + oracle.lib().or_rng_next(ctypes.byref(s)) % max_len
        out.append([lo + oracle.lib().or_rng_next(ctypes.byref(s)) % (hi - lo + 1) for _ in range(ln)])
    return out


@pytest.mark.parametrize("layers,k", [(1, 4), (3, 3), (1, 1)])
def test_speculative_greedy_matches_oracle(ctx, layers, k):
    """tests/engine.rs:134-160 on the device: speculative greedy decoding
    gives the target's own greedy tokens; the target as its own draft
    accepts every proposal."""
    hm = load_model(GOLDEN / "llama-gqa")
    om = oracle.Model(hm)
    tm = gpu.Model(ctx, hm)
    dm = tm.truncated(layers)
    odraft = om.truncated(layers)
    for prompt in rng_prompts(4, seed=4):
        want, _, _ = oracle.generate(om, None, prompt, 30, 0, kv_blocks=200)
        got_o, acc_o, st_o = oracle.generate(om, odraft, prompt, 30, k, kv_blocks=200)
        assert np.array_equal(got_o, want)
        got = generate(ctx, tm, dm, prompt, 30, k, kv_blocks=200)
        assert np.array_equal(got, want), (layers, k, prompt[:5])
        if layers == 3:
            assert st_o[1] == st_o[0]


def test_speculative_graph_replay_across_capacity(ctx):
    """A decode that crosses 1024 positions: the attention launch grows from
    16 to 32 span slots, so the cached step graphs are replayed, a new pair is
    captured, and that pair is replayed too; the tokens stay the target's own
    greedy tokens (tests/engine.rs:134-160 at a longer context)."""
    from ferrolm_amd.synth import random_model
    from ferrolm_amd.weights import Config
    cfg = Config(vocab=512, hidden=128, intermediate=256, layers=2, heads=4, kv_heads=2, head_dim=32,
                 rms_eps=1e-5, max_position=2048)
    hm = random_model(cfg, seed=7, std=0.05)
    om = oracle.Model(hm)
    tm = gpu.Model(ctx, hm)
    prompt = [int(x) for x in np.random.default_rng(3).integers(3, 500, 1000)]
    want, _, _ = oracle.generate(om, None, prompt, 48, 0, kv_blocks=80)
    got = generate(ctx, tm, tm.truncated(1), prompt, 48, 3, kv_blocks=80)
    assert np.array_equal(got, want)


def _batched_matches_oracle(ctx, hm, prompts, k, steps, kv_blocks, seed):
    """Prefill every prompt in one device forward, then run batched device spec
    steps; each sequence must emit what the oracle's spec step for that sequence
    alone emits from the same state, with the same rollback counters."""
    om = oracle.Model(hm)
    tm = gpu.Model(ctx, hm)
    dm, od = tm.truncated(1), om.truncated(1)
    b = Batch(ctx, tm, dm, prompts, k, kv_blocks=kv_blocks, seed=seed)
    first = b.prefill()
    okv, odkv = om.kv(kv_blocks), od.kv(kv_blocks)
    for i, p in enumerate(prompts):
        ol = om.forward(okv, [(p, 0, b.tb[i], 1)])
        assert int(np.argmax(ol[0])) == first[i], i
    otoks = [list(p) + [first[i]] for i, p in enumerate(prompts)]
    oc, odc = [len(p) for p in prompts], [0] * len(prompts)
    accepted = 0
    for step in range(steps):
        got = b.step()
        for i in range(len(prompts)):
            em, acc, c, dc = oracle.spec_step(om, okv, od, odkv, otoks[i], oc[i], odc[i], b.tb[i], b.db[i], k)
            assert [int(x) for x in em] == got[i], (step, i)
            assert (c, dc) == (b.computed[i], b.dcomp[i]), (step, i)
            otoks[i] += [int(x) for x in em]
            oc[i], odc[i] = c, dc
            accepted += acc
    return accepted


def _quantized(hm, kind):
    """Model::quantize of every projection (src/model.rs:192-219), no importance."""
    if kind == BF16:
        return hm
    for l in hm.layers:
        for name in ["wqkv", "wo", "w_gate_up", "w_down"]:
            mat = getattr(l, name)
            setattr(l, name, oracle.quantize(kind, bf16_to_f32(mat.bf16).reshape(mat.rows, mat.cols)))
    return hm


@pytest.mark.parametrize("kind", [BF16, INT8, INT4])
def test_batched_speculative_steps_over_shuffled_tables(ctx, kind):
    """Batched verify (five sequences of different lengths, k=4) over block tables
    drawn from a shuffled pool, at fixture size, with a bf16, int8 or int4 target
    (src/engine.rs:499-717 for every sequence of a step; src/kv.rs:139-151 tables)."""
    hm = _quantized(load_model(GOLDEN / "llama-gqa"), kind)
    rng = np.random.default_rng(11)
    prompts = [[int(x) for x in rng.integers(3, 500, n)] for n in (23, 61, 150, 97, 200)]
    accepted = _batched_matches_oracle(ctx, hm, prompts, k=4, steps=12, kv_blocks=128, seed=5)
    assert accepted > 0  # the one-layer draft agrees sometimes: varied tails and accept counts


def test_batched_speculative_steps_gqa_head_dim_128(ctx):
    """The larger-GQA attention shape (head_dim 128: 32-position spans; four query
    heads per kv head; rope theta 500000) in batched spec steps over contexts of
    300 to 700 positions."""
    from ferrolm_amd.synth import random_model
    from ferrolm_amd.weights import Config
    cfg = Config(vocab=512, hidden=256, intermediate=512, layers=2, heads=8, kv_heads=2, head_dim=128,
                 rms_eps=1e-5, rope_theta=500000.0, max_position=2048)
    hm = random_model(cfg, seed=9, std=0.05)
    rng = np.random.default_rng(12)
    prompts = [[int(x) for x in rng.integers(3, 500, n)] for n in (300, 451, 700)]
    _batched_matches_oracle(ctx, hm, prompts, k=4, steps=6, kv_blocks=160, seed=6)


def test_split_bf16_attention_head_dim_128_matches_oracle(ctx):
    """The split-operand bf16 MFMA attention (items of four 32-position
    sub-spans, 20 queries each: five verify rows of a GQA-4 model at head_dim
    128): four sequences of 4,100 to 4,300 positions make more than 1024
    one-span items, which is when the plan takes sub-spans. One forward of five
    rows per sequence, all logits and every layer's hidden state, against the
    oracle from a copy of the device's cache (src/model.rs:395-432,
    src/kernels.rs:671-756). Each product term is within 2^-16 of its f32 value;
    the bars are the ones the f32 paths hold (measured: logits 2.6e-5 and
    hidden states 2.3e-5 relative, against 1.2e-5 for both with f32 MFMA)."""
    from ferrolm_amd.synth import random_model
    from ferrolm_amd.weights import Config
    cfg = Config(vocab=512, hidden=1024, intermediate=1024, layers=2, heads=8, kv_heads=2, head_dim=128,
                 rms_eps=1e-5, rope_theta=500000.0, max_position=8192)
    hm = random_model(cfg, seed=21, std=0.05)
    rng = np.random.default_rng(22)
    lens = [4100, 4170, 4230, 4300]
    per_seq = max(lens) // 16 + 2
    nb = per_seq * len(lens)
    perm = [int(x) for x in rng.permutation(nb)]
    tables = [perm[i * per_seq:(i + 1) * per_seq] for i in range(len(lens))]
    prompts = [[int(x) for x in rng.integers(3, 500, n)] for n in lens]
    gm = gpu.Model(ctx, hm)
    kv = gpu.KvCache(ctx, cfg, nb)
    for p, tb in zip(prompts, tables):
        for a in range(0, len(p), 2048):
            gpu.forward(ctx, gm, kv, [(p[a:a + 2048], a, tb, gpu.LOGITS_NONE)], logits=False)
    om = oracle.Model(hm)
    okv = om.kv(nb)
    for i in range(cfg.layers):
        okv.set_layer(i, *kv.layer(i))
    chunks = [([int(x) for x in rng.integers(3, 500, 5)], n, tb, gpu.LOGITS_ALL) for n, tb in zip(lens, tables)]
    out = gpu.forward(ctx, gm, kv, chunks, hidden=True)
    ol, oh = om.forward(okv, chunks, hidden=True)
    lrel = np.abs(out.logits - ol).max(axis=1) / np.abs(ol).max(axis=1)
    hrel = np.linalg.norm(out.hidden - oh, axis=-1) / np.linalg.norm(oh, axis=-1)
    print(f"split bf16 attention, hd 128: logits rel max {lrel.max():.2e}, hidden rel max {hrel.max():.2e}")
    assert out.logits.shape == (20, cfg.vocab)
    assert lrel.max() <= 1e-4 and hrel.max() <= 1e-4, (lrel.max(), hrel.max())
    assert_argmax_parity(out.argmax, ol, tol=2e-3, max_ties=1)
    for i in range(cfg.layers):  # the new rows' cache slots
        gk, gv = kv.layer(i)
        ok, ov = okv.layer(i)
        assert np.abs(gk - ok).max() <= 1e-4 * np.abs(ok).max()
        assert np.abs(gv - ov).max() <= 1e-4 * np.abs(ov).max()


@pytest.mark.parametrize("hd,heads,kv_heads,rows", [(64, 8, 4, 1), (64, 16, 4, 2), (128, 8, 2, 1), (128, 16, 2, 1)])
def test_register_decode_attention_matches_oracle(ctx, hd, heads, kv_heads, rows):
    """The decode attention that keeps keys and values in registers
    (k_attn_dec): launches of one-span items with at most 8 queries and at
    least 1024 workgroups. Eight sequences of 2,090 to 2,160 positions over
    shuffled tables give 33 to 34 spans of 64 positions each (hd 64; 1,056 to
    1,088 workgroups over 4 kv heads, under the 4,096 from which hd 64 takes two
    sub-spans) or 66 to 68 of 32 (hd 128, 2 kv heads); rows x the GQA group
    makes 2, 8, 4 and 8 queries per item (the 4- and 8-query instances). One
    forward of those rows, all logits and every layer's hidden state, against
    the oracle from a copy of the device's cache (src/model.rs:395-432), and
    the new rows' cache slots."""
    from ferrolm_amd.synth import random_model
    from ferrolm_amd.weights import Config
    cfg = Config(vocab=512, hidden=heads * hd, intermediate=512, layers=2, heads=heads, kv_heads=kv_heads,
                 head_dim=hd, rms_eps=1e-5, rope_theta=10000.0, max_position=4096)
    hm = random_model(cfg, seed=31 + hd + heads, std=0.05)
    rng = np.random.default_rng(32)
    lens = [int(x) for x in rng.integers(2090, 2161, 8)]
    per_seq = (max(lens) + rows) // 16 + 2
    nb = per_seq * len(lens)
    perm = [int(x) for x in rng.permutation(nb)]
    tables = [perm[i * per_seq:(i + 1) * per_seq] for i in range(len(lens))]
    prompts = [[int(x) for x in rng.integers(3, 500, n)] for n in lens]
    gm = gpu.Model(ctx, hm)
    kv = gpu.KvCache(ctx, cfg, nb)
    for p, tb in zip(prompts, tables):
        for a in range(0, len(p), 2048):
            gpu.forward(ctx, gm, kv, [(p[a:a + 2048], a, tb, gpu.LOGITS_NONE)], logits=False)
    om = oracle.Model(hm)
    okv = om.kv(nb)
    for i in range(cfg.layers):
        okv.set_layer(i, *kv.layer(i))
    chunks = [([int(x) for x in rng.integers(3, 500, rows)], n, tb, gpu.LOGITS_ALL) for n, tb in zip(lens, tables)]
    out = gpu.forward(ctx, gm, kv, chunks, hidden=True)
    ol, oh = om.forward(okv, chunks, hidden=True)
    lrel = np.abs(out.logits - ol).max(axis=1) / np.abs(ol).max(axis=1)
    hrel = np.linalg.norm(out.hidden - oh, axis=-1) / np.linalg.norm(oh, axis=-1)
    print(f"register decode attention, hd {hd}, {heads}/{kv_heads} heads, {rows} rows: "
          f"logits rel max {lrel.max():.2e}, hidden rel max {hrel.max():.2e}")
    assert out.logits.shape == (8 * rows, cfg.vocab)
    assert lrel.max() <= 1e-4 and hrel.max() <= 1e-4, (lrel.max(), hrel.max())
    assert_argmax_parity(out.argmax, ol, tol=2e-3, max_ties=1)
    for i in range(cfg.layers):  # the new rows' cache slots
        gk, gv = kv.layer(i)
        ok, ov = okv.layer(i)
        assert np.abs(gk - ok).max() <= 1e-4 * np.abs(ok).max()
        assert np.abs(gv - ov).max() <= 1e-4 * np.abs(ov).max()


@pytest.mark.parametrize("n_seqs", [1, 2])
def test_speculative_steps_head_dim_64_one_and_two_passes(ctx, n_seqs):
    """Head dim 64 (64-position spans, three query heads per kv head): one sequence
    keeps every step within one pass of rows (up to 4); two sequences make a 6-row
    verify. Each step is checked against the oracle."""
    from ferrolm_amd.synth import random_model
    from ferrolm_amd.weights import Config
    cfg = Config(vocab=512, hidden=192, intermediate=384, layers=2, heads=6, kv_heads=2, head_dim=64,
                 rms_eps=1e-5, max_position=2048)
    hm = random_model(cfg, seed=13, std=0.05)
    rng = np.random.default_rng(14)
    prompts = [[int(x) for x in rng.integers(3, 500, n)] for n in (333, 150)[:n_seqs]]
    _batched_matches_oracle(ctx, hm, prompts, k=2, steps=10, kv_blocks=80, seed=8)


def test_quantized_forward_matches_oracle(ctx):
    hm = load_model(GOLDEN / "llama-gqa")
    for kind in [INT8, INT4]:
        for l in hm.layers:
            for name in ["wqkv", "wo", "w_gate_up", "w_down"]:
                mat = getattr(l, name)
                if mat.kind == BF16:
                    setattr(l, name, oracle.quantize(kind, bf16_to_f32(mat.bf16).reshape(mat.rows, mat.cols)))
                else:
                    setattr(l, name, oracle.quantize(kind, mat.to_f32()))
        prompt = list(range(3, 99))
        table = list(range(8))
        m = gpu.Model(ctx, hm)
        kv = gpu.KvCache(ctx, hm.cfg, 8)
        out = gpu.forward(ctx, m, kv, [(prompt, 0, table, gpu.LOGITS_ALL)])
        om = oracle.Model(hm)
        ol = om.forward(om.kv(8), [(prompt, 0, table, 2)])
        assert np.abs(out.logits - ol).max() < 1e-4 * np.abs(ol).max(), kind


@pytest.mark.parametrize("kind", [BF16, INT8, INT4])
def test_gemm_path_forward_and_batched_steps(ctx, kind):
    """Steps of more than 16 rows on a model 1024 wide run every projection as the
    bf16-MFMA GEMM (activations as hi + lo bf16 pieces, split K for the narrow
    products): a 40-token prefill with all logits and the hidden states against the
    oracle, then batched speculative steps whose 20-row verifies are GEMMs, each
    sequence's tokens against the oracle's spec step."""
    from ferrolm_amd.synth import random_model
    from ferrolm_amd.weights import Config
    cfg = Config(vocab=1024, hidden=1024, intermediate=2048, layers=2, heads=16, kv_heads=4, head_dim=64,
                 rms_eps=1e-5, max_position=2048)
    hm = _quantized(random_model(cfg, seed=21, std=0.03), kind)
    rng = np.random.default_rng(22)
    prompt = [int(x) for x in rng.integers(3, 1000, 40)]
    table, blocks = scattered_table(64)
    m = gpu.Model(ctx, hm)
    kv = gpu.KvCache(ctx, hm.cfg, blocks)
    out = gpu.forward(ctx, m, kv, [(prompt, 0, table, gpu.LOGITS_ALL)], hidden=True)
    om = oracle.Model(hm)
    ol, oh = om.forward(om.kv(blocks), [(prompt, 0, table, 2)], hidden=True)
    assert np.abs(out.logits - ol).max() < 1e-4 * np.abs(ol).max(), kind
    rel = np.linalg.norm(out.hidden - oh, axis=-1) / np.linalg.norm(oh, axis=-1)
    assert rel.max() < 1e-4, rel.max()
    prompts = [[int(x) for x in rng.integers(3, 1000, n)] for n in (40, 90, 17, 130)]
    _batched_matches_oracle(ctx, hm, prompts, k=4, steps=6, kv_blocks=64, seed=23)


@pytest.mark.parametrize("shape", [(576, 9, 3, 64), (512, 4, 2, 128), (256, 8, 8, 32)])
def test_output_projection_merge_matches_separate_merge(ctx, shape, monkeypatch):
    """Decode steps of 1 to 4 rows on bf16 models run the output projection
    with the attention merge folded in (the span partials merged in each
    workgroup); a context created with FERRO_SEPARATE_MERGE=1 runs the merge
    kernel instead. The operands are built with the same arithmetic (both
    merge a row's spans in one batch at these contexts), so logits, hidden
    states and the cache agree bit for bit; both agree with the oracle."""
    from ferrolm_amd.synth import random_model
    from ferrolm_amd.weights import Config
    hidden, heads, kv_heads, hd = shape
    cfg = Config(vocab=512, hidden=hidden, intermediate=2 * hidden, layers=2, heads=heads, kv_heads=kv_heads,
                 head_dim=hd, rms_eps=1e-5, max_position=2048)
    hm = random_model(cfg, seed=31, std=0.05)
    monkeypatch.setenv("FERRO_SEPARATE_MERGE", "1")
    ctx2 = gpu.Context()
    monkeypatch.delenv("FERRO_SEPARATE_MERGE")
    table, blocks = scattered_table(340)
    rng = np.random.default_rng(32)
    prompt = [int(x) for x in rng.integers(3, 500, 320)]
    runs = []
    for c in (ctx, ctx2):
        m = gpu.Model(c, hm)
        kv = gpu.KvCache(c, hm.cfg, blocks)
        gpu.forward(c, m, kv, [(prompt, 0, table, gpu.LOGITS_LAST)])
        outs, pos = [], len(prompt)
        for n in (1, 2, 3, 4):
            toks = [int(x) for x in rng.integers(3, 500, n)] if c is ctx else runs[0][2][len(outs)]
            o = gpu.forward(c, m, kv, [(toks, pos, table, gpu.LOGITS_ALL)], hidden=True)
            outs.append((o.logits, o.hidden, toks))
            pos += n
        runs.append(([x[0] for x in outs], [x[1] for x in outs], [x[2] for x in outs],
                     [kv.layer(i) for i in range(cfg.layers)]))
        del kv, m
    ctx2.close()
    (l1, h1, t1, kv1), (l2, h2, t2, kv2) = runs
    for a, b in zip(l1, l2):
        assert np.array_equal(a, b)
    for a, b in zip(h1, h2):
        assert np.array_equal(a, b)
    for (k1, v1), (k2, v2) in zip(kv1, kv2):
        assert np.array_equal(k1, k2) and np.array_equal(v1, v2)
    om = oracle.Model(hm)
    okv = om.kv(blocks)
    om.forward(okv, [(prompt, 0, table, 1)])
    pos = len(prompt)
    for toks, lg in zip(t1, l1):
        ol = om.forward(okv, [(toks, pos, table, 2)])
        assert np.abs(lg - ol).max() < 1e-4 * np.abs(ol).max()
        pos += len(toks)


@pytest.mark.parametrize("shape", [(576, 9, 3, 64, 1536), (512, 4, 2, 128, 1024), (1024, 16, 4, 64, 2048)],
                         ids=["draft-135m", "hd128", "wide1024"])
def test_fused_mlp_matches_unfused_and_oracle(ctx, shape, monkeypatch):
    """Decode steps of 1 to 4 rows on bf16 models fuse each layer's gate/up
    and down but the last (EPI_MLP: the down projection's output summed
    exactly in a fixed-point accumulator, 2^-36; the next q/k/v forms x + acc
    and its norm, AX). A context created with FERRO_NO_MLP_FUSE=1 runs the
    separate kernels. Logits and cache slots of the two agree to the rounding
    of the different summation orders, and both agree with the oracle's to the
    bars of the other forward tests; the greedy ids are equal (near-tie rule)."""
    from ferrolm_amd.synth import random_model
    from ferrolm_amd.weights import Config
    hidden, heads, kv_heads, hd, inter = shape
    cfg = Config(vocab=512, hidden=hidden, intermediate=inter, layers=4, heads=heads, kv_heads=kv_heads,
                 head_dim=hd, rms_eps=1e-5, max_position=2048)
    hm = random_model(cfg, seed=41, std=0.05)
    monkeypatch.setenv("FERRO_NO_MLP_FUSE", "1")
    ctx2 = gpu.Context()
    monkeypatch.delenv("FERRO_NO_MLP_FUSE")
    table, blocks = scattered_table(200)
    rng = np.random.default_rng(42)
    prompt = [int(x) for x in rng.integers(3, 500, 150)]
    steps = [[int(x) for x in rng.integers(3, 500, n)] for n in (1, 2, 3, 4, 1)]
    runs = []
    for c in (ctx, ctx2):
        m = gpu.Model(c, hm)
        kv = gpu.KvCache(c, hm.cfg, blocks)
        gpu.forward(c, m, kv, [(prompt, 0, table, gpu.LOGITS_LAST)])
        outs, pos = [], len(prompt)
        for toks in steps:
            o = gpu.forward(c, m, kv, [(toks, pos, table, gpu.LOGITS_ALL)])
            outs.append((o.logits, o.argmax))
            pos += len(toks)
        runs.append((outs, [kv.layer(i) for i in range(cfg.layers)]))
        del kv, m
    ctx2.close()
    (o1, kv1), (o2, kv2) = runs
    for (l1, a1), (l2, a2) in zip(o1, o2):
        assert np.abs(l1 - l2).max() <= 1e-5 * np.abs(l2).max()
    for (k1, v1), (k2, v2) in zip(kv1, kv2):
        assert np.array_equal(k1 != 0, k2 != 0)
        assert np.abs(k1 - k2).max() <= 1e-5 * np.abs(k2).max() and np.abs(v1 - v2).max() <= 1e-5 * np.abs(v2).max()
    om = oracle.Model(hm)
    okv = om.kv(blocks)
    om.forward(okv, [(prompt, 0, table, 1)])
    pos = len(prompt)
    for toks, (lg, am) in zip(steps, o1):
        ol = om.forward(okv, [(toks, pos, table, 2)])
        assert np.abs(lg - ol).max() < 1e-4 * np.abs(ol).max()
        assert_argmax_parity(am, ol)
        pos += len(toks)


@pytest.mark.parametrize("hd,heads,kv_heads,n", [(64, 16, 4, 1100), (128, 8, 2, 700), (64, 16, 16, 520)],
                         ids=["hd64", "hd128", "mha-hd64"])
def test_long_gqa_prefill_runs_multi_span_attention(ctx, hd, heads, kv_heads, n):
    """A prefill of n tokens whose row groups hold 32 queries (8 rows x GQA 4)
    launches more than 1024 attention work items of one span, so each item
    covers 128 positions: 2 (hd 64) or 4 (hd 128) sub-spans whose loads
    overlap the previous sub-span's scores, merged online. All logits and the
    hidden states against the oracle, and the cache slots."""
    from ferrolm_amd.synth import random_model
    from ferrolm_amd.weights import Config
    cfg = Config(vocab=512, hidden=heads * hd, intermediate=512, layers=2, heads=heads, kv_heads=kv_heads,
                 head_dim=hd, rms_eps=1e-5, rope_theta=500000.0, max_position=2048)
    hm = random_model(cfg, seed=51, std=0.05)
    prompt = [int(x) for x in np.random.default_rng(52).integers(3, 500, n)]
    table, blocks = scattered_table(n)
    m = gpu.Model(ctx, hm)
    kv = gpu.KvCache(ctx, hm.cfg, blocks)
    out = gpu.forward(ctx, m, kv, [(prompt, 0, table, gpu.LOGITS_ALL)], hidden=True)
    om = oracle.Model(hm)
    okv = om.kv(blocks)
    ol, oh = om.forward(okv, [(prompt, 0, table, 2)], hidden=True)
    assert np.abs(out.logits - ol).max() < 1e-4 * np.abs(ol).max()
    rel = np.linalg.norm(out.hidden - oh, axis=-1) / np.linalg.norm(oh, axis=-1)
    assert rel.max() < 1e-4, rel.max()
    for li in range(cfg.layers):
        gk, gv = kv.layer(li)
        ok, ov = okv.layer(li)
        assert np.abs(gk - ok).max() <= 1e-4 * np.abs(ok).max()
        assert np.abs(gv - ov).max() <= 1e-4 * np.abs(ov).max()


@pytest.mark.gpu
@pytest.mark.parametrize("kind", [BF16, INT8, INT4], ids=["bf16", "int8", "int4"])
def test_narrow_model_long_prefill_takes_the_gemm(ctx, kind):
    """A model narrower than 1024 (the 135M draft's 576: 18 k-blocks, padded
    to 20 on the device) runs a prefill of 256 rows or more on the GEMM.
    All logits, the hidden states and the cache slots against the oracle,
    and the profiler's records show every projection on the GEMM path."""
    from ferrolm_amd.synth import quantize_model, random_model
    from ferrolm_amd.weights import Config
    cfg = Config(vocab=512, hidden=576, intermediate=1536, layers=2, heads=9, kv_heads=3, head_dim=64,
                 rms_eps=1e-5, rope_theta=100000.0, max_position=2048)
    hm = quantize_model(random_model(cfg, seed=61, std=0.05), kind)
    n = 300
    prompt = [int(x) for x in np.random.default_rng(62).integers(3, 500, n)]
    table, blocks = scattered_table(n)
    m = gpu.Model(ctx, hm)
    kv = gpu.KvCache(ctx, hm.cfg, blocks)
    gpu.profile(ctx, True)
    gpu.profile_read(ctx, reset=True)
    try:
        out = gpu.forward(ctx, m, kv, [(prompt, 0, table, gpu.LOGITS_ALL)], hidden=True)
        recs = gpu.profile_read(ctx, reset=True)
    finally:
        gpu.profile(ctx, False)
    assert sum(r["launches"] for r in recs if r["gemm"]) >= 1 + 4 * cfg.layers, recs
    assert not any(r["launches"] for r in recs if not r["gemm"]), recs
    om = oracle.Model(hm)
    okv = om.kv(blocks)
    ol, oh = om.forward(okv, [(prompt, 0, table, 2)], hidden=True)
    assert np.abs(out.logits - ol).max() < 1e-4 * np.abs(ol).max()
    rel = np.linalg.norm(out.hidden - oh, axis=-1) / np.linalg.norm(oh, axis=-1)
    assert rel.max() < 1e-4, rel.max()
    for li in range(cfg.layers):
        gk, gv = kv.layer(li)
        ok, ov = okv.layer(li)
        assert np.abs(gk - ok).max() <= 1e-4 * np.abs(ok).max()
        assert np.abs(gv - ov).max() <= 1e-4 * np.abs(ov).max()


@pytest.mark.gpu
@pytest.mark.parametrize("heads,kv_heads,hd", [(32, 32, 64), (27, 9, 64), (32, 8, 128)],
                         ids=["mha-hd64", "gqa3-hd64", "gqa4-hd128"])
def test_flash_prefill_attention_across_chunks_and_sequences(ctx, heads, kv_heads, hd):
    """Long chunks at hd 64 and 128 run the flash attention items (64 rows of
    an MHA model, 20 of a GQA-3 one, 16 of a GQA-4 one, each walking the
    positions it sees in blocks of 64 or 32, split into parts of at most 256
    positions merged as spans). Two forwards:
    the first 520 tokens of one sequence; then its remaining 580 tokens (the
    items read the cached 520 positions) beside a fresh 300-token sequence.
    All logits, the hidden states and both sequences' cache slots against the
    oracle running the same chunks."""
    from ferrolm_amd.synth import random_model
    from ferrolm_amd.weights import Config
    cfg = Config(vocab=512, hidden=heads * hd, intermediate=512, layers=2, heads=heads, kv_heads=kv_heads,
                 head_dim=hd, rms_eps=1e-5, rope_theta=10000.0, max_position=2048)
    hm = random_model(cfg, seed=71, std=0.03)
    rng = np.random.default_rng(72)
    a = [int(x) for x in rng.integers(3, 500, 1100)]
    b = [int(x) for x in rng.integers(3, 500, 300)]
    ta, na = scattered_table(1100)
    tb, nb = scattered_table(300)
    tb = [x + na for x in tb]
    m = gpu.Model(ctx, hm)
    kv = gpu.KvCache(ctx, hm.cfg, na + nb)
    om = oracle.Model(hm)
    okv = om.kv(na + nb)
    steps = [[(a[:520], 0, ta, gpu.LOGITS_ALL)],
             [(a[520:], 520, ta, gpu.LOGITS_ALL), (b, 0, tb, gpu.LOGITS_ALL)]]
    for chunks in steps:
        out = gpu.forward(ctx, m, kv, chunks, hidden=True)
        ol, oh = om.forward(okv, [(t, p, tab, 2) for t, p, tab, _ in chunks], hidden=True)
        assert np.abs(out.logits - ol).max() < 1e-4 * np.abs(ol).max()
        rel = np.linalg.norm(out.hidden - oh, axis=-1) / np.linalg.norm(oh, axis=-1)
        assert rel.max() < 1e-4, rel.max()
    for li in range(cfg.layers):
        gk, gv = kv.layer(li)
        ok, ov = okv.layer(li)
        assert np.abs(gk - ok).max() <= 1e-4 * np.abs(ok).max()
        assert np.abs(gv - ov).max() <= 1e-4 * np.abs(ov).max()
