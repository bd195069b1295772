"""Load-time host routines of the product library (include/ferro_host.h) and
the Python weight containers, against the oracle. CPU only."""
import numpy as np
import pytest

import oracle
from ferrolm_amd import host, synth
from ferrolm_amd.weights import BF16, INT4, INT8, Config, bf16_to_f32, dequantize, load_model, shape

from conftest import GOLDEN


@pytest.mark.parametrize("kind", [INT8, INT4])
def test_product_quantizer_matches_oracle_bit_for_bit(kind):
    """QMatrix::quantize (src/quant.rs:78-143): codes and scales identical."""
    rng = np.random.default_rng(kind)
    for rows, cols in [(32, 32), (96, 544), (64, 2048)]:
        w = bf16_to_f32(host.random_bf16(5, rows, rows, cols, 0.02)).reshape(rows, cols)
        w[:, 3] *= 40.0
        imp = np.abs(rng.standard_normal(cols)).astype(np.float32) + 1e-8
        for importance in [None, imp]:
            a = host.quantize(kind, w, importance)
            b = oracle.quantize(kind, w, importance)
            assert np.array_equal(a.q, b.q) and np.array_equal(a.s, b.s)
    z = host.quantize(kind, np.zeros((32, 64), np.float32))
    assert not z.q.any() if kind == INT8 else np.all(z.q == 0x88)
    assert not z.s.any()


def test_dequantize_matches_oracle():
    w = bf16_to_f32(host.random_bf16(9, 1, 64, 256, 1.0)).reshape(64, 256)
    for kind in [INT8, INT4]:
        q = host.quantize(kind, w)
        ref = np.zeros((64, 256), np.float32)
        oracle.lib().or_dequantize(kind, 64, 256, oracle.ptr(q.q, oracle.u8p), oracle.ptr(q.s, oracle.f32p),
                                   oracle.ptr(ref, oracle.f32p))
        assert np.array_equal(dequantize(q), ref)


def test_random_weights_are_deterministic_normal_and_thread_independent():
    a = host.random_bf16(1, 7, 200, 96, 0.02)
    b = host.random_bf16(1, 7, 200, 96, 0.02)
    assert np.array_equal(a, b)
    assert not np.array_equal(a, host.random_bf16(1, 8, 200, 96, 0.02))
    f = bf16_to_f32(a).astype(np.float64)
    assert abs(f.mean()) < 0.002 and abs(f.std() - 0.02) < 0.001
    # rows are drawn in 64-row blocks from their own stream: the first block
    # of a taller matrix is the same matrix
    assert np.array_equal(host.random_bf16(1, 7, 64, 96, 0.02), a[:64])
    # block 0 is Rng::new(stream_seed) followed by Box-Muller, as the oracle's rng
    import ctypes
    st = ctypes.c_uint64(oracle.lib().or_rng_new(host.stream_seed(1, 7, 0)))
    vals = [oracle.lib().or_rng_normal(ctypes.byref(st)) * 0.02 for _ in range(5)]
    want = [oracle.lib().or_f32_to_bf16(float(np.float32(v))) for v in vals]
    assert list(a[0, :5]) == want


def test_awq_fold_keeps_the_function_before_rounding():
    """src/awq.rs:81-122: folding 1/s into the producers and s into the
    projection leaves the model's function unchanged (up to f32 rounding)."""
    cfg = Config(vocab=256, hidden=64, intermediate=96, layers=2, heads=4, kv_heads=4, head_dim=16,
                 rms_eps=1e-5, max_position=256)
    hm = synth.random_model(cfg, seed=3, std=0.05)
    # The same fold with the quantizer replaced by exact bf16->f32 storage.
    orig = synth.awq_apply
    try:
        captured = {}

        def fake_apply(kind, w, s, sq):
            from ferrolm_amd.weights import Matrix
            return Matrix(BF16, w.shape[0], w.shape[1], bf16=None, q=None, s=(w * s[None, :]).astype(np.float32))

        synth.awq_apply = fake_apply
        folded = synth.awq_model(hm, INT4, seed=1)
    finally:
        synth.awq_apply = orig
    x = np.random.default_rng(0).standard_normal((5, 64)).astype(np.float32)
    for l0, l1 in zip(hm.layers, folded.layers):
        wq0 = bf16_to_f32(l0.wqkv.bf16).reshape(l0.wqkv.rows, -1)
        xn0 = x * l0.attn_norm
        xn1 = x * l1.attn_norm
        y0 = xn0 @ wq0.T
        y1 = xn1 @ l1.wqkv.s.T
        # the o-fold divides v rows of qkv by s_o and multiplies wo columns by it
        qd = cfg.q_dim
        np.testing.assert_allclose(y1[:, :qd * 2], y0[:, :qd * 2], rtol=2e-5, atol=2e-6)
        v0 = y0[:, 2 * qd:]
        v1 = y1[:, 2 * qd:]
        o0 = v0 @ bf16_to_f32(l0.wo.bf16).reshape(l0.wo.rows, -1).T
        o1 = v1 @ l1.wo.s.T
        np.testing.assert_allclose(o1, o0, rtol=2e-4, atol=2e-6)


def test_awq_model_quantizes_every_projection():
    cfg = Config(vocab=256, hidden=64, intermediate=96, layers=1, heads=4, kv_heads=2, head_dim=16,
                 rms_eps=1e-5, max_position=256)
    hm = synth.awq_model(synth.random_model(cfg, seed=3), INT4, seed=2)
    l = hm.layers[0]
    assert all(getattr(l, n).kind == INT4 for n in ["wqkv", "wo", "w_gate_up", "w_down"])
    assert not np.all(l.attn_norm == 1) and not np.all(l.mlp_norm == 1)


def test_fixture_loader_stacks_projections():
    hm = load_model(GOLDEN / "llama-gqa")
    c = hm.cfg
    assert (c.hidden, c.heads, c.kv_heads, c.head_dim, c.layers) == (128, 8, 2, 16, 3)
    l = hm.layers[0]
    assert l.wqkv.rows == c.qkv_dim and l.w_gate_up.rows == 2 * c.intermediate
    assert hm.lm_head is not None and not c.tie_embeddings
    q = load_model(GOLDEN / "qwen2")
    assert q.cfg.qkv_bias and q.layers[0].bqkv.shape == (q.cfg.qkv_dim,)
    t = load_model(GOLDEN / "llama3-tied")
    assert t.cfg.rope_llama3 and t.cfg.tie_embeddings and t.lm_head is None


def test_benchmark_shapes():
    s = shape("smollm2-1.7b")
    assert (s.layers, s.hidden, s.heads, s.kv_heads, s.intermediate, s.vocab) == (24, 2048, 32, 32, 8192, 49152)
    # parameters in layers match the survey's count for the 1.7B shape
    per = s.hidden * s.qkv_dim + s.q_dim * s.hidden + 3 * s.hidden * s.intermediate
    assert per * s.layers == 1_610_612_736
    t, d, kind, k, plen = synth.shapes_for(2)
    assert kind == INT4 and k == 3 and plen == 1024 and d.hidden == 576


def test_table_cache_reuses_a_table_until_it_grows_or_is_replaced():
    from ferrolm_amd.spec import TableCache
    c = TableCache()
    t = [5, 9]
    a = c.get("s", t)
    assert a.dtype == np.uint32 and list(a) == [5, 9]
    assert c.get("s", t) is a              # unchanged: the same array
    t.append(2)
    b = c.get("s", t)
    assert list(b) == [5, 9, 2] and b is not a
    u = [7, 7, 7]                          # a released table's replacement, same length
    assert list(c.get("s", u)) == [7, 7, 7]
    c.drop("s")
    assert list(c.get("s", u)) == [7, 7, 7]
