"""The AWQ restatement in the oracle (src/awq.rs) and the host's channel
statistics and scales, on the CPU: the channel statistics and scales against
their closed forms, the search's errors against an independent f64
recomputation, its alpha against a brute-force argmin, and the reference's
own AWQ test (tests/quant.rs:60-82) on the llama-gqa fixture."""
import numpy as np
import pytest

import oracle
from ferrolm_amd import awq, host
from ferrolm_amd.weights import INT4, INT8, bf16_to_f32, dequantize, f32_to_bf16, load_model

from conftest import GOLDEN, oracle_awq, plain_quantized, reference_tokens, rel_error


def _calibration(seed, m, k):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[:, rng.choice(k, max(1, k // 16), replace=False)] *= 12.0  # outlier channels
    return x


def test_stats_and_scales_match_their_closed_forms_and_the_host():
    x = _calibration(1, 37, 96)
    a, q = oracle.awq_stats(x)
    ha, hq = host.awq_stats(x)
    assert np.array_equal(a, ha) and np.array_equal(q, hq)
    assert np.allclose(a, np.mean(np.abs(x.astype(np.float64)), axis=0), rtol=1e-6)
    assert np.allclose(q, np.mean(np.square(x.astype(np.float64)), axis=0), rtol=1e-6)
    for alpha in (0.0, 0.3, 1.0):
        s = oracle.awq_scales(a, alpha)
        assert np.array_equal(s, host.awq_scales(a, alpha))
        if alpha == 0.0:
            assert np.all(s == 1.0)
        else:
            # s_c proportional to a_c^alpha, normalised so that max * min = 1
            want = np.power(np.maximum(a, 1e-5).astype(np.float64), alpha)
            want /= np.sqrt(want.max() * want.min())
            assert np.allclose(s, want, rtol=1e-5)
            assert abs(float(s.max()) * float(s.min()) - 1.0) < 1e-5


def _errors_by_alpha(kind, w, cal):
    """Independent f64 evaluation of every alpha's output error: the
    dequantized apply() matrix on the scaled rows against the bf16 product."""
    a, sq = oracle.awq_stats(cal)
    yref = cal.astype(np.float64) @ bf16_to_f32(f32_to_bf16(w)).astype(np.float64).T
    errs = []
    for step in range(11):
        s = oracle.awq_scales(a, np.float32(step) / np.float32(10.0))
        m = oracle.quantize(kind, (w * s[None, :]).astype(np.float32), (sq / (s * s) + np.float32(1e-8)))
        y = (cal / s[None, :]).astype(np.float64) @ dequantize(m).astype(np.float64).T
        errs.append(float(np.mean(np.square(y - yref))))
    return errs


@pytest.mark.parametrize("kind", [INT8, INT4])
def test_search_picks_the_argmin_alpha_and_reports_its_errors(kind):
    rng = np.random.default_rng(7)
    w = (rng.standard_normal((96, 160)) * 0.05).astype(np.float32)
    cal = _calibration(3, 48, 160)
    s, alpha, ep, ea, m = oracle.awq_search(kind, w, cal)
    errs = _errors_by_alpha(kind, w, cal)
    assert ea <= ep
    assert ep == pytest.approx(errs[0], rel=1e-5)
    step = int(round(alpha * 10))
    assert ea == pytest.approx(errs[step], rel=1e-5)
    # the chosen alpha is the argmin, up to near-ties of the f32 chains
    assert errs[step] <= min(errs) * (1 + 1e-5)
    # the returned matrix is apply() at the chosen scales
    a, sq = oracle.awq_stats(cal)
    assert np.array_equal(s, oracle.awq_scales(a, np.float32(step) / np.float32(10.0)))
    again = oracle.quantize(kind, (w * s[None, :]).astype(np.float32), sq / (s * s) + np.float32(1e-8))
    assert np.array_equal(m.q, again.q) and np.array_equal(m.s, again.s)


def test_calibration_keeps_a_reservoir_of_projection_inputs():
    hm = load_model(GOLDEN / "llama-gqa")
    om = oracle.Model(hm)
    seqs = [reference_tokens(64, 10 + i) for i in range(8)]
    acts = oracle.calibrate(om, seqs, 256)
    c = hm.cfg
    assert len(acts) == c.layers
    widths = [c.hidden, c.heads * c.head_dim, c.hidden, c.intermediate]
    for l in acts:
        assert [a.shape for a in l] == [(256, w) for w in widths]
    # a stream that fits is kept whole, in order: two 64-token forwards
    small = oracle.calibrate(om, seqs[:2], 256)
    for i in range(2):
        kv = om.kv(4)
        _, taps = om.forward(kv, [(seqs[i], 0, list(range(4)), 0)], taps=True)
        assert np.array_equal(small[1][3][64 * i:64 * (i + 1)], taps[1][3])
    # every kept row is a row of some sequence's taps
    allrows = []
    for sq in seqs:
        kv = om.kv(4)
        _, t = om.forward(kv, [(sq, 0, list(range(4)), 0)], taps=True)
        allrows.append(t[2][0])
    allrows = np.concatenate(allrows)
    for r in acts[2][0][::37]:
        assert np.any(np.all(allrows == r, axis=1))


def test_reference_awq_folds_scales_and_reduces_held_out_error():
    """tests/quant.rs:60-82 on the oracle: int4 AWQ with calibration from
    8 x 64 tokens keeps every projection's error at or below plain int4's
    on the calibration sample, and lowers the held-out logit error."""
    hm = load_model(GOLDEN / "llama-gqa")
    om = oracle.Model(hm)
    acts = oracle.calibrate(om, [reference_tokens(64, 10 + i) for i in range(8)], 256)
    held = reference_tokens(96, 99)

    def logits(m):
        kv = m.kv(6)
        return m.forward(kv, [(held, 0, list(range(6)), 2)])

    ref = logits(om)
    plain = oracle.Model(plain_quantized(hm, INT4, oracle.quantize))
    search, apply = oracle_awq()
    qm, choices = awq.quantize_awq(hm, INT4, acts, search, apply)
    assert len(choices) == 3 * hm.cfg.layers  # 8 heads / 2 kv heads: o is not searched
    assert all(c.error_awq <= c.error_plain for c in choices)
    e_plain = rel_error(logits(plain), ref)
    e_awq = rel_error(logits(oracle.Model(qm)), ref)
    print(f"held-out relative logit error: int4 {e_plain:.4f}, int4+AWQ {e_awq:.4f}")
    assert e_awq < e_plain


@pytest.mark.parametrize("fixture", ["llama-gqa", "qwen2"])
def test_quantized_model_round_trips_through_its_file(tmp_path, fixture):
    """save_quantized / load_quantized: every array, the config and the
    oracle's logits come back identical (AWQ int4 with the oracle's search;
    qwen2 carries a q/k/v bias; a bf16 model round-trips too)."""
    from ferrolm_amd.weights import load_quantized, save_quantized
    hm = load_model(GOLDEN / fixture)
    om = oracle.Model(hm)
    acts = oracle.calibrate(om, [reference_tokens(48, 20 + i) for i in range(3)], 64)
    qm, _ = awq.quantize_awq(hm, INT4, acts, *oracle_awq())
    toks = reference_tokens(40, 5)
    for model in (qm, hm):
        path = tmp_path / "model.safetensors"
        save_quantized(model, path)
        back = load_quantized(path)
        assert back.cfg == model.cfg
        assert np.array_equal(back.embed, model.embed) and np.array_equal(back.norm, model.norm)
        for a, b in zip(back.layers, model.layers):
            for name in ("wqkv", "wo", "w_gate_up", "w_down"):
                x, y = getattr(a, name), getattr(b, name)
                assert (x.kind, x.rows, x.cols) == (y.kind, y.rows, y.cols)
                for f in ("bf16", "q", "s"):
                    assert (getattr(x, f) is None) == (getattr(y, f) is None)
                    if getattr(x, f) is not None:
                        assert np.array_equal(getattr(x, f), getattr(y, f))
            assert np.array_equal(a.attn_norm, b.attn_norm) and np.array_equal(a.mlp_norm, b.mlp_norm)
            assert (a.bqkv is None) == (b.bqkv is None)
        lo = [oracle.Model(m).forward(oracle.Model(m).kv(3), [(toks, 0, [0, 1, 2], 2)]) for m in (back, model)]
        assert np.array_equal(lo[0], lo[1])


def test_reservoir_generator_known_answers():
    """Model::record's generator is Marsaglia's xorshift64 (13, 7, 17): the
    first three outputs from his example seed 88172645463325252, as printed
    in "Xorshift RNGs" (J. Stat. Softw. 8(14), 2003)."""
    v, out = 88172645463325252, []
    for _ in range(3):
        v = awq.xorshift64(v)
        out.append(v)
    assert out == [8748534153485358512, 3040900993826735515, 3453997556048239312]


def test_host_reservoir_keeps_the_rows_model_record_keeps():
    """The product's reservoir (awq.Reservoir, fed per forward as the device
    capture delivers rows) keeps the same rows in the same slots as the
    oracle's Model::calibrate, for a stream that overflows max_rows many
    times (8 x 64 rows into 24) and one that fits."""
    hm = load_model(GOLDEN / "llama-gqa")
    om = oracle.Model(hm)
    seqs = [reference_tokens(64, 10 + i) for i in range(8)]
    for max_rows in (24, 600):
        want = oracle.calibrate(om, seqs, max_rows)
        res = awq.Reservoir(hm.cfg.layers, max_rows)
        for s in seqs:
            kv = om.kv(4)
            _, taps = om.forward(kv, [(s, 0, list(range(4)), 0)], taps=True)
            for li in range(hm.cfg.layers):
                for which in range(4):
                    res.record(li, which, taps[li][which])
        got = res.result()
        for gl, wl in zip(got, want):
            for g, w in zip(gl, wl):
                assert g.shape == w.shape and np.array_equal(g, w)
