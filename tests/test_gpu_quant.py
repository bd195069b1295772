"""Load-time quantization on the device (fg_quantize, fg_awq_search) against
the oracle's QMatrix::quantize and awq::search restatements: codes, scales,
the chosen alpha and both errors bit for bit; then the reference's AWQ test
(tests/quant.rs:60-82) with the device search and the device forward."""
import numpy as np
import pytest

import oracle
from ferrolm_amd import awq, gpu
from ferrolm_amd.weights import INT4, INT8, load_model

from conftest import GOLDEN, oracle_awq, plain_quantized, reference_tokens, rel_error

pytestmark = pytest.mark.gpu


def _weights(seed, rows, cols):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((rows, cols)) * 0.05).astype(np.float32)
    w[:, :32] = 0.0                                   # all-zero groups: scale 0, codes 0
    w[1, 32:64] = 1e-30                               # tiny groups (scale near the f32 floor)
    w[2, 64:96] = rng.choice([-1.0, 0.5, 1.0], 32)    # round-half cases
    w[3, 96:128] *= 100.0
    return w


@pytest.mark.parametrize("kind", [INT8, INT4], ids=["int8", "int4"])
@pytest.mark.parametrize("shape", [(32, 128), (96, 160), (256, 544)], ids=["32x128", "96x160", "256x544"])
def test_device_quantizer_reproduces_the_reference_codes(ctx, kind, shape):
    rows, cols = shape
    w = _weights(rows + cols, rows, cols)
    imp = np.random.default_rng(5).uniform(0.01, 4.0, cols).astype(np.float32)
    for importance in (None, imp):
        got = gpu.quantize(ctx, kind, w, importance)
        want = oracle.quantize(kind, w, importance)
        assert np.array_equal(got.s, want.s), shape
        assert np.array_equal(got.q, want.q), shape


def test_device_quantizer_rejects_bad_shapes(ctx):
    with pytest.raises(gpu.FgError, match="multiples of 32"):
        gpu.quantize(ctx, INT4, np.zeros((32, 48), np.float32))
    with pytest.raises(gpu.FgError, match="FG_INT8 or FG_INT4"):
        gpu.quantize(ctx, 0, np.zeros((32, 64), np.float32))


def _cal(seed, m, k):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[:, rng.choice(k, max(1, k // 16), replace=False)] *= 12.0
    return x


@pytest.mark.parametrize("kind", [INT8, INT4], ids=["int8", "int4"])
def test_device_awq_search_matches_the_oracle_bit_for_bit(ctx, kind):
    hm = load_model(GOLDEN / "llama-gqa")
    acts = oracle.calibrate(oracle.Model(hm), [reference_tokens(64, 10 + i) for i in range(8)], 256)
    l = hm.layers[1]
    cases = [(l.wqkv.to_f32(), acts[1][0]), (l.wo.to_f32(), acts[1][1]), (l.w_gate_up.to_f32(), acts[1][2]),
             (l.w_down.to_f32(), acts[1][3]), (_weights(9, 384, 512), _cal(4, 37, 512))]
    for w, cal in cases:
        s, alpha, ep, ea, m = gpu.awq_search(ctx, kind, w, cal)
        os_, oalpha, oep, oea, om = oracle.awq_search(kind, w, cal)
        assert alpha == oalpha and ep == oep and ea == oea, (w.shape, alpha, oalpha, ep, oep, ea, oea)
        assert np.array_equal(s, os_)
        assert np.array_equal(m.q, om.q) and np.array_equal(m.s, om.s)


def test_reference_awq_test_on_the_device(ctx):
    """tests/quant.rs:60-82 with every projection's search on the device:
    the model equals the oracle-searched one bit for bit, and the device
    forward's held-out logit error is lower than plain int4's."""
    c = ctx
    hm = load_model(GOLDEN / "llama-gqa")
    om = oracle.Model(hm)
    acts = oracle.calibrate(om, [reference_tokens(64, 10 + i) for i in range(8)], 256)
    held = reference_tokens(96, 99)
    search, apply = awq.device(c)
    qm, choices = awq.quantize_awq(hm, INT4, acts, search, apply)
    oqm, ochoices = awq.quantize_awq(hm, INT4, acts, *oracle_awq())
    assert [(x.alpha, x.error_plain, x.error_awq) for x in choices] == \
        [(x.alpha, x.error_plain, x.error_awq) for x in ochoices]
    for a, b in zip(qm.layers, oqm.layers):
        for name in ("wqkv", "wo", "w_gate_up", "w_down"):
            assert np.array_equal(getattr(a, name).q, getattr(b, name).q)
            assert np.array_equal(getattr(a, name).s, getattr(b, name).s)
        assert np.array_equal(a.attn_norm, b.attn_norm) and np.array_equal(a.mlp_norm, b.mlp_norm)

    def logits(host_model):
        m = gpu.Model(c, host_model)
        kv = gpu.KvCache(c, host_model.cfg, 6)
        return gpu.forward(c, m, kv, [(held, 0, list(range(6)), gpu.LOGITS_ALL)]).logits

    ref = logits(hm)
    e_plain = rel_error(logits(plain_quantized(hm, INT4, lambda k, w: gpu.quantize(c, k, w))), ref)
    e_awq = rel_error(logits(qm), ref)
    print(f"device held-out relative logit error: int4 {e_plain:.4f}, int4+AWQ {e_awq:.4f}")
    assert all(x.error_awq <= x.error_plain for x in choices)
    assert e_awq < e_plain


def test_device_awq_search_rejects_bad_arguments(ctx):
    w = np.zeros((64, 64), np.float32)
    with pytest.raises(gpu.FgError, match="calibration rows"):
        gpu.awq_search(ctx, INT4, w, np.zeros((0, 64), np.float32))
    with pytest.raises(gpu.FgError, match="input width"):
        gpu.awq_search(ctx, INT4, w, np.zeros((4, 32), np.float32))
    with pytest.raises(gpu.FgError, match="multiples of 32"):
        gpu.awq_search(ctx, INT8, np.zeros((48, 64), np.float32), np.zeros((4, 64), np.float32))
    # an all-zero matrix quantizes to zero codes and scales at every alpha, error 0
    s, alpha, ep, ea, m = gpu.awq_search(ctx, INT4, w, np.random.default_rng(0).standard_normal((8, 64)).astype(
        np.float32))
    assert (alpha, ep, ea) == (0.0, 0.0, 0.0)
    assert not m.s.any() and np.all(m.q == 0x88)


def _captures_close(dev, ora, tol=1e-4):
    """Same rows in the same slots (the reservoir draws depend only on the
    row counts), values within tol of the oracle's, row by row (relative L2;
    the residual stream's own bar in the forward tests)."""
    assert len(dev) == len(ora)
    for li, (dl, ol) in enumerate(zip(dev, ora)):
        for which, (d, o) in enumerate(zip(dl, ol)):
            assert d.shape == o.shape, (li, which, d.shape, o.shape)
            if d.size:
                rel = np.linalg.norm(d - o, axis=-1) / np.maximum(np.linalg.norm(o, axis=-1), 1e-30)
                assert rel.max() < tol, (li, which, float(rel.max()))


def test_device_calibration_matches_model_calibrate(ctx):
    """Model::calibrate (src/awq.rs:38-62) with the capture on the device
    (fg_forward_capture: the norms of the residual rows, the merged attention
    output and the SwiGLU activation of the gate/up epilogue) and the host
    reservoir, against the oracle's: sequences of 1 to 64 tokens (decode-sized
    GEMV steps, the bf16 merge-in-projection path at up to 4 rows), a stream
    that overflows the reservoir and one that fits. The device's rows then
    drive the AWQ search on the device, bit-equal to the oracle's search on
    the same rows: calibration, search and quantization end to end without
    the checker."""
    hm = load_model(GOLDEN / "llama-gqa")
    om = oracle.Model(hm)
    m = gpu.Model(ctx, hm)
    seqs = [reference_tokens(n, 30 + i) for i, n in enumerate((64, 3, 37, 64, 1, 64, 20, 64))]
    for max_rows in (256, 40):
        dev = awq.calibrate(ctx, m, seqs, max_rows)
        _captures_close(dev, oracle.calibrate(om, seqs, max_rows))
    qm, choices = awq.quantize_awq(hm, INT4, dev, *awq.device(ctx))
    oqm, ochoices = awq.quantize_awq(hm, INT4, dev, *oracle_awq())
    assert [(x.alpha, x.error_plain, x.error_awq) for x in choices] == \
        [(x.alpha, x.error_plain, x.error_awq) for x in ochoices]
    for a, b in zip(qm.layers, oqm.layers):
        for name in ("wqkv", "wo", "w_gate_up", "w_down"):
            assert np.array_equal(getattr(a, name).q, getattr(b, name).q)
            assert np.array_equal(getattr(a, name).s, getattr(b, name).s)


@pytest.mark.parametrize("kind", [0, INT8, INT4], ids=["bf16", "int8", "int4"])
def test_device_calibration_on_the_gemm_path(ctx, kind):
    """A 1024-wide model: 40- and 1024-token sequences run every projection
    as the MFMA GEMM (the SwiGLU capture in the GEMM epilogue, with split K),
    the 1024-token one with the flash prefill attention's partials; the
    captured rows against the oracle's."""
    from ferrolm_amd.synth import random_model
    from ferrolm_amd.weights import Config
    cfg = Config(vocab=1024, hidden=1024, intermediate=2048, layers=2, heads=16, kv_heads=4, head_dim=64,
                 rms_eps=1e-5, max_position=2048)
    hm = random_model(cfg, seed=41, std=0.03)
    if kind:
        hm = plain_quantized(hm, kind, lambda k, w: gpu.quantize(ctx, k, w))
    rng = np.random.default_rng(42)
    seqs = [[int(x) for x in rng.integers(3, 1000, n)] for n in (40, 1024)]
    dev = awq.calibrate(ctx, gpu.Model(ctx, hm), seqs, 2048)
    _captures_close(dev, oracle.calibrate(oracle.Model(hm), seqs, 2048))
