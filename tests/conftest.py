import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

GOLDEN = ROOT / "tests" / "golden"
FIXTURES = ["llama-gqa", "llama3-tied", "qwen2"]


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def ctx():
    from ferrolm_amd import gpu
    c = gpu.Context(0)
    yield c
    c.close()


def reference_prompts(n, seed):
    """tests/engine.rs:19-27 of the reference: n prompts from Rng(seed),
    lengths between(1, 150), ids between(3, 511)."""
    import ctypes
    import oracle
    rng = ctypes.c_uint64(oracle.lib().or_rng_new(seed))
    nxt = lambda: oracle.lib().or_rng_next(ctypes.byref(rng))
    out = []
    for _ in range(n):
        ln = 1 + nxt() % 150
        out.append([3 + nxt() % 509 for _ in range(ln)])
    return out


def reference_tokens(n, seed):
    """tests/quant.rs:36-39 of the reference: n ids between(3, 511) from Rng(seed)."""
    import ctypes
    import oracle
    rng = ctypes.c_uint64(oracle.lib().or_rng_new(seed))
    return [3 + oracle.lib().or_rng_next(ctypes.byref(rng)) % 509 for _ in range(n)]


def oracle_awq():
    """The oracle's AWQ search and apply, in the shape ferrolm_amd.awq takes."""
    import numpy as np
    import oracle

    def apply(kind, w, s, cal):
        _, sq = oracle.awq_stats(cal)
        ws = (np.ascontiguousarray(w, np.float32) * s[None, :]).astype(np.float32)
        imp = (sq / (s * s) + np.float32(1e-8)).astype(np.float32)
        return oracle.quantize(kind, ws, imp)

    return oracle.awq_search, apply


def plain_quantized(hm, kind, quantize):
    """Model::quantize(kind, None) (src/model.rs:192-219) with the given
    quantize(kind, w) -> Matrix."""
    from dataclasses import replace
    out = [replace(l, wqkv=quantize(kind, l.wqkv.to_f32()), wo=quantize(kind, l.wo.to_f32()),
                   w_gate_up=quantize(kind, l.w_gate_up.to_f32()), w_down=quantize(kind, l.w_down.to_f32()))
           for l in hm.layers]
    return replace(hm, layers=out)


def rel_error(a, b) -> float:
    """tests/quant.rs:30-34: sqrt(sum (a - b)^2 / sum b^2), f64."""
    import numpy as np
    a = np.asarray(a, np.float32).ravel()
    b = np.asarray(b, np.float32).ravel()
    num = np.sum(np.square((a - b).astype(np.float64)))
    den = np.sum(np.square(b.astype(np.float64)))
    return float(np.sqrt(num / den))


def exact_two_token_distribution(m, prompt, params):
    """tests/engine.rs:163-194 of the reference on the oracle model m: the
    probability of each two-token continuation of prompt under params =
    (temperature, top_p, top_k)."""
    import oracle

    def nxt(tokens):
        kv = m.kv(16)
        lg = m.forward(kv, [(tokens, 0, list(range(16)), 1)])[0]
        return zip(*oracle.distribution(lg, *params))

    out = []
    for t1, p1 in nxt(prompt):
        for t2, p2 in nxt(list(prompt) + [int(t1)]):
            out.append(((int(t1), int(t2)), float(p1) * float(p2)))
    return out


def chi_square(counts: dict, exact, n: int) -> float:
    """Pearson's statistic of observed continuation counts against exact."""
    assert set(counts) <= {s for s, _ in exact}, "impossible continuation sampled"
    return sum((counts.get(s, 0) - p * n) ** 2 / (p * n) for s, p in exact)


# Near-tie rule for greedy tokens. The device's logits agree with the oracle's
# to LOGIT_TOL x the row's largest |logit| (the fixture and config tests hold
# them to that), so the device may pick a different token only where the
# oracle's top two are within twice that of each other. Such a row is a
# documented near-tie; any other difference fails.
LOGIT_TOL = 1e-4
NEAR_TIE = 2 * LOGIT_TOL


def assert_argmax_parity(dev_argmax, ref_logits, tol: float = NEAR_TIE, max_ties: int | None = None) -> int:
    """Per-row greedy token of the device against sampler::argmax of the
    reference logits (first index of the maximum, src/sampler.rs:42-51).
    A row may differ only at a near-tie: the reference logit of the device's
    token is within tol x max|logit| of the row's maximum. Returns the number
    of excused rows (at most max_ties, default 1% of the rows + 1)."""
    import numpy as np
    dev = np.asarray(dev_argmax).astype(np.int64).ravel()
    ref = np.asarray(ref_logits, np.float32).reshape(len(dev), -1)
    want = ref.argmax(axis=1)
    ties = 0
    for r in np.nonzero(dev != want)[0]:
        gap = float(ref[r, want[r]]) - float(ref[r, dev[r]])
        scale = float(np.abs(ref[r]).max())
        assert 0.0 <= gap <= tol * scale, (
            f"row {r}: device token {dev[r]} vs {want[r]}, logit gap {gap:.3e} above the near-tie bar "
            f"{tol * scale:.3e}")
        ties += 1
    limit = max_ties if max_ties is not None else len(dev) // 100 + 1
    assert ties <= limit, f"{ties} near-tie rows of {len(dev)}"
    return ties
