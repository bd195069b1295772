"""ctypes binding of the CPU oracle (liboracle.so, built from ferro_oracle.c).

TEST INFRASTRUCTURE ONLY. The oracle is a C restatement of the reference's
CPU path (Rust, /root/reference/src), used as the parity checker for the
HIP path and as bench.py's timed CPU baseline. Only tests/, the smoke()
entry point and bench.py's cpu_baseline leg import this module; nothing in
the ferrolm_amd package does.

Parity pins (tests/test_oracle.py): the three transformers fixtures of the
reference's tests/reference.rs (logits within 1e-3 of the largest logit and
40 exact greedy tokens), the reference's kernel and quantizer unit-test
properties (src/kernels.rs:758-818, src/quant.rs:456-523), closed forms
(f64 matmul, dense softmax attention) and engine invariants
(speculative greedy == target alone, self-draft accepts everything,
tests/engine.rs:134-160).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np

from ferrolm_amd.weights import BF16, INT8, HostModel, Matrix

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"

f32p = C.POINTER(C.c_float)
u16p = C.POINTER(C.c_uint16)
u8p = C.POINTER(C.c_uint8)
u32p = C.POINTER(C.c_uint32)
i32p = C.POINTER(C.c_int32)
i64p = C.POINTER(C.c_int64)


class OrConfig(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("vocab", "hidden", "intermediate", "layers", "heads", "kv_heads",
                                          "head_dim")] + [
        ("rms_eps", C.c_float), ("rope_theta", C.c_float), ("rope_llama3", C.c_int32),
        ("rope_factor", C.c_float), ("rope_low_freq", C.c_float), ("rope_high_freq", C.c_float),
        ("rope_orig_max_pos", C.c_int32), ("max_position", C.c_int32), ("tie_embeddings", C.c_int32),
        ("qkv_bias", C.c_int32)]


class OrMatrix(C.Structure):
    _fields_ = [("kind", C.c_int32), ("rows", C.c_int32), ("cols", C.c_int32), ("_pad", C.c_int32),
                ("bf16", u16p), ("q", u8p), ("s", f32p)]


class OrLayer(C.Structure):
    _fields_ = [("attn_norm", f32p), ("wqkv", OrMatrix), ("bqkv", f32p), ("wo", OrMatrix),
                ("mlp_norm", f32p), ("w_gate_up", OrMatrix), ("w_down", OrMatrix)]


class OrChunk(C.Structure):
    _fields_ = [("tokens", u32p), ("n", C.c_int32), ("pos", C.c_int32), ("blocks", u32p),
                ("n_blocks", C.c_int32), ("logits", C.c_int32)]


def build() -> None:
    """Compiles liboracle.so with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", str(HERE), "-B"], check=True)


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        l = C.CDLL(str(LIB))
        sig = {
            "or_rng_new": (C.c_uint64, [C.c_uint64]),
            "or_rng_next": (C.c_uint64, [C.POINTER(C.c_uint64)]),
            "or_rng_uniform": (C.c_double, [C.POINTER(C.c_uint64)]),
            "or_rng_normal": (C.c_double, [C.POINTER(C.c_uint64)]),
            "or_f32_to_bf16": (C.c_uint16, [C.c_float]),
            "or_exp": (C.c_float, [C.c_float]),
            "or_dot": (C.c_float, [f32p, f32p, C.c_int32]),
            "or_rms_norm": (None, [f32p, f32p, C.c_int32, C.c_int32, C.c_float, f32p]),
            "or_silu_mul": (None, [f32p, C.c_int32, C.c_int32, f32p]),
            "or_argmax": (C.c_uint32, [f32p, C.c_int32]),
            "or_distribution": (C.c_int32, [f32p, C.c_int32, C.c_float, C.c_float, C.c_int32, u32p, f32p]),
            "or_draw": (C.c_uint32, [u32p, f32p, C.c_int32, C.POINTER(C.c_uint64)]),
            "or_set_threads": (None, [C.c_int32]),
            "or_set_fast": (C.c_int32, [C.c_int32, C.c_int32]),
            "or_quantize": (C.c_int32, [C.c_int32, C.c_int32, C.c_int32, f32p, f32p, u8p, f32p]),
            "or_dequantize": (None, [C.c_int32, C.c_int32, C.c_int32, u8p, f32p, f32p]),
            "or_matmul": (C.c_int32, [C.POINTER(OrMatrix), f32p, C.c_int32, f32p, f32p]),
            "or_model_create": (C.c_void_p, [C.POINTER(OrConfig), C.POINTER(OrLayer), u16p, f32p, u16p]),
            "or_model_truncated": (C.c_void_p, [C.c_void_p, C.c_int32]),
            "or_model_destroy": (None, [C.c_void_p]),
            "or_kv_create": (C.c_void_p, [C.c_int32] * 5),
            "or_kv_destroy": (None, [C.c_void_p]),
            "or_kv_read": (C.c_int32, [C.c_void_p, C.c_int32, f32p, f32p]),
            "or_kv_write_layer": (C.c_int32, [C.c_void_p, C.c_int32, f32p, f32p]),
            "or_forward": (C.c_int32, [C.c_void_p, C.c_void_p, C.POINTER(OrChunk), C.c_int32, f32p, f32p]),
            "or_forward_taps": (C.c_int32, [C.c_void_p, C.c_void_p, C.POINTER(OrChunk), C.c_int32, f32p, f32p,
                                            f32p]),
            "or_awq_stats": (None, [f32p, C.c_int32, C.c_int32, f32p, f32p]),
            "or_awq_scales": (None, [f32p, C.c_int32, C.c_float, f32p]),
            "or_awq_search": (C.c_int32, [C.c_int32, C.c_int32, C.c_int32, f32p, C.c_int32, f32p, f32p,
                                          f32p, C.POINTER(C.c_double), u8p, f32p]),
            "or_generate": (C.c_int32, [C.c_void_p, C.c_void_p, u32p, C.c_int32, C.c_int32, C.c_int32,
                                        C.c_int32, C.c_int32, u32p, i32p, i64p]),
            "or_spec_step": (C.c_int32, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, u32p, C.c_int32, i32p,
                                         i32p, u32p, C.c_int32, u32p, C.c_int32, C.c_int32, u32p, i32p]),
            "or_verify": (C.c_int32, [C.c_void_p, C.c_void_p, u32p, C.c_int32, C.c_int32, C.c_uint32, u32p,
                                      C.c_int32, u32p, i32p, f32p]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(l, name)
            fn.restype = res
            fn.argtypes = args
        _lib = l
    return _lib


def ptr(a: np.ndarray | None, t):
    if a is None:
        return C.cast(None, t)
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(t)


def config_struct(cfg) -> OrConfig:
    return OrConfig(cfg.vocab, cfg.hidden, cfg.intermediate, cfg.layers, cfg.heads, cfg.kv_heads, cfg.head_dim,
                    cfg.rms_eps, cfg.rope_theta, int(cfg.rope_llama3), cfg.rope_factor, cfg.rope_low_freq,
                    cfg.rope_high_freq, cfg.rope_orig_max_pos, cfg.max_position, int(cfg.tie_embeddings),
                    int(cfg.qkv_bias))


def matrix_struct(m: Matrix) -> OrMatrix:
    return OrMatrix(m.kind, m.rows, m.cols, 0, ptr(m.bf16, u16p), ptr(m.q, u8p), ptr(m.s, f32p))


def threads(n: int) -> None:
    lib().or_set_threads(n)


def fast(on: bool, threads: int = 0) -> bool:
    """The CPU baseline's fast path (AVX-512 register tiles and a spinning
    pool of `threads` threads, bit-identical to the portable loops) on or
    off; False when this CPU cannot take it."""
    return lib().or_set_fast(int(on), threads) == 0


class Model:
    """An oracle copy of a HostModel (Model::forward on the CPU)."""

    def __init__(self, hm: HostModel, _handle=None, _base=None):
        self.cfg = hm.cfg
        self._base = _base
        if _handle is not None:
            self.h = _handle
            return
        ls = (OrLayer * len(hm.layers))()
        for i, l in enumerate(hm.layers):
            ls[i] = OrLayer(ptr(l.attn_norm, f32p), matrix_struct(l.wqkv), ptr(l.bqkv, f32p), matrix_struct(l.wo),
                            ptr(l.mlp_norm, f32p), matrix_struct(l.w_gate_up), matrix_struct(l.w_down))
        cs = config_struct(hm.cfg)
        self.h = lib().or_model_create(C.byref(cs), ls, ptr(hm.embed, u16p), ptr(hm.norm, f32p),
                                       ptr(hm.lm_head, u16p))
        if not self.h:
            raise ValueError("oracle rejected the model (shape mismatch)")

    def truncated(self, n: int) -> "Model":
        from dataclasses import replace
        h = lib().or_model_truncated(self.h, n)
        m = Model.__new__(Model)
        m.cfg = replace(self.cfg, layers=min(n, self.cfg.layers))
        m.h = h
        m._base = self
        return m

    def __del__(self):
        if getattr(self, "h", None) and lib:
            lib().or_model_destroy(self.h)
            self.h = None

    def kv(self, blocks: int, block_size: int = 16) -> "KvCache":
        return KvCache(self.cfg, blocks, block_size)

    def forward(self, kv: "KvCache", chunks, hidden: bool = False, taps: bool = False):
        """chunks: list of (tokens, pos, blocks, logits_mode) with logits_mode
        0 none, 1 last, 2 all. Returns logits [rows, vocab] (and the hidden
        states [(layers+1), t, hidden] if asked; and, with taps, per layer
        the four projection inputs of Model::record, src/model.rs:312-333:
        a list of [xn (t x hidden), attention (t x heads*hd), xn (t x
        hidden), act (t x intermediate)])."""
        arr = (OrChunk * len(chunks))()
        keep = []
        rows = 0
        t = 0
        for i, (tok, pos, blocks, mode) in enumerate(chunks):
            tok = np.ascontiguousarray(tok, dtype=np.uint32)
            blocks = np.ascontiguousarray(blocks, dtype=np.uint32)
            keep += [tok, blocks]
            arr[i] = OrChunk(ptr(tok, u32p), len(tok), pos, ptr(blocks, u32p), len(blocks), mode)
            rows += len(tok) if mode == 2 else (1 if mode == 1 and len(tok) else 0)
            t += len(tok)
        logits = np.zeros((rows, self.cfg.vocab), dtype=np.float32)
        hid = np.zeros((self.cfg.layers + 1, t, self.cfg.hidden), dtype=np.float32) if hidden else None
        c = self.cfg
        H, qd, inter = c.hidden, c.heads * c.head_dim, c.intermediate
        per = t * (2 * H + qd + inter)
        tp = np.zeros(c.layers * per, dtype=np.float32) if taps else None
        n = lib().or_forward_taps(self.h, kv.h, arr, len(chunks), ptr(logits, f32p), ptr(hid, f32p),
                                  ptr(tp, f32p))
        if n < 0:
            raise ValueError("chunk overruns its cache blocks")
        out = [logits]
        if hidden:
            out.append(hid)
        if taps:
            lay = []
            for li in range(c.layers):
                b = tp[li * per:(li + 1) * per]
                o = [0, t * H, t * (H + qd), t * (2 * H + qd), per]
                lay.append([b[o[0]:o[1]].reshape(t, H), b[o[1]:o[2]].reshape(t, qd),
                            b[o[2]:o[3]].reshape(t, H), b[o[3]:o[4]].reshape(t, inter)])
            out.append(lay)
        return out[0] if len(out) == 1 else tuple(out)


class KvCache:
    def __init__(self, cfg, blocks: int, block_size: int = 16):
        self.cfg = cfg
        self.blocks = blocks
        self.block_size = block_size
        self.h = lib().or_kv_create(cfg.layers, cfg.kv_heads, cfg.head_dim, block_size, blocks)

    def layer(self, i: int):
        n = self.blocks * self.block_size * self.cfg.kv_heads * self.cfg.head_dim
        k = np.zeros(n, np.float32)
        v = np.zeros(n, np.float32)
        lib().or_kv_read(self.h, i, ptr(k, f32p), ptr(v, f32p))
        return k, v

    def set_layer(self, i: int, k: np.ndarray, v: np.ndarray) -> None:
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        lib().or_kv_write_layer(self.h, i, ptr(k, f32p), ptr(v, f32p))

    def __del__(self):
        if getattr(self, "h", None):
            lib().or_kv_destroy(self.h)
            self.h = None


def generate(target: Model, draft: Model | None, prompt, max_tokens: int, k: int, kv_blocks: int = 1024,
             max_batch_tokens: int = 512):
    """Greedy generation through the reference engine's speculative loop.
    Returns (tokens, per-step accepted counts, (proposed, accepted, steps))."""
    prompt = np.ascontiguousarray(prompt, dtype=np.uint32)
    out = np.zeros(max_tokens, np.uint32)
    acc = np.zeros(max_tokens, np.int32)
    st = np.zeros(3, np.int64)
    n = lib().or_generate(target.h, draft.h if draft else None, ptr(prompt, u32p), len(prompt), max_tokens, k,
                          kv_blocks, max_batch_tokens, ptr(out, u32p), ptr(acc, i32p), ptr(st, i64p))
    if n < 0:
        raise RuntimeError("oracle generate failed")
    return out[:n], acc[:int(st[2])], tuple(int(x) for x in st)


def verify(target: Model, kv: KvCache, blocks, pos: int, last: int, drafts):
    """One greedy verify step (returns emitted ids, accepted count, logits)."""
    blocks = np.ascontiguousarray(blocks, dtype=np.uint32)
    drafts = np.ascontiguousarray(drafts, dtype=np.uint32)
    k = len(drafts)
    out = np.zeros(k + 1, np.uint32)
    acc = C.c_int32(0)
    logits = np.zeros((k + 1, target.cfg.vocab), np.float32)
    n = lib().or_verify(target.h, kv.h, ptr(blocks, u32p), len(blocks), pos, last, ptr(drafts, u32p), k,
                        ptr(out, u32p), C.byref(acc), ptr(logits, f32p))
    if n < 0:
        raise RuntimeError("oracle verify failed")
    return out[:n], acc.value, logits


def spec_step(target: Model, tkv: KvCache, draft: Model, dkv: KvCache, tokens, computed: int, draft_computed: int,
              blocks, draft_blocks, k: int):
    """One greedy speculative step from an existing state. Returns
    (emitted ids, accepted, computed, draft_computed)."""
    tokens = np.ascontiguousarray(tokens, dtype=np.uint32)
    blocks = np.ascontiguousarray(blocks, dtype=np.uint32)
    draft_blocks = np.ascontiguousarray(draft_blocks, dtype=np.uint32)
    out = np.zeros(k + 1, np.uint32)
    acc = C.c_int32(0)
    c = C.c_int32(computed)
    dc = C.c_int32(draft_computed)
    n = lib().or_spec_step(target.h, tkv.h, draft.h, dkv.h, ptr(tokens, u32p), len(tokens), C.byref(c), C.byref(dc),
                           ptr(blocks, u32p), len(blocks), ptr(draft_blocks, u32p), len(draft_blocks), k,
                           ptr(out, u32p), C.byref(acc))
    if n < 0:
        raise RuntimeError("oracle spec step failed")
    return out[:n], acc.value, c.value, dc.value


def quantize(kind: int, w: np.ndarray, importance: np.ndarray | None = None) -> Matrix:
    rows, cols = w.shape
    w = np.ascontiguousarray(w, dtype=np.float32)
    bpk = 32 if kind == 1 else 16
    q = np.zeros(rows // 32 * cols * bpk, np.uint8)
    s = np.zeros(rows // 32 * (cols // 32) * 32, np.float32)
    imp = None if importance is None else np.ascontiguousarray(importance, np.float32)
    if lib().or_quantize(kind, rows, cols, ptr(w, f32p), ptr(imp, f32p), ptr(q, u8p), ptr(s, f32p)):
        raise ValueError("bad shape for quantization")
    return Matrix(kind, rows, cols, q=q, s=s)


def matmul(w: Matrix, x: np.ndarray, bias: np.ndarray | None = None) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    m = x.shape[0]
    y = np.zeros((m, w.rows), np.float32)
    ms = matrix_struct(w)
    if lib().or_matmul(C.byref(ms), ptr(x, f32p), m, ptr(bias, f32p), ptr(y, f32p)):
        raise ValueError("bad matrix")
    return y


def exp(x: float) -> float:
    return lib().or_exp(x)


def argmax(v: np.ndarray) -> int:
    v = np.ascontiguousarray(v, np.float32)
    return int(lib().or_argmax(ptr(v, f32p), len(v)))


# ---------------------------------------------------------------------------
# Sampling (src/sampler.rs:52-103) and the engine's sampling branch
# (src/engine.rs:575-610, 658-717).
# ---------------------------------------------------------------------------
class Rng:
    """The reference's Rng (src/rng.rs:5-36): xorshift64* seeded by
    seed * 0x9E3779B97F4A7C15 | 1."""

    def __init__(self, seed: int = 0, state: int | None = None):
        self.s = C.c_uint64(lib().or_rng_new(seed) if state is None else state)

    @property
    def state(self) -> int:
        return self.s.value

    def uniform(self) -> float:
        return lib().or_rng_uniform(C.byref(self.s))


def distribution(logits, temperature: float, top_p: float, top_k: int):
    """sampler::distribution: (tokens, probabilities) in the reference's order."""
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    v = len(logits)
    tok = np.zeros(v, np.uint32)
    pr = np.zeros(v, np.float32)
    n = lib().or_distribution(ptr(logits, f32p), v, temperature, top_p, top_k, ptr(tok, u32p), ptr(pr, f32p))
    return tok[:n].copy(), pr[:n].copy()


def draw(tok, pr, rng: Rng) -> int:
    """sampler::draw over (tok, pr) in the given order."""
    tok = np.ascontiguousarray(tok, dtype=np.uint32)
    pr = np.ascontiguousarray(pr, dtype=np.float32)
    return int(lib().or_draw(ptr(tok, u32p), ptr(pr, f32p), len(tok), C.byref(rng.s)))


def sample(logits, params, rng: Rng) -> int:
    """sampler::sample: params = (temperature, top_p, top_k); greedy when
    temperature <= 0 (no draw from the generator)."""
    t, top_p, top_k = params
    if t <= 0.0:
        return int(lib().or_argmax(ptr(np.ascontiguousarray(logits, np.float32), f32p), len(logits)))
    return draw(*distribution(logits, t, top_p, top_k), rng)


def _dense(tok, pr, vocab: int):
    d = np.zeros(vocab, np.float32)
    d[tok] = pr
    return d


def spec_step_sampled(target: Model, tkv: KvCache, draft: Model, dkv: KvCache, tokens, computed: int,
                      draft_computed: int, blocks, draft_blocks, k: int, params, rng: Rng):
    """One speculative step of Engine::propose + Engine::execute for one
    sequence under `params` = (temperature, top_p, top_k), drawing from
    `rng` in the reference's order: the k draft draws, then one uniform per
    verified proposal whose draft probability is positive, then the
    residual draw (src/engine.rs:575-594) or the bonus draw. Returns
    (emitted ids, accepted, computed, draft_computed)."""
    greedy = params[0] <= 0.0
    vocab = target.cfg.vocab
    tokens = [int(x) for x in tokens]
    base = len(tokens)
    drafts, qd = [], []
    for r in range(k):
        if r == 0:
            tok, pos = tokens[draft_computed:], draft_computed
        else:
            tok, pos = [drafts[-1]], base + r - 1
        lg = draft.forward(dkv, [(tok, pos, draft_blocks, 1)])[0]
        if greedy:
            t = int(lib().or_argmax(ptr(lg, f32p), vocab))
        else:
            tk, pr = distribution(lg, *params)
            t = draw(tk, pr, rng)
            qd.append(_dense(tk, pr, vocab))
        drafts.append(t)
    draft_computed = base + k - 1
    rows = target.forward(tkv, [([tokens[computed]] + drafts, computed, blocks, 2)])
    new, accepted = [], 0
    for j, d in enumerate(drafts):
        lg = rows[j]
        if greedy:
            t = int(lib().or_argmax(ptr(lg, f32p), vocab))
            take = None if t == d else t
        else:
            pd = _dense(*distribution(lg, *params), vocab)
            q = qd[j]
            px, qx = pd[d], q[d]
            if qx > 0 and rng.uniform() < float(min(np.float32(px / qx), np.float32(1.0))):
                take = None
            else:
                mask = pd > q
                if mask.any():
                    rt = np.nonzero(mask)[0]
                    take = draw(rt, (pd - q)[mask], rng)
                else:
                    rt = np.nonzero(pd > 0)[0]
                    take = draw(rt, pd[rt], rng)
        if take is None:
            new.append(d)
            accepted += 1
        else:
            new.append(int(take))
            break
    if accepted == k:
        new.append(sample(rows[k], params, rng))
    return new, accepted, base + accepted, min(draft_computed, base + accepted)


def generate_sampled(target: Model, draft: Model | None, prompt, max_tokens: int, k: int, params, seed: int,
                     kv_blocks: int = 256, max_batch_tokens: int = 512):
    """One request through the engine loop with sampling parameters
    (src/engine.rs:374-654, ignore_eos): chunked prefill, the first token
    sampled from the prompt's last row, then speculative steps. Returns
    (tokens, (proposed, accepted, steps))."""
    rng = Rng(seed)
    if draft is None:
        k = 0
    bs = 16
    max_len = min(target.cfg.max_position, kv_blocks * bs)
    tokens = [int(x) for x in prompt]
    if not tokens or len(tokens) >= max_len:
        raise ValueError("prompt does not fit")
    tkv = target.kv(kv_blocks)
    dkv = draft.kv(kv_blocks) if draft else None
    table = list(range(kv_blocks))
    computed = draft_computed = 0
    out = []
    proposed = acc_total = steps = 0
    while len(out) < max_tokens and len(tokens) < max_len:
        left = len(tokens) - computed
        spec = left == 1 and k > 0 and len(tokens) + k < max_len and max_batch_tokens > k
        if spec:
            emit, a, computed, draft_computed = spec_step_sampled(target, tkv, draft, dkv, tokens, computed,
                                                                  draft_computed, table, table, k, params, rng)
            proposed += k
            acc_total += a
            steps += 1
        else:
            n = min(left, max_batch_tokens)
            last = computed + n == len(tokens)
            lg = target.forward(tkv, [(tokens[computed:computed + n], computed, table, 1 if last else 0)])
            computed += n
            emit = [sample(lg[0], params, rng)] if last else []
        for t in emit:
            tokens.append(t)
            out.append(t)
            if len(out) >= max_tokens or len(tokens) >= max_len:
                break
    return np.array(out, np.uint32), (proposed, acc_total, steps)


# ---------------------------------------------------------------------------
# Calibration capture and AWQ (src/model.rs:56-70, 364-392; src/awq.rs)
# ---------------------------------------------------------------------------

def calibrate(m: Model, seqs, max_rows: int):
    """Model::calibrate (src/awq.rs:38-62): each sequence's forward from
    position 0 in a fresh cache, keeping up to max_rows input rows per
    projection by Model::record's reservoir sampling (src/model.rs:364-392:
    one xorshift generator shared by every layer and projection, advanced
    for each row past the first max_rows). Returns per layer the four lists
    [qkv, o, gate_up, down] of rows, as float32 arrays [rows, width]."""
    rng = 0x9E3779B97F4A7C15
    mask = (1 << 64) - 1
    layers = [[[] for _ in range(4)] for _ in range(m.cfg.layers)]
    seen = [[0] * 4 for _ in range(m.cfg.layers)]
    for s in seqs:
        s = [int(v) for v in s]
        nb = (len(s) + 15) // 16
        kv = m.kv(nb)
        _, taps = m.forward(kv, [(s, 0, list(range(nb)), 0)], taps=True)
        for li in range(m.cfg.layers):
            for which in range(4):
                for r in taps[li][which]:
                    n = seen[li][which]
                    seen[li][which] += 1
                    if n < max_rows:
                        layers[li][which].append(r.copy())
                    else:
                        rng ^= (rng << 13) & mask
                        rng ^= rng >> 7
                        rng ^= (rng << 17) & mask
                        j = rng % (n + 1)
                        if j < max_rows:
                            layers[li][which][j] = r.copy()
    return [[np.stack(rows).astype(np.float32) if rows else np.zeros((0, 0), np.float32) for rows in l]
            for l in layers]


def awq_stats(cal: np.ndarray):
    """stats (src/awq.rs:128-142): mean |x| and mean x^2 per channel."""
    cal = np.ascontiguousarray(cal, np.float32)
    m, k = cal.shape
    a = np.zeros(k, np.float32)
    q = np.zeros(k, np.float32)
    lib().or_awq_stats(ptr(cal, f32p), m, k, ptr(a, f32p), ptr(q, f32p))
    return a, q


def awq_scales(abs_mean: np.ndarray, alpha: float) -> np.ndarray:
    """scales (src/awq.rs:144-150) for one alpha."""
    abs_mean = np.ascontiguousarray(abs_mean, np.float32)
    s = np.zeros(abs_mean.size, np.float32)
    lib().or_awq_scales(ptr(abs_mean, f32p), abs_mean.size, alpha, ptr(s, f32p))
    return s


def awq_search(kind: int, w: np.ndarray, cal: np.ndarray):
    """search + apply (src/awq.rs:152-217): returns (scales, alpha,
    error_plain, error_awq, Matrix) for weights w (rows x k, f32) and
    calibration rows cal (m x k)."""
    w = np.ascontiguousarray(w, np.float32)
    cal = np.ascontiguousarray(cal, np.float32)
    rows, k = w.shape
    m = cal.shape[0]
    assert cal.shape[1] == k
    bpk = 32 if kind == INT8 else 16
    q = np.zeros(rows // 32 * k * bpk, np.uint8)
    s = np.zeros(rows // 32 * (k // 32) * 32, np.float32)
    sc = np.zeros(k, np.float32)
    alpha = C.c_float()
    errs = (C.c_double * 2)()
    if lib().or_awq_search(kind, rows, k, ptr(w, f32p), m, ptr(cal, f32p), ptr(sc, f32p), C.byref(alpha), errs,
                           ptr(q, u8p), ptr(s, f32p)):
        raise ValueError("awq_search: bad shape")
    return sc, float(alpha.value), float(errs[0]), float(errs[1]), Matrix(kind, rows, k, q=q, s=s)
