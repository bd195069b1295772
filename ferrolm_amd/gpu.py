"""ctypes binding of libferro_gpu.so (the C ABI in include/ferro_gpu.h).

This is the product path: every call runs the HIP kernels for gfx950. There
is no CPU fallback — if the library is missing or no GPU is present, the
calls raise.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass
from pathlib import Path

import numpy as np

from .weights import BF16, INT8, Config, HostModel, Matrix

PKG = Path(__file__).resolve().parent
# FERRO_STAMPS=1 loads the library built with the in-kernel timeline (python -m
# ferrolm_amd.build --stamps): the same kernels, each recording its entry and exit
LIB_PATH = PKG / ("libferro_gpu_stamps.so" if os.environ.get("FERRO_STAMPS") == "1" else "libferro_gpu.so")

f32p = C.POINTER(C.c_float)
u16p = C.POINTER(C.c_uint16)
u8p = C.POINTER(C.c_uint8)
u32p = C.POINTER(C.c_uint32)
i32p = C.POINTER(C.c_int32)

LOGITS_NONE, LOGITS_LAST, LOGITS_ALL = 0, 1, 2


class FgConfig(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("vocab", "hidden", "intermediate", "layers", "heads", "kv_heads",
                                          "head_dim")] + [
        ("rms_eps", C.c_float), ("rope_theta", C.c_float), ("rope_llama3", C.c_int32),
        ("rope_factor", C.c_float), ("rope_low_freq", C.c_float), ("rope_high_freq", C.c_float),
        ("rope_orig_max_pos", C.c_int32), ("max_position", C.c_int32), ("tie_embeddings", C.c_int32),
        ("qkv_bias", C.c_int32)]


class FgMatrix(C.Structure):
    _fields_ = [("format", C.c_int32), ("rows", C.c_int32), ("cols", C.c_int32), ("_pad", C.c_int32),
                ("bf16", u16p), ("q", u8p), ("s", f32p)]


class FgLayer(C.Structure):
    _fields_ = [("attn_norm", f32p), ("wqkv", FgMatrix), ("bqkv", f32p), ("wo", FgMatrix),
                ("mlp_norm", f32p), ("w_gate_up", FgMatrix), ("w_down", FgMatrix)]


class FgChunk(C.Structure):
    _fields_ = [("tokens", u32p), ("n", C.c_int32), ("pos", C.c_int32), ("blocks", u32p),
                ("n_blocks", C.c_int32), ("logits", C.c_int32)]


class FgSpecSeq(C.Structure):
    _fields_ = [("tail", u32p), ("n_tail", C.c_int32), ("draft_pos", C.c_int32), ("pos", C.c_int32),
                ("blocks", u32p), ("n_blocks", C.c_int32), ("draft_blocks", u32p), ("n_draft_blocks", C.c_int32)]


class FgSampling(C.Structure):
    _fields_ = [("temperature", C.c_float), ("top_p", C.c_float), ("top_k", C.c_int32), ("reserved", C.c_int32)]


u64p = C.POINTER(C.c_uint64)


class FgAwqChoice(C.Structure):
    _fields_ = [("alpha", C.c_float), ("_pad", C.c_int32), ("error_plain", C.c_double),
                ("error_awq", C.c_double)]


@dataclass
class SamplingParams:
    """The sampling fields of the reference's SamplingParams
    (src/sampler.rs:8-19): temperature <= 0 is greedy; top_k 0 is no limit.
    `seed` seeds the request's Rng (src/engine.rs:292-299)."""
    temperature: float = 0.0
    top_p: float = 1.0
    top_k: int = 0
    seed: int = 0

    @property
    def greedy(self) -> bool:
        return self.temperature <= 0.0

    def struct(self) -> FgSampling:
        return FgSampling(self.temperature, self.top_p, self.top_k, 0)


def rng_init(seed: int) -> int:
    """Rng::new (src/rng.rs:8-10): the generator state of a seed."""
    return ((seed * 0x9E3779B97F4A7C15) & 0xFFFFFFFFFFFFFFFF) | 1


EXPORTS = {
    "fg_ctx_create": (C.c_int, [C.c_int, C.POINTER(C.c_void_p)]),
    "fg_ctx_destroy": (None, [C.c_void_p]),
    "fg_last_error": (C.c_char_p, []),
    "fg_ctx_sync": (C.c_int, [C.c_void_p]),
    "fg_config_check": (C.c_int, [C.POINTER(FgConfig)]),
    "fg_model_upload": (C.c_int, [C.c_void_p, C.POINTER(FgConfig), C.POINTER(FgLayer), u16p, f32p, u16p,
                                  C.POINTER(C.c_void_p)]),
    "fg_model_truncated": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int32, C.POINTER(C.c_void_p)]),
    "fg_model_destroy": (None, [C.c_void_p]),
    "fg_model_weight_bytes": (C.c_int64, [C.c_void_p]),
    "fg_kv_create": (C.c_int, [C.c_void_p, C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_int32,
                               C.POINTER(C.c_void_p)]),
    "fg_kv_destroy": (None, [C.c_void_p]),
    "fg_kv_read": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int32, f32p, f32p]),
    "fg_kv_write": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int32, f32p, f32p]),
    "fg_forward": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.POINTER(FgChunk), C.c_int32, f32p, u32p, i32p,
                             f32p]),
    "fg_forward_capture": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.POINTER(FgChunk), C.c_int32, f32p]),
    "fg_spec_step": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.POINTER(FgSpecSeq),
                               C.c_int32, C.c_int32, u32p, i32p, i32p]),
    "fg_spec_step_mixed": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                     C.POINTER(FgSpecSeq), C.c_int32, C.c_int32, C.POINTER(FgChunk), C.c_int32,
                                     u32p, i32p, i32p, u32p]),
    "fg_spec_step_sampled": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                       C.POINTER(FgSpecSeq), C.c_int32, C.c_int32, C.POINTER(FgSampling), u64p,
                                       u32p, i32p, i32p]),
    "fg_forward_sampled": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.POINTER(FgChunk), C.c_int32,
                                     C.POINTER(FgSampling), u64p, u32p, i32p]),
    "fg_last_step_times": (C.c_int, [C.c_void_p, f32p]),
    "fg_profile": (C.c_int, [C.c_void_p, C.c_int32]),
    "fg_stamps_reset": (C.c_int, [C.c_void_p]),
    "fg_stamps_read": (C.c_int, [C.c_void_p, C.c_int32, C.c_void_p, C.c_char_p, C.c_int32]),
    "fg_profile_read": (C.c_int, [C.c_void_p, C.c_int32, i32p, C.POINTER(C.c_int64), C.POINTER(C.c_double),
                                  C.POINTER(C.c_double), C.POINTER(C.c_double), C.c_int32]),
    "fg_mat_upload": (C.c_int, [C.c_void_p, C.POINTER(FgMatrix), C.POINTER(C.c_void_p)]),
    "fg_mat_destroy": (None, [C.c_void_p]),
    "fg_matmul": (C.c_int, [C.c_void_p, C.c_void_p, f32p, C.c_int32, f32p, f32p]),
    "fg_matmul_device": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int32, C.c_void_p]),
    "fg_matmul_device_noalloc": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int32, C.c_void_p]),
    "fg_quantize": (C.c_int, [C.c_void_p, C.c_int32, C.c_int32, C.c_int32, f32p, f32p, u8p, f32p]),
    "fg_awq_search": (C.c_int, [C.c_void_p, C.c_int32, C.c_int32, C.c_int32, f32p, C.c_int32, f32p, f32p,
                                C.POINTER(FgAwqChoice), u8p, f32p]),
}

_lib = None


def lib():
    """Loads libferro_gpu.so (built by ferrolm_amd.build); raises if absent."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is not built: run `python -m ferrolm_amd.build`")
        l = C.CDLL(str(LIB_PATH))
        for name, (res, args) in EXPORTS.items():
            fn = getattr(l, name)
            fn.restype = res
            fn.argtypes = args
        _lib = l
    return _lib


class FgError(RuntimeError):
    pass


def check(rc: int) -> None:
    if rc != 0:
        raise FgError(f"ferro_gpu error {rc}: {lib().fg_last_error().decode()}")


def ptr(a, t):
    if a is None:
        return C.cast(None, t)
    assert a.flags["C_CONTIGUOUS"], "arrays passed to the library must be contiguous"
    return a.ctypes.data_as(t)


def config_struct(c: Config) -> FgConfig:
    return FgConfig(c.vocab, c.hidden, c.intermediate, c.layers, c.heads, c.kv_heads, c.head_dim, c.rms_eps,
                    c.rope_theta, int(c.rope_llama3), c.rope_factor, c.rope_low_freq, c.rope_high_freq,
                    c.rope_orig_max_pos, c.max_position, int(c.tie_embeddings), int(c.qkv_bias))


def check_config(c: Config) -> None:
    """fg_config_check: the reference's config shape checks plus the device's
    limits (host only, no GPU needed). Raises FgError on a refused shape."""
    cs = config_struct(c)
    check(lib().fg_config_check(C.byref(cs)))


def _need(a, dtype, n: int, what: str) -> None:
    if a is None or a.dtype != dtype or a.size != n or not a.flags["C_CONTIGUOUS"]:
        got = "None" if a is None else f"{a.dtype} x {a.size}"
        raise ValueError(f"{what}: expected {n} contiguous {np.dtype(dtype)} values, got {got}")


def check_matrix(m: Matrix, what: str) -> None:
    """The host arrays of a weight matrix match its shape and format, so the
    upload never reads past them: bf16 rows x cols uint16; quantized codes
    rows x cols (int8) or rows x cols / 2 (int4) bytes and (rows / 32) x
    (cols / 32) x 32 f32 scales (QMatrix, src/quant.rs:64-76)."""
    if m.rows <= 0 or m.cols <= 0:
        raise ValueError(f"{what}: empty matrix")
    if m.kind == BF16:
        _need(m.bf16, np.uint16, m.rows * m.cols, f"{what} bf16")
        return
    if m.rows % 32 or m.cols % 32:
        raise ValueError(f"{what}: quantized matrices need rows and cols that are multiples of 32")
    _need(m.q, np.uint8, m.rows * m.cols // (1 if m.kind == INT8 else 2), f"{what} codes")
    _need(m.s, np.float32, m.rows * m.cols // 32, f"{what} scales")


def matrix_struct(m: Matrix) -> FgMatrix:
    return FgMatrix(m.kind, m.rows, m.cols, 0, ptr(m.bf16, u16p), ptr(m.q, u8p), ptr(m.s, f32p))


class Context:
    """A device context: one HIP stream and its workspace (fg_ctx)."""

    def __init__(self, device: int = 0):
        h = C.c_void_p()
        check(lib().fg_ctx_create(device, C.byref(h)))
        self.h = h

    def sync(self) -> None:
        check(lib().fg_ctx_sync(self.h))

    def close(self) -> None:
        if getattr(self, "h", None):
            lib().fg_ctx_destroy(self.h)
            self.h = None

    def __del__(self):
        if lib is not None:  # at interpreter exit the module's globals are already cleared
            self.close()


class Model:
    """Device copy of a HostModel (fg_model_upload)."""

    def __init__(self, ctx: Context, hm: HostModel | None, _handle=None, _base=None, cfg: Config | None = None):
        self.ctx = ctx
        self._base = _base
        if _handle is not None:
            self.h = _handle
            self.cfg = cfg
            return
        self.cfg = hm.cfg
        c = hm.cfg
        check_config(c)
        if len(hm.layers) != c.layers:
            raise ValueError(f"{len(hm.layers)} layers given for a config of {c.layers}")
        _need(hm.embed, np.uint16, c.vocab * c.hidden, "embed")
        _need(hm.norm, np.float32, c.hidden, "norm")
        if hm.lm_head is not None and not c.tie_embeddings:
            _need(hm.lm_head, np.uint16, c.vocab * c.hidden, "lm_head")
        for i, l in enumerate(hm.layers):
            _need(l.attn_norm, np.float32, c.hidden, f"layer {i} attn_norm")
            _need(l.mlp_norm, np.float32, c.hidden, f"layer {i} mlp_norm")
            if c.qkv_bias:
                _need(l.bqkv, np.float32, c.qkv_dim, f"layer {i} bqkv")
            for name, m, rows, cols in (("wqkv", l.wqkv, c.qkv_dim, c.hidden), ("wo", l.wo, c.hidden, c.q_dim),
                                        ("w_gate_up", l.w_gate_up, 2 * c.intermediate, c.hidden),
                                        ("w_down", l.w_down, c.hidden, c.intermediate)):
                if (m.rows, m.cols) != (rows, cols):
                    raise ValueError(f"layer {i} {name}: {m.rows} x {m.cols}, the config needs {rows} x {cols}")
                check_matrix(m, f"layer {i} {name}")
        ls = (FgLayer * max(1, len(hm.layers)))()
        for i, l in enumerate(hm.layers):
            ls[i] = FgLayer(ptr(l.attn_norm, f32p), matrix_struct(l.wqkv), ptr(l.bqkv, f32p), matrix_struct(l.wo),
                            ptr(l.mlp_norm, f32p), matrix_struct(l.w_gate_up), matrix_struct(l.w_down))
        cs = config_struct(hm.cfg)
        h = C.c_void_p()
        check(lib().fg_model_upload(ctx.h, C.byref(cs), ls, ptr(hm.embed, u16p), ptr(hm.norm, f32p),
                                    ptr(hm.lm_head, u16p), C.byref(h)))
        self.h = h

    def truncated(self, n: int) -> "Model":
        from dataclasses import replace
        h = C.c_void_p()
        check(lib().fg_model_truncated(self.ctx.h, self.h, n, C.byref(h)))
        return Model(self.ctx, None, _handle=h, _base=self, cfg=replace(self.cfg, layers=min(n, self.cfg.layers)))

    def weight_bytes(self) -> int:
        return int(lib().fg_model_weight_bytes(self.h))

    def close(self) -> None:
        if getattr(self, "h", None):
            lib().fg_model_destroy(self.h)
            self.h = None

    def __del__(self):
        if lib is not None:  # at interpreter exit the module's globals are already cleared
            self.close()


class KvCache:
    """Paged f32 KV cache on the device (fg_kv_create), reference layout."""

    def __init__(self, ctx: Context, cfg: Config, blocks: int, block_size: int = 16):
        self.ctx = ctx
        self.cfg = cfg
        self.blocks = blocks
        self.block_size = block_size
        h = C.c_void_p()
        check(lib().fg_kv_create(ctx.h, cfg.layers, cfg.kv_heads, cfg.head_dim, block_size, blocks, C.byref(h)))
        self.h = h

    def _n(self) -> int:
        return self.blocks * self.block_size * self.cfg.kv_heads * self.cfg.head_dim

    def layer(self, i: int):
        k = np.zeros(self._n(), np.float32)
        v = np.zeros(self._n(), np.float32)
        check(lib().fg_kv_read(self.ctx.h, self.h, i, ptr(k, f32p), ptr(v, f32p)))
        return k, v

    def set_layer(self, i: int, k: np.ndarray, v: np.ndarray) -> None:
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        check(lib().fg_kv_write(self.ctx.h, self.h, i, ptr(k, f32p), ptr(v, f32p)))

    def close(self) -> None:
        if getattr(self, "h", None):
            lib().fg_kv_destroy(self.h)
            self.h = None

    def __del__(self):
        if lib is not None:  # at interpreter exit the module's globals are already cleared
            self.close()


@dataclass
class ForwardOut:
    logits: np.ndarray | None
    argmax: np.ndarray
    hidden: np.ndarray | None


def forward(ctx: Context, model: Model, kv: KvCache, chunks, logits: bool = True, hidden: bool = False) -> ForwardOut:
    """Model::forward on the device. chunks: (tokens, pos, blocks, mode)."""
    arr = (FgChunk * max(1, len(chunks)))()
    keep = []
    rows = 0
    t = 0
    for i, (tok, pos, blocks, mode) in enumerate(chunks):
        tok = np.ascontiguousarray(tok, dtype=np.uint32)
        blocks = np.ascontiguousarray(blocks, dtype=np.uint32)
        keep += [tok, blocks]
        arr[i] = FgChunk(ptr(tok, u32p), len(tok), pos, ptr(blocks, u32p), len(blocks), mode)
        rows += len(tok) if mode == LOGITS_ALL else (1 if mode == LOGITS_LAST and len(tok) else 0)
        t += len(tok)
    lg = np.zeros((rows, model.cfg.vocab), np.float32) if logits else None
    am = np.zeros(rows, np.uint32)
    hid = np.zeros((model.cfg.layers + 1, t, model.cfg.hidden), np.float32) if hidden else None
    nrows = C.c_int32(0)
    check(lib().fg_forward(ctx.h, model.h, kv.h, arr, len(chunks), ptr(lg, f32p), ptr(am, u32p), C.byref(nrows),
                           ptr(hid, f32p)))
    assert nrows.value == rows
    return ForwardOut(lg, am, hid)


def forward_capture(ctx: Context, model: Model, kv: KvCache, chunks) -> list:
    """Model::forward with Model::record's taps (src/model.rs:312-333) on the
    device (fg_forward_capture). chunks: (tokens, pos, blocks). Returns per
    layer the four projection inputs [qkv, o, gate_up, down] of every token
    in chunk order, as float32 arrays [tokens, width]."""
    c = model.cfg
    arr = (FgChunk * max(1, len(chunks)))()
    keep = []
    t = 0
    for i, (tok, pos, blocks) in enumerate(chunks):
        tok = np.ascontiguousarray(tok, dtype=np.uint32)
        blocks = np.ascontiguousarray(blocks, dtype=np.uint32)
        keep += [tok, blocks]
        arr[i] = FgChunk(ptr(tok, u32p), len(tok), pos, ptr(blocks, u32p), len(blocks), LOGITS_NONE)
        t += len(tok)
    widths = (c.hidden, c.heads * c.head_dim, c.hidden, c.intermediate)
    out = np.zeros((c.layers, t * sum(widths)), np.float32)
    if t and c.layers:
        check(lib().fg_forward_capture(ctx.h, model.h, kv.h, arr, len(chunks), ptr(out, f32p)))
    layers = []
    for li in range(c.layers):
        o, four = 0, []
        for w in widths:
            four.append(out[li, o:o + t * w].reshape(t, w))
            o += t * w
        layers.append(four)
    return layers


@dataclass
class SpecSeq:
    tail: np.ndarray
    draft_pos: int
    pos: int
    blocks: np.ndarray
    draft_blocks: np.ndarray


def _sampling_arrays(params: list):
    arr = (FgSampling * len(params))()
    for i, p in enumerate(params):
        arr[i] = p.struct()
    return arr


def forward_sampled(ctx: Context, model: Model, kv: KvCache, chunks, params: list, rng: np.ndarray) -> np.ndarray:
    """Model::forward with each selected row sampled on the device
    (fg_forward_sampled): params[r] for selected row r, rng (uint64, one
    state per selected row) advanced in place. Returns the tokens."""
    arr = (FgChunk * max(1, len(chunks)))()
    keep = []
    rows = 0
    for i, (tok, pos, blocks, mode) in enumerate(chunks):
        tok = np.ascontiguousarray(tok, dtype=np.uint32)
        blocks = np.ascontiguousarray(blocks, dtype=np.uint32)
        keep += [tok, blocks]
        arr[i] = FgChunk(ptr(tok, u32p), len(tok), pos, ptr(blocks, u32p), len(blocks), mode)
        rows += len(tok) if mode == LOGITS_ALL else (1 if mode == LOGITS_LAST and len(tok) else 0)
    if len(params) != rows or rng.dtype != np.uint64 or len(rng) != rows or not rng.flags.c_contiguous:
        raise ValueError("one parameter set and one uint64 generator state per selected row")
    out = np.zeros(rows, np.uint32)
    nrows = C.c_int32(0)
    check(lib().fg_forward_sampled(ctx.h, model.h, kv.h, arr, len(chunks), _sampling_arrays(params),
                                   rng.ctypes.data_as(u64p), ptr(out, u32p), C.byref(nrows)))
    assert nrows.value == rows
    return out


def spec_step(ctx: Context, target: Model, tkv: KvCache, draft: Model, dkv: KvCache, seqs: list, k: int,
              params: list | None = None, rng: np.ndarray | None = None):
    """One speculative step on device (fg_spec_step, or fg_spec_step_sampled
    with per-sequence params and uint64 generator states, advanced in place).
    Returns (tokens per sequence, accepted counts)."""
    n = len(seqs)
    arr = (FgSpecSeq * n)()
    keep = []
    for i, s in enumerate(seqs):
        tail = np.ascontiguousarray(s.tail, np.uint32)
        bl = np.ascontiguousarray(s.blocks, np.uint32)
        db = np.ascontiguousarray(s.draft_blocks, np.uint32)
        keep += [tail, bl, db]
        arr[i] = FgSpecSeq(ptr(tail, u32p), len(tail), s.draft_pos, s.pos, ptr(bl, u32p), len(bl), ptr(db, u32p),
                           len(db))
    out = np.zeros((n, k + 1), np.uint32)
    cnt = np.zeros(n, np.int32)
    acc = np.zeros(n, np.int32)
    if params is None:
        check(lib().fg_spec_step(ctx.h, target.h, tkv.h, draft.h, dkv.h, arr, n, k, ptr(out, u32p), ptr(cnt, i32p),
                                 ptr(acc, i32p)))
    else:
        if len(params) != n or rng is None or rng.dtype != np.uint64 or len(rng) != n or not rng.flags.c_contiguous:
            raise ValueError("one parameter set and one uint64 generator state per sequence")
        check(lib().fg_spec_step_sampled(ctx.h, target.h, tkv.h, draft.h, dkv.h, arr, n, k, _sampling_arrays(params),
                                         rng.ctypes.data_as(u64p), ptr(out, u32p), ptr(cnt, i32p), ptr(acc, i32p)))
    return [out[i, :cnt[i]].copy() for i in range(n)], acc


def spec_step_mixed(ctx: Context, target: Model, tkv: KvCache, draft: Model, dkv: KvCache, seqs: list, k: int,
                    chunks: list):
    """A greedy speculative step whose verify pass also carries other
    sequences' chunks (fg_spec_step_mixed): chunks are (tokens, pos, blocks,
    mode) with mode LOGITS_NONE or LOGITS_LAST. Returns (tokens per sequence,
    accepted counts, the argmax of each LOGITS_LAST chunk in order)."""
    n = len(seqs)
    arr = (FgSpecSeq * n)()
    keep = []
    for i, s in enumerate(seqs):
        tail = np.ascontiguousarray(s.tail, np.uint32)
        bl = np.ascontiguousarray(s.blocks, np.uint32)
        db = np.ascontiguousarray(s.draft_blocks, np.uint32)
        keep += [tail, bl, db]
        arr[i] = FgSpecSeq(ptr(tail, u32p), len(tail), s.draft_pos, s.pos, ptr(bl, u32p), len(bl), ptr(db, u32p),
                           len(db))
    carr = (FgChunk * max(1, len(chunks)))()
    last = 0
    for i, (tok, pos, blocks, mode) in enumerate(chunks):
        tok = np.ascontiguousarray(tok, dtype=np.uint32)
        blocks = np.ascontiguousarray(blocks, dtype=np.uint32)
        keep += [tok, blocks]
        carr[i] = FgChunk(ptr(tok, u32p), len(tok), pos, ptr(blocks, u32p), len(blocks), mode)
        last += 1 if mode == LOGITS_LAST and len(tok) else 0
    out = np.zeros((n, k + 1), np.uint32)
    cnt = np.zeros(n, np.int32)
    acc = np.zeros(n, np.int32)
    am = np.zeros(max(1, last), np.uint32)
    check(lib().fg_spec_step_mixed(ctx.h, target.h, tkv.h, draft.h, dkv.h, arr, n, k, carr, len(chunks),
                                   ptr(out, u32p), ptr(cnt, i32p), ptr(acc, i32p), ptr(am, u32p)))
    return [out[i, :cnt[i]].copy() for i in range(n)], acc, am[:last]


def last_step_times(ctx: Context) -> np.ndarray:
    t = np.zeros(3, np.float32)
    check(lib().fg_last_step_times(ctx.h, ptr(t, f32p)))
    return t


KIND_LABEL = {0: "bf16", 1: "int8", 2: "int4"}


def stamps_reset(ctx: Context) -> None:
    """Clears the in-kernel timeline (fg_stamps_reset; a library built with stamps)."""
    check(lib().fg_stamps_reset(ctx.h))


def stamps_read(ctx: Context, slots: int = 1024):
    """(ticks [slots][1024 workgroups][entry, exit] uint64 at 100 MHz, 0 = no record;
    labels of the labelled slots) (fg_stamps_read)."""
    ticks = np.zeros((slots, 1024, 2), np.uint64)
    buf = C.create_string_buffer(1 << 16)
    n = lib().fg_stamps_read(ctx.h, slots, ticks.ctypes.data_as(C.c_void_p), buf, len(buf))
    if n < 0:
        check(n)
    return ticks, buf.value.decode().split("\n")[:n]


def profile(ctx: Context, on: bool) -> None:
    """Brackets every GEMV launch with HIP events while on (fg_profile)."""
    check(lib().fg_profile(ctx.h, int(on)))


def profile_read(ctx: Context, reset: bool = True) -> list:
    """Per kernel class: dict(kind, passes, gemm, launches, us, bytes, flops); gemm is True for
    the GEMM path (more than 16 rows), whose passes is reported as 0."""
    cap = 12
    cls = np.zeros(cap, np.int32)
    n = np.zeros(cap, np.int64)
    us = np.zeros(cap, np.float64)
    by = np.zeros(cap, np.float64)
    fl = np.zeros(cap, np.float64)
    dp = C.POINTER(C.c_double)
    r = lib().fg_profile_read(ctx.h, cap, ptr(cls, i32p), n.ctypes.data_as(C.POINTER(C.c_int64)),
                              us.ctypes.data_as(dp), by.ctypes.data_as(dp), fl.ctypes.data_as(dp), int(reset))
    if r < 0:
        check(r)
    return [dict(kind=KIND_LABEL[int(cls[i]) // 4], passes=(1, 2, 4, 0)[int(cls[i]) % 4],
                 gemm=int(cls[i]) % 4 == 3, launches=int(n[i]),
                 us=float(us[i]), bytes=float(by[i]), flops=float(fl[i])) for i in range(min(r, cap))]


class Mat:
    """A single device matrix (kernels::matmul's operand)."""

    def __init__(self, ctx: Context, m: Matrix):
        self.ctx = ctx
        self.rows, self.cols, self.kind = m.rows, m.cols, m.kind
        check_matrix(m, "matrix")
        ms = matrix_struct(m)
        h = C.c_void_p()
        check(lib().fg_mat_upload(ctx.h, C.byref(ms), C.byref(h)))
        self.h = h

    def matmul(self, x: np.ndarray, bias: np.ndarray | None = None) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        y = np.zeros((x.shape[0], self.rows), np.float32)
        b = None if bias is None else np.ascontiguousarray(bias, np.float32)
        check(lib().fg_matmul(self.ctx.h, self.h, ptr(x, f32p), x.shape[0], ptr(b, f32p), ptr(y, f32p)))
        return y

    def close(self) -> None:
        if getattr(self, "h", None):
            lib().fg_mat_destroy(self.h)
            self.h = None

    def __del__(self):
        if lib is not None:  # at interpreter exit the module's globals are already cleared
            self.close()


def _qmatrix_buffers(kind: int, rows: int, cols: int):
    q = np.zeros(rows * cols // (1 if kind == INT8 else 2), np.uint8)
    s = np.zeros(rows * cols // 32, np.float32)
    return q, s


def quantize(ctx: Context, kind: int, w: np.ndarray, importance: np.ndarray | None = None) -> Matrix:
    """QMatrix::quantize (src/quant.rs:78-143) on the device (fg_quantize):
    the reference's codes and scales for a rows x cols f32 matrix."""
    w = np.ascontiguousarray(w, np.float32)
    rows, cols = w.shape
    q, s = _qmatrix_buffers(kind, rows, cols)
    imp = None if importance is None else np.ascontiguousarray(importance, np.float32)
    check(lib().fg_quantize(ctx.h, kind, rows, cols, ptr(w, f32p), ptr(imp, f32p), ptr(q, u8p), ptr(s, f32p)))
    return Matrix(kind, rows, cols, q=q, s=s)


def awq_search(ctx: Context, kind: int, w: np.ndarray, cal: np.ndarray):
    """awq::search + apply (src/awq.rs:152-217) on the device
    (fg_awq_search): returns (scales, alpha, error_plain, error_awq, Matrix)
    for weights w (rows x k) and calibration rows cal (m x k)."""
    w = np.ascontiguousarray(w, np.float32)
    cal = np.ascontiguousarray(cal, np.float32)
    rows, k = w.shape
    if cal.ndim != 2 or cal.shape[1] != k:
        raise FgError("calibration rows must have the projection's input width")
    q, s = _qmatrix_buffers(kind, rows, k)
    sc = np.zeros(k, np.float32)
    ch = FgAwqChoice()
    check(lib().fg_awq_search(ctx.h, kind, rows, k, ptr(w, f32p), cal.shape[0], ptr(cal, f32p), ptr(sc, f32p),
                              C.byref(ch), ptr(q, u8p), ptr(s, f32p)))
    return sc, float(ch.alpha), float(ch.error_plain), float(ch.error_awq), Matrix(kind, rows, k, q=q, s=s)
