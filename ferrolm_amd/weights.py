"""Host-side model description: configuration, weight containers and loaders.

Mirrors the reference's `Config` (src/config.rs:21-135), the weight fields of
`Model`/`Layer` (src/model.rs:28-51) and its checkpoint loading
(`Model::load`, src/model.rs:92-153). Weights are held as numpy arrays in the
formats the reference's own types hold them, so the same buffers feed both
the device upload (ferrolm_amd.gpu) and the CPU checker in the tests:

* bf16 matrices: row-major ``uint16`` bit patterns, ``rows x cols``
  (`Matrix::new`, src/kernels.rs:53).
* int8/int4 matrices: the reference's QMatrix byte layout — codes per
  32-row panel and input position, int4 as low/high nibbles offset by 8 —
  plus f32 scales ``[panel][group][32]`` (src/quant.rs:64-76).
"""
from __future__ import annotations

import json
import struct
from dataclasses import dataclass, field, replace
from pathlib import Path

import numpy as np

BF16, INT8, INT4 = 0, 1, 2
KIND_NAMES = {BF16: "bf16", INT8: "int8", INT4: "int4"}
PANEL = 32
GROUP = 32


@dataclass
class Config:
    """Model hyperparameters (src/config.rs:21-39)."""

    vocab: int
    hidden: int
    intermediate: int
    layers: int
    heads: int
    kv_heads: int
    head_dim: int
    rms_eps: float = 1e-6
    rope_theta: float = 10000.0
    rope_llama3: bool = False
    rope_factor: float = 1.0
    rope_low_freq: float = 1.0
    rope_high_freq: float = 4.0
    rope_orig_max_pos: int = 8192
    max_position: int = 4096
    tie_embeddings: bool = False
    qkv_bias: bool = False
    eos: tuple = ()

    @property
    def qkv_dim(self) -> int:
        return (self.heads + 2 * self.kv_heads) * self.head_dim

    @property
    def q_dim(self) -> int:
        return self.heads * self.head_dim

    def kv_bytes_per_token(self) -> int:
        """src/config.rs:147-150 (f32 K and V)."""
        return 2 * self.layers * self.kv_heads * self.head_dim * 4

    @staticmethod
    def from_hf(d: dict) -> "Config":
        """`Config::parse` (src/config.rs:48-135)."""
        arch = d.get("model_type", "llama")
        if arch not in ("llama", "mistral", "qwen2"):
            raise ValueError(f"unsupported model_type {arch!r}")
        if arch != "llama" and d.get("use_sliding_window") is True:
            raise ValueError("sliding-window attention is not supported")
        hidden = d["hidden_size"]
        heads = d["num_attention_heads"]
        kv = d.get("num_key_value_heads") or heads
        hd = d.get("head_dim") or hidden // heads
        if heads % kv or hd % 16 or hidden % 16:
            raise ValueError(f"unsupported shape: {heads} heads, {kv} kv heads, head_dim {hd}, hidden {hidden}")
        rope = d.get("rope_parameters") if isinstance(d.get("rope_parameters"), dict) else None
        theta = (rope or {}).get("rope_theta", d.get("rope_theta", 10000.0))
        scaling = rope if rope is not None else d.get("rope_scaling")
        llama3, factor, low, high, orig = False, 1.0, 1.0, 4.0, 8192
        if scaling:
            kind = scaling.get("rope_type") or scaling.get("type") or ""
            if kind == "llama3":
                llama3 = True
                if "factor" not in scaling:
                    raise ValueError("llama3 rope_scaling without factor")
                factor = float(scaling["factor"])
                low = float(scaling.get("low_freq_factor", 1.0))
                high = float(scaling.get("high_freq_factor", 4.0))
                orig = int(scaling.get("original_max_position_embeddings", 8192))
            elif kind != "default":
                raise ValueError(f"unsupported rope_scaling {kind!r}")
        eos = d.get("eos_token_id")
        eos = tuple(eos) if isinstance(eos, list) else ((eos,) if isinstance(eos, int) else ())
        return Config(
            vocab=d["vocab_size"], hidden=hidden, intermediate=d["intermediate_size"],
            layers=d["num_hidden_layers"], heads=heads, kv_heads=kv, head_dim=hd,
            rms_eps=float(d.get("rms_norm_eps", 1e-6)), rope_theta=float(theta),
            rope_llama3=llama3, rope_factor=factor, rope_low_freq=low, rope_high_freq=high,
            rope_orig_max_pos=orig, max_position=int(d.get("max_position_embeddings", 4096)),
            tie_embeddings=bool(d.get("tie_word_embeddings", False)),
            qkv_bias=arch == "qwen2" or d.get("attention_bias") is True, eos=eos,
        )


def shape(name: str) -> Config:
    """Named model shapes: the reference's presets (src/main.rs:149-176) plus
    the Llama shapes the benchmark configurations name."""
    table = {
        # hidden, inter, layers, heads, kv, hd, vocab, theta, tied
        "smollm2-135m": (576, 1536, 30, 9, 3, 64, 49152, 100000.0, True),
        "smollm2-360m": (960, 2560, 32, 15, 5, 64, 49152, 100000.0, True),
        "smollm2-1.7b": (2048, 8192, 24, 32, 32, 64, 49152, 130000.0, True),
        "llama3-8b": (4096, 14336, 32, 32, 8, 128, 128256, 500000.0, False),
        "llama3.2-1b": (2048, 8192, 16, 32, 8, 64, 128256, 500000.0, True),
    }
    if name not in table:
        raise ValueError(f"unknown shape {name!r}")
    h, i, l, nh, kv, hd, v, theta, tied = table[name]
    return Config(vocab=v, hidden=h, intermediate=i, layers=l, heads=nh, kv_heads=kv, head_dim=hd,
                  rms_eps=1e-5, rope_theta=theta, max_position=8192, tie_embeddings=tied, eos=(0,))


@dataclass
class Matrix:
    """One weight matrix (see module docstring for the layouts)."""

    kind: int
    rows: int
    cols: int
    bf16: np.ndarray | None = None  # uint16 [rows, cols]
    q: np.ndarray | None = None     # uint8 QMatrix codes
    s: np.ndarray | None = None     # float32 QMatrix scales

    def nbytes(self) -> int:
        """`Matrix::bytes` (src/kernels.rs:132-134, src/quant.rs:170-172)."""
        if self.kind == BF16:
            return self.rows * self.cols * 2
        return self.q.nbytes + self.s.nbytes

    def to_f32(self) -> np.ndarray:
        if self.kind == BF16:
            return bf16_to_f32(self.bf16)
        return dequantize(self)


@dataclass
class Layer:
    attn_norm: np.ndarray
    wqkv: Matrix
    bqkv: np.ndarray | None
    wo: Matrix
    mlp_norm: np.ndarray
    w_gate_up: Matrix
    w_down: Matrix


@dataclass
class HostModel:
    cfg: Config
    embed: np.ndarray          # uint16 [vocab, hidden]
    norm: np.ndarray           # float32 [hidden]
    layers: list = field(default_factory=list)
    lm_head: np.ndarray | None = None  # uint16 [vocab, hidden], untied only

    def truncated(self, n: int) -> "HostModel":
        """`Model::truncated` (src/model.rs:235-241)."""
        return HostModel(cfg=replace(self.cfg, layers=min(n, len(self.layers))), embed=self.embed,
                         norm=self.norm, layers=self.layers[:n], lm_head=self.lm_head)

    def quant(self) -> int:
        return self.layers[0].wqkv.kind if self.layers else BF16

    def weight_bytes(self) -> int:
        """`Model::weight_bytes` (src/model.rs:221-229)."""
        per = sum(l.wqkv.nbytes() + l.wo.nbytes() + l.w_gate_up.nbytes() + l.w_down.nbytes()
                  for l in self.layers)
        return per + self.embed.nbytes + (self.lm_head.nbytes if self.lm_head is not None else 0)


def bf16_to_f32(u: np.ndarray) -> np.ndarray:
    """src/safetensors.rs:166-168"""
    return (u.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """Round to nearest even, NaN kept NaN (src/safetensors.rs:170-178)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    b = x.view(np.uint32)
    rnd = np.uint32(0x7FFF) + ((b >> np.uint32(16)) & np.uint32(1))
    out = ((b + rnd) >> np.uint32(16)).astype(np.uint16)
    nan = np.isnan(x)
    if nan.any():
        out[nan] = ((b[nan] >> np.uint32(16)) | np.uint32(0x40)).astype(np.uint16)
    return out


def dequantize(m: Matrix) -> np.ndarray:
    """`QMatrix::row_f32` over all rows (src/quant.rs:145-168)."""
    P, K, G = m.rows // PANEL, m.cols, m.cols // GROUP
    if m.kind == INT8:
        codes = m.q.view(np.int8).reshape(P, K, PANEL).astype(np.float32)
    else:
        b = m.q.reshape(P, K, PANEL // 2)
        lo = (b & 0x0F).astype(np.int32) - 8
        hi = (b >> 4).astype(np.int32) - 8
        codes = np.concatenate([lo, hi], axis=2).astype(np.float32)
    s = m.s.reshape(P, G, PANEL)
    sk = np.repeat(s, GROUP, axis=1)  # [P, K, 32]
    w = (codes * sk).transpose(0, 2, 1).reshape(m.rows, K)
    return np.ascontiguousarray(w, dtype=np.float32)


def read_safetensors(path: Path) -> dict:
    """Minimal safetensors reader (header + raw little-endian data), the
    format `Checkpoint::open` reads (src/safetensors.rs:44-145)."""
    raw = Path(path).read_bytes()
    (n,) = struct.unpack("<Q", raw[:8])
    header = json.loads(raw[8:8 + n])
    base = 8 + n
    out = {}
    dt = {"BF16": np.uint16, "F32": np.float32, "F16": np.float16, "I64": np.int64, "U8": np.uint8}
    for name, info in header.items():
        if name == "__metadata__":
            continue
        a, b = info["data_offsets"]
        arr = np.frombuffer(raw[base + a:base + b], dtype=dt[info["dtype"]]).reshape(info["shape"])
        out[name] = (info["dtype"], arr)
    return out


def _vec_f32(t) -> np.ndarray:
    kind, a = t
    if kind == "BF16":
        return bf16_to_f32(a).copy()
    return np.asarray(a, dtype=np.float32).copy()


def _bf16(t) -> np.ndarray:
    kind, a = t
    if kind == "BF16":
        return np.ascontiguousarray(a)
    return f32_to_bf16(np.asarray(a, dtype=np.float32))


def load_model(d: str | Path) -> HostModel:
    """`Model::load` (src/model.rs:92-153): q/k/v and gate/up stacked."""
    d = Path(d)
    cfg = Config.from_hf(json.loads((d / "config.json").read_text()))
    t = read_safetensors(d / "model.safetensors")

    def stack(names):
        rows = [_bf16(t[n]) for n in names]
        w = np.ascontiguousarray(np.concatenate(rows, axis=0))
        return Matrix(BF16, w.shape[0], w.shape[1], bf16=w)

    layers = []
    for i in range(cfg.layers):
        p = f"model.layers.{i}"
        a = f"{p}.self_attn"
        b = None
        if cfg.qkv_bias:
            b = np.concatenate([_vec_f32(t[f"{a}.{x}_proj.bias"]) for x in "qkv"]).astype(np.float32)
        layers.append(Layer(
            attn_norm=_vec_f32(t[f"{p}.input_layernorm.weight"]),
            wqkv=stack([f"{a}.{x}_proj.weight" for x in "qkv"]), bqkv=b,
            wo=stack([f"{a}.o_proj.weight"]),
            mlp_norm=_vec_f32(t[f"{p}.post_attention_layernorm.weight"]),
            w_gate_up=stack([f"{p}.mlp.{x}_proj.weight" for x in ("gate", "up")]),
            w_down=stack([f"{p}.mlp.down_proj.weight"]),
        ))
    lm = None
    if not cfg.tie_embeddings and "lm_head.weight" in t:
        lm = _bf16(t["lm_head.weight"])
    return HostModel(cfg=cfg, embed=_bf16(t["model.embed_tokens.weight"]),
                     norm=_vec_f32(t["model.norm.weight"]), layers=layers, lm_head=lm)


# ---------------------------------------------------------------------------
# On-disk quantized models (the reference has none: it quantizes at load
# time, README.md:373-376). One safetensors file holds a HostModel as the
# device upload takes it: bf16 matrices as BF16 [rows, cols]; int8/int4
# matrices as their QMatrix codes (U8, flat) and scales (F32, flat) in the
# reference's layouts (src/quant.rs:64-76); norms, bias and embeddings as
# they are. The header's __metadata__ holds the Config and each matrix's
# format as JSON, so loading needs no config.json and repeats no search.
# ---------------------------------------------------------------------------

_MATS = ("wqkv", "wo", "w_gate_up", "w_down")
_DTYPE = {np.dtype(np.uint16): "BF16", np.dtype(np.float32): "F32", np.dtype(np.uint8): "U8"}


def write_safetensors(path: Path, tensors: dict, metadata: dict | None = None) -> None:
    """Writes name -> (safetensors dtype, array) as one safetensors file
    (8-byte little-endian header length, JSON header, data)."""
    header, blobs, off = {}, [], 0
    for name, (dtype, arr) in tensors.items():
        b = np.ascontiguousarray(arr).tobytes()
        header[name] = {"dtype": dtype, "shape": list(np.shape(arr)), "data_offsets": [off, off + len(b)]}
        blobs.append(b)
        off += len(b)
    if metadata:
        header["__metadata__"] = {k: str(v) for k, v in metadata.items()}
    h = json.dumps(header, separators=(",", ":")).encode()
    h += b" " * (-len(h) % 8)  # data starts 8-aligned
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for b in blobs:
            f.write(b)


def save_quantized(hm: HostModel, path: str | Path) -> None:
    """Saves a (quantized or bf16) HostModel to one safetensors file."""
    t, formats = {}, {}
    t["embed"] = ("BF16", hm.embed)
    t["norm"] = ("F32", hm.norm)
    if hm.lm_head is not None:
        t["lm_head"] = ("BF16", hm.lm_head)
    for i, l in enumerate(hm.layers):
        p = f"layers.{i}"
        t[f"{p}.attn_norm"] = ("F32", l.attn_norm)
        t[f"{p}.mlp_norm"] = ("F32", l.mlp_norm)
        if l.bqkv is not None:
            t[f"{p}.bqkv"] = ("F32", l.bqkv)
        for name in _MATS:
            m = getattr(l, name)
            formats[f"{p}.{name}"] = [m.kind, m.rows, m.cols]
            if m.kind == BF16:
                t[f"{p}.{name}"] = ("BF16", m.bf16)
            else:
                t[f"{p}.{name}.q"] = ("U8", m.q)
                t[f"{p}.{name}.s"] = ("F32", m.s)
    cfg = {k: (list(v) if isinstance(v, tuple) else v) for k, v in hm.cfg.__dict__.items()}
    write_safetensors(Path(path), t, {"format": "ferrolm-quantized-1", "config": json.dumps(cfg),
                                      "matrices": json.dumps(formats)})


def load_quantized(path: str | Path) -> HostModel:
    """Loads a model written by save_quantized."""
    raw = Path(path).read_bytes()
    (n,) = struct.unpack("<Q", raw[:8])
    meta = json.loads(raw[8:8 + n]).get("__metadata__", {})
    if meta.get("format") != "ferrolm-quantized-1":
        raise ValueError(f"{path}: not a ferrolm quantized model")
    c = json.loads(meta["config"])
    c["eos"] = tuple(c.get("eos", ()))
    cfg = Config(**c)
    formats = json.loads(meta["matrices"])
    t = read_safetensors(Path(path))

    def arr(name, dtype):
        return np.array(t[name][1], dtype=dtype, copy=True)

    def mat(key):
        kind, rows, cols = formats[key]
        if kind == BF16:
            return Matrix(BF16, rows, cols, bf16=arr(key, np.uint16).reshape(rows, cols))
        return Matrix(kind, rows, cols, q=arr(key + ".q", np.uint8), s=arr(key + ".s", np.float32))

    layers = []
    for i in range(cfg.layers):
        p = f"layers.{i}"
        layers.append(Layer(attn_norm=arr(f"{p}.attn_norm", np.float32), wqkv=mat(f"{p}.wqkv"),
                            bqkv=arr(f"{p}.bqkv", np.float32) if f"{p}.bqkv" in t else None,
                            wo=mat(f"{p}.wo"), mlp_norm=arr(f"{p}.mlp_norm", np.float32),
                            w_gate_up=mat(f"{p}.w_gate_up"), w_down=mat(f"{p}.w_down")))
    return HostModel(cfg=cfg, embed=arr("embed", np.uint16), norm=arr("norm", np.float32), layers=layers,
                     lm_head=arr("lm_head", np.uint16) if "lm_head" in t else None)
