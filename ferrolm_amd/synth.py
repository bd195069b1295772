"""Synthetic models and workloads for the benchmark configurations.

`random_model` is Model::random (src/model.rs:156-190) with the benchmark's
N(0, 0.02) weights (all matrices, embedding included; norms 1.0).
`quantize_model` is Model::quantize (src/model.rs:196-219).
`awq_model` is Model::quantize_awq (src/awq.rs:69-126) with the benchmark's
per-input-channel scales drawn log-uniform in [0.5, 2] instead of the
alpha search, and importance weights from synthetic calibration
activations (seeded N(0, 1) with 1% of channels at 20x): the same fold
order and the same `apply` (src/awq.rs:152-164).
"""
from __future__ import annotations

from dataclasses import dataclass, replace

import numpy as np

from . import host
from .weights import BF16, INT4, INT8, Config, HostModel, Layer, Matrix, bf16_to_f32, shape

EMBED_TENSOR = 1 << 40


def tensor_id(layer: int, which: int) -> int:
    return 16 * layer + which


def random_model(cfg: Config, seed: int, std: float = 0.02) -> HostModel:
    H, I = cfg.hidden, cfg.intermediate
    layers = []
    for l in range(cfg.layers):
        def mat(which, rows, cols):
            return Matrix(BF16, rows, cols, bf16=host.random_bf16(seed, tensor_id(l, which), rows, cols, std))
        layers.append(Layer(
            attn_norm=np.ones(H, np.float32), wqkv=mat(0, cfg.qkv_dim, H),
            bqkv=np.full(cfg.qkv_dim, 0.01, np.float32) if cfg.qkv_bias else None,
            wo=mat(1, H, cfg.q_dim), mlp_norm=np.ones(H, np.float32), w_gate_up=mat(2, 2 * I, H),
            w_down=mat(3, H, I)))
    embed = host.random_bf16(seed, EMBED_TENSOR, cfg.vocab, H, std)
    lm = None if cfg.tie_embeddings else host.random_bf16(seed, EMBED_TENSOR + 1, cfg.vocab, H, std)
    return HostModel(cfg=cfg, embed=embed, norm=np.ones(H, np.float32), layers=layers, lm_head=lm)


def _f32(m: Matrix) -> np.ndarray:
    return bf16_to_f32(m.bf16) if m.kind == BF16 else m.to_f32()


def quantize_model(hm: HostModel, kind: int) -> HostModel:
    """Model::quantize without importance weights."""
    if kind == BF16:
        return hm
    out = []
    for l in hm.layers:
        out.append(replace(l, wqkv=host.quantize(kind, _f32(l.wqkv)), wo=host.quantize(kind, _f32(l.wo)),
                           w_gate_up=host.quantize(kind, _f32(l.w_gate_up)),
                           w_down=host.quantize(kind, _f32(l.w_down))))
    return replace(hm, layers=out)


def _calibration_sq(seed: int, layer: int, which: int, k: int, rows: int = 64) -> np.ndarray:
    """Mean x^2 per input channel (awq::stats, src/awq.rs:128-142) of synthetic
    calibration rows: N(0, 1), with 1% of the channels scaled by 20."""
    rng = np.random.default_rng(host.stream_seed(seed, 2 * tensor_id(layer, which), 1))
    x = rng.standard_normal((rows, k))
    outl = rng.choice(k, size=max(1, k // 100), replace=False)
    x[:, outl] *= 20.0
    return (np.square(x).sum(axis=0) / rows).astype(np.float32)


def _scales(seed: int, layer: int, which: int, k: int) -> np.ndarray:
    """Per-input-channel AWQ scales, log-uniform in [0.5, 2]."""
    rng = np.random.default_rng(host.stream_seed(seed, 2 * tensor_id(layer, which) + 1, 2))
    return np.exp(rng.uniform(np.log(0.5), np.log(2.0), size=k)).astype(np.float32)


def awq_apply(kind: int, w: np.ndarray, s: np.ndarray, sq: np.ndarray) -> Matrix:
    """awq::apply (src/awq.rs:152-164): quantize W diag(s) with importance
    E[x^2]/s^2 + 1e-8, all in f32."""
    ws = (w * s[None, :]).astype(np.float32)
    imp = (sq / (s * s) + np.float32(1e-8)).astype(np.float32)
    return host.quantize(kind, ws, imp)


def awq_model(hm: HostModel, kind: int, seed: int) -> HostModel:
    """Model::quantize_awq's fold (src/awq.rs:75-123) with synthetic scales."""
    cfg = hm.cfg
    qd, kvd, inter, H = cfg.q_dim, cfg.kv_heads * cfg.head_dim, cfg.intermediate, cfg.hidden
    out = []
    for li, l in enumerate(hm.layers):
        qkv = _f32(l.wqkv).copy()
        gate_up = _f32(l.w_gate_up).copy()
        attn_norm = l.attn_norm.copy()
        mlp_norm = l.mlp_norm.copy()
        o = _f32(l.wo)
        sq_o = _calibration_sq(seed, li, 1, qd)
        if cfg.heads == cfg.kv_heads:
            s = _scales(seed, li, 1, qd)
            qkv[qd + kvd:qd + kvd + qd, :] /= s[:, None]
            wo = awq_apply(kind, o, s, sq_o)
        else:
            wo = awq_apply(kind, o, np.ones(qd, np.float32), sq_o)
        down = _f32(l.w_down)
        s = _scales(seed, li, 3, inter)
        gate_up[inter:2 * inter, :] /= s[:, None]
        w_down = awq_apply(kind, down, s, _calibration_sq(seed, li, 3, inter))
        s = _scales(seed, li, 2, H)
        mlp_norm /= s
        w_gate_up = awq_apply(kind, gate_up, s, _calibration_sq(seed, li, 2, H))
        s = _scales(seed, li, 0, H)
        attn_norm /= s
        wqkv = awq_apply(kind, qkv, s, _calibration_sq(seed, li, 0, H))
        out.append(Layer(attn_norm=attn_norm.astype(np.float32), wqkv=wqkv, bqkv=l.bqkv, wo=wo,
                         mlp_norm=mlp_norm.astype(np.float32), w_gate_up=w_gate_up, w_down=w_down))
    return replace(hm, layers=out)


def prompt_ids(n: int, vocab: int, seed: int) -> np.ndarray:
    """n uniform token ids in [0, vocab): numpy's PCG64 seeded with stream_seed(seed, 99, 3).

    The prompt only has to be the same on every run and in every test; the
    synthetic weights, not the prompt, come from the reference's Rng.
    """
    rng = np.random.default_rng(host.stream_seed(seed, 99, 3))
    return rng.integers(0, vocab, size=n, dtype=np.int64).astype(np.uint32)


@dataclass
class Workload:
    name: str
    target: HostModel
    draft: HostModel | None
    draft_layers: int | None  # the draft is the target's first layers when set
    k: int
    prompt_len: int
    new_tokens: int
    batch: int
    target_kind: int
    seed: int


def shapes_for(config: int) -> tuple[Config, Config, int, int, int]:
    """(target shape, draft shape, target quant, k, prompt) of each benchmark config."""
    s135 = shape("smollm2-135m")
    if config == 0:
        return replace(s135, rope_theta=10000.0), None, BF16, 3, 64
    if config == 1:
        return shape("smollm2-360m"), s135, INT8, 4, 512
    if config == 2:
        return shape("smollm2-1.7b"), s135, INT4, 3, 1024
    if config == 3:
        return shape("smollm2-1.7b"), s135, INT8, 4, 0
    if config == 4:
        return shape("llama3-8b"), shape("llama3.2-1b"), INT4, 4, 0
    raise ValueError(config)


def build(config: int, seed: int = 2024, layers: int | None = None) -> Workload:
    """The models of a benchmark configuration. `layers` truncates the target
    (for quick tests only; the benchmark uses the full shapes)."""
    tcfg, dcfg, kind, k, plen = shapes_for(config)
    if layers is not None:
        tcfg = replace(tcfg, layers=layers)
    target = random_model(tcfg, seed)
    if config == 0:
        return Workload("cfg0", target, None, 4, k, 64, 128, 1, BF16, seed)
    if kind == INT4 and config in (2, 4):
        target = awq_model(target, INT4, seed)
    else:
        target = quantize_model(target, kind)
    draft = random_model(dcfg, seed + 1)
    new = {1: 256, 2: 128, 3: 128, 4: 128}[config]
    batch = {1: 1, 2: 1, 3: 8, 4: 16}[config]
    return Workload(f"cfg{config}", target, draft, None, k, plen, new, batch, kind, seed)
