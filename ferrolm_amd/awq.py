"""Activation-aware weight quantization of a host model with calibration
activations (Model::quantize_awq, src/awq.rs:65-126), the alpha search of
every projection running on the device (fg_awq_search).

Per layer, in the reference's order:
  - o: searched, and its scales folded into v's rows of wqkv, only when every
    query head has its own kv head; otherwise quantized plainly (scales 1),
    still with the calibration importance (src/awq.rs:84-96);
  - down: searched, scales folded into the up rows of w_gate_up (:98-107);
  - gate/up (after that fold): searched, folded into mlp_norm (:109-115);
  - qkv (after the v fold): searched, folded into attn_norm (:117-122).
A fold divides in f32 (`*v /= s`). The q/k/v bias is left as it is, as the
reference leaves it.

`calib[layer][which]` holds the projection's calibration input rows
(which: 0 qkv, 1 o, 2 gate/up, 3 down), as Model::calibrate returns them.
"""
from __future__ import annotations

from dataclasses import dataclass, replace
from typing import Callable

import numpy as np

from . import host
from .weights import HostModel, Layer, Matrix

NAMES = ("qkv", "o", "gate_up", "down")


@dataclass
class Choice:
    """awq::Choice (src/awq.rs:24-31)."""

    layer: int
    which: str
    alpha: float
    error_plain: float
    error_awq: float


# search(kind, w, cal) -> (scales, alpha, error_plain, error_awq, Matrix)
Search = Callable[[int, np.ndarray, np.ndarray], tuple]
# apply(kind, w, scales, cal) -> Matrix
Apply = Callable[[int, np.ndarray, np.ndarray, np.ndarray], Matrix]


def xorshift64(v: int) -> int:
    """Marsaglia's xorshift64 step with shifts (13, 7, 17), as Model::record
    advances its generator (src/model.rs:383-385)."""
    m = (1 << 64) - 1
    v ^= (v << 13) & m
    v ^= v >> 7
    v ^= (v << 17) & m
    return v


class Reservoir:
    """Model::record's sample (src/model.rs:56-70, 364-392): up to max_rows
    rows per (layer, projection), a uniform reservoir over every row seen.
    One xorshift generator (13, 7, 17; seeded 0x9E3779B97F4A7C15) is shared
    by every layer and projection and advanced once per row past the first
    max_rows, so rows must arrive in the reference's order: per forward,
    layer by layer, qkv, o, gate_up, down, tokens in chunk order."""

    def __init__(self, layers: int, max_rows: int):
        self.max_rows = max_rows
        self.rng = 0x9E3779B97F4A7C15
        self.rows = [[[] for _ in range(4)] for _ in range(layers)]
        self.seen = [[0] * 4 for _ in range(layers)]

    def record(self, layer: int, which: int, x: np.ndarray) -> None:
        kept, mx = self.rows[layer][which], self.max_rows
        for r in np.asarray(x, np.float32):
            n = self.seen[layer][which]
            self.seen[layer][which] += 1
            if n < mx:
                kept.append(r.copy())
                continue
            self.rng = xorshift64(self.rng)
            j = self.rng % (n + 1)
            if j < mx:
                kept[j] = r.copy()

    def result(self) -> list:
        """Per layer the four row sets as float32 [rows, width] arrays."""
        return [[np.stack(rows).astype(np.float32) if rows else np.zeros((0, 0), np.float32) for rows in l]
                for l in self.rows]


def calibrate(ctx, model, seqs, max_rows: int) -> list:
    """Model::calibrate (src/awq.rs:38-62) on the device: each sequence's
    forward from position 0 in a fresh cache of its own 16-token blocks,
    with the four projection inputs of every layer captured on the device
    (fg_forward_capture) and sampled by Model::record's reservoir. Returns
    calib[layer][which] for quantize_awq."""
    from . import gpu

    c = model.cfg
    res = Reservoir(c.layers, max_rows)
    for s in seqs:
        s = np.ascontiguousarray(s, np.uint32)
        nb = (len(s) + 15) // 16
        kv = gpu.KvCache(ctx, c, max(nb, 1), 16)
        try:
            taps = gpu.forward_capture(ctx, model, kv, [(s, 0, np.arange(nb, dtype=np.uint32))])
        finally:
            kv.close()
        for li in range(c.layers):
            for which in range(4):
                res.record(li, which, taps[li][which])
    return res.result()


def device(ctx) -> tuple[Search, Apply]:
    """The device's search and apply (fg_awq_search, fg_quantize) on ctx."""
    from . import gpu

    def search(kind, w, cal):
        return gpu.awq_search(ctx, kind, w, cal)

    def apply(kind, w, s, cal):
        # apply (src/awq.rs:152-165): W diag(s), importance E[x^2] / s^2 + 1e-8, in f32
        _, sq = host.awq_stats(cal)
        ws = (np.ascontiguousarray(w, np.float32) * s[None, :]).astype(np.float32)
        imp = (sq / (s * s) + np.float32(1e-8)).astype(np.float32)
        return gpu.quantize(ctx, kind, ws, imp)

    return search, apply


def quantize_awq(hm: HostModel, kind: int, calib, search: Search, apply: Apply) -> tuple[HostModel, list]:
    """Model::quantize_awq (src/awq.rs:65-126): a new HostModel whose layers
    are quantized to `kind` with the searched scales folded into their
    producers, and the list of Choices (three or four per layer)."""
    cfg = hm.cfg
    qd, kvd, inter = cfg.heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim, cfg.intermediate
    layers, choices = [], []
    for li, l in enumerate(hm.layers):
        cal = calib[li]
        qkv = np.array(l.wqkv.to_f32(), np.float32, copy=True)
        gate_up = np.array(l.w_gate_up.to_f32(), np.float32, copy=True)
        attn_norm = np.array(l.attn_norm, np.float32, copy=True)
        mlp_norm = np.array(l.mlp_norm, np.float32, copy=True)

        o = l.wo.to_f32()
        if cfg.heads == cfg.kv_heads:
            s, alpha, ep, ea, wo = search(kind, o, cal[1])
            qkv[qd + kvd:qd + kvd + qd, :] /= s[:, None]
            choices.append(Choice(li, NAMES[1], alpha, ep, ea))
        else:
            wo = apply(kind, o, np.ones(qd, np.float32), cal[1])

        s, alpha, ep, ea, w_down = search(kind, l.w_down.to_f32(), cal[3])
        gate_up[inter:2 * inter, :] /= s[:, None]
        choices.append(Choice(li, NAMES[3], alpha, ep, ea))

        s, alpha, ep, ea, w_gate_up = search(kind, gate_up, cal[2])
        mlp_norm /= s
        choices.append(Choice(li, NAMES[2], alpha, ep, ea))

        s, alpha, ep, ea, wqkv = search(kind, qkv, cal[0])
        attn_norm /= s
        choices.append(Choice(li, NAMES[0], alpha, ep, ea))

        layers.append(Layer(attn_norm=attn_norm, wqkv=wqkv, bqkv=l.bqkv, wo=wo, mlp_norm=mlp_norm,
                            w_gate_up=w_gate_up, w_down=w_down))
    return replace(hm, layers=layers), choices
