"""Greedy speculative generation for one sequence over the device path.

A host-side mirror of the reference engine's single-sequence greedy loop
(Engine::schedule/execute/propose, src/engine.rs:395-717): chunked prompt
prefill under the token budget, then speculative steps of k draft proposals
verified in one target pass, with the reference's rollback of the
`computed` / `draft_computed` counters. The device does all model work
(ferrolm_amd.gpu); this loop only does the reference's bookkeeping.
"""
from __future__ import annotations

import time
from dataclasses import dataclass, field

import numpy as np

from . import gpu


@dataclass
class GenStats:
    proposed: int = 0
    accepted: int = 0
    spec_steps: int = 0
    accepted_per_step: list = field(default_factory=list)
    token_times: list = field(default_factory=list)
    verify_us: list = field(default_factory=list)
    draft_us: list = field(default_factory=list)


class BlockPool:
    """Hands out block ids in order (BlockManager::allocate without the
    prefix cache, src/kv.rs:139-151)."""

    def __init__(self, blocks: int):
        self.next = 0
        self.blocks = blocks

    def grow(self, table: list, tokens: int, bs: int = 16) -> bool:
        while len(table) * bs < tokens:
            if self.next >= self.blocks:
                return False
            table.append(self.next)
            self.next += 1
        return True


def generate(ctx: gpu.Context, target: gpu.Model, draft: gpu.Model | None, prompt, max_tokens: int, k: int,
             kv_blocks: int = 1024, max_batch_tokens: int = 512, max_seqs: int = 64, tkv=None, dkv=None,
             stats: GenStats | None = None):
    """Returns the generated ids (the first from the prompt's prefill)."""
    bs = 16
    cfg = target.cfg
    if draft is None:
        k = 0
    max_len = min(cfg.max_position, kv_blocks * bs)
    prompt = [int(t) for t in prompt]
    if not prompt or len(prompt) >= max_len:
        raise ValueError(f"prompt of {len(prompt)} tokens; this server fits 1 to {max_len - 1}")
    tkv = tkv or gpu.KvCache(ctx, cfg, kv_blocks)
    if draft is not None:
        dkv = dkv or gpu.KvCache(ctx, draft.cfg, kv_blocks + max_seqs)
    tpool, dpool = BlockPool(kv_blocks), BlockPool(kv_blocks + max_seqs)
    tb, db = [], []
    tokens = list(prompt)
    computed = dcomp = 0
    out = []
    st = stats or GenStats()
    while True:
        budget = max_batch_tokens
        left = len(tokens) - computed
        spec = left == 1 and k > 0 and len(tokens) + k < max_len and budget > k
        n = k + 1 if spec else min(left, budget)
        if not tpool.grow(tb, computed + n) or (spec and not dpool.grow(db, len(tokens) + k - 1)):
            raise RuntimeError("out of cache blocks")
        if spec:
            seq = gpu.SpecSeq(tail=np.array(tokens[dcomp:], np.uint32), draft_pos=dcomp, pos=computed,
                              blocks=np.array(tb, np.uint32), draft_blocks=np.array(db, np.uint32))
            toks, acc = gpu.spec_step(ctx, target, tkv, draft, dkv, [seq], k)
            t_us = gpu.last_step_times(ctx)
            st.draft_us.append(float(t_us[0]))
            st.verify_us.append(float(t_us[1]))
            emitted = [int(x) for x in toks[0]]
            a = int(acc[0])
            st.proposed += k
            st.accepted += a
            st.spec_steps += 1
            st.accepted_per_step.append(a)
            base = len(tokens)
            computed = base + a
            dcomp = min(base + k - 1, base + a)
        else:
            last = computed + n == len(tokens)
            o = gpu.forward(ctx, target, tkv, [(tokens[computed:computed + n], computed, tb,
                                               gpu.LOGITS_LAST if last else gpu.LOGITS_NONE)], logits=False)
            computed += n
            emitted = [int(o.argmax[0])] if last else []
        now = time.perf_counter()
        for t in emitted:
            tokens.append(t)
            out.append(t)
            st.token_times.append(now)
            if len(out) >= max_tokens or len(tokens) >= max_len:
                return np.array(out, np.uint32)
