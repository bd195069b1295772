"""Speculative generation over the device path.

A host-side mirror of the reference engine's loop (Engine::schedule/execute/
propose, src/engine.rs:395-717): chunked prompt prefill under the token
budget, then speculative steps of k draft proposals verified in one target
pass, with the reference's rollback of the `computed` / `draft_computed`
counters (src/engine.rs:613-615). `Runner` drives one request; `Batch` drives
several that decode together, every step one device speculative step over
all of them. Requests are greedy unless given SamplingParams; then every draw
(the prompt's first token, the draft proposals, acceptance, residual and
bonus draws) happens on the device from the request's generator state, which
these loops carry between steps. The device does all model work
(ferrolm_amd.gpu); these loops only do the reference's bookkeeping.
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


class ShuffledPool(BlockPool):
    """Block ids in a seeded random order, so that block tables are not
    contiguous (the block pool of the batched configurations)."""

    def __init__(self, blocks: int, seed: int):
        super().__init__(blocks)
        self.order = [int(b) for b in np.random.default_rng(seed).permutation(blocks)]

    def grow(self, table: list, tokens: int, bs: int = 16) -> bool:
        while len(table) * bs < tokens:
            if self.next >= self.blocks:
                return False
            table.append(self.order[self.next])
            self.next += 1
        return True


class TableCache:
    """uint32 copies of block tables for the device calls, reused until a table
    grows: a table list only ever grows in place (a released table is replaced
    by a new list), so the same list object at the same length holds the same
    ids. At 32 sequences of up to 2k tokens, converting every table on every
    step cost about as much host time as the rest of the step's host work."""

    def __init__(self):
        self._c = {}

    def get(self, key, table: list) -> np.ndarray:
        e = self._c.get(key)
        if e is None or e[0] is not table or len(e[1]) != len(table):
            e = (table, np.array(table, np.uint32))
            self._c[key] = e
        return e[1]

    def drop(self, key) -> None:
        self._c.pop(key, None)


class Batch:
    """Several greedy requests decoded together (ignore_eos). The prompts are
    prefilled in one forward over all their chunks (Logits::Last each); then
    every step runs the reference's spec plan for every sequence at once
    (Engine::execute over decoding sequences, src/engine.rs:499-654): one
    device speculative step, then each sequence's rollback. Blocks come from a
    shuffled pool shared by all sequences."""

    def __init__(self, ctx: gpu.Context, target: gpu.Model, draft: gpu.Model, prompts, k: int, kv_blocks: int,
                 seed: int = 0, tkv=None, dkv=None, params: list | None = None):
        self.ctx, self.target, self.draft, self.k = ctx, target, draft, k
        # per-sequence sampling (None: every sequence greedy)
        self.params = params if params is not None and any(not p.greedy for p in params) else None
        self.rng = (np.array([gpu.rng_init(p.seed) for p in params], np.uint64) if self.params is not None
                    else None)
        self.max_len = target.cfg.max_position
        self.tkv = tkv or gpu.KvCache(ctx, target.cfg, kv_blocks)
        self.dkv = dkv or gpu.KvCache(ctx, draft.cfg, kv_blocks)
        self.tpool, self.dpool = ShuffledPool(kv_blocks, seed), ShuffledPool(kv_blocks, seed + 1)
        self.tokens = [[int(t) for t in p] for p in prompts]
        n = len(self.tokens)
        self.tb, self.db = [[] for _ in range(n)], [[] for _ in range(n)]
        self.computed, self.dcomp = [0] * n, [0] * n
        self.tables = TableCache()
        self.stats = GenStats()

    def prefill(self, max_tokens: int = 0) -> list:
        """The first token of every sequence. With max_tokens, the prompts go
        through forwards of at most that many tokens (a long prompt in chunks, as
        the reference's token budget does, src/engine.rs:455); otherwise all of
        them in one forward."""
        for i, t in enumerate(self.tokens):
            if not self.tpool.grow(self.tb[i], len(t)):
                raise RuntimeError("out of cache blocks")
        first = [0] * len(self.tokens)
        budget = max_tokens or sum(len(t) for t in self.tokens)
        work = [(i, 0) for i in range(len(self.tokens))]  # (sequence, next position)
        while work:
            chunks, rows, room = [], [], budget
            while work and room > 0:
                i, pos = work.pop(0)
                t = self.tokens[i]
                n = min(len(t) - pos, room)
                last = pos + n == len(t)
                chunks.append((t[pos:pos + n], pos, self.tb[i], gpu.LOGITS_LAST if last else gpu.LOGITS_NONE))
                if last:
                    rows.append(i)
                else:
                    work.insert(0, (i, pos + n))
                room -= n
            if self.params is None:
                o = gpu.forward(self.ctx, self.target, self.tkv, chunks, logits=False)
                for r, i in enumerate(rows):
                    first[i] = int(o.argmax[r])
            else:
                st = np.ascontiguousarray(self.rng[rows])
                toks = gpu.forward_sampled(self.ctx, self.target, self.tkv, chunks, [self.params[i] for i in rows], st)
                self.rng[rows] = st
                for r, i in enumerate(rows):
                    first[i] = int(toks[r])
        for i, t in enumerate(self.tokens):
            self.computed[i] = len(t)
            t.append(first[i])
        return first

    def step(self) -> list:
        """One speculative step for every sequence; the emitted ids of each."""
        k = self.k
        seqs = []
        for i, t in enumerate(self.tokens):
            if len(t) - self.computed[i] != 1 or len(t) + k >= self.max_len:
                raise RuntimeError("every sequence must be decoding, with room for k more tokens")
            if not self.tpool.grow(self.tb[i], self.computed[i] + k + 1) or \
                    not self.dpool.grow(self.db[i], len(t) + k - 1):
                raise RuntimeError("out of cache blocks")
            seqs.append(gpu.SpecSeq(tail=np.array(t[self.dcomp[i]:], np.uint32), draft_pos=self.dcomp[i],
                                    pos=self.computed[i], blocks=self.tables.get((i, 0), self.tb[i]),
                                    draft_blocks=self.tables.get((i, 1), self.db[i])))
        toks, acc = gpu.spec_step(self.ctx, self.target, self.tkv, self.draft, self.dkv, seqs, k, self.params,
                                  self.rng)
        t_us = gpu.last_step_times(self.ctx)
        st = self.stats
        st.draft_us.append(float(t_us[0]))
        st.verify_us.append(float(t_us[1]))
        st.spec_steps += 1
        out = []
        for i, t in enumerate(self.tokens):
            a = int(acc[i])
            st.proposed += k
            st.accepted += a
            base = len(t)
            self.computed[i] = base + a
            self.dcomp[i] = min(base + k - 1, base + a)
            em = [int(x) for x in toks[i]]
            t.extend(em)
            out.append(em)
        return out


class Runner:
    """One request through the engine's greedy loop (ignore_eos)."""

    def __init__(self, ctx: gpu.Context, target: gpu.Model, draft: gpu.Model | None, prompt, k: int,
                 kv_blocks: int = 1024, max_batch_tokens: int = 512, max_seqs: int = 64, tkv=None, dkv=None,
                 params: gpu.SamplingParams | None = None):
        self.ctx, self.target, self.draft = ctx, target, draft
        self.params = params if params is not None and not params.greedy else None
        self.rng = np.array([gpu.rng_init(params.seed)], np.uint64) if self.params is not None else None
        self.k = k if draft is not None else 0
        self.bs = 16
        self.max_len = min(target.cfg.max_position, kv_blocks * self.bs)
        self.budget = max_batch_tokens
        prompt = [int(t) for t in prompt]
        if not prompt or len(prompt) >= self.max_len:
            raise ValueError(f"prompt of {len(prompt)} tokens; this server fits 1 to {self.max_len - 1}")
        self.tkv = tkv or gpu.KvCache(ctx, target.cfg, kv_blocks)
        self.dkv = None
        if draft is not None:
            self.dkv = dkv or gpu.KvCache(ctx, draft.cfg, kv_blocks + max_seqs)
        self.tpool, self.dpool = BlockPool(kv_blocks), BlockPool(kv_blocks + max_seqs)
        self.tb, self.db = [], []
        self.tables = TableCache()
        self.tokens = list(prompt)
        self.computed = 0
        self.dcomp = 0
        self.generated = []
        self.stats = GenStats()

    def decoding(self) -> bool:
        return len(self.tokens) - self.computed == 1

    def step(self) -> list:
        """One engine step (src/engine.rs:374-393); returns the emitted ids."""
        k = self.k
        left = len(self.tokens) - self.computed
        spec = left == 1 and k > 0 and len(self.tokens) + k < self.max_len and self.budget > k
        n = k + 1 if spec else min(left, self.budget)
        if not self.tpool.grow(self.tb, self.computed + n) or (
                spec and not self.dpool.grow(self.db, len(self.tokens) + k - 1)):
            raise RuntimeError("out of cache blocks")
        if spec:
            seq = gpu.SpecSeq(tail=np.array(self.tokens[self.dcomp:], np.uint32), draft_pos=self.dcomp,
                              pos=self.computed, blocks=self.tables.get(0, self.tb),
                              draft_blocks=self.tables.get(1, self.db))
            toks, acc = gpu.spec_step(self.ctx, self.target, self.tkv, self.draft, self.dkv, [seq], k,
                                      None if self.params is None else [self.params], self.rng)
            t_us = gpu.last_step_times(self.ctx)
            st = self.stats
            st.draft_us.append(float(t_us[0]))
            st.verify_us.append(float(t_us[1]))
            emitted = [int(x) for x in toks[0]]
            a = int(acc[0])
            st.proposed += k
            st.accepted += a
            st.spec_steps += 1
            st.accepted_per_step.append(a)
            base = len(self.tokens)
            self.computed = base + a
            self.dcomp = min(base + k - 1, base + a)
        else:
            last = self.computed + n == len(self.tokens)
            chunk = (self.tokens[self.computed:self.computed + n], self.computed, self.tb,
                     gpu.LOGITS_LAST if last else gpu.LOGITS_NONE)
            if last and self.params is not None:
                emitted = [int(gpu.forward_sampled(self.ctx, self.target, self.tkv, [chunk], [self.params],
                                                   self.rng)[0])]
            else:
                o = gpu.forward(self.ctx, self.target, self.tkv, [chunk], logits=False)
                emitted = [int(o.argmax[0])] if last else []
            self.computed += n
        out = []
        for t in emitted:
            if len(self.tokens) >= self.max_len:
                break
            self.tokens.append(t)
            self.generated.append(t)
            out.append(t)
        return out

    def prefill(self) -> list:
        """Steps until the prompt is processed and the first token exists."""
        out = []
        while not out:
            out = self.step()
        return out


def generate(ctx: gpu.Context, target: gpu.Model, draft: gpu.Model | None, prompt, max_tokens: int, k: int,
             kv_blocks: int = 1024, max_batch_tokens: int = 512, stats: GenStats | None = None, **kw):
    """The generated ids (the first from the prompt's prefill), stopping at
    max_tokens or the context limit (src/engine.rs:633-636). params=
    SamplingParams samples instead of decoding greedily."""
    r = Runner(ctx, target, draft, prompt, k, kv_blocks, max_batch_tokens, **kw)
    while len(r.generated) < max_tokens and len(r.tokens) < r.max_len:
        r.step()
    if stats is not None:
        stats.__dict__.update(r.stats.__dict__)
    return np.array(r.generated[:max_tokens], np.uint32)
