"""The reference's serving engine on the device: continuous batching over a
paged KV cache (Engine::schedule / execute, src/engine.rs:150-654) with the
prefix cache of BlockManager (src/kv.rs:74-212).

The host keeps what the reference's engine keeps: the waiting queue, the
running sequences, their block tables, the block manager with its prefix
cache, the token budget of a step, preemption with recompute. Every step's
work runs on the device through the C ABI:

  - a greedy step with both speculating sequences and prefill chunks or plain
    rows: one fg_spec_step_mixed, whose verify forward carries the chunks after
    the verify rows, as the reference runs one target forward per step;
  - otherwise prefill chunks and plain decode rows: one fg_forward (greedy:
    its argmax gives the token; with sampling requests fg_forward_sampled
    draws it), and speculating sequences: one fg_spec_step
    (fg_spec_step_sampled when any of them samples): the draft rounds, the
    target's verify pass over k+1 rows, acceptance and the draft/target
    rollback counters, on the device.

Steps with a sampled request make those two calls; they touch disjoint cache
blocks (shared prefix blocks are full prompt blocks, never written), so the
result is the same as one forward's.

Block ids from the block manager index the device caches directly. Prefix
keys are 64-bit hashes of (parent key, block tokens) of this build's own
(kv::chain, src/kv.rs:101-106, uses Rust's DefaultHasher): only equality of
keys matters, and a hit also compares the tokens, as the reference does, so a
hash collision can only turn a hit into a miss.
"""
from __future__ import annotations

import hashlib
from collections import OrderedDict, deque
from dataclasses import dataclass, field

import numpy as np

from . import gpu
from .spec import TableCache

ROOT = 0  # the key before a sequence's first block (src/kv.rs:98)


def chain(parent: int, tokens) -> int:
    """The prefix-cache key of a block holding `tokens` after the prefix
    whose key is `parent`."""
    h = hashlib.blake2b(digest_size=8)
    h.update(int(parent).to_bytes(8, "little"))
    h.update(np.asarray(tokens, np.uint32).tobytes())
    return int.from_bytes(h.digest(), "little")


@dataclass
class PrefixStats:
    queried: int = 0  # full prompt blocks looked up
    hit: int = 0
    evicted: int = 0


class BlockManager:
    """BlockManager (src/kv.rs:74-212): reference-counted cache blocks; full
    blocks published under their prefix key stay cached when no sequence
    uses them (idle) until allocation evicts the least recently released."""

    def __init__(self, blocks: int, block_size: int, prefix_enabled: bool):
        self.block_size = block_size
        self.prefix_enabled = prefix_enabled
        self._refs = [0] * blocks
        self.free = deque(range(blocks))
        self.key: list = [None] * blocks
        self.tokens: list = [None] * blocks
        self.by_key: dict = {}
        self.idle: OrderedDict = OrderedDict()  # release clock -> block (clocks increase)
        self.idle_since = [0] * blocks
        self.clock = 0
        self.stats = PrefixStats()

    def total(self) -> int:
        return len(self._refs)

    def available(self) -> int:
        """How many allocate() calls would succeed now: never-used blocks plus idle cached ones."""
        return len(self.free) + len(self.idle)

    def used(self) -> int:
        return self.total() - self.available()

    def allocate(self) -> int | None:
        if self.free:
            b = self.free.popleft()
        elif self.idle:
            _, b = self.idle.popitem(last=False)
            self._forget(b)
            self.stats.evicted += 1
        else:
            return None
        self._refs[b] = 1
        return b

    def _forget(self, b: int) -> None:
        k = self.key[b]
        if k is not None:
            self.key[b] = None
            self.by_key.pop(k, None)
            self.tokens[b] = None

    def release(self, b: int) -> None:
        if self._refs[b] <= 0:
            raise AssertionError(f"block {b} has no reference left to drop")
        self._refs[b] -= 1
        if self._refs[b] == 0:
            if self.key[b] is not None:
                self.clock += 1
                self.idle_since[b] = self.clock
                self.idle[self.clock] = b
            else:
                self.free.append(b)

    def lookup(self, parent: int, tokens) -> int | None:
        """The cached block holding exactly `tokens` after `parent`, now shared."""
        if not self.prefix_enabled:
            return None
        self.stats.queried += 1
        b = self.by_key.get(chain(parent, tokens))
        if b is None or self.tokens[b] != tuple(int(t) for t in tokens):
            return None
        if self._refs[b] == 0:
            del self.idle[self.idle_since[b]]
        self._refs[b] += 1
        self.stats.hit += 1
        return b

    def publish(self, b: int, parent: int, tokens) -> int:
        """Publishes a block the caller has just filled; returns its key."""
        k = chain(parent, tokens)
        if self.prefix_enabled and self.key[b] is None and k not in self.by_key:
            self.by_key[k] = b
            self.key[b] = k
            self.tokens[b] = tuple(int(t) for t in tokens)
        return k

    def refs(self, b: int) -> int:
        return self._refs[b]


@dataclass
class EngineConfig:
    """EngineConfig (src/engine.rs:45-73)."""

    block_size: int = 16
    kv_blocks: int = 1024
    max_batch_tokens: int = 512  # tokens processed per step, across all sequences
    max_seqs: int = 64
    prefix_cache: bool = True
    admission: str = "continuous"  # or "static"
    reserve_tokens: int | None = None  # slots reserved per sequence at admission
    spec_k: int = 4


@dataclass
class Params:
    """SamplingParams (src/sampler.rs:8-33)."""

    temperature: float = 0.0  # 0: greedy
    top_p: float = 1.0
    top_k: int = 0  # 0: no limit
    seed: int = 0
    max_tokens: int = 64
    stop_ids: tuple = ()
    ignore_eos: bool = False

    @property
    def greedy(self) -> bool:
        return self.temperature <= 0.0

    def device(self) -> gpu.SamplingParams:
        return gpu.SamplingParams(self.temperature, self.top_p, self.top_k, self.seed)


LENGTH, STOP, CANCELLED, REJECTED = "length", "stop", "cancelled", "rejected"


@dataclass
class Request:
    """A submitted request: its prompt, parameters, the tokens generated so
    far and, once done, why it finished (Event::Token / Event::Done)."""

    prompt: list
    params: Params
    tokens: list = field(default_factory=list)
    finish: str | None = None
    reason: str = ""
    cancelled: bool = False

    def cancel(self) -> None:
        self.cancelled = True


@dataclass
class Stats:
    """Stats (src/engine.rs:96-130)."""

    requests: int = 0
    finished: int = 0
    prompt_tokens: int = 0
    generated_tokens: int = 0
    computed_tokens: int = 0
    cached_tokens: int = 0
    steps: int = 0
    preemptions: int = 0
    spec_proposed: int = 0
    spec_accepted: int = 0
    mixed_steps: int = 0  # steps whose verify forward also carried chunks (no reference counterpart)
    peak_running: int = 0
    running: int = 0
    waiting: int = 0
    kv_used_blocks: int = 0
    kv_total_blocks: int = 0


class _Seq:
    def __init__(self, req: Request):
        self.req = req
        self.tokens = [int(t) for t in req.prompt]
        self.computed = 0
        self.blocks: list = []
        self.keys: list = []
        self.generated = 0
        self.rng = gpu.rng_init(req.params.seed)
        self.draft_computed = 0
        self.draft_blocks: list = []


class Engine:
    """Engine (src/engine.rs:176-717) over one device context: `model` and
    the optional `draft` are gpu.Models sharing a vocabulary."""

    def __init__(self, ctx: gpu.Context, model: gpu.Model, draft: gpu.Model | None = None,
                 cfg: EngineConfig | None = None):
        self.ctx, self.model, self.draft = ctx, model, draft
        self.cfg = cfg = cfg or EngineConfig()
        if cfg.block_size != 16:
            raise ValueError("the device caches use 16-token blocks")
        c = model.cfg
        self.kv = gpu.KvCache(ctx, c, cfg.kv_blocks)
        self.blocks = BlockManager(cfg.kv_blocks, cfg.block_size, cfg.prefix_cache)
        self.tables = TableCache()  # uint32 copies of the running sequences' block tables
        if draft is not None:
            if draft.cfg.vocab != c.vocab:
                raise ValueError("draft and target must share a vocabulary")
            n = cfg.kv_blocks + cfg.max_seqs  # as many slots as the target, plus room for proposals
            self.dkv = gpu.KvCache(ctx, draft.cfg, n)
            self.dblocks = BlockManager(n, cfg.block_size, False)
        self.max_len = min(c.max_position, cfg.kv_blocks * cfg.block_size)
        self.waiting: deque = deque()
        self.running: list = []
        self.stats = Stats(kv_total_blocks=cfg.kv_blocks)

    # ---- requests -------------------------------------------------------
    def submit(self, prompt, params: Params | None = None) -> Request:
        """Handle::submit + Engine::enqueue (src/engine.rs:271-301)."""
        req = Request(list(int(t) for t in prompt), params or Params())
        self.stats.requests += 1
        n = len(req.prompt)
        if n == 0 or n >= self.max_len:
            return self._reject(req, f"prompt of {n} tokens; this server fits 1 to {self.max_len - 1}")
        bad = next((t for t in req.prompt if t >= self.model.cfg.vocab), None)
        if bad is not None:
            return self._reject(req, f"token {bad} is outside the vocabulary")
        if not req.params.greedy and req.params.top_k < 0:
            return self._reject(req, "top_k must be 0 (no limit) or positive")
        self.stats.prompt_tokens += n
        self.waiting.append(_Seq(req))
        return req

    def _reject(self, req: Request, why: str) -> Request:
        req.finish, req.reason = REJECTED, why
        self.stats.finished += 1
        return req

    def run_until_idle(self) -> None:
        while self.running or self.waiting:
            self.step()

    # ---- bookkeeping ----------------------------------------------------
    def _release(self, s: _Seq) -> None:
        self.tables.drop((id(s), 0))
        self.tables.drop((id(s), 1))
        for b in s.blocks:
            self.blocks.release(b)
        s.blocks, s.keys, s.computed = [], [], 0
        if self.draft is not None:
            for b in s.draft_blocks:
                self.dblocks.release(b)
        s.draft_blocks, s.draft_computed = [], 0

    def _finish(self, s: _Seq, why: str) -> None:
        self._release(s)
        s.req.finish = why
        self.stats.finished += 1

    def _preempt(self, s: _Seq) -> None:
        self._release(s)
        self.stats.preemptions += 1
        self.waiting.appendleft(s)

    def _grow(self, i: int, target: int, draft: int) -> bool:
        bs = self.cfg.block_size
        s = self.running[i]
        while len(s.blocks) * bs < target:
            b = self.blocks.allocate()
            if b is None:
                return False
            s.blocks.append(b)
        if self.draft is not None:
            while len(s.draft_blocks) * bs < draft:
                b = self.dblocks.allocate()
                if b is None:
                    return False
                s.draft_blocks.append(b)
        return True

    def _reserve_for(self, i: int) -> int:
        r = self.cfg.reserve_tokens
        return 0 if r is None else max(min(r, self.max_len), len(self.running[i].tokens))

    def _reap_cancelled(self) -> None:
        i = 0
        while i < len(self.running):
            if self.running[i].req.cancelled:
                self._finish(self.running.pop(i), CANCELLED)
            else:
                i += 1
        keep = deque()
        for s in self.waiting:
            if s.req.cancelled:
                self._finish(s, CANCELLED)
            else:
                keep.append(s)
        self.waiting = keep

    # ---- one step -------------------------------------------------------
    def step(self) -> None:
        self._reap_cancelled()
        plans = self._schedule()
        if plans:
            self._execute(plans)
        st = self.stats
        st.steps += 1
        st.peak_running = max(st.peak_running, len(self.running))
        st.running, st.waiting = len(self.running), len(self.waiting)
        st.kv_used_blocks = self.blocks.used()

    def _schedule(self) -> list:
        """Engine::schedule (src/engine.rs:395-479): (sequence index, tokens)."""
        cfg, bs = self.cfg, self.cfg.block_size
        k = cfg.spec_k if self.draft is not None else 0
        budget = cfg.max_batch_tokens
        plans = []
        # Sequences already in flight are served in admission order. When the
        # block pool cannot cover one of them, the most recently admitted
        # sequence gives its blocks back and is requeued.
        i = 0
        while i < len(self.running) and budget > 0:
            s = self.running[i]
            left = len(s.tokens) - s.computed
            spec = left == 1 and k > 0 and len(s.tokens) + k < self.max_len and budget > k
            n = k + 1 if spec else min(left, budget)
            target = s.computed + n
            draft = len(s.tokens) + k - 1 if spec else 0
            if self._grow(i, max(target, self._reserve_for(i)), draft):
                plans.append([i, n])
                budget -= n
                i += 1
                continue
            self._preempt(self.running.pop())
        # Then the queue, strictly in arrival order: admission stops at the first
        # request that does not fit.
        static_open = not self.running
        while self.waiting:
            s = self.waiting[0]
            if len(self.running) >= cfg.max_seqs:
                break
            if cfg.admission == "continuous" and budget == 0:
                break
            if cfg.admission == "static" and not static_open:
                break
            # Reuse published blocks for the prompt's whole leading blocks. The
            # block that holds the final prompt token is always recomputed: its
            # forward produces the logits of the first new token.
            if not s.blocks:
                parent = ROOT
                body = s.tokens[:len(s.tokens) - 1]
                for c0 in range(0, len(body) - bs + 1, bs):
                    chunk = body[c0:c0 + bs]
                    b = self.blocks.lookup(parent, chunk)
                    if b is None:
                        break
                    parent = chain(parent, chunk)
                    s.blocks.append(b)
                    s.keys.append(parent)
                s.computed = len(s.blocks) * bs
            n = min(len(s.tokens) - s.computed, budget)
            r = cfg.reserve_tokens
            want = min(max(r, s.computed + n), self.max_len) if r is not None else s.computed + n
            need = max(0, -(-want // bs) - len(s.blocks))
            headroom = 0 if not self.running else max(self.blocks.total() // 100, 1)
            if self.blocks.available() < need + headroom:
                self._release(s)
                break
            self.waiting.popleft()
            self.stats.cached_tokens += s.computed
            self.running.append(s)
            ok = self._grow(len(self.running) - 1, want, 0)
            assert ok
            if n > 0:
                plans.append([len(self.running) - 1, n])
                budget -= n
        return plans

    def _spec_seq(self, i: int) -> gpu.SpecSeq:
        s = self.running[i]
        return gpu.SpecSeq(tail=np.array(s.tokens[s.draft_computed:], np.uint32), draft_pos=s.draft_computed,
                           pos=s.computed, blocks=self.tables.get((id(s), 0), s.blocks),
                           draft_blocks=self.tables.get((id(s), 1), s.draft_blocks))

    def _accept(self, plans: list, spec: list, toks, acc, rng, new: list) -> None:
        """The rollback of src/engine.rs:613-615 for each speculating plan."""
        k = self.cfg.spec_k
        for r, j in enumerate(spec):
            s = self.running[plans[j][0]]
            if rng is not None:
                s.rng = int(rng[r])
            a = int(acc[r])
            base = len(s.tokens)
            self.stats.spec_proposed += k
            self.stats.spec_accepted += a
            s.computed = base + a  # both caches hold the accepted proposals
            s.draft_computed = min(base + k - 1, base + a)
            new[j] = [int(t) for t in toks[r]]

    def _execute(self, plans: list) -> None:
        """Engine::execute (src/engine.rs:499-654) with the device calls."""
        bs = self.cfg.block_size
        k = self.cfg.spec_k
        is_spec = [self.draft is not None and len(self.running[i].tokens) - self.running[i].computed == 1 and n > 1
                   for i, n in plans]
        new = [[] for _ in plans]
        plain = [j for j, sp in enumerate(is_spec) if not sp]
        spec = [j for j, sp in enumerate(is_spec) if sp]
        # One target pass over every plan (src/engine.rs:511-542) when every
        # request of the step is greedy: the speculative step carries the prefill
        # chunks and plain rows in its verify forward. Otherwise (a sampled
        # request) two device calls.
        greedy = all(self.running[i].req.params.greedy for i, _ in plans)
        if plain and spec and greedy:
            chunks, last = [], []
            for j in plain:
                i, n = plans[j]
                s = self.running[i]
                done = s.computed + n == len(s.tokens)
                chunks.append((s.tokens[s.computed:s.computed + n], s.computed, s.blocks,
                               gpu.LOGITS_LAST if done else gpu.LOGITS_NONE))
                if done:
                    last.append(j)
            seqs = [self._spec_seq(plans[j][0]) for j in spec]
            toks, acc, am = gpu.spec_step_mixed(self.ctx, self.model, self.kv, self.draft, self.dkv, seqs, k,
                                                chunks)
            self.stats.mixed_steps += 1
            for r, j in enumerate(last):
                new[j] = [int(am[r])]
            for j in plain:
                i, n = plans[j]
                self.running[i].computed += n
            self._accept(plans, spec, toks, acc, None, new)
            plain, spec = [], []
        # prefill chunks and plain decode rows: one forward
        if plain:
            chunks, last = [], []
            for j in plain:
                i, n = plans[j]
                s = self.running[i]
                done = s.computed + n == len(s.tokens)
                chunks.append((s.tokens[s.computed:s.computed + n], s.computed, s.blocks,
                               gpu.LOGITS_LAST if done else gpu.LOGITS_NONE))
                if done:
                    last.append(j)
            if any(not self.running[plans[j][0]].req.params.greedy for j in last):
                ps = [self.running[plans[j][0]].req.params.device() for j in last]
                st = np.array([self.running[plans[j][0]].rng for j in last], np.uint64)
                toks = gpu.forward_sampled(self.ctx, self.model, self.kv, chunks, ps, st)
                for r, j in enumerate(last):
                    self.running[plans[j][0]].rng = int(st[r])
            else:
                toks = gpu.forward(self.ctx, self.model, self.kv, chunks, logits=False).argmax
            for r, j in enumerate(last):
                new[j] = [int(toks[r])]
            for j in plain:
                i, n = plans[j]
                self.running[i].computed += n
        # speculating sequences: one device speculative step
        if spec:
            seqs = [self._spec_seq(plans[j][0]) for j in spec]
            sampled = any(not self.running[plans[j][0]].req.params.greedy for j in spec)
            params = [self.running[plans[j][0]].req.params.device() for j in spec] if sampled else None
            rng = np.array([self.running[plans[j][0]].rng for j in spec], np.uint64) if sampled else None
            toks, acc = gpu.spec_step(self.ctx, self.model, self.kv, self.draft, self.dkv, seqs, k, params, rng)
            self._accept(plans, spec, toks, acc, rng, new)
        # tokens out, finished sequences, newly full blocks into the prefix cache
        eos = set(self.model.cfg.eos)
        finished = []
        for j, (i, n) in enumerate(plans):
            self.stats.computed_tokens += n
            s = self.running[i]
            p = s.req.params
            for t in new[j]:
                if (not p.ignore_eos and t in eos) or t in p.stop_ids:
                    finished.append((i, STOP))
                    break
                s.tokens.append(t)
                s.generated += 1
                s.req.tokens.append(t)
                self.stats.generated_tokens += 1
                if s.generated >= p.max_tokens or len(s.tokens) >= self.max_len:
                    finished.append((i, LENGTH))
                    break
            while len(s.keys) < min(s.computed, len(s.tokens)) // bs:
                b = len(s.keys)
                parent = s.keys[-1] if s.keys else ROOT
                s.keys.append(self.blocks.publish(s.blocks[b], parent, s.tokens[b * bs:(b + 1) * bs]))
        for i, why in sorted(finished, key=lambda f: -f[0]):
            self._finish(self.running.pop(i), why)
