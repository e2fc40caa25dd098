"""Continuous batching over the paged KV cache: the request scheduler of ggmlc's runtime
(runtime/include/ggmlc/batch_scheduler.h, runtime/src/batch_scheduler.cpp:130-405) on
`paged.BatchDecoder`.

Same surface and the same iteration-level policy: `step()` first admits pending
requests into free slots — each is prefilled alone (after mapping the pages of its
longest cached prompt prefix), its first token sampled, its new full prompt pages
offered to the prefix tree — and returns if it admitted any; otherwise it decodes one
token for every active slot in one batched step over the bucket {1, 2, 4, 8, 16} that
covers the highest active slot. Where the reference decodes the whole batch at the
largest position of any slot (batch_scheduler.cpp:302-321), every slot here runs at its
own position, so a sequence's tokens do not depend on what else is in the batch.
Other differences, by design: a request waits in the queue while the page pool (after
evicting unreferenced prefix pages) cannot hold prompt + max_new_tokens rows; prefix
pages are kept alive by the tree's own page reference; greedy sampling is the argmax on
the device; temperature sampling draws from this module's own generator.
"""

from __future__ import annotations

from collections import deque
from dataclasses import dataclass, field

import numpy as np

from .paged import BatchDecoder, PagedRadixTree


@dataclass
class GenerationRequest:
    request_id: int = 0
    prompt_tokens: list = field(default_factory=list)
    generated_tokens: list = field(default_factory=list)
    slot_id: int = -1
    current_pos: int = 0
    max_new_tokens: int = 32
    temperature: float = 0.0
    eos_token_id: int = -1
    finished: bool = False
    finish_reason: str = ""
    matched_radix_nodes: list = field(default_factory=list)
    prefix_tokens_matched: int = 0


@dataclass
class StepResult:
    new_tokens: list = field(default_factory=list)  # (request_id, token_id)
    completed_request_ids: list = field(default_factory=list)


BUCKETS = (1, 2, 4, 8, 16)


class ContinuousBatchScheduler:
    def __init__(self, executor, max_batch_size: int = 8, eos_token_id: int = 0, seed: int = 1337):
        if not isinstance(executor, BatchDecoder):  # a runner's executor: its paged decoder
            executor = executor.paged_decoder(max_batch_size)
        if max_batch_size > executor.max_batch:
            raise ValueError("max_batch_size exceeds the executor's slots")
        self.executor = executor
        self._max_batch = max_batch_size
        self.default_eos = eos_token_id
        self._next_id = 1
        self.radix_tree = PagedRadixTree(executor.P)
        self.prefix_caching = True
        self.total_prefix_cache_hits = 0
        self.total_prefix_tokens_saved = 0
        self.pending: deque = deque()
        self.active: list = [None] * max_batch_size
        self.requests: dict = {}
        self.use_graphs = True
        self._rng = np.random.default_rng(seed)

    # -- queue ---------------------------------------------------------------------
    def add_request(self, prompt_tokens, max_new_tokens: int = 32, temperature: float = 0.0,
                    eos_token_id: int = -1) -> int:
        toks = [int(t) for t in prompt_tokens]
        if not toks:
            raise ValueError("empty prompt")
        if min(toks) < 0 or max(toks) >= self.executor.cfg.n_vocab:
            raise ValueError("token id outside the vocabulary")
        if len(toks) + max_new_tokens > self.executor.max_ctx:
            raise ValueError("prompt + max_new_tokens exceeds the executor's context")
        r = GenerationRequest(self._next_id, toks, [], -1, 0, int(max_new_tokens), float(temperature),
                              eos_token_id if eos_token_id >= 0 else self.default_eos)
        self._next_id += 1
        self.pending.append(r)
        self.requests[r.request_id] = r
        return r.request_id

    def has_work(self) -> bool:
        return bool(self.pending) or any(a is not None for a in self.active)

    def active_count(self) -> int:
        return sum(a is not None for a in self.active)

    def pending_count(self) -> int:
        return len(self.pending)

    def max_batch_size(self) -> int:
        return self._max_batch

    def get_request(self, request_id: int) -> GenerationRequest | None:
        return self.requests.get(request_id)

    def enable_prefix_caching(self, enable: bool) -> None:
        self.prefix_caching = bool(enable)

    def is_prefix_caching_enabled(self) -> bool:
        return self.prefix_caching

    # -- internals -------------------------------------------------------------------
    def _sample(self, logits, temperature: float) -> int:
        """argmax (first maximum) at temperature <= 0, else a draw from softmax(logits / T)."""
        x = np.asarray(logits, np.float64)
        if temperature <= 0.0:
            return int(np.argmax(x))
        p = np.exp((x - x.max()) / temperature)
        return int(self._rng.choice(x.size, p=p / p.sum()))

    def _evict(self, n_pages: int) -> int:
        dropped = self.radix_tree.evict_lru(n_pages)
        for p in dropped:
            self.executor.kv.pool.release(p)
        return len(dropped)

    def _finish(self, r: GenerationRequest, res: StepResult, reason: str) -> None:
        r.finished, r.finish_reason = True, reason
        res.completed_request_ids.append(r.request_id)
        for node in r.matched_radix_nodes:
            self.radix_tree.release_node(node)
        r.matched_radix_nodes = []
        self.executor.kv.free_slot(r.slot_id)
        self.active[r.slot_id] = None

    def _emit(self, r: GenerationRequest, tok: int, res: StepResult) -> None:
        r.generated_tokens.append(tok)
        res.new_tokens.append((r.request_id, tok))
        if r.eos_token_id >= 0 and tok == r.eos_token_id:
            self._finish(r, res, "stop")
        elif len(r.generated_tokens) >= r.max_new_tokens:
            self._finish(r, res, "length")

    def _pages_free(self, keep=()) -> int:
        """pool pages free now plus the cached pages only the tree holds (unreferenced
        subtrees evict leaf by leaf), not counting the nodes in keep"""
        kv = self.executor.kv
        keep = {id(n) for n in keep}
        held = 0
        stack = [self.radix_tree.root]
        while stack:
            n = stack.pop()
            for ch in n.children.values():
                stack.append(ch)
                if ch.ref_count == 0 and id(ch) not in keep and kv.pool.refcount(ch.page) == 1:
                    held += 1
        return kv.pool.free_count + held

    def _admit(self, r: GenerationRequest, slot: int, res: StepResult) -> bool:
        ex, kv, P = self.executor, self.executor.kv, self.executor.P
        match = self.radix_tree.match_prefix(r.prompt_tokens) if self.prefix_caching else None
        matched = match.matched_tokens if match else 0
        need = -(-(len(r.prompt_tokens) + r.max_new_tokens) // P) - (match.matched_pages if match else 0)
        if need > self._pages_free(match.matched_nodes if match else ()):
            return False  # stays queued until pages come back
        r.slot_id = slot
        self.active[slot] = r
        kv.alloc_slot(slot)
        if match and match.matched_pages:
            for node in match.matched_nodes:
                self.radix_tree.retain_node(node)
            r.matched_radix_nodes = list(match.matched_nodes)
            r.prefix_tokens_matched = matched
            kv.map_existing_pages(slot, 0, match.pages)
            self.total_prefix_cache_hits += 1
            self.total_prefix_tokens_saved += matched
        kv.ensure_tokens(slot, len(r.prompt_tokens) + r.max_new_tokens, evict=self._evict)
        logits = ex.prefill(slot, r.prompt_tokens, matched)
        if self.prefix_caching:
            n_full = len(r.prompt_tokens) // P
            first = matched // P
            if n_full > first:
                adopted = self.radix_tree.insert_prefix(r.prompt_tokens, first, kv.pages[slot][first:n_full])
                for p in adopted:  # the tree's own reference
                    kv.pool.retain(p)
        tok = self._sample(logits.cpu().numpy(), r.temperature)
        r.current_pos = len(r.prompt_tokens)
        self._emit(r, tok, res)
        return True

    # -- one iteration -------------------------------------------------------------------
    def step(self) -> StepResult:
        res = StepResult()
        admitted = False
        while self.pending:
            slot = next((i for i, a in enumerate(self.active) if a is None), -1)
            if slot < 0:
                break
            if not self._admit(self.pending[0], slot, res):
                break
            self.pending.popleft()
            admitted = True
        if admitted:
            return res
        live = [i for i, a in enumerate(self.active) if a is not None]
        if not live:
            return res
        top = max(live) + 1  # rows [0, top) must run; idle rows in between compute nothing useful
        B = max(top, min(self._max_batch, next((b for b in BUCKETS if b >= top), top)))
        tokens = np.zeros(B, np.int32)
        for i in live:
            tokens[i] = self.active[i].generated_tokens[-1]
        ex = self.executor
        nxt = ex.decode(B, tokens, live=live, use_graph=self.use_graphs)
        logits = None
        for i in live:
            r = self.active[i]
            if r.temperature > 0.0:
                if logits is None:
                    logits = ex._buffers(B)["logits"].cpu().numpy()
                tok = self._sample(logits[i], r.temperature)
            else:
                tok = int(nxt[i])
            r.current_pos += 1
            self._emit(r, tok, res)
        return res
