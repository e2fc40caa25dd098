"""Paged KV cache, prefix radix tree and the batched paged decoder (continuous batching).

What ggmlc's runtime does (runtime/src/executor.cpp:634-920 paged slots over the VMM
windows of vmm_pool.cu, radix_tree.cpp prefix pages, batch_scheduler.cpp:130-405)
re-designed for one MI355X:

* `PagePool`: pages of `page_size` KV rows, refcounted on the host. Page p is rows
  [p*P, (p+1)*P) of every layer's K and V pool (device fp16 [1, Hkv, n_pages*P, hd]),
  so one page id addresses a token range in all layers at once. Page 0 is a trash page
  that absorbs the KV writes of idle batch rows.
* `PagedRadixTree`: full pages of prompt tokens keyed by their FNV-1a chunk hash (the
  tree of radix_tree.cpp). The tree holds a reference on each page it adopts, so a page
  outlives the request that computed it until it is evicted (LRU leaves first).
* `PagedKVCache`: the pools plus one page table row per batch slot (host mirror +
  device int32 [max_batch, max_pages]); slots share prefix pages by listing them.
* `BatchDecoder`: prefill of one sequence at a time on a contiguous cache (`Decoder`,
  the GEMM path), whose rows are then stored into the slot's pages (shared prefix pages
  are loaded first, so only the suffix is computed); batched decode of B slots per step
  with every sequence at its own position: the fused GEMV layer stack over B rows, KV
  writes to each row's pool row and `gq_flash_attn_paged` over each row's own pages.
  One HIP graph per (B, context bucket).
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np
import torch

from . import ops
from .model import Decoder, ModelWeights, _Recorder, forward, pad_kv_len, q8_chain_ok

FNV_OFFSET = 0xCBF29CE484222325
FNV_PRIME = 0x100000001B3
_M64 = (1 << 64) - 1


class PagePool:
    """Refcounted page ids [reserved, n_pages); ids below `reserved` are never handed out."""

    def __init__(self, n_pages: int, reserved: int = 1):
        if n_pages <= reserved:
            raise ValueError("the pool needs more pages than it reserves")
        self.n_pages, self.reserved = n_pages, reserved
        self._ref = np.zeros(n_pages, np.int64)
        self._free = list(range(n_pages - 1, reserved - 1, -1))  # pop() hands out low ids first

    def alloc(self) -> int:
        if not self._free:
            raise MemoryError("KV page pool exhausted")
        p = self._free.pop()
        self._ref[p] = 1
        return p

    def retain(self, p: int) -> None:
        if self._ref[p] <= 0:
            raise ValueError(f"page {p} is not allocated")
        self._ref[p] += 1

    def release(self, p: int) -> bool:
        """Drop one reference; True when the page went back to the free list."""
        if self._ref[p] <= 0:
            raise ValueError(f"page {p} is not allocated")
        self._ref[p] -= 1
        if self._ref[p] == 0:
            self._free.append(p)
            return True
        return False

    def refcount(self, p: int) -> int:
        return int(self._ref[p])

    @property
    def free_count(self) -> int:
        return len(self._free)

    @property
    def used_count(self) -> int:
        return self.n_pages - self.reserved - len(self._free)


@dataclass(eq=False)
class RadixNode:
    token_chunk: tuple = ()
    chunk_hash: int = 0
    page: int = -1
    parent: "RadixNode | None" = None
    children: dict = field(default_factory=dict)
    ref_count: int = 0
    last_accessed: int = 0


@dataclass
class PrefixMatchResult:
    matched_tokens: int = 0
    matched_pages: int = 0
    pages: list = field(default_factory=list)
    matched_nodes: list = field(default_factory=list)


class PagedRadixTree:
    """Prompt prefixes in whole pages (radix_tree.h / radix_tree.cpp): each edge is one
    page of tokens, matched by hash and then by exact token equality."""

    def __init__(self, tokens_per_page: int = 1024):
        self._tpp = tokens_per_page if tokens_per_page > 0 else 1024
        self._tick = 0
        self.root = RadixNode()

    @property
    def tokens_per_page(self) -> int:
        return self._tpp

    @staticmethod
    def hash_token_chunk(tokens) -> int:
        """64-bit FNV-1a over the little-endian bytes of the int32 tokens."""
        h = FNV_OFFSET
        for t in np.asarray(tokens, np.int64).tolist():
            v = t & 0xFFFFFFFF
            for sh in (0, 8, 16, 24):
                h = ((h ^ ((v >> sh) & 0xFF)) * FNV_PRIME) & _M64
        return h

    def _chunk(self, tokens, p):
        c = tuple(int(t) for t in tokens[p * self._tpp:(p + 1) * self._tpp])
        return c, self.hash_token_chunk(c)

    def match_prefix(self, prompt_tokens) -> PrefixMatchResult:
        r = PrefixMatchResult()
        cur = self.root
        for p in range(len(prompt_tokens) // self._tpp):
            chunk, h = self._chunk(prompt_tokens, p)
            nxt = cur.children.get(h)
            if nxt is None or nxt.token_chunk != chunk:  # a hash collision is a miss
                break
            cur = nxt
            self._tick += 1
            cur.last_accessed = self._tick
            r.matched_nodes.append(cur)
            r.pages.append(cur.page)
            r.matched_pages += 1
            r.matched_tokens += self._tpp
        return r

    def insert_prefix(self, prompt_tokens, start_page: int, pages: list) -> list:
        """Attach pages[j] as page start_page + j of this prompt (whole pages only).
        Returns the pages the tree adopted (chunks already present keep their page);
        the caller adds a pool reference for each of them on the tree's behalf."""
        cur = self.root
        for p in range(start_page):
            if (p + 1) * self._tpp > len(prompt_tokens):
                return []
            chunk, h = self._chunk(prompt_tokens, p)
            nxt = cur.children.get(h)
            if nxt is None or nxt.token_chunk != chunk:
                return []
            cur = nxt
        adopted = []
        for j, page in enumerate(pages):
            pi = start_page + j
            if (pi + 1) * self._tpp > len(prompt_tokens):
                break
            chunk, h = self._chunk(prompt_tokens, pi)
            self._tick += 1
            nxt = cur.children.get(h)
            if nxt is not None and nxt.token_chunk == chunk:
                nxt.last_accessed = self._tick
                cur = nxt
                continue
            if nxt is not None:  # same hash, other tokens: keep the resident chunk
                break
            node = RadixNode(chunk, h, int(page), cur, {}, 0, self._tick)
            cur.children[h] = node
            cur = node
            adopted.append(int(page))
        return adopted

    def retain_node(self, node: RadixNode) -> None:
        node.ref_count += 1
        self._tick += 1
        node.last_accessed = self._tick

    def release_node(self, node: RadixNode) -> None:
        if node.ref_count > 0:
            node.ref_count -= 1

    def evict_lru(self, max_pages: int) -> list:
        """Unlink up to max_pages unreferenced leaves, oldest first; returns their pages."""
        freed = []
        while len(freed) < max_pages:
            leaves = []
            stack = [self.root]
            while stack:
                n = stack.pop()
                for ch in n.children.values():
                    if not ch.children and ch.ref_count == 0:
                        leaves.append(ch)
                    else:
                        stack.append(ch)
            if not leaves:
                break
            t = min(leaves, key=lambda n: n.last_accessed)
            del t.parent.children[t.chunk_hash]
            t.parent = None
            freed.append(t.page)
        return freed

    def _count(self) -> int:
        n, stack = 0, [self.root]
        while stack:
            x = stack.pop()
            n += 1
            stack.extend(x.children.values())
        return n

    @property
    def total_cached_pages(self) -> int:
        return self._count() - 1

    @property
    def total_nodes(self) -> int:
        return self._count()

    def reset(self) -> list:
        """Drop every node; returns the pages the tree held."""
        pages = []
        stack = list(self.root.children.values())
        while stack:
            x = stack.pop()
            pages.append(x.page)
            stack.extend(x.children.values())
        self.root.children.clear()
        self._tick = 0
        return pages


class PagedKVCache:
    """Device K/V page pools of every layer plus the per-slot page tables."""

    def __init__(self, cfg, max_batch: int, max_ctx: int, page_size: int, n_pages: int, device):
        if page_size < 64 or page_size & (page_size - 1) or (cfg.head_dim == 64 and page_size < 128):
            raise ValueError("page_size must be a power of two >= 64 (>= 128 for head_dim 64)")
        self.cfg, self.P, self.max_batch, self.max_ctx = cfg, page_size, max_batch, max_ctx
        self.max_pages = -(-max_ctx // page_size)
        self.n_pages = n_pages
        rows = n_pages * page_size
        self.k = [torch.zeros((1, cfg.n_head_kv, rows, cfg.head_dim), dtype=torch.float16, device=device)
                  for _ in range(cfg.n_layer)]
        self.v = [torch.zeros_like(t) for t in self.k]
        self.pool = PagePool(n_pages, reserved=1)  # page 0: the idle rows' trash page
        self.trash_row = 0
        self.table_host = np.full((max_batch, self.max_pages), -1, np.int32)
        self.table = torch.full((max_batch, self.max_pages), -1, dtype=torch.int32, device=device)
        self.pages: list[list[int]] = [[] for _ in range(max_batch)]
        self.active = [False] * max_batch
        self._dirty = set()

    @property
    def page_bytes(self) -> int:
        """device bytes of one page over all layers, K and V"""
        c = self.cfg
        return 2 * c.n_layer * c.n_head_kv * self.P * c.head_dim * 2

    def active_bytes(self) -> int:
        return self.pool.used_count * self.page_bytes

    def _set(self, slot: int) -> None:
        row = self.table_host[slot]
        row[:] = -1
        row[:len(self.pages[slot])] = self.pages[slot]
        self._dirty.add(slot)

    def sync(self) -> None:
        """Copy the changed page-table rows to the device."""
        for slot in sorted(self._dirty):
            self.table[slot].copy_(torch.from_numpy(self.table_host[slot]))
        self._dirty.clear()

    def alloc_slot(self, slot: int) -> None:
        if self.active[slot]:
            self.free_slot(slot)
        self.active[slot] = True

    def free_slot(self, slot: int) -> None:
        for p in self.pages[slot]:
            self.pool.release(p)
        self.pages[slot] = []
        self.active[slot] = False
        self._set(slot)

    def map_existing_pages(self, slot: int, start_page: int, pages: list) -> None:
        """Share pages (e.g. a matched prefix) as pages start_page.. of the slot."""
        if start_page != len(self.pages[slot]):
            raise ValueError("shared pages must continue the slot's page list")
        for p in pages:
            self.pool.retain(p)
            self.pages[slot].append(int(p))
        self._set(slot)

    def ensure_tokens(self, slot: int, n_tokens: int, evict=None) -> None:
        """Give the slot pages for rows [0, n_tokens); evict(k) may drop up to k cached
        pages (returns how many it dropped) when the pool is empty."""
        need = -(-n_tokens // self.P)
        if need > self.max_pages:
            raise ValueError(f"{n_tokens} tokens exceed the slot's {self.max_pages * self.P} rows")
        while len(self.pages[slot]) < need:
            while self.pool.free_count == 0 and evict is not None and evict(1) > 0:
                pass
            self.pages[slot].append(self.pool.alloc())
        self._set(slot)

    def extract_page(self, slot: int, page_idx: int) -> int:
        return self.pages[slot][page_idx]


class BatchDecoder:
    """Prefill one sequence at a time into its pages; decode B slots per step, each at
    its own position, over the paged pools."""

    CTX_BUCKET = 512

    def __init__(self, w: ModelWeights, max_batch: int, max_ctx: int, page_size: int = 128,
                 n_pages: int | None = None, device=None, prefill_ubatch: int = 512):
        self.w, self.cfg = w, w.cfg
        self.dev = device if device is not None else w.embed.data.device
        self.max_batch, self.max_ctx, self.P = max_batch, max_ctx, page_size
        if n_pages is None:
            n_pages = max_batch * -(-max_ctx // page_size) + 1
        self.kv = PagedKVCache(self.cfg, max_batch, max_ctx, page_size, n_pages, self.dev)
        self.pre = Decoder(w, max_ctx, self.dev)  # contiguous prefill cache (one sequence at a time)
        self.ubatch = prefill_ubatch
        self.pos = torch.zeros(max_batch, dtype=torch.int32, device=self.dev)
        self.pos_host = np.zeros(max_batch, np.int64)
        self.ws = ops.Workspace(self.dev)
        self._bufs: dict[int, dict[str, torch.Tensor]] = {}
        self.graphs: dict[tuple[int, int], torch.cuda.CUDAGraph] = {}
        self._q8_chain: bool | None = None  # q8_chain_ok(w), computed on the first step
        self.use_q8 = True  # the int8 path's quantized-row handoffs when they apply (forward's q8)

    # -- prefill ----------------------------------------------------------------
    def prefill(self, slot: int, tokens, start: int = 0) -> torch.Tensor:
        """Compute rows [start, n) of the slot's sequence (rows [0, start) are already in
        its pages, e.g. a shared prefix) and store them into its pages; returns the last
        token's logits (device fp32 [vocab]). With start == n the last token is run again
        for its logits and nothing is stored (its row is already in a page)."""
        tokens = np.asarray(tokens, np.int32).reshape(-1)
        n = tokens.size
        if n == 0 or start > n or n > self.max_ctx:
            raise ValueError("prefill needs 0 <= start <= n <= max_ctx tokens")
        if len(self.kv.pages[slot]) * self.P < n:
            raise ValueError("the slot has no pages for its prompt (ensure_tokens first)")
        self.kv.sync()
        dec, pages = self.pre, self.kv.table[slot]
        first = start if start < n else n - 1
        for li in range(self.cfg.n_layer):  # the rows the prefill attends to but does not compute
            ops.kv_pages_copy(self.kv.k[li][0], dec.k_cache[li][0], pages, self.P, 0, first, to_pool=False)
            ops.kv_pages_copy(self.kv.v[li][0], dec.v_cache[li][0], pages, self.P, 0, first, to_pool=False)
        dec.reset(first)
        i, last_s = first, 0
        while i < n:
            s = min(self.ubatch, n - i)
            ids = torch.from_numpy(tokens[i:i + s].copy()).to(self.dev)
            dec.step(s, pad_kv_len(i + s, self.max_ctx), ids)
            i, last_s = i + s, s
        logits = dec._buffers(last_s)["logits"][0]
        for li in range(self.cfg.n_layer):
            ops.kv_pages_copy(self.kv.k[li][0], dec.k_cache[li][0], pages, self.P, start, n, to_pool=True)
            ops.kv_pages_copy(self.kv.v[li][0], dec.v_cache[li][0], pages, self.P, start, n, to_pool=True)
        for s_ in [k for k in dec._bufs if k not in (1, self.ubatch)]:  # odd tail sizes: do not keep
            del dec._bufs[s_]
        self.set_pos(slot, n)
        return logits

    def set_pos(self, slot: int, pos: int) -> None:
        self.pos_host[slot] = pos
        self.pos[slot:slot + 1].fill_(pos)

    # -- batched decode -------------------------------------------------------------
    def _buffers(self, B: int) -> dict[str, torch.Tensor]:
        if B not in self._bufs:
            c, d = self.cfg, self.dev
            f32 = dict(dtype=torch.float32, device=d)
            self._bufs[B] = {
                "ids": torch.zeros(B, dtype=torch.int32, device=d),
                "x": torch.empty((B, c.n_embd), **f32),
                "x_alt": torch.empty((B, c.n_embd), **f32),
                "h": torch.empty((B, c.n_embd), **f32),
                "qkv": torch.empty((B, c.q_dim + 2 * c.kv_dim), **f32),
                "q": torch.empty((1, B, c.n_head, c.head_dim), **f32),
                "k": torch.empty((1, B, c.n_head_kv, c.head_dim), **f32),
                "attn": torch.empty((B, c.n_head, c.head_dim), **f32),
                "proj": torch.empty((B, c.n_embd), **f32),
                "proj2": torch.empty((2, B, c.n_embd), **f32),  # a product's two halves of K
                "gu": torch.empty((B, 2 * c.n_ff), **f32),
                "act": torch.empty((B, c.n_ff), **f32),
                "logits": torch.empty((B, c.n_vocab), **f32),
                "next": torch.zeros(B, dtype=torch.int32, device=d),
                "kv_idx": torch.zeros(B, dtype=torch.int64, device=d),
                "seq_len": torch.zeros(B, dtype=torch.int32, device=d),
                "rope_cs": torch.zeros((B, c.head_dim), dtype=torch.float32, device=d),
                # the int8 path's quantized rows: the o projection's input, down's input
                "q8_o": torch.zeros(ops.q8_rows_bytes(c.q_dim), dtype=torch.uint8, device=d),
                "q8_d": torch.zeros(ops.q8_rows_bytes(c.n_ff), dtype=torch.uint8, device=d),
            }
        return self._bufs[B]

    def _ws_need(self, B: int, max_len: int) -> int:
        c, L = self.cfg, self.w.layers[0]
        need = [ops.mul_mat_workspace_size(wt, B) for wt in (L.qkv, L.o, L.gate_up, L.down, self.w.lm_head)]
        need.append(ops.flash_attn_paged_workspace_size(c.head_dim, B, c.n_head, c.n_head_kv, max_len, self.P))
        return max(need)

    def step(self, B: int, max_len: int, trace: list | None = None) -> torch.Tensor:
        """One decode token for slots [0, B): row b runs the token in this bucket's ids[b]
        at position pos[b], writes its K/V row into slot b's pages and attends to rows
        [0, pos[b]] of them; then pos[b] += 1. Returns next tokens (device int32 [B]);
        the logits stay in the bucket's "logits" [B, vocab]. max_len must bound every
        pos[b] + 1 (it sizes the attention launch)."""
        c, b, ws = self.cfg, self._buffers(B), self.ws
        if max_len > self.max_ctx:
            raise ValueError("max_len exceeds the slots' context")
        ws.get(self._ws_need(B, max_len))
        if self._q8_chain is None:
            self._q8_chain = q8_chain_ok(self.w)
        # 2..16 slots: the int8 chain with the quantized-row handoffs where it applies
        # (one row keeps the fused GEMV)
        q8 = (self.use_q8 and trace is None and 1 < B <= 16 and self._q8_chain and
              ops.paged_q8_ok(c.head_dim, B, c.n_head, c.n_head_kv, max_len, self.P))
        fused = B <= 4 and trace is None and not q8
        b["pos_ids"] = self.pos[:B]
        ops.paged_step_inputs(self.pos, self.kv.table, self.P, self.kv.trash_row, b["kv_idx"], b["seq_len"], B=B)
        scale = 1.0 / math.sqrt(c.head_dim)
        table = self.kv.table[:B]

        def attend(li, q, out_q8=None):
            return ops.flash_attn_paged(q[0].permute(1, 0, 2), self.kv.k[li][0], self.kv.v[li][0], table,
                                        b["seq_len"], self.P, max_len, scale, out=b["attn"], ws=ws, out_q8=out_q8)

        logits = forward(self.w, B, b, b["ids"], self.kv.k, self.kv.v, attend, fused, _Recorder(trace), ws,
                         b["logits"], 0, q8=q8)
        ops.argmax(logits, out=b["next"])
        ops.paged_advance(self.pos, B=B)
        return b["next"]

    def ctx_bucket(self, max_len: int) -> int:
        return min(self.max_ctx, -(-max_len // self.CTX_BUCKET) * self.CTX_BUCKET)

    def decode(self, B: int, tokens, live=None, use_graph: bool = True) -> np.ndarray:
        """Feed tokens[b] to slot b (b < B) and return the argmax of each row's logits
        (host int32 [B]); every slot b advances by one position. live: the slots whose
        results are used (default all B); the others must hold no pages."""
        b = self._buffers(B)
        b["ids"].copy_(torch.as_tensor(np.asarray(tokens, np.int32)[:B]))
        self.kv.sync()
        live = list(range(B)) if live is None else list(live)
        L = self.ctx_bucket(int(self.pos_host[live].max()) + 1 if live else 1)
        if use_graph:
            self.capture(B, L).replay()
        else:
            self.step(B, L)
        self.pos_host[:B] += 1
        return b["next"].cpu().numpy()

    def capture(self, B: int, max_len: int) -> torch.cuda.CUDAGraph:
        key = (B, max_len)
        if key in self.graphs:
            return self.graphs[key]
        self.ws.get(self._ws_need(B, max_len))
        saved = self.pos.clone()
        self.step(B, max_len)  # warm-up outside the graph
        torch.cuda.synchronize()
        self.pos.copy_(saved)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self.step(B, max_len)
        torch.cuda.synchronize()
        self.pos.copy_(saved)
        self.graphs[key] = g
        return g
