"""Host-side bookkeeping of the paged KV path (no GPU): the page pool's refcounts and
the prefix radix tree (runtime/src/radix_tree.cpp semantics: whole-page chunks, exact
token check behind the hash, LRU eviction of unreferenced leaves)."""

from __future__ import annotations

import pytest

from ggmlc_amd.paged import PagePool, PagedRadixTree


def test_page_pool_refcounts():
    pool = PagePool(5, reserved=1)
    assert pool.free_count == 4 and pool.used_count == 0
    a, b = pool.alloc(), pool.alloc()
    assert (a, b) == (1, 2) and pool.used_count == 2
    pool.retain(a)
    assert not pool.release(a) and pool.refcount(a) == 1
    assert pool.release(a) and pool.refcount(a) == 0
    with pytest.raises(ValueError):
        pool.release(a)
    with pytest.raises(ValueError):
        pool.retain(a)
    for _ in range(3):
        pool.alloc()
    with pytest.raises(MemoryError):
        pool.alloc()
    assert pool.refcount(0) == 0  # the reserved page is never handed out


def _fnv1a_bytes(data: bytes) -> int:
    h = 0xCBF29CE484222325
    for byte in data:
        h = ((h ^ byte) * 0x100000001B3) % (1 << 64)
    return h


def test_fnv1a_on_token_bytes():
    import numpy as np

    # the byte-wise FNV-1a against its published 64-bit test vectors ...
    assert _fnv1a_bytes(b"") == 0xCBF29CE484222325
    assert _fnv1a_bytes(b"a") == 0xAF63DC4C8601EC8C
    assert _fnv1a_bytes(b"foobar") == 0x85944171F73967E8
    # ... and the chunk hash is that function over the tokens' little-endian int32 bytes
    h = PagedRadixTree.hash_token_chunk
    for toks in ([], [0x64636261], [1, 2], [2, 1], [-1, 7, 1 << 30]):
        assert h(toks) == _fnv1a_bytes(np.asarray(toks, "<i4").tobytes())
    assert h([1, 2]) != h([2, 1])


def test_radix_match_insert_and_sharing():
    t = PagedRadixTree(4)
    prompt = list(range(10))  # 2 full pages + a tail of 2
    assert t.match_prefix(prompt).matched_pages == 0
    assert t.insert_prefix(prompt, 0, [11, 12, 13]) == [11, 12]  # the tail never forms a page
    assert t.total_cached_pages == 2 and t.total_nodes == 3
    m = t.match_prefix(list(range(8)) + [99])
    assert (m.matched_pages, m.matched_tokens, m.pages) == (2, 8, [11, 12])
    m = t.match_prefix([0, 1, 2, 3, 7, 7, 7, 7])
    assert m.pages == [11]
    # a second prompt sharing page 0 adds a branch; re-inserting a present chunk keeps its page
    assert t.insert_prefix([0, 1, 2, 3, 9, 9, 9, 9], 1, [21]) == [21]
    assert t.insert_prefix(prompt, 0, [31, 32]) == []
    assert t.total_cached_pages == 3
    # a start page that is not cached cannot attach
    assert t.insert_prefix([5, 5, 5, 5, 6, 6, 6, 6], 1, [41]) == []


def test_radix_hash_collision_is_a_miss():
    t = PagedRadixTree(2)
    t.insert_prefix([1, 2], 0, [5])
    node = next(iter(t.root.children.values()))
    # plant a node whose hash matches another chunk's hash: the exact check must reject it
    other = [3, 4]
    h = PagedRadixTree.hash_token_chunk(other)
    t.root.children[h] = type(node)((9, 9), h, 6, t.root, {}, 0, 0)
    assert t.match_prefix(other).matched_pages == 0
    assert t.insert_prefix(other, 0, [7]) == []


def test_radix_lru_eviction_respects_references():
    t = PagedRadixTree(2)
    t.insert_prefix([1, 1, 2, 2], 0, [1, 2])
    t.insert_prefix([3, 3], 0, [3])
    m = t.match_prefix([1, 1, 2, 2])
    for n in m.matched_nodes:
        t.retain_node(n)
    assert t.evict_lru(5) == [3]  # only the unreferenced leaf goes
    for n in m.matched_nodes:
        t.release_node(n)
    t.match_prefix([1, 1])  # touch the parent: the leaf below it is now the oldest
    assert t.evict_lru(1) == [2]
    assert t.evict_lru(1) == [1]
    assert t.total_nodes == 1 and t.evict_lru(1) == []
    t.insert_prefix([8, 8], 0, [4])
    assert t.reset() == [4] and t.total_cached_pages == 0


# ---- work list of the matrix-core paged attention kernel (k_attn_dec_mma) ---------
# Host model of paged_item (csrc/attention.hip): each wave takes the sequence lengths
# in chunks of 64 lanes, forms the inclusive prefix sum of every sequence's
# min(cdiv(len, 128), n_split) splits, and locates split number c = i // Hkv with a
# ballot of the lanes whose prefix ends at or before c.
def _paged_item(lens, n_split, hkv, i):
    c, hk = divmod(i, hkv)
    base = 0
    for b0 in range(0, len(lens), 64):
        n = [0] * 64
        for lane in range(64):
            b = b0 + lane
            ln = lens[b] if b < len(lens) else 0
            n[lane] = min(-(-ln // 128), n_split) if ln > 0 else 0
        x, acc = [], 0
        for lane in range(64):
            acc += n[lane]
            x.append(acc)
        tot = x[63]
        if c < base + tot:
            k = sum(1 for lane in range(64) if base + x[lane] <= c)
            assert k < 64 and b0 + k < len(lens) and n[k] > 0
            return b0 + k, hk, c - base - (x[k] - n[k])
        base += tot
    return None


@pytest.mark.parametrize("lens,max_len,hkv", [
    ([2079, 3260, 3543, 2835, 652, 1167, 2993, 945, 3521, 1587, 2105, 840, 763, 1452, 3882, 1174], 4096, 2),
    ([2048] * 16, 4096, 2),
    ([0, 1, 127, 128, 129, 0, 5000, -3], 4096, 1),  # empty, partial, exact, past max_len, negative
    ([(i * 37) % 900 for i in range(130)], 1024, 3),  # three chunks of 64 lanes
    ([0] * 5, 256, 2),
])
def test_paged_mma_work_list(lens, max_len, hkv):
    """Every (sequence, kv head, split below the sequence's length and the grid's split
    count) is exactly one item, items come first in the grid and the rest report the end."""
    n_split = -(-max_len // 128)
    grid = n_split * hkv * len(lens)
    want = {(b, h, sp) for b, ln in enumerate(lens) if ln > 0
            for sp in range(min(-(-ln // 128), n_split)) for h in range(hkv)}
    got, ended = [], False
    for i in range(grid):
        it = _paged_item(lens, n_split, hkv, i)
        if it is None:
            ended = True
            continue
        assert not ended, "an item after the end of the list"
        got.append(it)
    assert len(got) == len(set(got)) == len(want)
    assert set(got) == want
    # the kernel reads rows [split * 128, min(len, split * 128 + 128)): inside the sequence
    for b, _, sp in got:
        assert sp * 128 < lens[b] and sp < n_split
