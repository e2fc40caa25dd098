"""Paged KV + continuous batching on the GPU (ggmlc_amd.paged, ggmlc_amd.batching).

* gq_flash_attn_paged against the exact softmax (float64, the query rounded to fp16 as
  in the CPU decode path) over each sequence's own pages — shared pages, ragged
  lengths, an empty sequence, garbage in every pool row a sequence does not own — and
  against gq_flash_attn_ext on the same rows gathered contiguously;
* the per-slot step inputs and the page copies, bit-exact;
* the batched decoder: every sequence of a batch (own position, pages shared with
  another sequence's prefix) against the reference ggml decoder graph run on that
  sequence alone (oracle.RefLlama), prefill and each decode step, at the end-to-end bar
  of tests/test_model.py (cosine >= 0.9999 on the tiny shapes);
* the scheduler: the reference's continuous-batching and prefix-caching scenarios
  (tests/e2e/test_continuous_batching.py, tests/e2e/test_prefix_caching.py), with every
  generated token checked against the reference graph fed the same tokens.
"""

from __future__ import annotations

import math
import os

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu


def _cos(a, b):
    a, b = np.asarray(a, np.float64).ravel(), np.asarray(b, np.float64).ravel()
    return float(a @ b / np.linalg.norm(a) / np.linalg.norm(b))


def _mar(got, want):
    return float(np.abs(np.asarray(got, np.float64) - want).max() / max(np.abs(want).max(), 1e-30))


def _exact(q, K, V, scale):
    """q [Hq, D] (fp16-rounded), K/V [Hkv, n, D] -> [Hq, D] in float64"""
    Hq, Hkv = q.shape[0], K.shape[0]
    out = np.zeros((Hq, q.shape[1]))
    if K.shape[1] == 0:
        return out
    for h in range(Hq):
        k, v = K[h // (Hq // Hkv)].astype(np.float64), V[h // (Hq // Hkv)].astype(np.float64)
        s = k @ q[h].astype(np.float64) * scale
        p = np.exp(s - s.max())
        out[h] = p @ v / p.sum()
    return out


def _init():
    import torch
    from ggmlc_amd import _lib

    _lib.check(_lib.load().gq_init())
    return torch.device("cuda")


@pytest.mark.parametrize("D,Hq,Hkv,P,lens", [
    (128, 12, 2, 128, [1, 127, 128, 129, 401, 0]),
    (128, 32, 32, 64, [64, 65, 200, 3]),
    (64, 15, 5, 128, [300, 1, 129, 128, 255]),
    (128, 8, 8, 256, [20]),                      # one split: the output is written directly
    (64, 4, 4, 256, [1000, 999, 513, 17, 256, 2, 700, 64]),
    (64, 32, 4, 128, [300, 1, 129, 0, 511]),     # 8 query heads per kv head (matrix-core kernel)
    (128, 16, 1, 256, [1000, 257, 3]),           # 16 per kv head, 256-row pages
    # 2..4 query heads per kv head on the matrix-core kernel
    (128, 12, 4, 128, [700, 1, 1300, 0, 129]),   # G = 3, the 12/4 x 128 shape
    (128, 16, 8, 256, [513, 900, 2, 256]),       # G = 2
    (64, 8, 4, 128, [300, 128, 0, 77]),          # G = 2, 64-dim heads
    (128, 16, 4, 128, [40, 17, 128, 99]),        # G = 4
    # one split (max_len <= 128): outputs written by the kernel itself, a sequence of
    # length 0 among them (zeros), into a NaN-filled output
    (128, 12, 4, 128, [100, 0, 128, 1]),         # G = 3
    (64, 8, 4, 128, [0, 64, 0]),                 # G = 2
    (128, 8, 2, 128, [3, 0]),                    # G = 4
])
def test_flash_attn_paged_vs_exact(D, Hq, Hkv, P, lens):
    import torch
    from ggmlc_amd import ops

    dev = _init()
    rng = np.random.default_rng(D + Hq + P + len(lens))
    B = len(lens)
    npg = [-(-n // P) for n in lens]
    max_pages = max(npg) + 1
    n_pages = 2 + sum(npg)
    rows = n_pages * P
    # every pool row starts as garbage (huge values and NaN); each sequence writes its own rows
    k_pool = np.full((Hkv, rows, D), np.float16(6.0e4), np.float16)
    v_pool = np.full((Hkv, rows, D), np.float16(np.nan), np.float16)
    perm = rng.permutation(np.arange(1, n_pages))
    table = np.full((B, max_pages), -1, np.int32)
    used = 0
    seqs = []
    for b, n in enumerate(lens):
        K = rng.standard_normal((Hkv, n, D)).astype(np.float16)
        V = rng.standard_normal((Hkv, n, D)).astype(np.float16)
        if b == 4 and lens[3] >= P and n >= P:  # sequence 4 shares sequence 3's first page
            K[:, :P], V[:, :P] = seqs[3][0][:, :P], seqs[3][1][:, :P]
            table[b, 0] = table[3, 0]
            own = range(1, npg[b])
        else:
            own = range(npg[b])
        for pi in own:
            table[b, pi] = perm[used]
            used += 1
        for r in range(n):
            pr = table[b, r // P] * P + r % P
            k_pool[:, pr], v_pool[:, pr] = K[:, r], V[:, r]
        seqs.append((K, V))
    q = rng.standard_normal((Hq, B, D)).astype(np.float32)
    scale = 1.0 / math.sqrt(D)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    out = torch.full((B, Hq, D), float("nan"), dtype=torch.float32, device=dev)
    out = ops.flash_attn_paged(t(q), t(k_pool), t(v_pool), t(table), t(np.array(lens, np.int32)), P, max(lens),
                               scale, out=out).cpu().numpy()
    q16 = q.astype(np.float16).astype(np.float32)
    worst = 0.0
    for b, n in enumerate(lens):
        want = _exact(q16[:, b], seqs[b][0], seqs[b][1], scale)
        if n == 0:
            assert np.all(out[b] == 0.0)
            continue
        worst = max(worst, _mar(out[b], want))
        # the same rows laid out contiguously through the unpaged kernel
        ref = ops.flash_attn_ext(t(q[:, b:b + 1]), t(seqs[b][0]), t(seqs[b][1]), None, scale).cpu().numpy()
        assert _mar(out[b], ref[0]) < 2e-6, b
    print(f"paged attention max-abs-rel vs exact {worst:.2e}")
    assert worst < 1e-5
    # the in-kernel split merge gives the bits of the separate merge launch
    with ops.separate_attn_merge():
        sep = ops.flash_attn_paged(t(q), t(k_pool), t(v_pool), t(table), t(np.array(lens, np.int32)), P, max(lens),
                                   scale).cpu().numpy()
    assert np.array_equal(sep, out, equal_nan=True)


@pytest.mark.parametrize("D,Hq,Hkv,lens,qtype", [
    (128, 12, 2, [2079, 3260, 1, 0, 652, 1167, 300, 945, 129, 128, 2105, 840, 763, 1452, 3882, 1174], O.Q8_0),
    (128, 12, 2, [700, 5, 1300, 257, 64, 900], O.Q8_0),
    (64, 32, 4, [500, 1, 129, 1000, 384], O.Q4_0),   # 8 q heads per kv head, K = 2048
    (128, 12, 4, [700, 0, 1300, 129, 3], O.Q8_0),    # 3 q heads per kv head, K = 1536
    (128, 16, 8, [900, 256, 5, 700, 130], O.Q4_0),   # 2 per kv head, K = 2048
])
def test_flash_attn_paged_q8_feeds_o_projection(D, Hq, Hkv, lens, qtype):
    """gq_flash_attn_paged_q8 writes the same fp32 rows as gq_flash_attn_paged and, from
    the split merge, those rows quantized for the output projection: the projection
    reading them (gq_mul_mat_fusion.b_q8) gives exactly the bits of MUL_MAT on the fp32
    rows (the int8 path's own prologue)."""
    import torch
    from ggmlc_amd import ops

    dev = _init()
    rng = np.random.default_rng(D + Hq + len(lens))
    P, B = 128, len(lens)
    npg = [-(-n // P) for n in lens]
    max_len = max(lens)
    n_pages = 1 + sum(npg)
    table = np.full((B, -(-max_len // P)), -1, np.int32)
    perm = rng.permutation(np.arange(1, n_pages))
    used = 0
    for b, n in enumerate(npg):
        table[b, :n] = perm[used:used + n]
        used += n
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    k_pool = t(rng.standard_normal((Hkv, n_pages * P, D)).astype(np.float16))
    v_pool = t(rng.standard_normal((Hkv, n_pages * P, D)).astype(np.float16))
    q = t(rng.standard_normal((Hq, B, D)).astype(np.float32))
    tb, sl = t(table), t(np.array(lens, np.int32))
    scale = 1.0 / math.sqrt(D)
    assert ops.paged_q8_ok(D, B, Hq, Hkv, max_len, P)
    want = ops.flash_attn_paged(q, k_pool, v_pool, tb, sl, P, max_len, scale)
    q8 = torch.full((ops.q8_rows_bytes(Hq * D),), 0x55, dtype=torch.uint8, device=dev)
    got = ops.flash_attn_paged(q, k_pool, v_pool, tb, sl, P, max_len, scale, out_q8=q8)
    g = torch.Generator(device=dev)
    g.manual_seed(B)
    w = ops.quantize_weights(torch.randn((1536, Hq * D), generator=g, device=dev) * 0.02, qtype)
    y_want = ops.mul_mat(w, want.view(B, Hq * D))
    y_got = ops.mul_mat_fused(w, got.view(B, Hq * D), x_q8=q8)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    assert torch.equal(y_got, y_want), (y_got - y_want).abs().max().item()
    # every row is written, those of sequences of length 0 included (zeros, quantized as
    # zeros), and a second call gives the same bits; quantized rows past B are written by
    # neither call, so both buffers start from the same bytes
    q8a = torch.full_like(q8, 0x5A)
    first = ops.flash_attn_paged(q, k_pool, v_pool, tb, sl, P, max_len, scale, out_q8=q8a)
    q8b = torch.full_like(q8, 0x5A)
    again = torch.full_like(first, float("nan"))
    ops.flash_attn_paged(q, k_pool, v_pool, tb, sl, P, max_len, scale, out=again, out_q8=q8b)
    torch.cuda.synchronize()
    assert torch.equal(again, first)
    assert torch.equal(q8b, q8a)


def test_paged_step_inputs_advance_and_copy():
    import torch
    from ggmlc_amd import ops

    dev = _init()
    P, B = 64, 4
    table = torch.tensor([[3, 1, -1], [2, -1, -1], [-1, -1, -1], [4, 5, 6]], dtype=torch.int32, device=dev)
    pos = torch.tensor([0, 63, 5, 130], dtype=torch.int32, device=dev)
    kv_idx = torch.zeros(B, dtype=torch.int64, device=dev)
    seq_len = torch.zeros(B, dtype=torch.int32, device=dev)
    ops.paged_step_inputs(pos, table, P, 7, kv_idx, seq_len)
    assert kv_idx.tolist() == [3 * 64, 2 * 64 + 63, 7, 6 * 64 + 2]
    assert seq_len.tolist() == [1, 64, 0, 131]
    pos[1] = 64  # past the slot's pages: the trash row
    ops.paged_step_inputs(pos, table, P, 7, kv_idx, seq_len)
    assert kv_idx.tolist()[1] == 7 and seq_len.tolist()[1] == 0
    ops.paged_advance(pos, torch.tensor([1, 0, 1, 1], dtype=torch.int32, device=dev))
    assert pos.tolist() == [1, 64, 6, 131]
    ops.paged_advance(pos)
    assert pos.tolist() == [2, 65, 7, 132]

    # rows [r0, r1) between a contiguous cache and pages [5, 2, 7] of a pool
    H, D, ctx = 3, 128, 192
    g = torch.Generator(device=dev).manual_seed(0)
    cache = torch.randn((H, ctx, D), generator=g, device=dev).half()
    pool = torch.zeros((H, 8 * P, D), dtype=torch.float16, device=dev)
    pages = torch.tensor([5, 2, 7], dtype=torch.int32, device=dev)
    ops.kv_pages_copy(pool, cache, pages, P, 10, 150, to_pool=True)
    rows = torch.tensor([[5, 2, 7][r // P] * P + r % P for r in range(10, 150)], device=dev)
    assert torch.equal(pool[:, rows], cache[:, 10:150])
    mask = torch.ones(8 * P, dtype=torch.bool, device=dev)
    mask[rows] = False
    assert torch.count_nonzero(pool[:, mask]) == 0
    back = torch.zeros_like(cache)
    ops.kv_pages_copy(pool, back, pages, P, 10, 150, to_pool=False)
    assert torch.equal(back[:, 10:150], cache[:, 10:150])
    assert torch.count_nonzero(back[:, :10]) == 0 and torch.count_nonzero(back[:, 150:]) == 0


def _model(cfg, seed=7):
    import torch
    from ggmlc_amd.model import host_weights, random_weights

    dev = _init()
    w = random_weights(cfg, dev, seed=seed)
    host = host_weights(w)
    torch.cuda.synchronize()
    return w, host


def _gqa_cfg(qtype, n_ff=512):
    from ggmlc_amd.model import LlamaConfig

    # configs[4]'s attention shape (12 q heads over 2 kv heads of 128) in a small model
    return LlamaConfig("tiny-gqa6", 2, 256, 12, 2, 128, n_ff, 512, qtype)


@pytest.mark.skipif(not O.ref_available(), reason="needs oracle/_ref")
@pytest.mark.parametrize("qtype", [O.Q8_0, O.Q4_0])
@pytest.mark.parametrize("B,graphs,q8", [(3, True, True), (3, True, False), (6, False, True), (6, True, True),
                                         (6, True, False)])
def test_batch_decoder_matches_reference_per_sequence(qtype, B, graphs, q8):
    """q8: 3..16 slots run the int8 chain with the quantized-row handoffs; without it 3
    slots run the fused GEMV layer stack and 6 the GEMM one with separate prologue and
    rope launches. Sequence 3 reuses sequence 1's first page (its prefix) and computes
    only its suffix."""
    from ggmlc_amd.paged import BatchDecoder

    cfg = _gqa_cfg(qtype)
    w, host = _model(cfg)
    P, max_ctx, n_new = 128, 1024, 4
    bd = BatchDecoder(w, max_batch=8, max_ctx=max_ctx, page_size=P)
    bd.use_q8 = q8
    rng = np.random.default_rng(5)
    lens = [37, 133, 300, 140, 260, 64][:B]
    prompts = [rng.integers(0, cfg.n_vocab, n).astype(np.int32) for n in lens]
    if B > 3:
        prompts[3][:P] = prompts[1][:P]
    refs = [O.RefLlama(cfg, host, max_ctx, n_threads=8) for _ in range(B)]
    tokens = np.zeros(B, np.int32)
    for b in range(B):
        bd.kv.alloc_slot(b)
        start = 0
        if b == 3:
            bd.kv.map_existing_pages(3, 0, [bd.kv.pages[1][0]])
            start = P
        bd.kv.ensure_tokens(b, lens[b] + n_new)
        got = bd.prefill(b, prompts[b], start).cpu().numpy()
        want, _ = refs[b].step(prompts[b])
        c = _cos(got, want)
        print(f"seq {b} prefill ({lens[b]} tokens, from row {start}): cos {c:.7f}")
        assert c >= 0.9999, (b, c)
        tokens[b] = int(np.argmax(got))
    if B > 3:  # slot 1 and slot 3 hold the shared page
        assert bd.kv.pool.refcount(bd.kv.pages[1][0]) == 2 and bd.kv.pages[3][0] == bd.kv.pages[1][0]
    for i in range(n_new):
        nxt = bd.decode(B, tokens, use_graph=graphs)
        logits = bd._buffers(B)["logits"].cpu().numpy()
        cs = []
        for b in range(B):
            want, _ = refs[b].step([int(tokens[b])])
            cs.append(_cos(logits[b], want))
            assert cs[-1] >= 0.9999, (i, b, cs[-1])
            assert nxt[b] == int(np.argmax(logits[b]))
        print(f"step {i}: min cos {min(cs):.7f}")
        tokens = nxt
    assert bd.pos_host[:B].tolist() == [n + n_new for n in lens]


@pytest.mark.parametrize("qtype,B,n_ff", [(O.Q8_0, 8, 512), (O.Q4_0, 5, 512), (O.Q8_0, 16, 512), (O.Q4_0, 16, 1024)])
def test_batch_decoder_q8_chain_bit_identical(qtype, B, n_ff):
    """The batched decode step with the quantized-row handoffs (rope in the QKV epilogue,
    the merge quantizing o's input, gate_up quantizing down's input; o, 1536 -> 256, and
    with n_ff 1024 down too, left in two halves of K for the next prologue's ADD) gives
    exactly the logits of the same step through the separate prologue and rope launches."""
    import torch
    from ggmlc_amd import ops
    from ggmlc_amd.paged import BatchDecoder

    cfg = _gqa_cfg(qtype, n_ff)
    w, _ = _model(cfg)
    P, max_ctx = 128, 1024
    rng = np.random.default_rng(11)
    lens = [int(n) for n in rng.integers(1, 700, B)]
    prompts = [rng.integers(0, cfg.n_vocab, n).astype(np.int32) for n in lens]
    decs = []
    for use_q8 in (False, True):
        bd = BatchDecoder(w, max_batch=B, max_ctx=max_ctx, page_size=P)
        bd.use_q8 = use_q8
        for b in range(B):
            bd.kv.alloc_slot(b)
            bd.kv.ensure_tokens(b, lens[b] + 3)
            bd.prefill(b, prompts[b])
        decs.append(bd)
    x = torch.empty((B, cfg.n_ff), device="cuda")
    assert ops.mul_mat_halves(w.layers[0].down, x, int8=True) == (n_ff == 1024)
    tokens = rng.integers(0, cfg.n_vocab, B).astype(np.int32)
    for i in range(3):
        outs = []
        for bd in decs:
            outs.append(bd.decode(B, tokens, use_graph=i > 0))
        l0, l1 = (bd._buffers(B)["logits"] for bd in decs)
        torch.cuda.synchronize()
        assert torch.equal(l0, l1), (i, (l0 - l1).abs().max().item())
        assert np.array_equal(outs[0], outs[1])
        tokens = outs[0]


def _near_argmax(tok, ref_logits, dev_frac=0.02):
    """the greedy token is the reference's argmax unless the reference's top two are
    closer than the pipeline's deviation (a few percent of the logits' spread)"""
    best = float(ref_logits.max())
    return tok == int(np.argmax(ref_logits)) or best - float(ref_logits[tok]) <= dev_frac * float(ref_logits.std())


def _check_against_reference(cfg, host, reqs, max_ctx):
    for r in reqs:
        ref = O.RefLlama(cfg, host, max_ctx, n_threads=8)
        logits, _ = ref.step(np.array(r.prompt_tokens, np.int32))
        for j, tok in enumerate(r.generated_tokens):
            assert _near_argmax(tok, logits), (r.request_id, j)
            if j + 1 < len(r.generated_tokens):
                logits, _ = ref.step([tok])


@pytest.mark.skipif(not O.ref_available(), reason="needs oracle/_ref")
def test_scheduler_continuous_batching():
    """tests/e2e/test_continuous_batching.py: three requests, a fourth admitted mid-flight,
    every request runs to max_new_tokens and no page stays allocated."""
    from ggmlc_amd.batching import ContinuousBatchScheduler
    from ggmlc_amd.paged import BatchDecoder

    cfg = _gqa_cfg(O.Q8_0)
    w, host = _model(cfg, seed=3)
    bd = BatchDecoder(w, max_batch=8, max_ctx=512, page_size=128)
    sched = ContinuousBatchScheduler(bd, max_batch_size=8, eos_token_id=-1)
    assert sched.max_batch_size() == 8
    r1 = sched.add_request([101], max_new_tokens=4)
    r2 = sched.add_request([202], max_new_tokens=8)
    r3 = sched.add_request([303, 7, 9], max_new_tokens=6)
    assert sched.pending_count() == 3 and sched.active_count() == 0
    steps, r4 = 0, None
    while sched.has_work():
        steps += 1
        if steps == 3:
            r4 = sched.add_request([404], max_new_tokens=5)
        sched.step()
        assert steps <= 30
    with pytest.raises(ValueError):  # token ids outside the vocabulary are refused
        sched.add_request([cfg.n_vocab], max_new_tokens=2)
    reqs = [sched.get_request(i) for i in (r1, r2, r3, r4)]
    for r in reqs:
        assert r.finished and r.finish_reason == "length" and len(r.generated_tokens) == r.max_new_tokens
        assert r.current_pos == len(r.prompt_tokens) + r.max_new_tokens - 1
    assert bd.kv.active_bytes() == 0
    _check_against_reference(cfg, host, reqs, 512)

    # an end-of-sequence token stops a request early
    eos = reqs[1].generated_tokens[2]
    r5 = sched.get_request(sched.add_request([202], max_new_tokens=8, eos_token_id=eos))
    while sched.has_work():
        sched.step()
    g5 = r5.generated_tokens
    print("eos", eos, "r2", reqs[1].generated_tokens, "r5", g5)
    assert r5.finished and eos not in g5[:-1]
    assert (r5.finish_reason == "stop" and g5[-1] == eos) or (r5.finish_reason == "length" and len(g5) == 8)
    if g5 == reqs[1].generated_tokens[:len(g5)]:  # the same greedy path as r2 stops where r2 met eos
        assert len(g5) == reqs[1].generated_tokens.index(eos) + 1


@pytest.mark.skipif(not O.ref_available(), reason="needs oracle/_ref")
def test_scheduler_prefix_caching():
    """tests/e2e/test_prefix_caching.py: a 128-token shared prefix (one page) computed by
    the first request is reused by the next three; a prompt that is exactly the cached
    page reruns only its last token; the tree keeps the page after the requests end."""
    from ggmlc_amd.batching import ContinuousBatchScheduler
    from ggmlc_amd.paged import BatchDecoder

    cfg = _gqa_cfg(O.Q8_0)
    w, host = _model(cfg, seed=4)
    bd = BatchDecoder(w, max_batch=8, max_ctx=512, page_size=128)
    sched = ContinuousBatchScheduler(bd, max_batch_size=8, eos_token_id=-1)
    sched.enable_prefix_caching(True)
    assert sched.is_prefix_caching_enabled()
    shared = [100 + (i % 300) for i in range(128)]
    rid1 = sched.add_request(shared + [401, 402], max_new_tokens=4)
    while sched.has_work():
        sched.step()
        if sched.get_request(rid1).current_pos >= 130:
            break
    assert sched.total_prefix_cache_hits == 0
    rids = [sched.add_request(shared + [k, k + 1], max_new_tokens=4) for k in (411, 421, 431)]
    sched.step()
    assert sched.total_prefix_cache_hits >= 3 and sched.total_prefix_tokens_saved >= 3 * 128
    for rid in rids:
        assert sched.get_request(rid).prefix_tokens_matched == 128
    while sched.has_work():
        sched.step()
    full = sched.get_request(sched.add_request(shared, max_new_tokens=3))  # the whole prompt is cached
    while sched.has_work():
        sched.step()
    assert full.prefix_tokens_matched == 128 and len(full.generated_tokens) == 3
    reqs = [sched.get_request(r) for r in [rid1] + rids] + [full]
    for r in reqs:
        assert r.finished and len(r.generated_tokens) == r.max_new_tokens
    assert sched.radix_tree.total_cached_pages == 1
    assert bd.kv.active_bytes() == bd.kv.page_bytes  # the tree's page
    _check_against_reference(cfg, host, reqs, 512)


@pytest.mark.skipif(not O.ref_available(), reason="needs oracle/_ref")
def test_scheduler_waits_for_pages_and_evicts():
    """A pool of 5 usable pages: a request that does not fit waits in the queue until
    pages come back; a cached prefix page no request holds is evicted for a new one."""
    from ggmlc_amd.batching import ContinuousBatchScheduler
    from ggmlc_amd.paged import BatchDecoder

    cfg = _gqa_cfg(O.Q8_0)
    w, host = _model(cfg, seed=5)
    bd = BatchDecoder(w, max_batch=4, max_ctx=512, page_size=128, n_pages=6)
    sched = ContinuousBatchScheduler(bd, max_batch_size=4, eos_token_id=-1)
    rng = np.random.default_rng(9)
    a = sched.add_request(rng.integers(0, cfg.n_vocab, 260).tolist(), max_new_tokens=4)  # 3 pages, 2 cached
    b = sched.add_request(rng.integers(0, cfg.n_vocab, 200).tolist(), max_new_tokens=250)  # 4 pages: must wait
    sched.step()
    assert sched.active_count() == 1 and sched.pending_count() == 1
    while sched.has_work():
        sched.step()
    ra, rb = sched.get_request(a), sched.get_request(b)
    assert ra.finished and rb.finished and len(rb.generated_tokens) == 250
    # a's two cached pages, one evicted for b, plus b's own full prompt page
    assert sched.radix_tree.total_cached_pages == 2
    assert bd.kv.pool.used_count == sched.radix_tree.total_cached_pages
    _check_against_reference(cfg, host, [ra, rb], 512)
