"""Host model of the prefill GEMM's addressing (csrc/gemm.hip k_gemm): every global load
offset, LDS address and store index that a launch generates, for the shapes the GPU tests
and the configs run, checked against the buffer resources, the LDS allocation and the
output extents on the CPU.

It restates the kernel's index formulas (loader mapping, the PF-deep register ring and its
K-step sequence, the LDS tile layout, MFMA operand reads, epilogue) and the host plan
(gemm_plan: tile height and K splits), so a change to either is checked here before it
reaches a GPU.
"""

from __future__ import annotations

import numpy as np
import pytest

QK = 32
BN, BK, LDK = 128, 64, 72
OOB = 0x80000000
BLOCK = {8: 34, 2: 18}  # Q8_0, Q4_0 block bytes


def cdiv(a, b):
    return -(-a // b)


def gemm_plan(N, K, M, ncu=256):
    """gemm.hip gemm_bm + gemm_plan"""
    if M > 64 and cdiv(N, BN) >= 16:
        bm = 128
    else:
        bm = 64 if cdiv(N, BN) * cdiv(M, 128) < ncu else 128
    tiles, nk = cdiv(N, BN) * cdiv(M, bm), cdiv(K, BK)
    per_cu = 1 if bm == 128 else 2
    ks = 1
    if tiles < ncu:
        ks = min(cdiv(per_cu * ncu, tiles), nk // 4, 16)
    ks = max(ks, 1)
    spk = cdiv(nk, ks)
    return bm, cdiv(nk, spk), spk


def gemm_tail(N, K, M, ncu=256):
    """gemm.hip gemm_plan's tail round: (n_head, ks_tail, spk_tail), or None. When the last
    round of 128-token tiles would be at most half full, the weight rows from n_head on run
    as a second launch with K split."""
    bm = gemm_plan(N, K, M, ncu)[0]
    n_tiles, m_tiles, nk = cdiv(N, BN), cdiv(M, bm), cdiv(K, BK)
    tiles = n_tiles * m_tiles
    if bm != 128 or tiles <= ncu or ncu % m_tiles:
        return None
    head = tiles // ncu * (ncu // m_tiles)
    tail_tiles = (n_tiles - head) * m_tiles
    if tail_tiles <= 0 or 2 * tail_tiles > ncu:
        return None
    kt = min(ncu // tail_tiles, nk // 4, 4)
    if kt < 2:
        return None
    spk = cdiv(nk, kt)
    return head * BN, cdiv(nk, spk), spk


def launches(N, K, M, ncu=256):
    """the launches of one GEMM: (weight rows, bm, ks, spk), the head first"""
    bm, ks, spk = gemm_plan(N, K, M, ncu)
    t = gemm_tail(N, K, M, ncu)
    if t is None:
        return [(N, bm, ks, spk)]
    n_head, kt, spkt = t
    return [(n_head, bm, 1, cdiv(K, BK)), (N - n_head, bm, kt, spkt)]


PF = {128: 2, 64: 2}  # gemm.hip GEMM_PF_WS (k_gemm_ws), GEMM_PF_64 (k_gemm): K steps of loads in flight
LDS_MAX = 160 * 1024  # LDS of one workgroup on gfx950


def lds_bytes(bm):
    """one stage: sAh, sAl (BM x LDK halves), sB (BN x LDK halves), sD[2][BN] floats"""
    return (2 * bm * LDK + BN * LDK) * 2 + 2 * BN * 4


def stages(bm):
    """k_gemm_ws (128-token tiles) double-buffers its stage in dynamic LDS; k_gemm (64) has one"""
    return 2 if bm == 128 else 1


def check_launch(qt, N, K, M, plan=None):
    bm, ks, spk = plan if plan is not None else gemm_plan(N, K, M)
    bb = BLOCK[qt]
    row_bytes = (K // QK) * bb
    lda = 2 * K
    nb = K // QK
    aq = bm // 32
    mi = bm // 64
    sb = lds_bytes(bm)
    if stages(bm) == 1:
        assert sb <= 64 * 1024  # static LDS of one workgroup
    else:
        assert stages(bm) * sb <= LDS_MAX and sb % 16 == 0  # stage 1 starts 16-byte aligned
    # loader threads: all 256 threads of k_gemm, the 256 producer threads (waves 4-7) of k_gemm_ws
    tid = np.arange(256)
    lane, wave = tid & 63, tid >> 6
    wm, wn = wave >> 1, wave & 1
    lrow, lhalf = tid >> 1, tid & 1
    arow = tid // (8 // aq)
    apiece = (tid % (8 // aq)) * aq
    assert arow.max() < bm and (apiece + aq - 1).max() < 8
    a_bytes = M * lda * 2  # the activation workspace: M rows of lda halves
    # every offset grows with the tile index, so the first and last tiles of each grid
    # dimension bound the rest (every K step of every split is checked for them)
    for bx in sorted({0, cdiv(N, BN) - 1}):
        n0 = bx * BN
        w_base = n0 * row_bytes
        w_rec = min(N - n0, BN) * row_bytes
        assert w_base + w_rec <= N * row_bytes  # the weight resource stays inside W
        for by in sorted({0, cdiv(M, bm) - 1}):
            m0 = by * bm
            a_base = m0 * lda * 2
            a_rec = min(M - m0, bm) * lda * 2
            assert a_base + a_rec <= a_bytes and a_rec < 2**31 and w_rec < 2**31
            arow_off = arow * lda * 2
            wrow_off = lrow * row_bytes
            for bz in range(ks):
                kt0 = bz * spk
                kt1 = min(cdiv(K, BK), kt0 + spk)
                assert kt0 < kt1  # no empty split
                # every step the ring loads: kt0 .. kt1 + PF (prologue and refills)
                for kt in range(kt0, kt1 + PF[bm] + 1):
                    k = kt * BK + apiece * 8
                    av = (k < K) & (kt < kt1)
                    ao = np.where(av, arow_off + k * 2, OOB)
                    lo = np.where(av, ao + K * 2, OOB)
                    for i in range(aq):
                        for off in (ao + 16 * i, lo + 16 * i):
                            ok = off >= OOB
                            inb = off + 16 <= a_rec
                            assert np.all(ok | inb | (arow + m0 >= M)), (qt, N, K, M, kt)
                            # an in-range read stays inside its own row's hi / lo halves
                            rowok = (off - arow_off) + 16 <= lda * 2
                            assert np.all(ok | rowok)
                    kb = kt * 2 + lhalf
                    valid = (kb < nb) & (kt < kt1)
                    off = wrow_off + kb * bb
                    even = (off & 3) == 0
                    doff = np.where(valid, np.where(even, off, off + 2), OOB)
                    uoff = np.where(valid, np.where(even, off + (32 if qt == 8 else 16), off), OOB)
                    nw = 8 if qt == 8 else 4
                    for o, width in [(doff + 4 * (nw - 1), 4), (uoff, 2)]:
                        ok = o >= OOB
                        assert np.all(ok | (o + width <= w_rec) | (lrow + n0 >= N))
                        # the block read stays inside its row
                        assert np.all(ok | (o + width - wrow_off <= row_bytes))
                    assert np.all(~valid | (doff % 4 == 0))
    # LDS: tile writes and MFMA operand reads (halves within a tile, then bytes); with two
    # stages every address below is also taken at + sb, which stays inside 2 * sb
    if stages(bm) == 2:
        # parity of the stage parked by iteration kt and the one read in it never coincide
        for r in range(40):
            assert ((r + 1) & 1) != (r & 1)
    for i in range(aq):
        ah = (arow * LDK + apiece * 8 + 8 * i) * 2
        assert (ah + 16).max() <= bm * LDK * 2
    sbw = (lrow * LDK + lhalf * 32 + 8 * 3) * 2 + 16
    assert sbw.max() <= BN * LDK * 2
    sd = (lhalf * BN + lrow) * 4 + 4
    assert sd.max() <= 2 * BN * 4
    for kb in range(2):
        for h in range(2):
            kk = kb * 32 + h * 16 + 8 * (lane >> 5)
            for i in range(mi):
                ro = (wm * (bm // 2) + i * 32 + (lane & 31)) * LDK + kk
                assert (ro + 8).max() * 2 <= bm * LDK * 2
            for j in range(2):
                rb = (wn * 64 + j * 32 + (lane & 31)) * LDK + kk
                assert (rb + 8).max() * 2 <= BN * LDK * 2
        dwi = kb * BN + wn * 64 + 32 + (lane & 31)
        assert dwi.max() < 2 * BN
    # epilogue rows / columns are guarded by m < M, n < N (the row scales rs[m] are read for
    # m < M only); partial tiles by z < ks
    m = np.arange(M)
    assert np.all(m * 4 + 4 <= M * 4)
    return bm, ks


def workspace_layout(N, K, M):
    """api.hip plan_mul_mat for the fp16 GEMM path: the hi + lo rows (M x 2K halves), the
    row scales (M floats) and the split-K partials, each 256-byte aligned"""
    r256 = lambda b: (b + 255) & ~255  # noqa: E731
    ws_rs = r256(M * K * 4)
    ws_act = ws_rs + r256(M * 4)
    bm, ks, spk = gemm_plan(N, K, M)
    part = ks * M * N * 4 if ks > 1 else 0
    t = gemm_tail(N, K, M)
    if t is not None:
        part = t[1] * M * (N - t[0]) * 4
    return ws_rs, ws_act, ws_act + r256(part)


@pytest.mark.parametrize("qt,N,K,M", [(2, 4096, 4096, 512), (2, 96, 11008, 17), (8, 1600, 960, 37), (2, 96, 17408, 17),
                                     (2, 12288, 4096, 512)])
def test_gemm_workspace_regions_disjoint(qt, N, K, M):
    ws_rs, ws_act, total = workspace_layout(N, K, M)
    assert M * 2 * K * 2 <= ws_rs  # the activation rows end before the row scales
    assert ws_rs + M * 4 <= ws_act  # the row scales end before the partials
    assert ws_rs % 256 == 0 and ws_act % 256 == 0
    # the library sizes the workspace the same way (no device: 256 CUs assumed, as here)
    from ggmlc_amd import _lib

    lib = _lib.load()
    bb = BLOCK[qt]
    w = _lib.make_tensor(0x1000, _lib.Q8_0 if qt == 8 else _lib.Q4_0, [K, N], [bb, K // QK * bb])
    x = _lib.make_tensor(0x1000, _lib.F32, [K, M], [4, 4 * K])
    assert lib.gq_mul_mat_workspace_size(w, x) == total


SHAPES = [
    (2, 64, 1024, 5),      # the shape a pipelined variant once faulted on
    (2, 12288, 4096, 512), (2, 4096, 4096, 512), (2, 22016, 4096, 512), (2, 4096, 11008, 512),
    (2, 32000, 4096, 37), (8, 1600, 960, 512), (8, 5120, 960, 512), (8, 960, 2560, 512),
    (8, 2048, 1536, 16), (8, 17920, 1536, 8), (8, 1536, 8960, 16), (8, 151936, 1536, 7),
    (2, 4096, 4096, 5), (2, 4096, 4096, 129), (8, 256, 512, 70), (2, 96, 64, 3),
]


@pytest.mark.parametrize("qt,N,K,M", SHAPES)
def test_gemm_addresses_in_bounds(qt, N, K, M):
    # each launch of the GEMM addresses its own weight rows (the tail launch: from n_head,
    # with the output and bias offset the same way) over the same activation
    for n, bm, ks, spk in launches(N, K, M):
        check_launch(qt, n, K, M, (bm, ks, spk))


def test_gemm_tail_round_plans():
    """7B qkv at M = 512: 384 tiles = 256 + 128; the 128 (32 tile columns x 4 token tiles)
    run with K split 2 ways; gate_up's last round (176 of 256) stays whole"""
    assert launches(12288, 4096, 512) == [(8192, 128, 1, 64), (4096, 128, 2, 32)]
    assert gemm_tail(22016, 4096, 512) is None
    assert gemm_tail(4096, 4096, 512) is None  # 128 tiles: one round, K split as before
    for n, bm, ks, spk in launches(12288, 4096, 512):
        assert n % BN == 0 and ks * spk >= cdiv(4096, BK)


def ws_schedule(kt0, kt1, pf):
    """k_gemm_ws's loop structure restated: the producers' ring loads and parks and the
    consumers' reads, per barrier interval. Returns (producer barriers, consumer barriers,
    intervals), each interval a dict of the step parked (and its stage) and the step read."""
    ring = {}
    intervals = [{"park": None, "read": None}]
    for s in range(pf):  # prologue loads
        ring[s] = kt0 + s
    intervals[0]["park"] = (ring[0], 0)
    ring[0] = kt0 + pf
    pbar = 1

    def iter_(kt, slot):
        nonlocal pbar
        intervals.append({"park": (ring[slot], (kt + 1 - kt0) & 1), "read": None})
        assert ring[slot] == kt + 1  # the slot holds the step being parked
        ring[slot] = kt + 1 + pf
        pbar += 1

    kt = kt0
    while kt + pf <= kt1:
        for s in range(pf):
            iter_(kt + s, (s + 1) % pf)
        kt += pf
    for s in range(pf - 1):
        if kt + s < kt1:
            iter_(kt + s, (s + 1) % pf)
    cbar = 1
    for kt in range(kt0, kt1):
        intervals[cbar]["read"] = (kt, (kt - kt0) & 1)
        cbar += 1
    return pbar, cbar, intervals


@pytest.mark.parametrize("pf", [1, 2, 3, 4])
def test_gemm_ws_schedule(pf):
    for kt0 in (0, 3, 16):
        for n in range(1, 40):
            kt1 = kt0 + n
            pbar, cbar, iv = ws_schedule(kt0, kt1, pf)
            assert pbar == cbar == n + 1  # both roles pass the same barriers
            parked = {}
            for i, d in enumerate(iv):
                if d["read"] is not None:
                    step, buf = d["read"]
                    assert parked[buf] == step  # parked in an earlier interval, not overwritten since
                    assert d["park"][1] != buf  # the stage being parked is not the one being read
                if d["park"] is not None:
                    parked[d["park"][1]] = d["park"][0]
            reads = [d["read"][0] for d in iv if d["read"] is not None]
            assert reads == list(range(kt0, kt1))
