"""Host model of the int8-MFMA MUL_MAT for 5..16 activation rows (csrc/gemm_i8.hip k_gemm_i8,
csrc/quantize.hip act_prep_i8): the launch plan, every global offset, LDS address and store
index a launch generates (checked against the buffer resources, the LDS arrays and the
output extents), and a numpy emulation of a whole launch's data path - the LDS image of the
staged row segments, each lane's 8 operand bytes, v_mfma_i32_16x16x32_i8's lane layout (A:
lane l = row l % 16, K 8 (l / 16) ..; D: column l % 16, rows 4 (l / 16) ..; checked on the
GPU), the Q4_0 nibble correction and the per-block scale fmas - against the block formula of
ggml's vec_dot (isum exact, then isum * (d_w * d_x) accumulated in fp32).

All CPU; a change to the kernel's index formulas is checked here before a GPU runs it.
"""

from __future__ import annotations

import numpy as np
import pytest

QK, NBS = 32, 8
BLOCK = {8: 34, 2: 18}  # Q8_0, Q4_0
OOB = 0x80000000


def cdiv(a, b):
    return -(-a // b)


def plan(N, K):
    """gemm_i8.hip gemm_i8_plan: (K parts, waves per workgroup, workgroups)"""
    tiles, nsteps = cdiv(N, 16), K // (QK * NBS)
    ks, waves = 1, 4
    if tiles < 512 and nsteps >= 4:
        ks = 4
    elif tiles < 4096 and nsteps >= 4:
        ks = 2
    return ks, waves, cdiv(tiles, waves // ks)


def halves(N, K):
    """gemm_i8.hip gemm_i8_halves: plain products of at most 128 tiles in 4 K parts"""
    return plan(N, K)[0] == 4 and cdiv(N, 16) <= 128


def half_range(spl, bx, wave, nsteps, ks=4):
    """k_gemm_i8's steps of a wave with SPL (1: 8 waves per tile; 2: two workgroups per
    tile, bx & 1 the half): (tile, half, part within the half, s0, s1)"""
    parts = ks * (2 if spl == 1 else 1)
    tile = (bx >> 1 if spl == 2 else bx) * (4 // ks) + wave // parts
    kp = wave % parts
    half = bx & 1 if spl == 2 else kp // ks
    kh = kp % ks if spl == 1 else kp
    nhs = (nsteps + 1) // 2
    hbeg = half * nhs
    hend = min(nsteps, hbeg + nhs)
    sp = cdiv(nhs, ks)
    s0 = min(hend, hbeg + kh * sp)
    return tile, half, kh, s0, min(hend, s0 + sp)


def wave_range(bx, wave, ks, nsteps, waves=4):
    tile = bx * (waves // ks) + wave // ks
    kp = wave % ks
    sp = cdiv(nsteps, ks)
    s0 = min(nsteps, kp * sp)
    return tile, kp, s0, min(nsteps, s0 + sp)


def check_addresses(qt, N, K, M):
    bb = BLOCK[qt]
    rb = NBS * bb
    cpr = rb // 16
    cpw = 16 * cpr
    lpl = cdiv(cpw, 64)
    nb = K // QK
    nsteps = nb // NBS
    row_bytes = nb * bb
    assert K % 256 == 0 and rb % 16 == 0 and row_bytes == nsteps * rb and row_bytes % 16 == 0
    ks, waves, wgs = plan(N, K)
    lane = np.arange(64)
    g, lr = lane >> 4, lane & 15
    stage_bytes = 16 * rb
    # every wave of every workgroup: the first and last workgroups bound the rest (offsets
    # grow with the tile), plus one in the middle
    seen_parts = {}
    for bx in sorted({0, wgs // 2, wgs - 1}):
        for wave in range(waves):
            tile, kp, s0, s1 = wave_range(bx, wave, ks, nsteps, waves)
            seen_parts.setdefault(tile, []).append((kp, s0, s1))
            n0 = tile * 16
            rows = N - n0
            w_bytes = min(rows, 16) * row_bytes if rows > 0 else 0
            # weight chunks: every step the ring issues, s0 .. s1 + 1 (prologue and refills)
            for i in range(lpl):
                c = lane + 64 * i
                cval = c < cpw
                coff = np.where(cval, (c // cpr) * row_bytes + (c % cpr) * 16, 0)
                for s in range(s0, s1 + 2):
                    live = s < s1
                    off = np.where(live & cval, coff + s * rb, OOB)
                    ok = off >= OOB
                    assert np.all(ok | (off + 16 <= w_bytes) | ((c // cpr) + n0 >= N)), (qt, N, K, tile, s)
                    assert np.all(ok | (off % 16 == 0))
                    assert np.all(off < 2**32)
                # park: LDS chunk c of the wave's slice
                assert np.all(~cval | (c * 16 + 16 <= stage_bytes))
            # activation operand, scales, block sums
            for s in range(s0, s1 + 2):
                live = s < s1
                for b in range(NBS):
                    e = (s * NBS + b) * 16 + lr
                    qo = np.where(live, e * 32 + 8 * g, OOB)
                    do = np.where(live, e * 4, OOB)
                    assert np.all((qo >= OOB) | (qo + 8 <= nb * 512))
                    assert np.all((do >= OOB) | (do + 4 <= nb * 64))
                    assert np.all((qo >= OOB) | (qo % 8 == 0))
    # LDS operand reads of a step
    gq = g if qt == 8 else (g & 1)
    for b in range(NBS):
        rp = lr * rb + b * bb + 2 + 8 * gq
        if b % 2 == 0:
            base = rp - 2
            assert np.all(base % 4 == 0) and np.all(base + 12 <= stage_bytes)
        else:
            assert np.all(rp % 4 == 0) and np.all(rp + 8 <= stage_bytes)
        for r in range(4):
            dwo = (4 * g + r) * rb + b * bb
            assert np.all(dwo % 2 == 0) and np.all(dwo + 2 <= stage_bytes)
    # the K parts of a tile cover every step once
    for tile, parts in seen_parts.items():
        if len(parts) == ks:
            steps = sorted(s for _, s0, s1 in parts for s in range(s0, s1))
            assert steps == list(range(nsteps))
    return ks, waves, wgs


SHAPES = [
    (8, 2048, 1536, 16), (8, 1536, 1536, 16), (8, 17920, 1536, 16), (8, 1536, 8960, 16), (8, 151936, 1536, 16),
    (2, 4096, 4096, 8), (2, 12288, 4096, 8), (2, 22016, 4096, 8), (2, 4096, 11008, 8), (2, 32000, 4096, 8),
    (8, 100, 512, 5), (2, 37, 256, 7), (8, 16, 2048, 16), (2, 1000, 8192, 12),
]


@pytest.mark.parametrize("qt,N,K,M", SHAPES)
def test_gemm_i8_addresses_in_bounds(qt, N, K, M):
    check_addresses(qt, N, K, M)


# ---- data path ------------------------------------------------------------------------

def f16(x):
    return np.float16(x)


def make_weights(qt, N, K, rng):
    """raw block rows: [d (fp16 LE)][quants] per block"""
    nb = K // QK
    bb = BLOCK[qt]
    raw = np.zeros((N, nb * bb), np.uint8)
    d = (rng.random((N, nb)) * 0.02 + 1e-3).astype(np.float16)
    if qt == 8:
        q = rng.integers(-128, 128, (N, nb, 32)).astype(np.int8)
        vals = q.astype(np.int64)
    else:
        nib = rng.integers(0, 16, (N, nb, 32)).astype(np.uint8)
        vals = nib.astype(np.int64) - 8
    for b in range(nb):
        raw[:, b * bb:b * bb + 2] = np.ascontiguousarray(d[:, b]).view(np.uint8).reshape(N, 2)
        if qt == 8:
            raw[:, b * bb + 2:b * bb + 34] = np.ascontiguousarray(q[:, b]).view(np.uint8)
        else:
            # byte j: quant j in the low nibble, quant j + 16 in the high nibble
            raw[:, b * bb + 2:b * bb + 18] = nib[:, b, :16] | (nib[:, b, 16:] << 4)
    return raw, d, vals


def make_act(M, K, rng):
    """the i8 layout of act_prep_i8 for quantized rows: quants, scales, block sums"""
    nb = K // QK
    qx = rng.integers(-127, 128, (M, nb, 32)).astype(np.int8)
    dx = (rng.random((M, nb)) * 0.05 + 1e-3).astype(np.float16).astype(np.float32)
    buf = np.zeros(nb * 640, np.uint8)
    qv = buf[:nb * 512].reshape(nb, 16, 32)
    dv = buf[nb * 512:nb * 576].view(np.float32).reshape(nb, 16)
    sv = buf[nb * 576:].view(np.int32).reshape(nb, 16)
    for m in range(M):
        qv[:, m, :] = np.ascontiguousarray(qx[m]).view(np.uint8)
        dv[:, m] = dx[m]
        sv[:, m] = qx[m].astype(np.int64).sum(1)
    # rows M..15 hold garbage in a reused workspace: fill them so that they must not leak
    qv[:, M:, :] = 0x5a
    dv[:, M:] = np.float32(1e30)
    sv[:, M:] = 123456
    return buf, qx, dx


def emulate(qt, N, K, M, wraw, act):
    """k_gemm_i8's arithmetic, lane by lane, in the kernel's order"""
    bb = BLOCK[qt]
    rb = NBS * bb
    nb = K // QK
    nsteps = nb // NBS
    row_bytes = nb * bb
    ks, waves, wgs = plan(N, K)
    flat = wraw.reshape(-1)
    qv = act[:nb * 512].reshape(nb, 16, 32).view(np.int8)
    dv = act[nb * 512:nb * 576].view(np.float32).reshape(nb, 16)
    sv = act[nb * 576:].view(np.int32).reshape(nb, 16)
    lane = np.arange(64)
    g, lr = lane >> 4, lane & 15
    gq = g if qt == 8 else (g & 1)
    nsh = np.zeros(64, np.int64) if qt == 8 else 4 * (g >> 1)
    out = np.zeros((M, N), np.float32)
    for bx in range(wgs):
        parts = {}
        for wave in range(waves):
            tile, kp, s0, s1 = wave_range(bx, wave, ks, nsteps, waves)
            n0 = tile * 16
            acc = np.zeros((64, 4), np.float32)
            for s in range(s0, s1):
                # the wave's LDS slice: 16 row segments of rb bytes (rows past N read 0)
                stage = np.zeros(16 * rb, np.uint8)
                for r in range(16):
                    n = n0 + r
                    if n < N:
                        stage[r * rb:(r + 1) * rb] = flat[n * row_bytes + s * rb:n * row_bytes + (s + 1) * rb]
                for b in range(NBS):
                    kb = s * NBS + b
                    rp = lr * rb + b * bb + 2 + 8 * gq
                    wop = np.stack([stage[rp + e] for e in range(8)], 1).astype(np.int64)  # [lane][8]
                    if qt == 2:
                        wop = (wop >> nsh[:, None]) & 0xF
                    else:
                        wop = wop.astype(np.uint8).view(np.int8).astype(np.int64)
                    A = np.zeros((16, 32), np.int64)
                    B = np.zeros((32, 16), np.int64)
                    for l in range(64):
                        A[l % 16, 8 * (l // 16):8 * (l // 16) + 8] = wop[l]
                        B[8 * (l // 16):8 * (l // 16) + 8, l % 16] = qv[kb, l % 16, 8 * (l // 16):8 * (l // 16) + 8]
                    D = A @ B  # D[i = weight row][j = activation row]
                    dx = dv[kb, lr]
                    for r in range(4):
                        i = 4 * g + r
                        isum = D[i, lr] if qt == 8 else D[i, lr] - 8 * sv[kb, lr].astype(np.int64)
                        dw = np.frombuffer(stage[(i * rb + b * bb)[:, None] + np.arange(2)].tobytes(),
                                           np.float16).astype(np.float32)
                        with np.errstate(over="ignore", invalid="ignore"):
                            acc[:, r] = np.float32(isum.astype(np.float32) * (dw * dx)) + acc[:, r]
            parts[wave] = (tile, kp, acc)
        for wave, (tile, kp, acc) in parts.items():
            if kp != 0:
                continue
            tot = acc.copy()
            for k in range(1, ks):
                tot = tot + parts[wave + k][2]
            n0 = tile * 16
            for l in range(64):
                m = l % 16
                if m >= M:
                    continue
                for r in range(4):
                    n = n0 + 4 * (l // 16) + r
                    if n < N:
                        out[m, n] = tot[l, r]
    return out


@pytest.mark.parametrize("qt", [8, 2])
@pytest.mark.parametrize("N,K,M", [(40, 512, 5), (16, 2048, 16), (70, 1024, 9)])
def test_gemm_i8_emulated_data_path_matches_block_formula(qt, N, K, M):
    rng = np.random.default_rng(N * 7 + K + M + qt)
    wraw, dw, wvals = make_weights(qt, N, K, rng)
    act, qx, dx = make_act(M, K, rng)
    got = emulate(qt, N, K, M, wraw, act)
    # ggml's block formula in float64: sum_b isum * d_w * d_x
    isum = np.einsum("nbj,mbj->mnb", wvals, qx.astype(np.int64))
    ref = (isum * dw.astype(np.float64)[None, :, :] * dx.astype(np.float64)[:, None, :]).sum(-1)
    np.testing.assert_allclose(got, ref, rtol=2e-6, atol=1e-6 * np.abs(ref).max())


# ---- paired epilogues (rope, SWIGLU) and the quantized SWIGLU rows ----------------------

def pair_row(lo, h, r):
    """epilogue.h pair_row: logical row r -> physical row"""
    if lo == 0:
        return r
    return (r & ~lo) + ((r & lo) >> 1) + (r & 1) * h


@pytest.mark.parametrize("N,K,qt,lo,h", [
    (17920, 1536, 8, ~0, 8960),          # Qwen2.5-1.5B gate|up: SWIGLU pairs (c, c + N/2)
    (22016, 4096, 2, ~0, 11008),         # 7B gate|up
    (2048, 1536, 8, 127, 64),            # Qwen2.5-1.5B QKV: NEOX pairs of 128-dim heads
    (12288, 4096, 2, 127, 64),           # 7B QKV
    (1024, 1024, 2, 63, 32),             # 64-dim heads
    (1024, 2048, 8, 0, 0),               # normal rope: adjacent pairs, the identity
])
def test_paired_weight_rows_in_bounds(N, K, qt, lo, h):
    """k_gemm_i8 with a paired epilogue: tile n0's resource starts at physical row
    pbase = pair_row(n0) and spans (N - pbase) rows; every chunk offset stays inside it,
    the logical -> physical map is a bijection of [0, N), and a lane's rows 4g .. 4g + 3 are
    two whole pairs (even logical row and its partner)."""
    bb = BLOCK[qt]
    row_bytes = K // QK * bb
    rb = NBS * bb
    cpr = rb // 16
    assert N % 16 == 0
    phys = [pair_row(lo, h, r) for r in range(N)]
    assert sorted(phys) == list(range(N))
    for n0 in range(0, N, 16):
        pbase = pair_row(lo, h, n0)
        wbytes = (N - pbase) * row_bytes
        assert wbytes < 2**31
        rows = [pair_row(lo, h, n0 + r) for r in range(16)]
        assert min(rows) == pbase
        for c in range(16 * cpr):
            off = (rows[c // cpr] - pbase) * row_bytes + (c % cpr) * 16 + (K // 256 - 1) * rb
            assert 0 <= off and off + 16 <= wbytes
        for g in range(4):  # the lane's two pairs
            for p in range(2):
                row = n0 + 4 * g + 2 * p
                if lo == ~0:
                    assert phys[row + 1] == phys[row] + h
                elif lo:
                    assert phys[row + 1] == phys[row] + h and phys[row] // (lo + 1) == phys[row + 1] // (lo + 1)


@pytest.mark.parametrize("N,M", [(17920, 16), (17920, 5), (22016, 9), (1024, 16)])
def test_quantized_swiglu_rows_in_bounds(N, M):
    """EPI_GLU_Q8: workgroup b writes quant block b of every row m < M: 2 quant bytes per
    lane at (b * 16 + m) * 32 + 8 wave + 2 g, the scale and block sum after all quants,
    inside gq_q8_rows_bytes(N / 2); the blocks of all workgroups tile the layout."""
    Kq = N // 2
    nbq = Kq // 32
    size = nbq * 640
    assert N % 64 == 0 and N // 64 == nbq
    seen = set()
    for b in range(N // 64):
        for m in range(M):
            e = b * 16 + m
            for wave in range(4):
                for g in range(4):
                    o = e * 32 + 8 * wave + 2 * g
                    assert o % 2 == 0 and o + 2 <= nbq * 512
                    seen.update((o, o + 1))
            assert nbq * 512 + e * 4 + 4 <= nbq * 576 and nbq * 576 + e * 4 + 4 <= size
    assert len(seen) == (N // 64) * M * 32


@pytest.mark.parametrize("nsteps,ord_", [(6, 2), (6, 4), (35, 4), (3, 4), (5, 2), (16, 8)])
def test_emulated_split_order_equals_the_split(nsteps, ord_):
    """ORD: one wave walking every step, folding its sum at the part boundaries k * sp and
    adding the parts in order (empty ones 0), gives the float32 bits of the ord_-part
    launch, whose waves sum their own steps and are then added in part order."""
    rng = np.random.default_rng(nsteps * 10 + ord_)
    contrib = (rng.standard_normal((nsteps, 8)) * 10.0 ** rng.integers(-3, 3, (nsteps, 8))).astype(np.float32)
    sp = cdiv(nsteps, ord_)
    # the split launch
    parts = []
    for k in range(ord_):
        s0, s1 = min(nsteps, k * sp), min(nsteps, k * sp + sp)
        acc = np.zeros(8, np.float32)
        for s in range(s0, s1):
            acc = np.float32(acc + contrib[s])
        parts.append(acc)
    want = parts[0]
    for k in range(1, ord_):
        want = np.float32(want + parts[k])
    # the one-wave emulation (k_gemm_i8's fold)
    part = [np.zeros(8, np.float32) for _ in range(ord_)]
    acc = np.zeros(8, np.float32)
    for s in range(nsteps):
        for k in range(1, ord_):
            if s == k * sp:
                part[k - 1], acc = acc, np.zeros(8, np.float32)
        acc = np.float32(acc + contrib[s])
    part[(nsteps - 1) // sp] = acc
    got = part[0]
    for k in range(1, ord_):
        got = np.float32(got + part[k])
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("nsteps", [4, 5, 6, 7, 9, 35, 64])
def test_emulated_halves_order_equals_the_halves(nsteps):
    """SPL with ORD = 8 (one-part launches: the quantized SWIGLU rows): one wave walking
    every step, folding at the starts of the 8 parts of K's two halves (empty parts start
    where the next one does: the fold cascades in part order), then (half 0's parts in
    order) + (half 1's parts in order), gives the float32 bits of the halves over waves
    (8 waves, or two workgroups whose slabs are added)."""
    rng = np.random.default_rng(nsteps)
    contrib = (rng.standard_normal((nsteps, 8)) * 10.0 ** rng.integers(-3, 3, (nsteps, 8))).astype(np.float32)
    # the waves: part kh of half h sums steps half_range(...) from 0
    sums = {}
    for wave in range(8):
        _, h, kh, s0, s1 = half_range(1, 0, wave, nsteps)
        acc = np.zeros(8, np.float32)
        for s in range(s0, s1):
            acc = np.float32(acc + contrib[s])
        sums[(h, kh)] = acc
    a0, a1 = sums[(0, 0)], sums[(1, 0)]
    for k in range(1, 4):
        a0, a1 = np.float32(a0 + sums[(0, k)]), np.float32(a1 + sums[(1, k)])
    want = np.float32(a0 + a1)
    # the one-wave fold (k_gemm_i8's pstart / fold / kl)
    nhs = (nsteps + 1) // 2
    spo = cdiv(nhs, 4)

    def pstart(k):
        return min(nhs, k * spo) if k < 4 else min(nsteps, nhs + (k - 4) * spo)

    part = [np.zeros(8, np.float32) for _ in range(8)]
    acc = np.zeros(8, np.float32)
    for s in range(nsteps):
        for k in range(1, 8):
            if s == pstart(k):
                part[k - 1], acc = acc, np.zeros(8, np.float32)
        acc = np.float32(acc + contrib[s])
    kl = max([0] + [k for k in range(1, 8) if pstart(k) <= nsteps - 1])
    part[kl] = acc
    b0, b1 = part[0], part[4]
    for k in range(1, 4):
        b0, b1 = np.float32(b0 + part[k]), np.float32(b1 + part[4 + k])
    got = np.float32(b0 + b1)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_plan_of_the_configs():
    """the launch shapes of the configs' batched-decode products"""
    assert plan(2048, 1536) == (4, 4, 128)       # Qwen2.5-1.5B qkv
    assert plan(1536, 1536) == (4, 4, 96)        # o
    assert plan(17920, 1536) == (2, 4, 560)      # gate|up
    assert plan(1536, 8960) == (4, 4, 96)        # down
    assert plan(151936, 1536) == (1, 4, 2374)    # tied head
    assert plan(4096, 11008) == (4, 4, 256)      # 7B down


def test_halves_plan_of_the_configs():
    """the configs[4] o and down (96 tiles) take K in halves, QKV (128 tiles) would as a
    plain product; gate|up, the head and the 7B products (256 tiles and more) do not, nor
    products of fewer than 4 steps"""
    assert halves(1536, 1536) and halves(1536, 8960) and halves(2048, 1536)
    assert not halves(17920, 1536) and not halves(151936, 1536) and not halves(4096, 11008)
    assert not halves(4096, 4096) and not halves(256, 768)
    assert halves(2048, 1024) and not halves(2064, 1024)


@pytest.mark.parametrize("nsteps", [4, 5, 6, 7, 35, 64])
@pytest.mark.parametrize("spl", [1, 2])
def test_halves_cover_every_step_once(nsteps, spl):
    """every tile's waves (8 in one workgroup, or 4 in each of two) cover each step once:
    half 0 is the first ceil(steps / 2) steps, half 1 the rest, each in 4 consecutive
    parts in wave order (which is the order the sums are added in)"""
    tiles = 3
    wgs = tiles * (2 if spl == 2 else 1)
    waves = 8 if spl == 1 else 4
    seen = {t: [] for t in range(tiles)}
    for bx in range(wgs):
        for wave in range(waves):
            tile, half, kh, s0, s1 = half_range(spl, bx, wave, nsteps)
            assert 0 <= tile < tiles and 0 <= s0 <= s1 <= nsteps
            seen[tile].append((half, kh, s0, s1))
    nhs = (nsteps + 1) // 2
    for t, rs in seen.items():
        rs.sort()
        assert [(h, k) for h, k, _, _ in rs] == [(h, k) for h in range(2) for k in range(4)]
        steps = [s for _, _, s0, s1 in rs for s in range(s0, s1)]
        assert steps == list(range(nsteps))  # once each, in (half, part) order
        assert all(s1 <= nhs for h, _, _, s1 in rs if h == 0) and all(s0 >= nhs for h, _, s0, _ in rs if h == 1)


def staged_copy(qt, K, lac=10, lmh=8):
    """k_gemm_i8's compact activation copy (LMH rows of every block, LAC pieces per thread):
    per piece q of the 256 threads, the workspace offset it loads (None: OOB) and the LDS
    byte it stores to."""
    nb = K // QK
    qp, sp = lmh * 2, lmh // 4
    ppb = qp + sp * (2 if qt == 2 else 1)
    nq, ns = nb * qp, nb * sp
    out = []
    for i in range(lac):
        for t in range(256):
            q = t + 256 * i
            if q < nq:
                off = (q // qp) * 512 + (q % qp) * 16
            elif q < nq + ns:
                off = nb * 512 + ((q - nq) // sp) * 64 + ((q - nq) % sp) * 16
            else:
                off = nb * 576 + ((q - nq - ns) // sp) * 64 + ((q - nq - ns) % sp) * 16
            out.append((None if q >= nb * ppb else off, q * 16))
    return out


@pytest.mark.parametrize("qt,K", [(2, 4096), (8, 4096), (2, 256), (8, 3840), (2, 2048)])
def test_staged_activation_copy_and_reads(qt, K):
    """The copy stays inside the workspace's bytes and the LDS buffer, and every operand the
    steps read from it (quants, scale, block sum of (block, row) for rows < 8; rows 8..15 read
    row - 8) is the byte the per-step loads take from the workspace."""
    nb = K // QK
    lac, lmh = 10, 8
    abytes = nb * (640 if qt == 2 else 576)
    rng = np.random.default_rng(K + qt)
    ws = rng.integers(0, 256, size=nb * 640, dtype=np.uint8)
    lds = np.zeros(lac * 4096, dtype=np.uint8)
    for off, dst in staged_copy(qt, K, lac, lmh):
        assert dst + 16 <= lds.size
        if off is None:
            continue  # reads 0 (out of the resource), lands in the slack
        assert 0 <= off and off + 16 <= abytes
        lds[dst:dst + 16] = ws[off:off + 16]
    assert nb * lmh * (40 if qt == 2 else 36) <= lds.size
    lane = np.arange(64)
    g, lr = lane >> 4, lane & 15
    lra = lr & (lmh - 1)
    for s in range(nb // NBS):
        for b in range(NBS):
            e = (s * NBS + b) * lmh + lra          # compact (block, row)
            ef = (s * NBS + b) * 16 + lra          # the workspace's (block, row)
            for j in range(8):
                assert np.array_equal(lds[e * 32 + 8 * g + j], ws[ef * 32 + 8 * g + j])
            for j in range(4):
                assert np.array_equal(lds[nb * lmh * 32 + e * 4 + j], ws[nb * 512 + ef * 4 + j])
                if qt == 2:
                    assert np.array_equal(lds[nb * lmh * 36 + e * 4 + j], ws[nb * 576 + ef * 4 + j])
            assert (e * 32 + 8 * g + 8 <= nb * lmh * 32).all()
            assert (nb * lmh * 36 + e * 4 + 4 <= nb * lmh * 40).all()
