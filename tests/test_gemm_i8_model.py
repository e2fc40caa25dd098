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
    """gemm_i8.hip gemm_i8_plan"""
    tiles, nsteps = cdiv(N, 16), K // (QK * NBS)
    ks = 1
    if tiles < 512 and nsteps >= 4:
        ks = 4
    elif tiles < 4096 and nsteps >= 4:
        ks = 2
    return ks, cdiv(tiles, 4 // ks)


def wave_range(bx, wave, ks, nsteps):
    tile = bx * (4 // ks) + wave // ks
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
    ks, wgs = plan(N, K)
    lane = np.arange(64)
    g, lr = lane >> 4, lane & 15
    stage_bytes = 16 * rb
    # every wave of every workgroup: the first and last workgroups bound the rest (offsets
    # grow with the tile), plus one in the middle
    seen_parts = {}
    for bx in sorted({0, wgs // 2, wgs - 1}):
        for wave in range(4):
            tile, kp, s0, s1 = wave_range(bx, wave, ks, nsteps)
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
    return ks, wgs


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
    ks, wgs = plan(N, K)
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
        for wave in range(4):
            tile, kp, s0, s1 = wave_range(bx, wave, ks, nsteps)
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
