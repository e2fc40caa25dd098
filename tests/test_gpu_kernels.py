"""Parity of the HIP path (through the C ABI) with the oracle and the reference's
golden vectors. Needs an MI355X.

Bars: quantize_row_q8_0 and set_rows bit-exact; mul_mat within max-abs-rel 1e-5
(max|d| / max|ref|; the north star asks 1e-3: both paths form every block product
exactly, so only fp32 accumulation order differs); attention within 1e-3 of the exact
softmax, and within the reference's own deviation from it when compared to
the reference (its decode path accumulates V in fp16).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from ggmlc_amd import ops

pytestmark = pytest.mark.gpu

DEV = "cuda"


def mar(a, b):
    """max-abs-rel: max|a - b| / max|b|"""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


def f16(a):
    return np.asarray(a, np.float32).astype(np.float16).view(np.uint16)


def to_dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def qweight(wq: np.ndarray, qtype: int, K: int) -> ops.QWeight:
    return ops.QWeight(to_dev(wq), qtype, K)


@pytest.fixture(scope="module", autouse=True)
def _init():
    from ggmlc_amd import _lib

    _lib.check(_lib.load().gq_init())
    yield
    torch.cuda.synchronize()


# ------------------------------------------------------------ quantizers ---

def test_quantize_row_q8_0_golden(golden_dir):
    g = np.load(golden_dir / "quantize_q8_0.npz")
    got = ops.quantize_row_q8_0(to_dev(g["x"])).cpu().numpy()
    assert np.array_equal(got, g["q"])


@pytest.mark.parametrize("shape,scale", [((1, 4096), 1.0), ((512, 4096), 1.0), ((8, 11008), 30.0),
                                         ((3, 960), 1e-3), ((64, 2560), 1e-6)])
def test_quantize_row_q8_0_vs_oracle(shape, scale):
    rng = np.random.default_rng(hash(shape) % 2**32)
    x = (rng.standard_normal(shape) * scale).astype(np.float32)
    x[0, :64] = np.round(x[0, :64] * 4) / 4
    x[-1, :32] = 0
    got = ops.quantize_row_q8_0(to_dev(x)).cpu().numpy()
    assert np.array_equal(got, O.quantize_row_q8_0(x))


@pytest.mark.parametrize("qtype", [O.Q8_0, O.Q4_0])
def test_quantize_weights_vs_oracle(qtype):
    rng = np.random.default_rng(qtype)
    w = (rng.standard_normal((300, 1024)) * 0.02).astype(np.float32)
    w[0, :32] = 0
    w[1, :32] = np.round(w[1, :32] * 500) / 500
    got = ops.quantize_weights(to_dev(w), qtype).data.cpu().numpy()
    assert np.array_equal(got, O.quantize_weights(w, qtype))


# --------------------------------------------------------------- mul_mat ---

def test_mul_mat_golden(golden_dir):
    files = sorted(golden_dir.glob("mul_mat_*.npz"))
    assert files
    for f in files:
        g = np.load(f)
        K = int(g["K"])
        w = qweight(g["w"], int(g["wtype"]), K)
        y = ops.mul_mat(w, to_dev(g["x"])).cpu().numpy()
        r = mar(y, g["y"])
        print(f.name, f"{r:.2e}")
        assert r < 1e-5, (f.name, r)


def _check_mm(qtype, K, N, M, rows_checked=256, seed=0):
    rng = np.random.default_rng(seed)
    w = (torch.randn((N, K), generator=torch.Generator().manual_seed(seed)) * 0.02).to(DEV)
    qw = ops.quantize_weights(w.contiguous(), qtype)
    x = rng.standard_normal((M, K)).astype(np.float32)
    y = ops.mul_mat(qw, to_dev(x)).cpu().numpy()
    sel = np.sort(rng.choice(N, size=min(rows_checked, N), replace=False))
    sel[-1] = N - 1
    wq_sel = qw.data.cpu().numpy()[sel]
    msel = np.unique(np.concatenate([[0, M - 1], rng.choice(M, size=min(M, 64), replace=False)]))
    want = O.mul_mat(wq_sel, qtype, K, x[msel])
    r = mar(y[np.ix_(msel, sel)], want)
    print(f"qtype={qtype} K={K} N={N} M={M}: max-abs-rel {r:.2e}")
    assert r < 1e-5
    return r


@pytest.mark.parametrize("M", [1, 2, 3, 4])
def test_gemv_c1_q8_0(M):
    """config 1: Linear 4096 -> 4096, Q8_0 (decode GEMV)."""
    _check_mm(O.Q8_0, 4096, 4096, M)


@pytest.mark.parametrize("M", [1, 8, 128, 512])
def test_mlp_c2_q4_0(M):
    """config 2: SwiGLU MLP 4096/11008, Q4_0: fused gate_up 4096 -> 22016, down 11008 -> 4096."""
    _check_mm(O.Q4_0, 4096, 22016, M, seed=1)
    _check_mm(O.Q4_0, 11008, 4096, M, seed=2)


@pytest.mark.parametrize("qtype", [O.Q8_0, O.Q4_0])
@pytest.mark.parametrize("K,N,M", [(960, 1600, 1), (960, 5120, 3), (2560, 960, 1), (960, 960, 37),
                                   (1536, 2048, 16), (8960, 1536, 1), (256, 130, 5), (32, 7, 2),
                                   (8960, 1536, 16), (1536, 17920, 12),
                                   # 5..16 rows on int8 MFMA: row tails, K split in 1, 2 and 4 parts
                                   (2048, 100, 9), (4096, 33, 13), (11008, 300, 16), (4096, 16500, 6),
                                   # a last round of tiles run as its own launch with K split
                                   # (7B qkv at 512 tokens: 2 ways; Qwen2.5 gate|up: 4 ways)
                                   (4096, 12288, 512), (1536, 17920, 512)])
def test_mul_mat_shapes(qtype, K, N, M):
    _check_mm(qtype, K, N, M, seed=K + N + M)


def _big_rows(M, K, seed):
    """Activations whose blocks reach past the fp16 range of d * q on some rows: a block at
    amax 3e4 (no row scale needed), 7e4 and 1e6 (row scales 2 and 32), 8e6 (128: the largest
    finite fp16 block scale is 65504), a row whose other blocks sit 1e-3 low (wide range
    inside one row) and ordinary N(0, 1) rows."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((M, K)).astype(np.float32)
    nb = K // 32
    for m, amax in zip(range(M), (3e4, 7e4, 1e6, 8e6, 1e6, 7e4)):
        b = int(rng.integers(nb))
        blk = x[m, 32 * b:32 * b + 32]
        x[m, 32 * b:32 * b + 32] = blk / np.abs(blk).max() * np.float32(amax)
    if M > 4:
        x[4] *= np.float32(1e-3)
        b = int(rng.integers(nb))
        x[4, 32 * b:32 * b + 32] = np.linspace(-1e6, 1e6, 32, dtype=np.float32)
    return x


@pytest.mark.parametrize("qtype", [O.Q8_0, O.Q4_0])
@pytest.mark.parametrize("K,N,M", [(4096, 1024, 17), (4096, 1024, 128), (11008, 1024, 512), (11008, 96, 17),
                                   (4096, 300, 3), (4096, 300, 9),
                                   (17408, 96, 17)])  # K past the one-launch prologue: two-pass row scales
def test_mul_mat_large_activations(qtype, K, N, M):
    """Activation blocks with amax up to 8e6 (where d * q leaves the fp16 range) on every
    path: the GEMV (M <= 4), int8 MFMA (5..16) and the fp16 MFMA GEMM (row scales, split K at
    N = 96), within 1e-5 of the oracle and finite."""
    g = torch.Generator(device=DEV)
    g.manual_seed(K + N + M)
    qw = ops.quantize_weights(torch.randn((N, K), generator=g, device=DEV) * 0.02, qtype)
    x = _big_rows(M, K, K + M)
    y = ops.mul_mat(qw, to_dev(x)).cpu().numpy()
    assert np.isfinite(y).all()
    want = O.mul_mat(qw.data.cpu().numpy(), qtype, K, x)
    for m in range(min(M, 6)):  # each large row at the bar on its own
        r = mar(y[m], want[m])
        assert r < 1e-5, (m, r)
    r = mar(y, want)
    print(f"qtype={qtype} K={K} N={N} M={M}: max-abs-rel {r:.2e}")
    assert r < 1e-5


@pytest.mark.parametrize("K,N,M", [(4096, 1024, 17), (11008, 512, 128)])
def test_mul_mat_fused_large_activations(K, N, M):
    """The GEMM's fused prologues with inputs past the fp16 range of d * q: ADD (x + d of two
    large rows) and SWIGLU (silu(g) * u up to ~1e6) give the bits of the separate ops, which
    are within 1e-5 of the oracle."""
    g = torch.Generator(device=DEV)
    g.manual_seed(K + N)
    w = ops.quantize_weights(torch.randn((N, K), generator=g, device=DEV) * 0.02, O.Q4_0)
    x = to_dev(_big_rows(M, K, 1))
    d = to_dev(_big_rows(M, K, 2) * np.float32(0.03))  # sums below 127 * 65504 wherever the blocks meet
    got = ops.mul_mat_fused(w, x, x_add=d, x_sum=torch.empty_like(x))
    s = ops.add(x, d)
    want = ops.mul_mat(w, s)
    assert torch.equal(got, want)
    r = mar(want.cpu().numpy(), O.mul_mat(w.data.cpu().numpy(), O.Q4_0, K, s.cpu().numpy()))
    assert r < 1e-5, r
    gate = to_dev(np.random.default_rng(3).standard_normal((M, K)).astype(np.float32) * np.float32(3))
    up = to_dev(_big_rows(M, K, 4) * np.float32(0.05))  # |silu(g) * u| up to ~5e6 < 127 * 65504
    gu = torch.cat([gate, up], dim=1).contiguous()
    got = ops.mul_mat_fused(w, gu, x_swiglu=True)
    sw = ops.swiglu(gate, up)
    assert float(sw.abs().max()) > 7e4
    want = ops.mul_mat(w, sw)
    assert torch.equal(got, want)
    r = mar(want.cpu().numpy(), O.mul_mat(w.data.cpu().numpy(), O.Q4_0, K, sw.cpu().numpy()))
    assert r < 1e-5, r
    assert torch.isfinite(got).all()


def test_mul_mat_strided_rows():
    """src1 with a row stride wider than K (a view) and batch dims."""
    K, N = 512, 96
    rng = np.random.default_rng(4)
    w = (torch.randn((N, K), generator=torch.Generator().manual_seed(4)) * 0.02).to(DEV)
    qw = ops.quantize_weights(w, O.Q8_0)
    big = rng.standard_normal((2, 3, K + 64)).astype(np.float32)
    xt = to_dev(big)[:, :, :K]
    y = ops.mul_mat(qw, xt).cpu().numpy()
    want = O.mul_mat(qw.data.cpu().numpy(), O.Q8_0, K, big[:, :, :K].reshape(-1, K)).reshape(2, 3, N)
    assert mar(y, want) < 1e-5


@pytest.mark.parametrize("qtype,K,N,M,rms,glu,add", [
    (O.Q4_0, 4096, 12288, 1, True, False, False),   # 7B qkv: RMS_NORM -> MUL_MAT
    (O.Q4_0, 4096, 22016, 1, True, True, False),    # 7B gate_up: RMS_NORM -> MUL_MAT -> SWIGLU
    (O.Q4_0, 11008, 4096, 1, False, False, True),   # 7B down: MUL_MAT -> ADD (in place)
    (O.Q4_0, 4096, 4096, 3, True, False, True),     # three rows, both ends fused
    (O.Q8_0, 960, 5120, 1, True, True, False),      # K % 256 != 0 (block-wise kernel)
    (O.Q8_0, 2560, 960, 2, False, False, True),     # SmolLM2 down shape
    (O.Q8_0, 8960, 1536, 1, False, False, True),    # split-K over waves (KS = 4)
    (O.Q8_0, 8192, 1536, 1, True, True, False),     # split-K (KS = 2) with SWIGLU pairs
    (O.Q4_0, 4096, 4096, 4, True, True, False),
])
@pytest.mark.parametrize("pre_add", [False, True])
def test_mul_mat_fused_bit_identical_to_unfused(qtype, K, N, M, rms, glu, add, pre_add):
    """gq_mul_mat_fused gives exactly the bits of RMS_NORM / MUL_MAT / SWIGLU / ADD run
    one by one (those are pinned against the oracle above)."""
    g = torch.Generator(device=DEV)
    g.manual_seed(K + N + M)
    w = ops.quantize_weights(torch.randn((N, K), generator=g, device=DEV) * 0.02, qtype)
    x = torch.randn((M, K), generator=g, device=DEV) * 3.0
    eps = 1e-5
    xin = x
    if pre_add:  # ADD(x, d) feeding the node; the sum is stored for later nodes
        d = torch.randn((M, K), generator=g, device=DEV)
        x_sum_want = ops.add(x, d)
        xin = x_sum_want
    h = ops.rms_norm(xin, eps) if rms else xin
    y = ops.mul_mat(w, h)
    if glu:
        want = ops.swiglu(y)
    elif add:
        r = torch.randn((M, N), generator=g, device=DEV)
        want = ops.add(r, y)
    else:
        want = y
    kw = dict(rms_eps=eps if rms else None)
    x_sum = None
    if pre_add:
        x_sum = torch.full_like(x, float("nan"))
        kw.update(x_add=d, x_sum=x_sum)
    if add:
        got = r.clone()
        ops.mul_mat_fused(w, x, out=got, add=got, **kw)  # in place
    else:
        got = ops.mul_mat_fused(w, x, swiglu=glu, **kw)
    torch.cuda.synchronize()
    assert got.shape == want.shape
    assert torch.equal(got, want), (got - want).abs().max().item()
    if pre_add:
        assert torch.equal(x_sum, x_sum_want)


@pytest.mark.parametrize("qtype,K,N,M,mode", [
    (O.Q4_0, 4096, 12288, 37, "rms"),        # 7B QKV prefill rows: RMS_NORM in the prologue
    (O.Q4_0, 4096, 22016, 64, "add_rms"),    # 7B gate_up after the residual ADD
    (O.Q8_0, 1536, 2048, 16, "add_rms"),     # Qwen2.5-1.5B QKV at batch 16 (split K)
    (O.Q8_0, 8960, 1536, 16, "swiglu"),      # Qwen2.5-1.5B down: SWIGLU of gate|up in front
    (O.Q4_0, 11008, 4096, 9, "swiglu"),      # 7B down, 9 rows
    (O.Q8_0, 960, 960, 5, "add_rms"),        # K = 960 (not a multiple of 64)
    (O.Q4_0, 14336, 64, 6, "rms"),           # K near the prologue's limit
])
def test_mul_mat_fused_gemm_prologue_bit_identical(qtype, K, N, M, mode):
    """More than 4 rows: ADD / RMS_NORM / SWIGLU fused into the prologue that quantizes
    the GEMM's activation give exactly the bits of the ops run one by one."""
    g = torch.Generator(device=DEV)
    g.manual_seed(K + N + M)
    w = ops.quantize_weights(torch.randn((N, K), generator=g, device=DEV) * 0.02, qtype)
    eps = 1e-5
    if mode == "swiglu":
        gu = torch.randn((M, 2 * K), generator=g, device=DEV) * 2.0
        want = ops.mul_mat(w, ops.swiglu(gu))
        got = ops.mul_mat_fused(w, gu, x_swiglu=True)
    else:
        x = torch.randn((M, K), generator=g, device=DEV) * 3.0
        kw = dict(rms_eps=eps)
        xin = x
        if mode == "add_rms":
            d = torch.randn((M, K), generator=g, device=DEV)
            x_sum_want = ops.add(x, d)
            xin = x_sum_want
            x_sum = torch.full_like(x, float("nan"))
            kw.update(x_add=d, x_sum=x_sum)
        want = ops.mul_mat(w, ops.rms_norm(xin, eps))
        got = ops.mul_mat_fused(w, x, **kw)
        if mode == "add_rms":
            torch.cuda.synchronize()
            assert torch.equal(x_sum, x_sum_want)
    torch.cuda.synchronize()
    assert got.shape == want.shape
    assert torch.equal(got, want), (got - want).abs().max().item()


@pytest.mark.parametrize("qtype,K,Hq,Hkv,hd,M,mode,n_dims", [
    (O.Q4_0, 4096, 32, 32, 128, 1, 2, 128),   # 7B QKV (MHA)
    (O.Q8_0, 1536, 12, 2, 128, 3, 2, 128),    # Qwen2.5-1.5B QKV (GQA 6), three tokens
    (O.Q8_0, 960, 15, 5, 64, 2, 2, 64),       # SmolLM2 QKV: K = 960, block-wise kernel
    (O.Q4_0, 1024, 4, 2, 128, 4, 0, 96),      # normal rope, partial n_dims, four tokens
    (O.Q8_0, 1536, 12, 2, 128, 16, 2, 128),   # batch 16: the int8 MFMA GEMM's epilogue, K in parts
    (O.Q4_0, 1024, 8, 2, 64, 7, 2, 64),       # int8 path, 64-dim NEOX heads, 7 tokens
    (O.Q4_0, 4096, 32, 32, 128, 5, 0, 128),   # int8 path, normal rope (adjacent pairs), 7B MHA
    (O.Q8_0, 2048, 4, 2, 128, 9, 0, 96),      # int8 path, normal rope with partial n_dims
])
@pytest.mark.parametrize("cached", [False, True])
def test_mul_mat_fused_rope_kv_bit_identical(qtype, K, Hq, Hkv, hd, M, mode, n_dims, cached):
    """The QKV product with the rope + KV-store epilogue (the GEMV for up to 4 tokens, the
    int8 MFMA GEMM for 5..16) gives exactly the bits of RMS_NORM -> MUL_MAT ->
    gq_rope_kv_store (pinned by the decoder-op tests): q_out, both caches (untouched rows
    included) and the count of out-of-range rows."""
    g = torch.Generator(device=DEV)
    g.manual_seed(K + Hq + M)
    N = (Hq + 2 * Hkv) * hd
    w = ops.quantize_weights(torch.randn((N, K), generator=g, device=DEV) * 0.02, qtype)
    x = torch.randn((M, K), generator=g, device=DEV) * 3.0
    d = torch.randn((M, K), generator=g, device=DEV)
    pos = torch.arange(700, 700 + M, dtype=torch.int32, device=DEV)
    idx = torch.tensor(([5, 63, -1, 64] + list(range(6, 60, 4)))[:M], dtype=torch.int64, device=DEV)
    kc1 = torch.randn((1, Hkv, 64, hd), generator=g, device=DEV).half()
    vc1 = torch.randn((1, Hkv, 64, hd), generator=g, device=DEV).half()
    kc2, vc2 = kc1.clone(), vc1.clone()
    bad1 = torch.zeros(1, dtype=torch.int32, device=DEV)
    bad2 = torch.zeros(1, dtype=torch.int32, device=DEV)
    eps = 1e-5
    # unfused: ADD, RMS_NORM, MUL_MAT, then the rope/set_rows node
    y = ops.mul_mat(w, ops.rms_norm(ops.add(x, d), eps))
    qv = y[:, :Hq * hd].view(1, M, Hq, hd)
    kv = y[:, Hq * hd:(Hq + Hkv) * hd].view(1, M, Hkv, hd)
    vv = y[:, (Hq + Hkv) * hd:].view(1, M, Hkv, hd)
    q1 = torch.empty((1, M, Hq, hd), device=DEV)
    ops.rope_kv_store(qv, kv, vv, pos, n_dims, mode, 10000.0, idx, q1, kc1, vc1, n_bad=bad1)
    # fused
    q2 = torch.full_like(q1, float("nan"))
    x_sum = torch.empty_like(x)
    cache = ops.rope_cache(pos, n_dims, 10000.0) if cached else None
    ret = ops.mul_mat_fused(w, x, rms_eps=eps, x_add=d, x_sum=x_sum, rope_kv=ops.RopeKv(
        Hq, Hkv, hd, pos, n_dims, mode, 10000.0, idx, q2, kc2, vc2, n_bad=bad2, cache=cache))
    torch.cuda.synchronize()
    assert ret is None
    assert torch.equal(q1, q2), (q1 - q2).abs().max().item()
    assert torch.equal(kc1.view(torch.int16), kc2.view(torch.int16))
    assert torch.equal(vc1.view(torch.int16), vc2.view(torch.int16))
    n_bad_rows = int(((idx < 0) | (idx >= 64)).sum())
    assert int(bad1.item()) == int(bad2.item()) == 2 * Hkv * n_bad_rows


@pytest.mark.parametrize("qtype,K,N,M,epi", [
    (O.Q8_0, 1536, 2048, 1, "plain"),       # Qwen2.5-1.5B QKV shape, decode
    (O.Q8_0, 960, 1600, 3, "plain"),        # K = 960 (block-wise kernel), three rows
    (O.Q4_0, 4096, 22016, 1, "swiglu"),     # bias on both halves before SWIGLU
    (O.Q8_0, 2560, 960, 2, "add"),          # bias, then the residual ADD
    (O.Q8_0, 1536, 2048, 16, "gemm"),       # batch 16: int8 MFMA path, K in 4 parts, bias in the store
    (O.Q4_0, 4096, 4096, 5, "gemm"),        # 5 rows: int8 MFMA path
    (O.Q4_0, 4096, 12288, 37, "gemm"),      # prompt rows: GEMM path, bias in the tile store
    (O.Q8_0, 1536, 17920, 16, "swiglu"),    # batch 16: SWIGLU in the int8 GEMM's epilogue
    (O.Q4_0, 4096, 22016, 6, "swiglu"),     # 6 rows, Q4_0
    (O.Q8_0, 4096, 12288, 512, "gemm"),     # the last round's rows as a split-K launch: bias offset with them
])
def test_mul_mat_fused_bias_bit_identical(qtype, K, N, M, epi):
    """MUL_MAT with its bias input (executor.cpp:2436-2445: ADD(MUL_MAT(W, x), b)) fused
    into the GEMV epilogue or the GEMM store gives exactly the bits of MUL_MAT then ADD."""
    g = torch.Generator(device=DEV)
    g.manual_seed(K + N + M + 1)
    w = ops.quantize_weights(torch.randn((N, K), generator=g, device=DEV) * 0.02, qtype)
    x = torch.randn((M, K), generator=g, device=DEV) * 3.0
    b = torch.randn(N, generator=g, device=DEV) * 0.5
    y = ops.add(ops.mul_mat(w, ops.rms_norm(x, 1e-5)), b)
    kw = dict(rms_eps=1e-5, bias=b)
    if epi == "swiglu":
        want, got = ops.swiglu(y), ops.mul_mat_fused(w, x, swiglu=True, **kw)
    elif epi == "add":
        r = torch.randn((M, N), generator=g, device=DEV)
        want = ops.add(r, y)
        got = r.clone()
        ops.mul_mat_fused(w, x, out=got, add=got, **kw)
    else:
        want, got = y, ops.mul_mat_fused(w, x, **kw)
    torch.cuda.synchronize()
    assert torch.equal(got, want), (got - want).abs().max().item()


@pytest.mark.parametrize("M", [1, 3, 16])
def test_mul_mat_fused_rope_kv_with_bias_bit_identical(M):
    """Qwen2's q/k/v biases ahead of the rope + KV-store epilogue (the decode QKV launch)."""
    g = torch.Generator(device=DEV)
    g.manual_seed(77 + M)
    K, Hq, Hkv, hd = 1536, 12, 2, 128
    N = (Hq + 2 * Hkv) * hd
    w = ops.quantize_weights(torch.randn((N, K), generator=g, device=DEV) * 0.02, O.Q8_0)
    x = torch.randn((M, K), generator=g, device=DEV) * 3.0
    b = torch.randn(N, generator=g, device=DEV)
    pos = torch.arange(300, 300 + M, dtype=torch.int32, device=DEV)
    idx = pos.to(torch.int64)
    kc1 = torch.zeros((1, Hkv, 512, hd), dtype=torch.float16, device=DEV)
    vc1, kc2, vc2 = kc1.clone(), kc1.clone(), kc1.clone()
    y = ops.add(ops.mul_mat(w, ops.rms_norm(x, 1e-5)), b)
    q1 = torch.empty((1, M, Hq, hd), device=DEV)
    ops.rope_kv_store(y[:, :Hq * hd].view(1, M, Hq, hd), y[:, Hq * hd:(Hq + Hkv) * hd].view(1, M, Hkv, hd),
                      y[:, (Hq + Hkv) * hd:].view(1, M, Hkv, hd), pos, hd, 2, 1e6, idx, q1, kc1, vc1)
    q2 = torch.full_like(q1, float("nan"))
    ops.mul_mat_fused(w, x, rms_eps=1e-5, bias=b, rope_kv=ops.RopeKv(
        Hq, Hkv, hd, pos, hd, 2, 1e6, idx, q2, kc2, vc2, cache=ops.rope_cache(pos, hd, 1e6)))
    torch.cuda.synchronize()
    assert torch.equal(q1, q2)
    assert torch.equal(kc1.view(torch.int16), kc2.view(torch.int16))
    assert torch.equal(vc1.view(torch.int16), vc2.view(torch.int16))


@pytest.mark.parametrize("qtype,K,F,M", [
    (O.Q8_0, 1536, 8960, 16),   # Qwen2.5-1.5B gate_up -> down at batch 16
    (O.Q8_0, 1536, 8960, 5),
    (O.Q4_0, 4096, 11008, 9),   # 7B MLP, 9 rows
    (O.Q8_0, 1536, 1024, 16),   # gate_up 2048 x 1536 and down 1536 x 1024 in K halves (whole tiles)
    (O.Q4_0, 2048, 512, 9),     # gate_up 1024 x 2048 in K halves (the ring)
])
def test_swiglu_quantized_rows_feed_down_bit_identical(qtype, K, F, M):
    """gate_up with SWIGLU in the int8 GEMM's epilogue also writes its rows quantized
    (out_q8); the down projection reading them (x_q8) gives exactly the bits of
    MUL_MAT(down, SWIGLU(MUL_MAT(gate_up, RMS_NORM(x)))) run one by one, with and without
    the fp32 SWIGLU rows written."""
    g = torch.Generator(device=DEV)
    g.manual_seed(K + F + M)
    wgu = ops.quantize_weights(torch.randn((2 * F, K), generator=g, device=DEV) * 0.02, qtype)
    wd = ops.quantize_weights(torch.randn((K, F), generator=g, device=DEV) * 0.02, qtype)
    x = torch.randn((M, K), generator=g, device=DEV) * 3.0
    bd = torch.randn(K, generator=g, device=DEV) * 0.1
    act = ops.swiglu(ops.mul_mat(wgu, ops.rms_norm(x, 1e-5)))
    want = ops.add(ops.mul_mat(wd, act), bd)
    for no_out in (False, True):
        q8 = torch.full((ops.q8_rows_bytes(F),), 0x55, dtype=torch.uint8, device=DEV)
        a = ops.mul_mat_fused(wgu, x, rms_eps=1e-5, swiglu=True, out_q8=q8, no_out=no_out)
        got = ops.mul_mat_fused(wd, act, x_q8=q8, bias=bd)
        torch.cuda.synchronize()
        if not no_out:
            assert torch.equal(a, act)
        assert torch.equal(got, want), (got - want).abs().max().item()


@pytest.mark.parametrize("qtype,N,M,mode", [
    (O.Q8_0, 65536, 16, "plain"),   # one K part: a wave's whole tile requested at once
    (O.Q4_0, 65552, 5, "plain"),    # row tiles past N in the last workgroup
    (O.Q8_0, 17920, 16, "swiglu"),  # Qwen2.5-1.5B gate|up with the quantized rows (2-part order)
    (O.Q4_0, 1024, 9, "swiglu"),    # 4-part order
])
def test_gemm_i8_whole_tile_bits(qtype, N, M, mode):
    """Rows of 6 steps (K = 1536) on one K part stage the activation in LDS and request each
    wave's whole tile at once: the bits of the per-step ring (GQ_OPT_GEMM_I8_RING), and
    within 1e-5 of the oracle."""
    K = 1536
    g = torch.Generator(device=DEV)
    g.manual_seed(N + M)
    w = ops.quantize_weights(torch.randn((N, K), generator=g, device=DEV) * 0.02, qtype)
    x = torch.randn((M, K), generator=g, device=DEV)

    def run():
        if mode == "plain":
            return [ops.mul_mat(w, x)]
        q8 = torch.full((ops.q8_rows_bytes(N // 2),), 0x55, dtype=torch.uint8, device=DEV)
        y = ops.mul_mat_fused(w, x, swiglu=True, out_q8=q8)
        return [y, q8]

    got = run()
    with ops.gemm_i8_ring():
        ring = run()
    torch.cuda.synchronize()
    for a, b in zip(got, ring):
        assert torch.equal(a, b)
    if mode == "plain":
        rng = np.random.default_rng(N)
        sel = np.unique(np.concatenate([rng.choice(N, size=256, replace=False), [0, N - 1]]))
        want = O.mul_mat(w.data.cpu().numpy()[sel], qtype, K, x.cpu().numpy())
        assert mar(got[0].cpu().numpy()[:, sel], want) < 1e-5


@pytest.mark.parametrize("qtype,K,N,M", [
    (O.Q4_0, 4096, 22016, 8),   # configs[1] gate_up at M = 8: 2 K parts, 2 tiles per workgroup
    (O.Q8_0, 4096, 16384, 7),   # Q8_0, 2 K parts
    (O.Q8_0, 2048, 65536, 6),   # one K part, 4 tiles per workgroup
    (O.Q4_0, 256, 70, 8),       # one step, a partial last tile
    (O.Q4_0, 4096, 8200, 3),    # 3 rows (int8 forced), rows past N in the last workgroup
    (O.Q8_0, 3840, 9000, 8),    # 15 steps: parts of 8 and 7
])
def test_gemm_i8_staged_activation_bits(qtype, K, N, M):
    """Up to 8 rows on the int8 ring with 2 or 4 tiles per workgroup: the activation copied
    into LDS once per workgroup gives the bits of the per-step activation loads
    (GQ_OPT_GEMM_I8_RING), and stays within 1e-5 of the oracle."""
    g = torch.Generator(device=DEV)
    g.manual_seed(K + N + M + 3)
    w = ops.quantize_weights(torch.randn((N, K), generator=g, device=DEV) * 0.02, qtype)
    x = torch.randn((M, K), generator=g, device=DEV)
    got = ops.mul_mat_fused(w, x, int8=True)
    with ops.gemm_i8_ring():
        ring = ops.mul_mat_fused(w, x, int8=True)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int32), ring.view(torch.int32))
    rng = np.random.default_rng(N + K)
    sel = np.unique(np.concatenate([rng.choice(N, size=min(N, 192), replace=False), [0, N - 1]]))
    want = O.mul_mat(w.data.cpu().numpy()[sel], qtype, K, x.cpu().numpy())
    assert mar(got.cpu().numpy()[:, sel], want) < 1e-5


@pytest.mark.parametrize("qtype,K,N,M", [
    (O.Q8_0, 1536, 1536, 16),   # Qwen2.5-1.5B o at batch 16: halves of 3 steps (a part of each empty)
    (O.Q8_0, 8960, 1536, 16),   # Qwen2.5-1.5B down: 35 steps, halves of 18 and 17
    (O.Q4_0, 1024, 2048, 5),    # 4 steps (one per part of each half), 128 tiles
    (O.Q4_0, 4096, 1000, 9),    # a partial last tile
    (O.Q8_0, 2048, 256, 3),     # 3 rows (int8 forced)
    (O.Q8_0, 2048, 1056, 9),    # the consumer (K = 1056) on the fp16 GEMM path's prologue
])
def test_gemm_i8_halves_bits(qtype, K, N, M):
    """Narrow plain products (at most 128 row tiles in 4 K parts) take K in two halves:
    with out_halves two workgroups per tile leave the halves' sums as two slabs whose fp32
    sum is the product's bits (one 8-wave workgroup per tile adding them in that order),
    which stay within 1e-5 of the oracle; the next prologue's ADD of the two slabs
    (x_add_halves, before RMS_NORM, the sum stored) gives the bits of adding the product."""
    g = torch.Generator(device=DEV)
    g.manual_seed(K + N + M + 5)
    w = ops.quantize_weights(torch.randn((N, K), generator=g, device=DEV) * 0.02, qtype)
    x = torch.randn((M, K), generator=g, device=DEV)
    assert ops.mul_mat_halves(w, x, int8=True)
    assert not ops.mul_mat_halves(w, x, torch.zeros(N, device=DEV), int8=True)
    want = ops.mul_mat_fused(w, x, int8=True)
    halves = torch.full((2, M, N), float("nan"), device=DEV)
    ops.mul_mat_fused(w, x, out=halves, int8=True, out_halves=True)
    torch.cuda.synchronize()
    assert torch.equal((halves[0] + halves[1]).view(torch.int32), want.view(torch.int32))
    rng = np.random.default_rng(N + K)
    sel = np.unique(np.concatenate([rng.choice(N, size=min(N, 192), replace=False), [0, N - 1]]))
    ref = O.mul_mat(w.data.cpu().numpy()[sel], qtype, K, x.cpu().numpy())
    assert mar(want.cpu().numpy()[:, sel], ref) < 1e-5
    if N % 32 == 0:  # the consumer: ADD + RMS_NORM + the next product (int8 path where K % 256 == 0)
        i8 = N % 256 == 0
        w2 = ops.quantize_weights(torch.randn((512, N), generator=g, device=DEV) * 0.02, qtype)
        r = torch.randn((M, N), generator=g, device=DEV) * 3.0
        s1, s2 = torch.empty_like(r), torch.empty_like(r)
        y1 = ops.mul_mat_fused(w2, r, rms_eps=1e-5, x_add=want, x_sum=s1, int8=i8)
        y2 = ops.mul_mat_fused(w2, r, rms_eps=1e-5, x_add=halves, x_add_halves=True, x_sum=s2, int8=i8)
        torch.cuda.synchronize()
        assert torch.equal(s1.view(torch.int32), s2.view(torch.int32))
        assert torch.equal(y1.view(torch.int32), y2.view(torch.int32))


@pytest.mark.parametrize("qtype,K,N", [(O.Q8_0, 1536, 2048), (O.Q4_0, 4096, 4096)])
@pytest.mark.parametrize("M", [1, 3, 4])
def test_int8_path_for_few_rows_matches_rows_of_a_batch(qtype, K, N, M):
    """int8 = 1 puts 1..4 rows on the int8 MFMA path (default: the GEMV): every row is
    computed on its own, so its bits equal the same row of a 16-row product (which is
    pinned against the oracle), with ADD + RMS_NORM in the prologue and the bias."""
    g = torch.Generator(device=DEV)
    g.manual_seed(K + N + M)
    w = ops.quantize_weights(torch.randn((N, K), generator=g, device=DEV) * 0.02, qtype)
    x = torch.randn((16, K), generator=g, device=DEV) * 3.0
    d = torch.randn((16, K), generator=g, device=DEV)
    b = torch.randn(N, generator=g, device=DEV) * 0.1
    want = ops.mul_mat_fused(w, x, rms_eps=1e-5, x_add=d, x_sum=torch.empty_like(x), bias=b)
    got = ops.mul_mat_fused(w, x[:M].contiguous(), rms_eps=1e-5, x_add=d[:M].contiguous(),
                            x_sum=torch.empty((M, K), device=DEV), bias=b, int8=True)
    torch.cuda.synchronize()
    assert torch.equal(got, want[:M]), (got - want[:M]).abs().max().item()


# --------------------------------------------------------------- set_rows ---

def test_set_rows_golden(golden_dir):
    g = np.load(golden_dir / "set_rows_f32_f16.npz")
    cache = to_dev(g["cache"]).view(torch.float16)
    ops.set_rows(cache, to_dev(g["src"]), to_dev(g["idx"]))
    assert np.array_equal(cache.view(torch.int16).cpu().numpy().view(np.uint16), g["out"])


@pytest.mark.parametrize("B,H,ctx,hd,s", [(1, 32, 2048, 128, 1), (1, 5, 1024, 64, 512), (2, 2, 300, 128, 7),
                                          (1, 3, 50, 6, 4)])
def test_set_rows_vs_oracle(B, H, ctx, hd, s):
    rng = np.random.default_rng(s + hd)
    cache = f16(rng.standard_normal((B, H, ctx, hd)))
    src = (rng.standard_normal((B, H, s, hd)) * 50).astype(np.float32)
    src.reshape(-1)[:6] = [65519.0, 65520.0, -1e-8, 3e-6, -0.0, 7e4]
    idx = rng.choice(ctx, size=s, replace=False).astype(np.int64)
    want = O.set_rows_f32_f16(cache, src, idx)
    dc = to_dev(cache).view(torch.float16)
    ops.set_rows(dc, to_dev(src), to_dev(idx))
    assert np.array_equal(dc.view(torch.int16).cpu().numpy().view(np.uint16), want)
    # i32 indices give the same bytes
    dc2 = to_dev(cache).view(torch.float16)
    ops.set_rows(dc2, to_dev(src), to_dev(idx.astype(np.int32)))
    assert torch.equal(dc2, dc)


def test_set_rows_out_of_range_is_skipped_and_counted():
    cache = torch.zeros((1, 2, 8, 64), dtype=torch.float16, device=DEV)
    src = torch.ones((1, 2, 3, 64), dtype=torch.float32, device=DEV)
    idx = torch.tensor([1, 8, -1], dtype=torch.int64, device=DEV)
    bad = torch.zeros(1, dtype=torch.int32, device=DEV)
    ops.set_rows(cache, src, idx, n_bad=bad)
    c = cache.cpu()
    assert int(bad.item()) == 2 * 2  # two bad rows x two heads
    assert (c[0, :, 1] == 1).all() and c[0, :, [0] + list(range(2, 8))].abs().sum() == 0


# -------------------------------------------------------------- attention ---

def _attn_dev(q, kc, vc, n_kv, mask, scale=None):
    Hq, S, D = q.shape
    scale = 1.0 / np.sqrt(np.float32(D)) if scale is None else scale
    kd = to_dev(kc).view(torch.float16)[:, :n_kv]
    vd = to_dev(vc).view(torch.float16)[:, :n_kv]
    md = to_dev(mask).view(torch.float16) if mask is not None else None
    return ops.flash_attn_ext(to_dev(q), kd, vd, md, float(scale)).cpu().numpy()


def test_flash_attn_golden(golden_dir):
    files = sorted(golden_dir.glob("flash_attn_*.npz"))
    assert files
    for f in files:
        g = np.load(f)
        n_kv = int(g["n_kv"])
        got = _attn_dev(g["q"], g["kc"], g["vc"], n_kv, g["mask"])
        exact = O.flash_attn_ext_f16(g["q"], g["kc"], g["vc"], n_kv, g["mask"], mode=1)
        r_exact, r_ref = mar(got, exact), mar(got, g["out"])
        ref_dev = mar(g["out"], exact)
        print(f.name, f"vs exact {r_exact:.2e}  vs reference {r_ref:.2e}  (reference vs exact {ref_dev:.2e})")
        assert r_exact < 1e-3
        assert r_ref < ref_dev + 1e-3


@pytest.mark.parametrize("Hq,Hkv,D,S,pos,ctx", [
    (32, 32, 128, 1, 1100, 2048),   # config 4 decode (MHA): n_kv 1280, 160-row splits
    (32, 32, 128, 1, 1400, 2048),   # n_kv 1536: 192-row splits
    (32, 32, 128, 1, 900, 2048),    # n_kv 1024: 128-row splits
    (15, 5, 64, 1, 600, 1024),      # config 3 decode (GQA 3)
    (12, 2, 128, 1, 4000, 4352),    # config 5 decode, long context (GQA 6)
    (15, 5, 64, 4, 300, 1024),      # small chunk
    (8, 2, 128, 64, 200, 512),      # prefill chunk, tiled-path precision
    (32, 32, 128, 512, 0, 1024),    # config 4 pp512 first chunk
    (4, 2, 128, 2, 100, 512),       # two query rows per kv head pair: per-row masks in the decode kernel
    (8, 8, 128, 1, 5, 32),          # one split (no merge)
    (10, 2, 64, 1, 777, 1024),      # G = 5 (decode kernel with 8 query slots, 5 used)
    (4, 4, 64, 1, 700, 1024),       # D = 64, MHA
])
def test_flash_attn_vs_exact(Hq, Hkv, D, S, pos, ctx):
    rng = np.random.default_rng(Hq * S + pos)
    n_kv = O.pad_kv_len(pos + S, ctx)
    q = rng.standard_normal((Hq, S, D)).astype(np.float32)
    kc = f16(rng.standard_normal((Hkv, ctx, D)))
    vc = f16(rng.standard_normal((Hkv, ctx, D)))
    mask = O.causal_mask_f16(pos, S, n_kv)
    got = _attn_dev(q, kc, vc, n_kv, mask)
    exact = O.flash_attn_ext_f16(q, kc, vc, n_kv, mask, mode=1)
    r = mar(got, exact)
    print(f"Hq={Hq} Hkv={Hkv} D={D} S={S} n_kv={n_kv}: vs exact {r:.2e}")
    assert r < 1e-3


@pytest.mark.parametrize("D", [40, 72, 80, 96, 112, 192, 256, 8])
@pytest.mark.parametrize("Hq,Hkv,S,pos,ctx", [
    (8, 8, 1, 1100, 2048),    # decode, MHA, splits merged inside the kernel
    (12, 2, 1, 3000, 4096),   # decode, GQA 6 (8 query slots), many splits: separate merge
    (4, 2, 3, 200, 512),      # three query rows per kv head pair
    (4, 1, 37, 450, 1024),    # prefill rows: the tiled kernel
    (6, 2, 1, 20, 64),        # one split
])
def test_flash_attn_other_head_dims_vs_exact(D, Hq, Hkv, S, pos, ctx):
    """Head dims other than 64 and 128 (the rest of the set ggmlc's executor sends to
    flash attention, executor.cpp:2306-2309, and one it sends to its soft_max fallback)
    run on the VALU kernels padded to 64, 128 or 256 dims: against the exact softmax at
    the bar of the 64/128 cases, with every dst row written at the real head stride."""
    rng = np.random.default_rng(D * 7 + Hq * S + pos)
    n_kv = O.pad_kv_len(pos + S, ctx)
    q = rng.standard_normal((Hq, S, D)).astype(np.float32)
    kc = f16(rng.standard_normal((Hkv, ctx, D)))
    vc = f16(rng.standard_normal((Hkv, ctx, D)))
    mask = O.causal_mask_f16(pos, S, n_kv)
    got = _attn_dev(q, kc, vc, n_kv, mask)
    exact = O.flash_attn_ext_f16(q, kc, vc, n_kv, mask, mode=1)
    assert got.shape == exact.shape and np.isfinite(got).all()
    r = mar(got, exact)
    print(f"Hq={Hq} Hkv={Hkv} D={D} S={S} n_kv={n_kv}: vs exact {r:.2e}")
    assert r < 1e-3


@pytest.mark.parametrize("D,G,masked", [(128, 1, 0xF800), (64, 4, 0xF800), (128, 2, 0xFC00)])
def test_flash_attn_banded_mask_prefill(D, G, masked):
    """Prefill (matrix-core path) under a band mask: query row i sees keys
    (pos + i - 150, pos + i], so each query tile meets fully masked KV blocks before
    its band (nothing accumulated yet: they must be computed) and after it (skipped),
    with -32768 or -inf as the masked value."""
    rng = np.random.default_rng(D + G)
    Hkv, S, pos, n_kv = 2, 256, 300, 640
    Hq = Hkv * G
    q = rng.standard_normal((Hq, S, D)).astype(np.float32)
    kc = f16(rng.standard_normal((Hkv, n_kv, D)))
    vc = f16(rng.standard_normal((Hkv, n_kv, D)))
    i = np.arange(S)[:, None]
    jj = np.arange(n_kv)[None, :]
    mask = np.where((jj <= pos + i) & (jj > pos + i - 150), 0, masked).astype(np.uint16)
    got = _attn_dev(q, kc, vc, n_kv, mask)
    exact = O.flash_attn_ext_f16(q, kc, vc, n_kv, mask, mode=1)
    r = mar(got, exact)
    print(f"D={D} G={G} masked={masked:#x}: vs exact {r:.2e}")
    assert r < 1e-3


@pytest.mark.parametrize("D,G", [(128, 1), (64, 1), (128, 6)])
def test_flash_attn_prefill_block_skip_sees_every_lane(D, G):
    """The prefill kernel skips a KV block only when no query of its tile needs it: here
    every query sees the first three blocks, and in the last block only one key of one
    query row (never the first query of a wave, nor the keys the first lane of a wave
    reads) is unmasked, so a vote that looked at one lane per wave would drop it."""
    rng = np.random.default_rng(D * 7 + G)
    Hkv, S, n_kv = 2, 64, 256
    Hq = Hkv * G
    q = rng.standard_normal((Hq, S, D)).astype(np.float32)
    kc = f16(rng.standard_normal((Hkv, n_kv, D)))
    vc = f16(rng.standard_normal((Hkv, n_kv, D)))
    mask = np.full((S, n_kv), 0xF800, dtype=np.uint16)  # -32768
    mask[:, :192] = 0
    mask[5, 200] = 0  # row 5: key 8 of the last block (lanes with g = 2 read it)
    got = _attn_dev(q, kc, vc, n_kv, mask)
    exact = O.flash_attn_ext_f16(q, kc, vc, n_kv, mask, mode=1)
    r = mar(got, exact)
    print(f"D={D} G={G}: vs exact {r:.2e}")
    assert r < 1e-3


@pytest.mark.parametrize("Hq,Hkv,D,S,pos,ctx", [
    (32, 32, 128, 1, 1100, 2048),   # 7B decode: 8 splits of 160 rows per kv head
    (12, 2, 128, 3, 4000, 4352),    # GQA 6 x 3 rows: 8 query vectors, many splits
])
def test_flash_attn_decode_workspace_and_replays(Hq, Hkv, D, S, pos, ctx):
    """Split decode (partials in the workspace, then the merge) needs no clean
    workspace: a workspace full of random bytes gives the same bits, and a captured
    graph of three calls sharing one workspace replays to the eager bits every time,
    with eager calls between the replays."""
    rng = np.random.default_rng(Hq + S)
    n_kv = O.pad_kv_len(pos + S, ctx)
    kc = to_dev(f16(rng.standard_normal((Hkv, ctx, D)))).view(torch.float16)[:, :n_kv]
    vc = to_dev(f16(rng.standard_normal((Hkv, ctx, D)))).view(torch.float16)[:, :n_kv]
    mask = to_dev(O.causal_mask_f16(pos, S, n_kv)).view(torch.float16)
    qs = [to_dev(rng.standard_normal((Hq, S, D)).astype(np.float32)) for _ in range(3)]
    need = ops.flash_attn_workspace_size(D, S, Hq, Hkv, n_kv)
    assert need > 0
    ws = ops.Workspace(torch.device(DEV))
    ws.get(need)
    ws.buf.zero_()
    scale = 1.0 / np.sqrt(D)
    clean = [ops.flash_attn_ext(q, kc, vc, mask, scale, ws=ws).clone() for q in qs]
    exact = O.flash_attn_ext_f16(qs[0].cpu().numpy(), kc.view(torch.int16).cpu().numpy().view(np.uint16),
                                 vc.view(torch.int16).cpu().numpy().view(np.uint16), n_kv,
                                 mask.view(torch.int16).cpu().numpy().view(np.uint16), mode=1)
    assert mar(clean[0].cpu().numpy(), exact) < 1e-3
    ws.buf.copy_(torch.randint(0, 256, ws.buf.shape, dtype=torch.uint8, device=DEV))
    dirty = ops.flash_attn_ext(qs[0], kc, vc, mask, scale, ws=ws)
    assert torch.equal(dirty, clean[0])
    outs = [torch.empty_like(c) for c in clean]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for q, o in zip(qs, outs):
            ops.flash_attn_ext(q, kc, vc, mask, scale, out=o, ws=ws)
    for r in range(3):
        for o in outs:
            o.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        for o, c in zip(outs, clean):
            assert torch.equal(o, c), r
        again = ops.flash_attn_ext(qs[1], kc, vc, mask, scale, ws=ws)  # eager call between replays
        assert torch.equal(again, clean[1])


@pytest.mark.parametrize("Hq,Hkv,D,S,pos,ctx", [
    (32, 32, 128, 1, 1100, 2048),   # 7B decode: 8 splits of 160 rows per kv head
    (12, 2, 128, 3, 4000, 4352),    # GQA 6 x 3 rows: 8 query vectors, 34 splits
    (15, 5, 64, 1, 700, 1024),      # SmolLM2 shape
])
def test_flash_attn_fused_merge_bits(Hq, Hkv, D, S, pos, ctx):  # noqa: PLR0913
    """The decode kernel merges its split partials itself (the last workgroup of each
    kv head, counted on a device counter); that gives the bits of the separate merge
    launch (gq_set_option GQ_OPT_ATTN_SEPARATE_MERGE), call after call."""
    rng = np.random.default_rng(Hq * D + S)
    n_kv = O.pad_kv_len(pos + S, ctx)
    kc = to_dev(f16(rng.standard_normal((Hkv, ctx, D)))).view(torch.float16)[:, :n_kv]
    vc = to_dev(f16(rng.standard_normal((Hkv, ctx, D)))).view(torch.float16)[:, :n_kv]
    mask = to_dev(O.causal_mask_f16(pos, S, n_kv)).view(torch.float16)
    q = to_dev(rng.standard_normal((Hq, S, D)).astype(np.float32))
    scale = 1.0 / np.sqrt(D)
    fused = [ops.flash_attn_ext(q, kc, vc, mask, scale) for _ in range(4)]
    with ops.separate_attn_merge():
        sep = ops.flash_attn_ext(q, kc, vc, mask, scale)
    for f in fused:
        assert torch.equal(f, sep)
    # clearing the arrival counters between launches (gq_attn_reset_counters) changes nothing
    from ggmlc_amd import _lib
    _lib.check(_lib.load().gq_attn_reset_counters(ops._stream()))
    assert torch.equal(ops.flash_attn_ext(q, kc, vc, mask, scale), sep)
    exact = O.flash_attn_ext_f16(q.cpu().numpy(), kc.view(torch.int16).cpu().numpy().view(np.uint16),
                                 vc.view(torch.int16).cpu().numpy().view(np.uint16), n_kv,
                                 mask.view(torch.int16).cpu().numpy().view(np.uint16), mode=1)
    assert mar(fused[0].cpu().numpy(), exact) < 1e-3


@pytest.mark.parametrize("Hq,Hkv,D,n_kv", [(12, 2, 128, 1000), (24, 4, 64, 700), (16, 1, 128, 130),
                                            (10, 2, 128, 3000), (15, 5, 64, 700), (16, 8, 128, 1300),
                                            # odd lengths: the VALU kernel (the matrix-core one
                                            # reads the mask 4 keys per load)
                                            (12, 2, 128, 131), (6, 2, 64, 1001), (8, 4, 128, 1001),
                                            (15, 5, 64, 131), (10, 2, 128, 1002)])
def test_flash_attn_decode_many_heads_per_kv_masked_vs_exact(Hq, Hkv, D, n_kv):
    """One query row with 2..16 query heads per kv head (the matrix-core decode kernel over
    the contiguous cache, the KQ mask added to the scores) against the exact softmax in
    float64: -inf holes, a fully masked 256-row span, -32768 entries, n_kv not a multiple of
    128 and a cache longer than the view; a -inf on the last key (the mask's last element)."""
    rng = np.random.default_rng(Hq * D + n_kv)
    ctx = n_kv + 64
    kc = f16(rng.standard_normal((Hkv, ctx, D)))
    vc = f16(rng.standard_normal((Hkv, ctx, D)))
    q = rng.standard_normal((Hq, 1, D)).astype(np.float32)
    mask = np.zeros(n_kv, np.float32)
    mask[rng.random(n_kv) < 0.1] = -np.inf
    if n_kv > 400:
        mask[128:384] = -np.inf
    mask[rng.random(n_kv) < 0.05] = -32768.0
    mask[0] = 0.0
    mask[n_kv - 1] = -np.inf
    scale = 1.0 / np.sqrt(D)
    kd = to_dev(kc).view(torch.float16)[:, :n_kv]
    vd = to_dev(vc).view(torch.float16)[:, :n_kv]
    md = to_dev(f16(mask).reshape(1, n_kv)).view(torch.float16)
    out = ops.flash_attn_ext(to_dev(q), kd, vd, md, scale).cpu().numpy()[0]
    q16 = q[:, 0].astype(np.float16).astype(np.float64)
    K = kc.view(np.float16)[:, :n_kv].astype(np.float64)
    V = vc.view(np.float16)[:, :n_kv].astype(np.float64)
    m64 = f16(mask).view(np.float16).astype(np.float64)
    want = np.zeros((Hq, D))
    for h in range(Hq):
        s = K[h // (Hq // Hkv)] @ q16[h] * scale + m64
        p = np.exp(s - s.max())
        want[h] = p @ V[h // (Hq // Hkv)] / p.sum()
    r = mar(out, want)
    print(f"Hq={Hq} Hkv={Hkv} D={D} n_kv={n_kv}: vs exact {r:.2e}")
    assert r < 2e-5


def test_flash_attn_padding_and_gqa_invariants():
    rng = np.random.default_rng(21)
    Hq, Hkv, D, ctx, pos = 6, 2, 64, 1024, 300
    q = rng.standard_normal((Hq, 1, D)).astype(np.float32)
    kc = f16(rng.standard_normal((Hkv, ctx, D)))
    vc = f16(rng.standard_normal((Hkv, ctx, D)))
    a = _attn_dev(q, kc, vc, 512, O.causal_mask_f16(pos, 1, 512))
    b = _attn_dev(q, kc, vc, 768, O.causal_mask_f16(pos, 1, 768))
    assert np.abs(a - b).max() < 1e-6  # masked padding contributes nothing
    # GQA head h reads kv head h // 3: expanding K/V to MHA gives the same result
    ke = np.repeat(kc, 3, axis=0)
    ve = np.repeat(vc, 3, axis=0)
    c = _attn_dev(q, ke, ve, 512, O.causal_mask_f16(pos, 1, 512))
    assert np.abs(a - c).max() < 1e-6


# ---------------------------------------------------------------- softmax ---

def test_soft_max_golden(golden_dir):
    g = np.load(golden_dir / "soft_max_f32.npz")
    y = ops.soft_max_ext(to_dev(g["x"]), to_dev(g["mask"]).view(torch.float16), float(g["scale"]))
    assert np.abs(y.cpu().numpy() - g["y"]).max() < 1e-6


def test_soft_max_alibi_vs_torch():
    rng = np.random.default_rng(5)
    H, R, C = 6, 5, 77
    x = rng.standard_normal((H, R, C)).astype(np.float32)
    m = rng.standard_normal((R, C)).astype(np.float32)
    mb = 8.0
    y = ops.soft_max_ext(to_dev(x), to_dev(m).half(), 0.5, mb).cpu().numpy()
    n_log2 = 1 << int(np.floor(np.log2(H)))
    m0, m1 = 2.0 ** (-mb / n_log2), 2.0 ** (-mb / 2 / n_log2)
    slopes = np.array([m0 ** (h + 1) if h < n_log2 else m1 ** (2 * (h - n_log2) + 1) for h in range(H)])
    z = x * 0.5 + slopes[:, None, None] * m.astype(np.float16).astype(np.float32)[None]
    z = np.exp(z - z.max(-1, keepdims=True))
    assert np.abs(y - z / z.sum(-1, keepdims=True)).max() < 1e-6


@pytest.mark.parametrize("pos,s,max_ctx", [
    (0, 1, 256), (0, 37, 512), (255, 1, 512), (256, 1, 512), (700, 4, 1024), (1023, 1, 2048), (100, 512, 2048),
])
def test_kv_step_inputs_bits(pos, s, max_ctx):
    """gq_kv_step_inputs against the executor's host-side step inputs restated in the
    oracle (executor.cpp:58-64 pad_kv_len, :136-148 fill_f16_causal_mask, :1181-1393
    positions and KV row indices), bit for bit, with garbage in every output first."""
    n_kv = O.pad_kv_len(pos + s, max_ctx)
    p = torch.tensor([pos], dtype=torch.int32, device=DEV)
    pos_ids = torch.full((s,), -7, dtype=torch.int32, device=DEV)
    kv_idx = torch.full((s,), -7, dtype=torch.int64, device=DEV)
    mask_full = torch.full((s, max_ctx), 12345, dtype=torch.int16, device=DEV)
    mask = mask_full.view(torch.float16)[:, :n_kv]
    ops.kv_step_inputs(p, s, pos_ids, kv_idx, mask)
    want = O.causal_mask_f16(pos, s, n_kv)
    assert np.array_equal(mask_full[:, :n_kv].cpu().numpy().view(np.uint16), want)
    assert (mask_full[:, n_kv:] == 12345).all()  # the view's columns past n_kv are untouched
    assert pos_ids.cpu().tolist() == list(range(pos, pos + s))
    assert kv_idx.cpu().tolist() == list(range(pos, pos + s))
    ops.kv_advance(p, s)
    assert int(p.item()) == pos + s


def test_flash_attn_config_goldens(golden_dir):
    """Decode attention at the configs' shapes (SmolLM2 GQA-3 n_kv 768, 7B MHA n_kv 1280,
    Qwen2.5 GQA-6 n_kv 3072 and 4096) against ggml's own output at 1, 4 and 16 threads.
    ggml's result moves with its thread count (split-KV chunks, fp16 V accumulator:
    ops.cpp:8682-8696, 9179-9209); the GPU accumulates in fp32. Bars: within 1e-3 of the
    exact softmax, and no farther from each reference output than the reference outputs
    are from each other (its thread spread) or, where one reference output is farther from
    the exact softmax than that spread, than the triangle bound through the exact result
    (the reference's distance from it plus the GPU's); and within that distance + 1e-3."""
    import sys

    sys.path.insert(0, str(golden_dir))
    from make_golden import CFG_THREADS, cfg_attn_inputs, inputs_digest

    files = sorted(golden_dir.glob("cfg_attn_*.npz"))
    assert len(files) == 4
    for f in files:
        g = np.load(f)
        q, kc, vc, mask, n_kv = cfg_attn_inputs(int(g["seed"]), int(g["Hq"]), int(g["Hkv"]), int(g["hd"]),
                                                int(g["pos"]))
        assert inputs_digest(q, kc, vc, mask) == str(g["digest"]), f.name
        got = _attn_dev(q, kc, vc, n_kv, mask)
        exact = O.flash_attn_ext_f16(q, kc, vc, n_kv, mask, mode=1)
        refs = {t: g[f"out_t{t}"] for t in CFG_THREADS}
        spread = max(mar(refs[a], refs[b]) for a in CFG_THREADS for b in CFG_THREADS if a != b)
        line = [f"{f.name}: vs exact {mar(got, exact):.2e}, spread {spread:.2e}"]
        assert mar(got, exact) < 1e-3, f.name
        for t, r in refs.items():
            dev = mar(r, exact)
            line.append(f"t{t} {mar(got, r):.2e} (ref vs exact {dev:.2e})")
            assert mar(got, r) <= max(spread, dev + mar(got, exact)), (f.name, t)
            assert mar(got, r) < dev + 1e-3, (f.name, t)
        print(" | ".join(line))


@pytest.mark.parametrize("Hq,Hkv,D,pos,ctx", [(32, 32, 128, 1100, 2048), (15, 5, 64, 700, 1024)])
def test_flash_attn_decode_on_two_streams(Hq, Hkv, D, pos, ctx):
    """Decode attention issued on two streams at once, each with its own workspace (the
    in-kernel split merge counts arrivals per stream): every output has the bits of the
    same call run alone."""
    rng = np.random.default_rng(Hq + D)
    n_kv = O.pad_kv_len(pos + 1, ctx)
    mask = to_dev(O.causal_mask_f16(pos, 1, n_kv)).view(torch.float16)
    scale = 1.0 / np.sqrt(D)
    inputs = []
    for _ in range(2):
        kc = to_dev(f16(rng.standard_normal((Hkv, ctx, D)))).view(torch.float16)[:, :n_kv]
        vc = to_dev(f16(rng.standard_normal((Hkv, ctx, D)))).view(torch.float16)[:, :n_kv]
        inputs.append((to_dev(rng.standard_normal((Hq, 1, D)).astype(np.float32)), kc, vc))
    alone = [ops.flash_attn_ext(q, k, v, mask, scale) for q, k, v in inputs]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    wss = [ops.Workspace(torch.device(DEV)), ops.Workspace(torch.device(DEV))]
    outs = [[], []]
    for _ in range(24):
        for i in range(2):
            with torch.cuda.stream(streams[i]):
                q, k, v = inputs[i]
                outs[i].append(ops.flash_attn_ext(q, k, v, mask, scale, ws=wss[i]))
    torch.cuda.synchronize()
    for i in range(2):
        for o in outs[i]:
            assert torch.equal(o, alone[i]), i
