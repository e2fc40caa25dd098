"""Decoder ops around the quantized path (SWIGLU, RMS_NORM, ROPE, GET_ROWS, ARGMAX, ADD).

CPU tests pin the golden vectors (written by the reference's compiled ggml) against the
closed forms; GPU tests check the HIP kernels against those golden vectors.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle as O


def _rope_np(x, pos, n_dims, mode, base):
    """closed form: theta_i = p * base^(-2i/n_dims), rotate pairs (NEOX: i, i+n/2; NORMAL: 2i, 2i+1)."""
    y = x.astype(np.float64).copy()
    half = n_dims // 2
    i = np.arange(half)
    for s, p in enumerate(pos):
        th = p * base ** (-2.0 * i / n_dims)
        c, sn = np.cos(th), np.sin(th)
        a = (i if mode == 2 else 2 * i)
        b = (i + half if mode == 2 else 2 * i + 1)
        x0, x1 = x[s][:, a].astype(np.float64), x[s][:, b].astype(np.float64)
        y[s][:, a] = x0 * c - x1 * sn
        y[s][:, b] = x0 * sn + x1 * c
    return y


def test_golden_decoder_ops_match_closed_forms(golden_dir):
    g = np.load(golden_dir / "swiglu.npz")
    a = g["a"].astype(np.float64)
    n = a.shape[1] // 2
    assert np.allclose(g["y"], a[:, :n] / (1 + np.exp(-a[:, :n])) * a[:, n:], rtol=1e-5, atol=1e-6)
    g = np.load(golden_dir / "rms_norm.npz")
    x = g["x"].astype(np.float64)
    assert np.allclose(g["y"], x / np.sqrt((x * x).mean(1, keepdims=True) + float(g["eps"])), rtol=1e-5, atol=1e-6)
    for name in ("neox", "normal"):
        g = np.load(golden_dir / f"rope_{name}.npz")
        want = _rope_np(g["x"], g["pos"], int(g["n_dims"]), int(g["mode"]), float(g["freq_base"]))
        # fp32 theta at positions up to 4095 carries ~5e-4 rad of rounding in the reference
        assert np.abs(g["y"] - want).max() < 5e-3
        assert np.abs(g["y"][:3] - want[:3]).max() < 1e-5
    for name in ("q8_0", "q4_0"):
        g = np.load(golden_dir / f"get_rows_{name}.npz")
        tab = O.dequantize(g["table"], int(g["wtype"]), int(g["n_embd"]))
        assert np.array_equal(g["y"], tab[g["ids"]])
    g = np.load(golden_dir / "argmax.npz")
    assert np.array_equal(g["y"], g["x"].argmax(1))


# ------------------------------------------------------------------- GPU

@pytest.fixture(scope="module")
def dev():
    import torch
    from ggmlc_amd import _lib

    _lib.check(_lib.load().gq_init())
    return torch.device("cuda")


def _t(a, dev):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


@pytest.mark.gpu
def test_swiglu_rms_norm_gpu(golden_dir, dev):
    from ggmlc_amd import ops

    g = np.load(golden_dir / "swiglu.npz")
    y = ops.swiglu(_t(g["a"], dev)).cpu().numpy()
    assert np.abs(y - g["y"]).max() <= 1e-6 * max(1.0, np.abs(g["y"]).max())
    g = np.load(golden_dir / "rms_norm.npz")
    y = ops.rms_norm(_t(g["x"], dev), float(g["eps"])).cpu().numpy()
    assert np.abs(y - g["y"]).max() < 2e-6


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["neox", "normal"])
def test_rope_gpu(golden_dir, dev, name):
    from ggmlc_amd import ops

    g = np.load(golden_dir / f"rope_{name}.npz")
    x = _t(g["x"], dev).unsqueeze(0)          # [1, seq, heads, hd] = ggml [hd, heads, seq, 1]
    y = ops.rope_ext(x, _t(g["pos"], dev), int(g["n_dims"]), int(g["mode"]), float(g["freq_base"]))
    assert np.abs(y[0].cpu().numpy() - g["y"]).max() < 1e-4


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["neox", "normal"])
def test_rope_cache_gpu(golden_dir, dev, name):
    """gq_rope_cache is the table the rope kernels rotate with: rotating the golden
    input by it in float32 numpy (y0 = x0 c - x1 s, y1 = x0 s + x1 c, each product
    rounded) gives exactly the bits of gq_rope_ext, and stays within the golden bar."""
    from ggmlc_amd import ops

    g = np.load(golden_dir / f"rope_{name}.npz")
    n_dims, mode = int(g["n_dims"]), int(g["mode"])
    pos = _t(g["pos"], dev)
    cs = ops.rope_cache(pos, n_dims, float(g["freq_base"])).cpu().numpy()  # [seq, n_dims]
    x = g["x"].astype(np.float32)  # [seq, heads, hd]
    y = ops.rope_ext(_t(x, dev).unsqueeze(0), pos, n_dims, mode, float(g["freq_base"]))[0].cpu().numpy()
    half = n_dims // 2
    j = np.arange(half)
    i0, i1 = (j, j + half) if mode == 2 else (2 * j, 2 * j + 1)
    c = cs[:, None, 0::2]
    s_ = cs[:, None, 1::2]
    want = x.copy()
    x0, x1 = x[..., i0], x[..., i1]
    want[..., i0] = np.float32(x0 * c) - np.float32(x1 * s_)
    want[..., i1] = np.float32(x0 * s_) + np.float32(x1 * c)
    assert np.array_equal(want, y)
    assert np.abs(want - g["y"]).max() < 1e-4


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["q8_0", "q4_0"])
def test_get_rows_gpu(golden_dir, dev, name):
    from ggmlc_amd import ops

    g = np.load(golden_dir / f"get_rows_{name}.npz")
    w = ops.QWeight(_t(g["table"], dev), int(g["wtype"]), int(g["n_embd"]))
    y = ops.get_rows(w, _t(g["ids"], dev)).cpu().numpy()
    assert np.array_equal(y, g["y"])


@pytest.mark.gpu
def test_argmax_add_gpu(golden_dir, dev):
    import torch
    from ggmlc_amd import ops

    g = np.load(golden_dir / "argmax.npz")
    assert np.array_equal(ops.argmax(_t(g["x"], dev)).cpu().numpy(), g["y"])
    rng = np.random.default_rng(0)
    a = rng.standard_normal((3, 4, 96)).astype(np.float32)
    b = rng.standard_normal((1, 4, 96)).astype(np.float32)
    y = ops.add(_t(a, dev), _t(b, dev)).cpu().numpy()
    assert np.array_equal(y, a + b)
    torch.cuda.synchronize()


@pytest.mark.gpu
@pytest.mark.parametrize("n,pad", [(151936, 0), (32000, 0), (49152, 1), (4099, 0), (5, 0)])
def test_argmax_first_maximum(dev, n, pad):
    """ggml_vec_argmax_f32: the first index of the maximum; -inf rows give 0. Ties are planted
    inside one 4-value chunk, across lanes and across passes of the 16-byte path (n % 4 == 0
    with 16-byte rows), and on the scalar path (n % 4 != 0, or rows padded by one float so
    they are not 16-byte aligned)."""
    from ggmlc_amd import ops

    rng = np.random.default_rng(n + pad)
    rows = 7
    x = rng.standard_normal((rows, n + pad)).astype(np.float32)
    top = np.float32(9.5)
    plants = [
        [n - 1],                              # the last entry
        [3, 2],                               # inside one chunk: 2 comes first
        [5 * 4 + 1, 4 * 1024 * 4 + 1],        # two lanes' chunks
        [min(n - 1, 40000), min(n - 1, 33000 * 4 % n)],  # far apart: different passes
        [0],
    ]
    for r, idx in enumerate(plants):
        for i in idx:
            if i < n:
                x[r, i] = top
    x[5, :n] = -np.inf
    x[6, :n] = np.float32(-3.0)  # all equal: index 0
    xt = _t(x, dev)[:, :n]
    got = ops.argmax(xt).cpu().numpy()
    want = np.array([0 if np.all(x[r, :n] == -np.inf) else int(np.argmax(x[r, :n])) for r in range(rows)],
                    np.int32)
    assert np.array_equal(got, want), (got, want)


@pytest.mark.gpu
@pytest.mark.parametrize("mode,n_dims,Hq,Hkv,hd,s", [(2, 128, 32, 32, 128, 1), (2, 64, 15, 5, 64, 7),
                                                     (0, 96, 4, 2, 128, 3)])
def test_rope_kv_store_bit_identical(dev, mode, n_dims, Hq, Hkv, hd, s):
    """gq_rope_kv_store == rope_ext(q), rope_ext(k), set_rows(k), set_rows(v), bit for bit,
    including the skipped out-of-range index and its count."""
    import torch
    from ggmlc_amd import ops

    g = torch.Generator(device=dev)
    g.manual_seed(hd + s)
    qkv = torch.randn((s, (Hq + 2 * Hkv) * hd), generator=g, device=dev) * 4
    qv = qkv[:, :Hq * hd].view(1, s, Hq, hd)
    kv = qkv[:, Hq * hd:(Hq + Hkv) * hd].view(1, s, Hkv, hd)
    vv = qkv[:, (Hq + Hkv) * hd:].view(1, s, Hkv, hd)
    pos = torch.arange(1000, 1000 + s, dtype=torch.int32, device=dev)
    idx = torch.tensor(([5, -1, 9, 63, 0, 7, 2])[:s], dtype=torch.int64, device=dev)
    kc1 = (torch.randn((1, Hkv, 64, hd), generator=g, device=dev)).half()
    vc1 = (torch.randn((1, Hkv, 64, hd), generator=g, device=dev)).half()
    kc2, vc2 = kc1.clone(), vc1.clone()
    bad1 = torch.zeros(1, dtype=torch.int32, device=dev)
    bad2 = torch.zeros(1, dtype=torch.int32, device=dev)
    q1 = ops.rope_ext(qv, pos, n_dims, mode, 10000.0)
    k1 = ops.rope_ext(kv, pos, n_dims, mode, 10000.0)
    ops.set_rows(kc1, k1.permute(0, 2, 1, 3), idx, n_bad=bad1)
    ops.set_rows(vc1, vv.permute(0, 2, 1, 3), idx, n_bad=bad1)
    q2 = torch.empty_like(q1)
    ops.rope_kv_store(qv, kv, vv, pos, n_dims, mode, 10000.0, idx, q2, kc2, vc2, n_bad=bad2)
    torch.cuda.synchronize()
    assert torch.equal(q1, q2)
    assert torch.equal(kc1.view(torch.int16), kc2.view(torch.int16))
    assert torch.equal(vc1.view(torch.int16), vc2.view(torch.int16))
    assert int(bad1.item()) == int(bad2.item()) == (2 * Hkv if s > 1 else 0)
