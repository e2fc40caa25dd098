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
