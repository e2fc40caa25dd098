"""gq_flash_attn_ext_noalloc (the allocation-free decode attention: split partials in a
static per-device array) against gq_flash_attn_ext with a caller workspace, through the
C ABI: the same bits, on calls in a row whose second one is smaller than the first, and
across the launch plans that use partials (the matrix-core decode with its merge launch,
the VALU decode with its merge in the kernel or in a separate launch, the tiled kernel).
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import oracle as O
from ggmlc_amd import _lib, ops

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _f16(rng, shape):
    return torch.from_numpy(rng.standard_normal(shape).astype(np.float32).astype(np.float16)).to(DEV)


def _case(rng, Hq, Hkv, D, S, pos, ctx):
    n_kv = O.pad_kv_len(pos + S, ctx)
    kc = _f16(rng, (Hkv, ctx, D))[:, :n_kv]
    vc = _f16(rng, (Hkv, ctx, D))[:, :n_kv]
    mask = torch.from_numpy(O.causal_mask_f16(pos, S, n_kv)).to(DEV).view(torch.float16)
    q = torch.from_numpy(rng.standard_normal((Hq, S, D)).astype(np.float32)).to(DEV)
    return q, kc, vc, mask, n_kv


def _noalloc(q, k, v, mask, scale):
    Hq, S, D = q.shape
    out = torch.full((S, Hq, D), float("nan"), dtype=torch.float32, device=DEV)
    L = _lib.load()
    d = [ops._desc(t) for t in (q, k, v, mask, out)]
    _lib.check(L.gq_flash_attn_ext_noalloc(ctypes.byref(d[0]), ctypes.byref(d[1]), ctypes.byref(d[2]),
                                           ctypes.byref(d[3]), scale, 0.0, 0.0, ctypes.byref(d[4]),
                                           ops._stream()))
    return out


@pytest.fixture(scope="module", autouse=True)
def _init():
    _lib.check(_lib.load().gq_init())
    yield
    torch.cuda.synchronize()


# (Hq, Hkv, D, S, pos, ctx): each case is run after the one before it, larger first
CASES = [
    (12, 2, 128, 1, 4000, 4352),   # GQA 6 decode: the matrix-core route, 32 splits of 128 rows
    (8, 8, 64, 1, 8000, 8192),     # MHA decode (VALU kernel): 32 splits, the separate merge launch
    (32, 32, 128, 1, 1100, 2048),  # 7B decode: 9 splits merged in the kernel
    (32, 32, 128, 16, 300, 1024),  # 16 rows: the tiled kernel with partials
    (15, 5, 64, 1, 200, 512),      # SmolLM2 decode, smallest
]


def test_noalloc_matches_workspace_entry_point():
    rng = np.random.default_rng(55)
    sizes = []
    for Hq, Hkv, D, S, pos, ctx in CASES:
        q, k, v, mask, n_kv = _case(rng, Hq, Hkv, D, S, pos, ctx)
        need = ops.flash_attn_workspace_size(D, S, Hq, Hkv, n_kv)
        assert 0 < need <= _lib.GQ_ATTN_SCRATCH_BYTES
        sizes.append(need)
        scale = 1.0 / np.sqrt(D)
        want = ops.flash_attn_ext(q, k, v, mask, scale)
        for _ in range(2):  # the array keeps the previous call's partials: same bits again
            got = _noalloc(q, k, v, mask, scale)
            torch.cuda.synchronize()
            assert torch.equal(got, want), (Hq, Hkv, D, S, pos)
        exact = O.flash_attn_ext_f16(q.cpu().numpy(), k.contiguous().view(torch.int16).cpu().numpy().view(np.uint16),
                                     v.contiguous().view(torch.int16).cpu().numpy().view(np.uint16), n_kv,
                                     mask.view(torch.int16).cpu().numpy().view(np.uint16), scale, mode=1)
        g = got.cpu().numpy().astype(np.float64)
        assert np.abs(g - exact).max() / np.abs(exact).max() < 1e-3
    assert sizes[0] > sizes[-1]  # the last call is smaller than the first


def test_noalloc_rejects_shapes_past_the_scratch():
    # 8 query rows of 32 MHA heads over 65536 rows: 1024 splits of partials = 136 MB
    Hq = Hkv = 32
    D, S, n_kv = 128, 8, 65536
    need = ops.flash_attn_workspace_size(D, S, Hq, Hkv, n_kv)
    assert need > _lib.GQ_ATTN_SCRATCH_BYTES
    q = torch.zeros((Hq, S, D), dtype=torch.float32, device=DEV)
    kv = torch.zeros((Hkv, n_kv, D), dtype=torch.float16, device=DEV)
    out = torch.zeros((S, Hq, D), dtype=torch.float32, device=DEV)
    L = _lib.load()
    d = [ops._desc(t) for t in (q, kv, kv, out)]
    rc = L.gq_flash_attn_ext_noalloc(ctypes.byref(d[0]), ctypes.byref(d[1]), ctypes.byref(d[2]), None, 0.1, 0.0,
                                     0.0, ctypes.byref(d[3]), ops._stream())
    assert rc == -3 and b"static scratch" in L.gq_last_error()
