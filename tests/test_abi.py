"""The C ABI library loads, exports every entry point of include/gq.h, and rejects
bad calls on the host before touching a device. CPU only: nothing here launches
a kernel."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from ggmlc_amd import _lib

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "gq.h"


def declared_functions() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(gq_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not _lib.LIB_PATH.exists():
        pytest.fail("libgq.so not built (python -m ggmlc_amd.build)")
    return _lib.load()


def test_exports_every_declared_symbol(lib):
    names = declared_functions()
    assert len(names) >= 11
    for n in names:
        assert hasattr(lib, n), n
    # the Python binding covers exactly the header's entry points
    assert sorted(_lib.SIGNATURES) == names


def test_abi_version_and_struct_layout(lib):
    assert lib.gq_abi_version() == 3
    # gq_tensor: void* + 2 x int32 + 4 x int64 + 4 x size_t
    assert ctypes.sizeof(_lib.gq_tensor) == 8 + 8 + 32 + 32


def _t(gtype, ne, nb):
    return _lib.make_tensor(0x1000, gtype, ne, nb)


def test_mul_mat_rejects_bad_shapes_without_device(lib):
    w = _t(_lib.Q8_0, [4096, 64], [34, 4352])
    x_bad = _t(_lib.F32, [4000, 1], [4, 16000])
    d = _t(_lib.F32, [64, 1], [4, 256])
    rc = lib.gq_mul_mat(w, x_bad, d, None, 0, None)
    assert rc == -1
    assert b"shape" in lib.gq_last_error()
    w_f32 = _t(_lib.F32, [4096, 64], [4, 16384])
    x = _t(_lib.F32, [4096, 1], [4, 16384])
    assert lib.gq_mul_mat(w_f32, x, d, None, 0, None) == -2
    # decode (M <= 4) needs no workspace; prefill does, and a missing one is
    # reported before any launch
    assert lib.gq_mul_mat_workspace_size(w, x) == 0
    x64 = _t(_lib.F32, [4096, 64], [4, 16384])
    d64 = _t(_lib.F32, [64, 64], [4, 256])
    assert lib.gq_mul_mat_workspace_size(w, x64) >= 64 * 4096 * 2
    assert lib.gq_mul_mat(w, x64, d64, None, 0, None) == -3
    # K not a multiple of 32
    w33 = _t(_lib.Q8_0, [33, 4], [34, 34])
    assert lib.gq_mul_mat(w33, _t(_lib.F32, [33, 1], [4, 132]), _t(_lib.F32, [4, 1], [4, 16]), None, 0, None) == -1


def test_other_entry_points_validate_on_host(lib):
    assert lib.gq_quantize_row_q8_0(None, None, 33, None) == -1
    assert lib.gq_quantize_weights(0, None, None, 32, None) == -2
    cache = _t(_lib.F16, [64, 16, 2, 1], [2, 128, 2048, 4096])
    src = _t(_lib.F32, [64, 3, 2, 1], [4, 256, 768, 1536])
    idx_bad = _t(_lib.I64, [4, 1, 1, 1], [8, 32, 32, 32])
    assert lib.gq_set_rows(cache, src, idx_bad, None, None) == -1
    # head dims: multiples of 8 up to 256 (a 100-dim head is rejected; a 96-dim one passes
    # validation and then needs its split workspace)
    q = _t(_lib.F32, [100, 1, 4, 1], [4, 400, 400, 1600])
    k = _t(_lib.F16, [100, 256, 2, 1], [2, 208, 53248, 106496])
    d = _t(_lib.F32, [100, 4, 1, 1], [4, 400, 1600, 1600])
    assert lib.gq_flash_attn_ext(q, k, k, None, 0.1, 0.0, 0.0, d, None, 0, None) == -2
    q = _t(_lib.F32, [96, 1, 4, 1], [4, 384, 384, 1536])
    k = _t(_lib.F16, [96, 256, 2, 1], [2, 192, 49152, 98304])
    d = _t(_lib.F32, [96, 4, 1, 1], [4, 384, 1536, 1536])
    assert lib.gq_flash_attn_ext(q, k, k, None, 0.1, 0.0, 0.0, d, None, 0, None) == -3
    x = _t(_lib.F32, [10, 3, 1, 1], [4, 40, 120, 120])
    y = _t(_lib.F32, [10, 4, 1, 1], [4, 40, 160, 160])
    assert lib.gq_soft_max(x, None, 1.0, 0.0, y, None) == -1
    assert lib.gq_soft_max(x, None, 1.0, 0.5, _t(_lib.F32, [10, 3, 1, 1], [4, 40, 120, 120]), None) == -1


def test_mul_mat_halves_plan_and_rejects_without_device(lib):
    """gq_mul_mat_fused_halves: plain int8 products of at most 128 row tiles in 4 K parts
    and no bias take K in two halves; out_halves elsewhere, slabs of the wrong shape and
    b_add_halves without b_add or off the GEMM path are refused before any launch (a
    valid request reaches the workspace check)."""
    w = _t(_lib.Q8_0, [1536, 1536], [34, 1632])     # Qwen2.5-1.5B o: 96 tiles, 6 steps
    wide = _t(_lib.Q8_0, [1536, 4096], [34, 1632])  # 256 tiles
    short = _t(_lib.Q8_0, [768, 1536], [34, 816])   # 3 steps: one K part
    x = _t(_lib.F32, [1536, 16], [4, 6144])
    i8 = _lib.gq_mul_mat_fusion()
    i8.int8 = 1
    assert lib.gq_mul_mat_fused_halves(w, x, ctypes.byref(i8)) == 1
    assert lib.gq_mul_mat_fused_halves(wide, x, ctypes.byref(i8)) == 0
    assert lib.gq_mul_mat_fused_halves(short, _t(_lib.F32, [768, 16], [4, 3072]), ctypes.byref(i8)) == 0
    bias = _t(_lib.F32, [1536, 1, 1, 1], [4, 6144, 6144, 6144])
    ib = _lib.gq_mul_mat_fusion()
    ib.int8, ib.bias = 1, ctypes.pointer(bias)
    assert lib.gq_mul_mat_fused_halves(w, x, ctypes.byref(ib)) == 0
    sw = _lib.gq_mul_mat_fusion()
    sw.int8, sw.swiglu = 1, 1
    assert lib.gq_mul_mat_fused_halves(w, x, ctypes.byref(sw)) == 0
    assert lib.gq_mul_mat_fused_halves(w, _t(_lib.F32, [1536, 17], [4, 6144]), ctypes.byref(i8)) == -2
    # M 1..4 without int8: the GEMV path, no halves
    assert lib.gq_mul_mat_fused_halves(w, _t(_lib.F32, [1536, 2], [4, 6144]), ctypes.byref(_lib.gq_mul_mat_fusion())) == 0
    two = _t(_lib.F32, [1536, 16, 2, 1], [4, 6144, 98304, 196608])
    oh = _lib.gq_mul_mat_fusion()
    oh.int8, oh.out_halves = 1, 1
    assert lib.gq_mul_mat_fused(w, x, two, ctypes.byref(oh), None) == -3  # accepted: needs the workspace
    assert lib.gq_mul_mat_fused(wide, x, _t(_lib.F32, [4096, 16, 2, 1], [4, 16384, 262144, 524288]),
                                ctypes.byref(oh), None) == -1
    assert b"out_halves" in lib.gq_last_error()
    one = _t(_lib.F32, [1536, 16, 1, 1], [4, 6144, 98304, 98304])
    assert lib.gq_mul_mat_fused(w, x, one, ctypes.byref(oh), None) == -1
    overlap = _t(_lib.F32, [1536, 16, 2, 1], [4, 6144, 6144, 12288])
    assert lib.gq_mul_mat_fused(w, x, overlap, ctypes.byref(oh), None) == -1
    ohb = _lib.gq_mul_mat_fusion()
    ohb.int8, ohb.out_halves, ohb.bias = 1, 1, ctypes.pointer(bias)
    assert lib.gq_mul_mat_fused(w, x, two, ctypes.byref(ohb), None) == -1
    # the consumer's ADD of two slabs
    d = _t(_lib.F32, [1536, 16], [4, 6144])
    ba = _lib.gq_mul_mat_fusion()
    ba.int8, ba.rms_norm, ba.rms_eps, ba.b_add_halves = 1, 1, 1e-5, 1
    assert lib.gq_mul_mat_fused(w, x, d, ctypes.byref(ba), None) == -1  # no b_add
    ba.b_add = ctypes.pointer(one)
    assert lib.gq_mul_mat_fused(w, x, d, ctypes.byref(ba), None) == -1  # one slab
    ba.b_add = ctypes.pointer(two)
    assert lib.gq_mul_mat_fused(w, x, d, ctypes.byref(ba), None) == -3  # accepted
    g1 = _lib.gq_mul_mat_fusion()
    g1.rms_norm, g1.rms_eps, g1.b_add_halves = 1, 1e-5, 1
    two1 = _t(_lib.F32, [1536, 1, 2, 1], [4, 6144, 6144, 12288])
    g1.b_add = ctypes.pointer(two1)
    assert lib.gq_mul_mat_fused(w, _t(_lib.F32, [1536, 1], [4, 6144]), _t(_lib.F32, [1536, 1], [4, 6144]),
                                ctypes.byref(g1), None) == -2  # the GEMV path


def test_python_binding_raises(lib):
    with pytest.raises(_lib.GQError):
        _lib.check(-1)


def test_mul_mat_fused_rejects_without_device(lib):
    w = _t(_lib.Q4_0, [4096, 64], [18, 2304])
    x5 = _t(_lib.F32, [4096, 5], [4, 16384])
    d5 = _t(_lib.F32, [64, 5], [4, 256])
    f = _lib.gq_mul_mat_fusion(1, 1e-5, 0, None)
    # M > 4: the GEMM path, whose prologue fusions need the workspace it reports
    need = lib.gq_mul_mat_fused_workspace_size(w, x5, ctypes.byref(f))
    assert need >= 5 * 4096 * 2
    assert lib.gq_mul_mat_fused(w, x5, d5, ctypes.byref(f), None) == -3
    # output-side fusions: the GEMV (M <= 4) and the int8 path (M <= 16, K % 256 == 0,
    # 16-byte aligned weights: here it needs the workspace of its prologue), not beyond
    g5 = _lib.gq_mul_mat_fusion(0, 0.0, 1, None)
    assert lib.gq_mul_mat_fused(w, x5, _t(_lib.F32, [32, 5], [4, 128]), ctypes.byref(g5), None) == -3
    x17 = _t(_lib.F32, [4096, 17], [4, 16384])
    assert lib.gq_mul_mat_fused(w, x17, _t(_lib.F32, [32, 17], [4, 128]), ctypes.byref(g5), None) == -2
    assert b"M <= 4" in lib.gq_last_error()
    # quantized rows in and out: the int8 path only, out_q8 with swiglu, b_q8 without
    # the input-side fusions
    q = _lib.gq_mul_mat_fusion()
    q.out_q8 = 0x1000
    assert lib.gq_mul_mat_fused(w, x5, d5, ctypes.byref(q), None) == -1
    q.swiglu = 1
    assert lib.gq_mul_mat_fused(w, x17, _t(_lib.F32, [32, 17], [4, 128]), ctypes.byref(q), None) == -2
    bq = _lib.gq_mul_mat_fusion()
    bq.b_q8, bq.rms_norm, bq.rms_eps = 0x1000, 1, 1e-5
    assert lib.gq_mul_mat_fused(w, x5, d5, ctypes.byref(bq), None) == -1
    assert b"b_q8" in lib.gq_last_error()
    x1 = _t(_lib.F32, [4096, 1], [4, 16384])
    bq.rms_norm = 0
    assert lib.gq_mul_mat_fused(w, x1, _t(_lib.F32, [64, 1], [4, 256]), ctypes.byref(bq), None) == -2
    assert lib.gq_q8_rows_bytes(4096) == 4096 // 32 * 640 and lib.gq_q8_rows_bytes(100) == 0
    # int8: the int8 path for 1..16 rows (here its workspace is missing), nothing beyond
    i8 = _lib.gq_mul_mat_fusion()
    i8.int8 = 1
    assert lib.gq_mul_mat_fused_workspace_size(w, x1, ctypes.byref(i8)) == 4096 // 32 * 640
    assert lib.gq_mul_mat_fused(w, x1, _t(_lib.F32, [64, 1], [4, 256]), ctypes.byref(i8), None) == -3
    assert lib.gq_mul_mat_fused(w, x17, _t(_lib.F32, [64, 17], [4, 256]), ctypes.byref(i8), None) == -2
    wu = _lib.make_tensor(0x1004, _lib.Q4_0, [4096, 64], [18, 2304])  # not 16-byte aligned
    assert lib.gq_mul_mat_fused(wu, x1, _t(_lib.F32, [64, 1], [4, 256]), ctypes.byref(i8), None) == -2
    # the SWIGLU input needs 2K-wide rows, and only exists on the GEMM path
    s5 = _lib.gq_mul_mat_fusion()
    s5.b_swiglu = 1
    assert lib.gq_mul_mat_fused(w, x5, d5, ctypes.byref(s5), None) == -1
    x1w = _t(_lib.F32, [8192, 1], [4, 32768])
    assert lib.gq_mul_mat_fused(w, x1w, _t(_lib.F32, [64, 1], [4, 256]), ctypes.byref(s5), None) == -2
    x5w = _t(_lib.F32, [8192, 5], [4, 32768])
    assert lib.gq_mul_mat_fused_workspace_size(w, x5w, ctypes.byref(s5)) == need
    x = _t(_lib.F32, [4096, 1], [4, 16384])
    d64 = _t(_lib.F32, [64, 1], [4, 256])
    g = _lib.gq_mul_mat_fusion(0, 0.0, 1, None)
    assert lib.gq_mul_mat_fused(w, x, d64, ctypes.byref(g), None) == -1  # swiglu output is N/2 wide
    r = _t(_lib.F32, [64, 1], [4, 256])
    h = _lib.gq_mul_mat_fusion(0, 0.0, 1, ctypes.pointer(r))
    assert lib.gq_mul_mat_fused(w, x, _t(_lib.F32, [32, 1], [4, 128]), ctypes.byref(h), None) == -1
    assert b"exclusive" in lib.gq_last_error()


def test_mul_mat_fused_pre_add_validation(lib):
    w = _t(_lib.Q8_0, [4096, 64], [34, 4352])
    x = _t(_lib.F32, [4096, 1], [4, 16384])
    d = _t(_lib.F32, [64, 1], [4, 256])
    s = _lib.make_tensor(0x2000, _lib.F32, [4096, 1], [4, 16384])
    f = _lib.gq_mul_mat_fusion(0, 0.0, 0, None, None, ctypes.pointer(s))
    assert lib.gq_mul_mat_fused(w, x, d, ctypes.byref(f), None) == -1  # b_sum needs b_add
    a = _lib.make_tensor(0x3000, _lib.F32, [4096, 1], [4, 16384])
    g = _lib.gq_mul_mat_fusion(0, 0.0, 0, None, ctypes.pointer(a), ctypes.pointer(x))
    assert lib.gq_mul_mat_fused(w, x, d, ctypes.byref(g), None) == -1  # b_sum aliases b
    assert b"alias" in lib.gq_last_error()
    bad = _lib.make_tensor(0x3000, _lib.F32, [2048, 1], [4, 8192])
    h = _lib.gq_mul_mat_fusion(0, 0.0, 0, None, ctypes.pointer(bad), None)
    assert lib.gq_mul_mat_fused(w, x, d, ctypes.byref(h), None) == -1  # b_add shaped like b


def test_mul_mat_fused_rope_kv_validation(lib):
    """The rope + KV-store epilogue: dst must be NULL, the product rows must be the
    q/k/v heads, NEOX needs n_dims == head_dim (else the caller runs it unfused)."""
    Hq, Hkv, hd, M = 4, 2, 64, 1
    N = (Hq + 2 * Hkv) * hd
    w = _t(_lib.Q8_0, [256, N], [34, 272])
    x = _t(_lib.F32, [256, M], [4, 1024])
    pos = _lib.make_tensor(0x1000, _lib.I32, [M], [4])
    idx = _lib.make_tensor(0x2000, _lib.I64, [M], [8])
    qo = _lib.make_tensor(0x3000, _lib.F32, [hd, Hq, M, 1], [4, 4 * hd, 4 * hd * Hq, 4 * hd * Hq * M])
    kc = _lib.make_tensor(0x4000, _lib.F16, [hd, 32, Hkv, 1], [2, 2 * hd, 64 * hd, 128 * hd])
    vc = _lib.make_tensor(0x5000, _lib.F16, [hd, 32, Hkv, 1], [2, 2 * hd, 64 * hd, 128 * hd])

    def epi(**kw):
        a = dict(n_head=Hq, n_head_kv=Hkv, head_dim=hd, n_dims=hd, mode=2)
        a.update(kw)
        return _lib.gq_rope_kv_epilogue(a["n_head"], a["n_head_kv"], a["head_dim"], ctypes.pointer(pos), a["n_dims"],
                                        a["mode"], 10000.0, 1.0, 1.0, ctypes.pointer(idx), ctypes.pointer(qo),
                                        ctypes.pointer(kc), ctypes.pointer(vc), None)

    def call(e, dst=None, swiglu=0):
        f = _lib.gq_mul_mat_fusion(1, 1e-5, swiglu, None, None, None, ctypes.pointer(e))
        return lib.gq_mul_mat_fused(w, x, dst, ctypes.byref(f), None)

    d = _t(_lib.F32, [N, M], [4, 4 * N])
    assert call(epi(), dst=d) == -1 and b"NULL" in lib.gq_last_error()
    assert call(epi(), swiglu=1) == -1 and b"exclusive" in lib.gq_last_error()
    assert call(epi(n_head_kv=3)) == -1  # rows are not (Hq + 2 Hkv) * hd
    assert call(epi(n_dims=32)) == -2    # NEOX with partial rotation: unfused
    assert call(epi(mode=1)) == -2
    f = _lib.gq_mul_mat_fusion(0, 0.0, 0, None, None, None, None)
    assert lib.gq_mul_mat_fused(w, x, None, ctypes.byref(f), None) == -1  # no epilogue: dst required


@pytest.mark.parametrize("Hq,Hkv,D,S,n_kv", [
    (12, 2, 128, 1, 70000),    # GQA 6: 6 query vectors per kv head
    (16, 2, 64, 1, 140000),    # GQA 8, D = 64
    (12, 2, 128, 1, 4096),
    (32, 32, 128, 1, 1280),
])
def test_attention_split_plan_bounded(lib, Hq, Hkv, D, S, n_kv):
    """The decode plan never asks for more KV splits than the merge holds (1024): the
    workspace is n_split * Hkv * (Hq / Hkv * S) * (D + 2) floats."""
    q = _t(_lib.F32, [D, S, Hq, 1], [4, 4 * D, 4 * D * S, 4 * D * S * Hq])
    k = _t(_lib.F16, [D, n_kv, Hkv, 1], [2, 2 * D, 2 * D * n_kv, 2 * D * n_kv * Hkv])
    ws = lib.gq_flash_attn_ext_workspace_size(q, k)
    per_split = Hkv * (Hq // Hkv) * S * (D + 2) * 4
    assert ws % per_split == 0
    assert 1 <= ws // per_split <= 1024


def test_set_option_rejects_unknown(lib):
    assert lib.gq_set_option(_lib.GQ_OPT_ATTN_SEPARATE_MERGE, 0) == 0
    assert lib.gq_set_option(_lib.GQ_OPT_ATTN_SEPARATE_MERGE, 7) == -1
    assert lib.gq_set_option(999, 1) == -1
    assert b"unknown option" in lib.gq_last_error()


def test_flash_attn_rejects_heads_past_2gib(lib):
    D, n_kv, Hkv = 128, 1 << 20, 2
    q = _t(_lib.F32, [D, 1, 2, 1], [4, 4 * D, 4 * D, 8 * D])
    k = _t(_lib.F16, [D, n_kv, Hkv, 1], [2, 4096, 4096 * n_kv, 4096 * n_kv * Hkv])  # 4 GiB per head
    d = _t(_lib.F32, [D, 2, 1, 1], [4, 4 * D, 8 * D, 8 * D])
    assert lib.gq_flash_attn_ext(q, k, k, None, 1.0, 0.0, 0.0, d, None, 0, None) == -1
    assert b"2 GiB" in lib.gq_last_error()
