"""Device ops on torch tensors, each one call into libgq.so.

These mirror the ggml operators ggmlc's executor emits on the quantized path
(runtime/src/executor.cpp:2091-2447) with the same argument meaning:

* ``quantize_row_q8_0(x)``           — ggml x86 ``quantize_row_q8_0`` (bit-exact)
* ``mul_mat(w, x)``                  — ``ggml_mul_mat(W[Q8_0|Q4_0], X[f32])``
* ``set_rows(cache, src, idx)``      — ``ggml_set_rows`` F32 -> F16 (in place)
* ``flash_attn_ext(q, k, v, mask, scale)`` — ``ggml_flash_attn_ext`` over F16 K/V
* ``soft_max_ext(x, mask, scale, max_bias)`` — ``ggml_soft_max_ext``

Layout convention: a torch tensor of shape ``[d3, d2, d1, d0]`` is the ggml
tensor ``ne = [d0, d1, d2, d3]`` (ggml's innermost dimension is torch's last).
A quantized weight is a ``QWeight``: uint8 bytes ``[N, K/32 * block_bytes]``
exactly as stored in a .gguf, plus its type and K.

Work runs on torch's current HIP stream. Nothing here computes on the CPU; if
libgq.so is not built every call raises.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from . import _lib
from ._lib import BLOCK_BYTES, F16, F32, I32, I64, Q4_0, Q8_0, check, make_tensor

__all__ = [
    "QWeight", "Q8_0", "Q4_0", "quantize_row_q8_0", "quantize_weights", "mul_mat",
    "set_rows", "flash_attn_ext", "soft_max_ext", "Workspace",
    "swiglu", "rms_norm", "rope_ext", "add", "get_rows", "argmax",
    "kv_step_inputs", "kv_advance", "rope_cache",
]

_TORCH_TO_GQ = {torch.float32: F32, torch.float16: F16, torch.int64: I64, torch.int32: I32}


@dataclass
class QWeight:
    """A block-quantized weight: N rows of K elements (ggml ne = [K, N])."""

    data: torch.Tensor  # uint8 [N, K/32 * block_bytes], contiguous, on device
    qtype: int
    K: int

    @property
    def N(self) -> int:
        return self.data.shape[0]

    @property
    def nbytes(self) -> int:
        return self.data.numel()

    def desc(self):
        bb = BLOCK_BYTES[self.qtype]
        return make_tensor(self.data.data_ptr(), self.qtype, [self.K, self.N], [bb, self.K // 32 * bb])


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _desc(t: torch.Tensor, gtype: int | None = None):
    """ggml descriptor of a (up to 4-d) torch tensor, strides in bytes."""
    if gtype is None:
        gtype = _TORCH_TO_GQ[t.dtype]
    es = t.element_size()
    shape = list(t.shape)[::-1]
    strides = [s * es for s in list(t.stride())[::-1]]
    if len(shape) > 4:
        raise ValueError("at most 4 dimensions")
    while len(shape) < 4:
        strides.append(strides[-1] * shape[-1] if shape else es)
        shape.append(1)
    return make_tensor(t.data_ptr(), gtype, shape, strides)


class Workspace:
    """Grow-only device scratch buffer (256-byte aligned) shared by calls on one stream.

    HIP graphs captured while a smaller buffer was current keep its raw address, so a
    buffer replaced by a larger one is retired, not freed: it lives as long as the
    workspace (and so as long as the decoder whose graphs may still replay it)."""

    def __init__(self, device=None):
        self.device = device
        self.buf = None
        self.retired: list[torch.Tensor] = []

    def get(self, nbytes: int) -> tuple[int, int]:
        if nbytes == 0:
            return 0, 0
        if self.buf is None or self.buf.numel() < nbytes:
            if torch.cuda.is_current_stream_capturing():
                # a graph captured earlier may still point at the current buffer
                raise RuntimeError(f"Workspace: {nbytes} bytes needed during graph capture; size it first")
            dev = self.device or torch.device("cuda", torch.cuda.current_device())
            if self.buf is not None:
                self.retired.append(self.buf)
            self.buf = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=dev)
        return self.buf.data_ptr(), self.buf.numel()


_default_ws: dict[int, Workspace] = {}


def _ws(ws: Workspace | None) -> Workspace:
    if ws is not None:
        return ws
    dev = torch.cuda.current_device()
    if dev not in _default_ws:
        _default_ws[dev] = Workspace(torch.device("cuda", dev))
    return _default_ws[dev]


class separate_attn_merge:
    """Context manager: decode attention merges its KV splits in a second launch
    (gq_set_option GQ_OPT_ATTN_SEPARATE_MERGE) inside the block; same bits, for comparisons."""

    def __enter__(self):
        check(_lib.load().gq_set_option(_lib.GQ_OPT_ATTN_SEPARATE_MERGE, 1))
        return self

    def __exit__(self, *exc):
        check(_lib.load().gq_set_option(_lib.GQ_OPT_ATTN_SEPARATE_MERGE, 0))
        return False


class gemm_i8_ring:
    """Context manager: the int8 path streams every product's weights and activation through
    its per-step ring (gq_set_option GQ_OPT_GEMM_I8_RING) inside the block, with no whole-tile
    requests or LDS-staged activations; same bits, for comparisons."""

    def __enter__(self):
        check(_lib.load().gq_set_option(_lib.GQ_OPT_GEMM_I8_RING, 1))
        return self

    def __exit__(self, *exc):
        check(_lib.load().gq_set_option(_lib.GQ_OPT_GEMM_I8_RING, 0))
        return False


def quantize_row_q8_0(x: torch.Tensor) -> torch.Tensor:
    """x: fp32 contiguous, numel % 32 == 0 -> uint8 [..., K/32*34] block_q8_0 bytes."""
    if x.dtype != torch.float32 or not x.is_contiguous():
        raise ValueError("quantize_row_q8_0: x must be contiguous float32")
    K = x.shape[-1]
    out = torch.empty(x.shape[:-1] + (K // 32 * 34,), dtype=torch.uint8, device=x.device)
    L = _lib.load()
    check(L.gq_quantize_row_q8_0(x.data_ptr(), out.data_ptr(), x.numel(), _stream()))
    return out


def quantize_weights(w: torch.Tensor, qtype: int) -> QWeight:
    """ggmlc's compile-time quantizer (quantize.py) on device: w fp32 [N, K] -> QWeight."""
    if w.dtype != torch.float32 or not w.is_contiguous() or w.dim() != 2:
        raise ValueError("quantize_weights: w must be a contiguous float32 [N, K]")
    N, K = w.shape
    out = torch.empty((N, K // 32 * BLOCK_BYTES[qtype]), dtype=torch.uint8, device=w.device)
    check(_lib.load().gq_quantize_weights(qtype, w.data_ptr(), out.data_ptr(), w.numel(), _stream()))
    return QWeight(out, qtype, K)


def mul_mat(w: QWeight, x: torch.Tensor, out: torch.Tensor | None = None,
            ws: Workspace | None = None) -> torch.Tensor:
    """ggml_mul_mat(W, X): x fp32 [..., K] -> fp32 [..., N]."""
    if x.dtype != torch.float32:
        raise ValueError("mul_mat: x must be float32")
    if out is None:
        out = torch.empty(x.shape[:-1] + (w.N,), dtype=torch.float32, device=x.device)
    L = _lib.load()
    a, b, d = w.desc(), _desc(x), _desc(out)
    need = L.gq_mul_mat_workspace_size(a, b)
    ptr, size = _ws(ws).get(need)
    check(L.gq_mul_mat(a, b, d, ptr, size, _stream()))
    return out


@dataclass
class RopeKv:
    """The rope + KV-store epilogue of :func:`mul_mat_fused` (the arguments of
    :func:`rope_kv_store`, with q/k/v being the rows of the fused QKV product)."""
    n_head: int
    n_head_kv: int
    head_dim: int
    pos: torch.Tensor
    n_dims: int
    mode: int
    freq_base: float
    kv_idx: torch.Tensor
    q_out: torch.Tensor
    k_cache: torch.Tensor
    v_cache: torch.Tensor
    freq_scale: float = 1.0
    attn_factor: float = 1.0
    n_bad: torch.Tensor | None = None
    cache: torch.Tensor | None = None  # rope_cache(pos, ...) of the same arguments


def mul_mat_fused(w: QWeight, x: torch.Tensor, out: torch.Tensor | None = None, rms_eps: float | None = None,
                  swiglu: bool = False, add: torch.Tensor | None = None, x_add: torch.Tensor | None = None,
                  x_sum: torch.Tensor | None = None, rope_kv: RopeKv | None = None, x_swiglu: bool = False,
                  ws: Workspace | None = None, bias: torch.Tensor | None = None, out_q8: torch.Tensor | None = None,
                  x_q8: torch.Tensor | None = None, no_out: bool = False, int8: bool = False,
                  out_halves: bool = False, x_add_halves: bool = False) -> torch.Tensor | None:
    """MUL_MAT fused with its graph neighbours, bit-identical to the unfused ops:
    x_add -> x + x_add first (stored to x_sum when given); rms_eps -> RMS_NORM;
    x_swiglu -> the input is SWIGLU of x's two halves (x [..., 2K]); swiglu -> SWIGLU of
    the result's two halves (out [..., N/2]); add -> add + result (add may be out);
    rope_kv -> the result's q/k/v rows go through :func:`rope_kv_store` instead of
    being written (returns None); bias (fp32 [N]) -> the product + bias before the
    output-side fusions (MUL_MAT's bias ADD). Up to 4 rows run as one GEMV launch; more rows take
    the GEMM path (input-side fusions, with the workspace ws); on its int8 path (5..16 rows,
    K % 256 == 0) also swiglu and rope_kv, plus out_q8 (uint8 [q8_rows_bytes(N / 2)]: with
    swiglu, the result rows quantized for the next product; no_out: only those) and x_q8
    (x's rows already quantized, e.g. another product's out_q8: x gives the shape only);
    int8 -> the int8 path also for 1..4 rows. out_halves (where :func:`mul_mat_halves`
    says so; x 2-d): out [2, M, N] holds the sums over K's two halves, out[0] + out[1]
    being the product's bits; x_add_halves: x_add is such a pair [2, M, K], x + (x_add[0]
    + x_add[1]) being added."""
    if x.dtype != torch.float32:
        raise ValueError("mul_mat_fused: x must be float32")
    n_out = w.N // 2 if swiglu else w.N
    if out is None and rope_kv is None and not no_out:
        out = torch.empty(((2,) if out_halves else ()) + x.shape[:-1] + (n_out,), dtype=torch.float32,
                          device=x.device)
    f = _lib.gq_mul_mat_fusion()
    f.b_swiglu = 1 if x_swiglu else 0
    f.out_halves = 1 if out_halves else 0
    f.b_add_halves = 1 if x_add_halves else 0
    if out_q8 is not None:
        f.out_q8 = out_q8.data_ptr()
    if x_q8 is not None:
        f.b_q8 = x_q8.data_ptr()
    f.int8 = 1 if int8 else 0
    keep = []  # descriptors the fusion struct points at
    if rope_kv is not None:
        r = rope_kv
        descs = [_desc(t) for t in (r.pos, r.kv_idx, r.q_out, r.k_cache, r.v_cache)]
        cd = _desc(r.cache) if r.cache is not None else None
        keep += descs + [cd]
        e = _lib.gq_rope_kv_epilogue(r.n_head, r.n_head_kv, r.head_dim, ctypes.pointer(descs[0]), r.n_dims, r.mode,
                                     r.freq_base, r.freq_scale, r.attn_factor, ctypes.pointer(descs[1]),
                                     ctypes.pointer(descs[2]), ctypes.pointer(descs[3]), ctypes.pointer(descs[4]),
                                     r.n_bad.data_ptr() if r.n_bad is not None else None,
                                     ctypes.pointer(cd) if cd is not None else None)
        keep.append(e)
        f.rope_kv = ctypes.pointer(e)
    if rms_eps is not None:
        f.rms_norm, f.rms_eps = 1, float(rms_eps)
    f.swiglu = 1 if swiglu else 0
    ad = _desc(add) if add is not None else None
    if ad is not None:
        f.add = ctypes.pointer(ad)
    xa = _desc(x_add) if x_add is not None else None
    if xa is not None:
        f.b_add = ctypes.pointer(xa)
    xs = _desc(x_sum) if x_sum is not None else None
    if xs is not None:
        f.b_sum = ctypes.pointer(xs)
    bd = _desc(bias) if bias is not None else None
    if bd is not None:
        f.bias = ctypes.pointer(bd)
    od = _desc(out) if out is not None and not no_out else None
    L, wd, xd = _lib.load(), w.desc(), _desc(x)
    need = L.gq_mul_mat_fused_workspace_size(wd, xd, ctypes.byref(f))
    if need:
        f.workspace, f.workspace_bytes = _ws(ws).get(need)
    check(L.gq_mul_mat_fused(wd, xd, od, ctypes.byref(f), _stream()))
    del keep
    return out


def set_rows(cache: torch.Tensor, src: torch.Tensor, idx: torch.Tensor,
             n_bad: torch.Tensor | None = None) -> torch.Tensor:
    """ggml_set_rows(cache, src, idx) in place.

    cache fp16 ``[B, H, rows, hd]`` (ggml [hd, rows, H, B]); src fp32 ``[B, H, s, hd]``;
    idx int64/int32 ``[s]`` (or broadcast ``[ne_c2, ne_c1, s]``)."""
    L = _lib.load()
    nb_ptr = n_bad.data_ptr() if n_bad is not None else None
    check(L.gq_set_rows(_desc(cache), _desc(src), _desc(idx), nb_ptr, _stream()))
    return cache


def flash_attn_ext(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, mask: torch.Tensor | None,
                   scale: float, max_bias: float = 0.0, logit_softcap: float = 0.0,
                   out: torch.Tensor | None = None, ws: Workspace | None = None) -> torch.Tensor:
    """ggml_flash_attn_ext. q fp32 ``[Hq, S, D]``; k/v fp16 ``[Hkv, n_kv, D]`` (views of a
    cache are fine); mask fp16 ``[S, n_kv]`` or None. Returns fp32 ``[S, Hq, D]``."""
    Hq, S, D = q.shape
    if out is None:
        out = torch.empty((S, Hq, D), dtype=torch.float32, device=q.device)
    L = _lib.load()
    qd, kd, vd, od = _desc(q), _desc(k), _desc(v), _desc(out)
    md = _desc(mask) if mask is not None else None
    need = L.gq_flash_attn_ext_workspace_size(qd, kd)
    ptr, size = _ws(ws).get(need)
    check(L.gq_flash_attn_ext(qd, kd, vd, md, scale, max_bias, logit_softcap, od, ptr, size, _stream()))
    return out


def flash_attn_paged(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor, page_table: torch.Tensor,
                     seq_len: torch.Tensor, page_size: int, max_len: int, scale: float,
                     out: torch.Tensor | None = None, ws: Workspace | None = None,
                     out_q8: torch.Tensor | None = None) -> torch.Tensor:
    """Batched decode attention over a paged KV pool (gq_flash_attn_paged): q fp32
    ``[Hq, B, D]`` (row b = the new token of sequence b), pools fp16 ``[Hkv, rows, D]``,
    page_table int32 ``[>= B, max_pages]``, seq_len int32 ``[>= B]``. Returns fp32 ``[B, Hq, D]``.
    out_q8 (uint8 [q8_rows_bytes(Hq * D)]): also the rows quantized for the output
    projection (gq_flash_attn_paged_q8; see :func:`paged_q8_ok`)."""
    Hq, B, D = q.shape
    if out is None:
        out = torch.empty((B, Hq, D), dtype=torch.float32, device=q.device)
    L = _lib.load()
    qd, kd, vd, od = _desc(q), _desc(k_pool), _desc(v_pool), _desc(out)
    need = L.gq_flash_attn_paged_workspace_size(qd, kd, max_len, page_size)
    ptr, size = _ws(ws).get(need)
    if out_q8 is not None:
        check(L.gq_flash_attn_paged_q8(qd, kd, vd, _desc(page_table), _desc(seq_len), page_size, max_len, scale, od,
                                       out_q8.data_ptr(), ptr, size, _stream()))
    else:
        check(L.gq_flash_attn_paged(qd, kd, vd, _desc(page_table), _desc(seq_len), page_size, max_len, scale, od,
                                    ptr, size, _stream()))
    return out


def mul_mat_halves(w: QWeight, x: torch.Tensor, bias: torch.Tensor | None = None, int8: bool = False) -> bool:
    """Whether the plain product w x (bias optional; int8 as in :func:`mul_mat_fused`)
    takes K in two halves on the int8 path, so that :func:`mul_mat_fused` accepts
    out_halves (gq_mul_mat_fused_halves)."""
    f = _lib.gq_mul_mat_fusion()
    f.int8 = 1 if int8 else 0
    bd = _desc(bias) if bias is not None else None
    if bd is not None:
        f.bias = ctypes.pointer(bd)
    rc = _lib.load().gq_mul_mat_fused_halves(w.desc(), _desc(x), ctypes.byref(f))
    check(min(rc, 0))
    return rc == 1


def q8_rows_bytes(K: int) -> int:
    """Bytes of up to 16 activation rows of K values quantized for the int8 path
    (gq_q8_rows_bytes)."""
    return int(_lib.load().gq_q8_rows_bytes(K))


def paged_q8_ok(D: int, B: int, Hq: int, Hkv: int, max_len: int, page_size: int) -> bool:
    """Whether :func:`flash_attn_paged` can write out_q8 for this launch: B <= 16, 2..16 q
    heads per kv head, pages of a multiple of 128 rows, max_len > 128 (the library rejects
    the rest with GQ_ERR_UNSUPPORTED)."""
    G = Hq // Hkv if Hkv and Hq % Hkv == 0 else 0
    return (D in (64, 128) and 1 <= B <= 16 and 1 < G <= 16 and page_size % 128 == 0 and max_len > 128)


def flash_attn_paged_workspace_size(D: int, B: int, Hq: int, Hkv: int, max_len: int, page_size: int) -> int:
    L = _lib.load()
    q = make_tensor(0, F32, [D, B, Hq, 1], [4, 4 * D, 4 * D * B, 4 * D * B * Hq])
    k = make_tensor(0, F16, [D, page_size, Hkv, 1], [2, 2 * D, 2 * D * page_size, 2 * D * page_size * Hkv])
    return L.gq_flash_attn_paged_workspace_size(q, k, max_len, page_size)


def paged_step_inputs(pos: torch.Tensor, page_table: torch.Tensor, page_size: int, trash_row: int,
                      kv_idx: torch.Tensor, seq_len: torch.Tensor | None = None, B: int | None = None) -> None:
    """kv_idx[b] (int64) = pool row of position pos[b]; seq_len[b] (int32) = pos[b] + 1."""
    B = pos.numel() if B is None else B
    check(_lib.load().gq_paged_step_inputs(pos.data_ptr(), B, _desc(page_table), page_size, trash_row,
                                           kv_idx.data_ptr(), seq_len.data_ptr() if seq_len is not None else None,
                                           _stream()))


def paged_advance(pos: torch.Tensor, active: torch.Tensor | None = None, B: int | None = None) -> None:
    """pos[b] += 1 on the device where active[b] != 0 (all slots when active is None)."""
    B = pos.numel() if B is None else B
    check(_lib.load().gq_paged_advance(pos.data_ptr(), active.data_ptr() if active is not None else None, B,
                                       _stream()))


def kv_pages_copy(pool: torch.Tensor, cache: torch.Tensor, pages: torch.Tensor, page_size: int, r0: int, r1: int,
                  to_pool: bool) -> None:
    """Rows [r0, r1) of one sequence between a contiguous cache ``[H, ctx, D]`` and its
    pages (int32 device ids) in a pool ``[H, rows, D]`` (both fp16)."""
    if r1 <= r0:
        return
    check(_lib.load().gq_kv_pages_copy(_desc(pool), _desc(cache), pages.data_ptr(), pages.numel(), page_size, r0, r1,
                                       1 if to_pool else 0, _stream()))


def soft_max_ext(x: torch.Tensor, mask: torch.Tensor | None = None, scale: float = 1.0,
                 max_bias: float = 0.0, out: torch.Tensor | None = None) -> torch.Tensor:
    """ggml_soft_max_ext over the last dim of x (fp32, up to 4-d)."""
    if out is None:
        out = torch.empty_like(x)
    L = _lib.load()
    md = _desc(mask) if mask is not None else None
    check(L.gq_soft_max(_desc(x), md, scale, max_bias, _desc(out), _stream()))
    return out


# ---------------------------------------------------------------- decoder ops

def swiglu(a: torch.Tensor, b: torch.Tensor | None = None, swapped: bool = False,
           out: torch.Tensor | None = None) -> torch.Tensor:
    """ggml_swiglu(a): silu(a[..., :n]) * a[..., n:] (or ggml_swiglu_split(a, b))."""
    nc = a.shape[-1] if b is not None else a.shape[-1] // 2
    if out is None:
        out = torch.empty(a.shape[:-1] + (nc,), dtype=torch.float32, device=a.device)
    bd = _desc(b) if b is not None else None
    check(_lib.load().gq_swiglu(_desc(a), bd, _desc(out), int(swapped), _stream()))
    return out


def rms_norm(x: torch.Tensor, eps: float, out: torch.Tensor | None = None) -> torch.Tensor:
    """ggml_rms_norm(x, eps) over the last dim."""
    if out is None:
        out = torch.empty_like(x)
    check(_lib.load().gq_rms_norm(_desc(x), eps, _desc(out), _stream()))
    return out


def rope_ext(x: torch.Tensor, pos: torch.Tensor, n_dims: int, mode: int = 2, freq_base: float = 10000.0,
             freq_scale: float = 1.0, attn_factor: float = 1.0, out: torch.Tensor | None = None) -> torch.Tensor:
    """ggml_rope_ext: x fp32 ``[B, seq, heads, hd]`` (ggml [hd, heads, seq, B]), pos int32 ``[seq]``."""
    if out is None:
        out = torch.empty_like(x)
    check(_lib.load().gq_rope_ext(_desc(x), _desc(pos), n_dims, mode, 0, freq_base, freq_scale, 0.0,
                                  attn_factor, 0.0, 0.0, _desc(out), _stream()))
    return out


def rope_kv_store(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, pos: torch.Tensor, n_dims: int, mode: int,
                  freq_base: float, kv_idx: torch.Tensor, q_out: torch.Tensor, k_cache: torch.Tensor,
                  v_cache: torch.Tensor, freq_scale: float = 1.0, attn_factor: float = 1.0,
                  n_bad: torch.Tensor | None = None) -> torch.Tensor:
    """rope_ext(q) -> q_out and rope_ext(k), v -> set_rows into the F16 caches, one launch.
    q/k/v ``[1, s, H, hd]`` fp32 views; caches ``[1, Hkv, rows, hd]`` fp16; kv_idx int64 [s]."""
    nb_ptr = n_bad.data_ptr() if n_bad is not None else None
    check(_lib.load().gq_rope_kv_store(_desc(q), _desc(k), _desc(v), _desc(pos), n_dims, mode, freq_base, freq_scale,
                                       attn_factor, _desc(kv_idx), _desc(q_out), _desc(k_cache), _desc(v_cache),
                                       nb_ptr, _stream()))
    return q_out


def rope_cache(pos: torch.Tensor, n_dims: int, freq_base: float, freq_scale: float = 1.0, attn_factor: float = 1.0,
               out: torch.Tensor | None = None) -> torch.Tensor:
    """ggml_rope_cache_init for each position: fp32 [n, n_dims] of interleaved (cos, sin)."""
    if out is None:
        out = torch.empty((pos.shape[0], n_dims), dtype=torch.float32, device=pos.device)
    check(_lib.load().gq_rope_cache(_desc(pos), n_dims, freq_base, freq_scale, attn_factor, _desc(out), _stream()))
    return out


def add(a: torch.Tensor, b: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """ggml_add(a, b) with b repeated over a."""
    if out is None:
        out = torch.empty_like(a)
    check(_lib.load().gq_add(_desc(a), _desc(b), _desc(out), _stream()))
    return out


def get_rows(table, ids: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """ggml_get_rows(table, ids): table is a QWeight (rows of K) or an fp32/fp16 [rows, K] tensor."""
    if isinstance(table, QWeight):
        td, K = table.desc(), table.K
        dev = table.data.device
    else:
        td, K = _desc(table), table.shape[-1]
        dev = table.device
    if out is None:
        out = torch.empty((ids.shape[0], K), dtype=torch.float32, device=dev)
    check(_lib.load().gq_get_rows(td, _desc(ids), _desc(out), _stream()))
    return out


def argmax(x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """ggml_argmax over the last dim of a 2-d fp32 tensor -> int32 [rows]."""
    if out is None:
        out = torch.empty((x.shape[0],), dtype=torch.int32, device=x.device)
    check(_lib.load().gq_argmax(_desc(x), _desc(out), _stream()))
    return out


# ------------------------------------------------------------ KV step inputs

def kv_step_inputs(pos: torch.Tensor, s: int, pos_ids: torch.Tensor | None = None,
                   kv_idx: torch.Tensor | None = None, mask: torch.Tensor | None = None) -> None:
    """Fill pos_ids (int32 [s]), kv_idx (int64 [s]) and the fp16 causal mask [s, n_kv]
    from the device position ``pos`` (int32 [1])."""
    md = _desc(mask) if mask is not None else None
    check(_lib.load().gq_kv_step_inputs(pos.data_ptr(), s, pos_ids.data_ptr() if pos_ids is not None else None,
                                        kv_idx.data_ptr() if kv_idx is not None else None, md, _stream()))


def kv_advance(pos: torch.Tensor, s: int) -> None:
    """pos += s on the device."""
    check(_lib.load().gq_kv_advance(pos.data_ptr(), s, _stream()))


def mul_mat_workspace_size(w: QWeight, M: int) -> int:
    """Workspace bytes gq_mul_mat needs for M activation rows of this weight."""
    x = make_tensor(0, F32, [w.K, M], [4, w.K * 4])
    return int(_lib.load().gq_mul_mat_workspace_size(w.desc(), x))


def flash_attn_workspace_size(D: int, S: int, Hq: int, Hkv: int, n_kv: int) -> int:
    """Workspace bytes gq_flash_attn_ext needs for this shape."""
    q = make_tensor(0, F32, [D, S, Hq, 1], [4, D * 4, D * 4 * S, D * 4 * S * Hq])
    k = make_tensor(0, F16, [D, n_kv, Hkv, 1], [2, D * 2, D * 2 * n_kv, D * 2 * n_kv * Hkv])
    return int(_lib.load().gq_flash_attn_ext_workspace_size(q, k))
