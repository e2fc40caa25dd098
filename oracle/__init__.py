"""CPU oracle for the quantized hot path — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg import this package, and only as the checker. The product package
(``ggmlc_amd``) never imports it.

Two libraries are wrapped:

* ``liboracle.so`` — this repo's C restatement (``gq_oracle.c``) of the
  reference's quantize / mul_mat / set_rows / flash_attn_ext / soft_max.
* ``_ref/libggmlref.so`` — the reference's own ggml 0.20.2 CPU backend compiled
  from ``/root/reference/third_party/ggml`` by ``oracle/Makefile`` (present only
  where that build ran; tests that need it skip otherwise).
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ORACLE_SO = HERE / "liboracle.so"
REF_SO = HERE / "_ref" / "libggmlref.so"
REF_V4_SO = HERE / "_ref" / "v4" / "libggmlref.so"

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_f32 = ctypes.c_float

Q8_0, Q4_0 = 8, 2
BLOCK_BYTES = {Q8_0: 34, Q4_0: 18}


def _ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(_vp)


def build() -> None:
    """Compile the restatement (and the reference build where the tree exists)."""
    import subprocess

    subprocess.run(["make", "-s", "-C", str(HERE), "all"], check=True)


_lib = None
_ref = None


def lib():
    global _lib
    if _lib is None:
        if not ORACLE_SO.exists():
            build()
        L = ctypes.CDLL(str(ORACLE_SO))
        L.or_fp32_to_fp16.restype = ctypes.c_uint16
        L.or_fp32_to_fp16.argtypes = [_f32]
        L.or_fp16_to_fp32.restype = _f32
        L.or_fp16_to_fp32.argtypes = [ctypes.c_uint16]
        for n in ("or_fp32_to_fp16_row", "or_quantize_row_q8_0", "or_quantize_row_q8_0_ref",
                  "or_quantize_q8_0_py", "or_quantize_q4_0_py", "or_dequantize_row_q8_0",
                  "or_dequantize_row_q4_0"):
            getattr(L, n).argtypes = [_vp, _vp, _i64]
            getattr(L, n).restype = None
        L.or_mul_mat.argtypes = [_i32, _vp, _i64, _i64, _vp, _i64, _vp, _i32]
        L.or_mul_mat_q8act.argtypes = [_i32, _vp, _i64, _i64, _vp, _i64, _vp, _i32]
        L.or_set_rows_f32_f16.argtypes = [_vp, _i64, _i64, _i64, _i64, _vp, _i64, _vp]
        L.or_flash_attn_ext_f16.argtypes = [_vp, _i64, _i64, _i64, _vp, _vp, _i64, _i64, _i64,
                                            _vp, _f32, _vp, _i32, _i32]
        L.or_soft_max_f32.argtypes = [_vp, _i64, _i64, _vp, _f32, _vp]
        L.or_pad_kv_len.restype = _i64
        L.or_pad_kv_len.argtypes = [_i64, _i64, _i64]
        L.or_fill_causal_mask_f16.argtypes = [_vp, _i64, _i64, _i64]
        _lib = L
    return _lib


def ref_available() -> bool:
    return REF_SO.exists()


def ref(variant: str = "v3"):
    """The compiled reference ggml CPU backend (raises if it was not built). variant
    "v3" is the x86-64-v3 build the tests use; "v4" the AVX-512 + VNNI build of the same
    sources (oracle/Makefile ref-v4), for timing on hosts that support it."""
    global _ref
    if variant == "v4":
        return _load_ref(REF_V4_SO, "v4")
    if _ref is None:
        _ref = _load_ref(REF_SO, "v3")
    return _ref


_ref_v4 = None


def ref_v4_usable() -> bool:
    """The AVX-512 build exists and this host's CPU has the instructions it uses."""
    if not REF_V4_SO.exists():
        return False
    try:
        flags = set()
        for line in open("/proc/cpuinfo"):
            if line.startswith("flags"):
                flags = set(line.split(":", 1)[1].split())
                break
    except OSError:
        return False
    return {"avx512f", "avx512bw", "avx512dq", "avx512vl", "avx512cd", "avx512_vnni"} <= flags


def _load_ref(path, variant):
    global _ref_v4
    if variant == "v4" and _ref_v4 is not None:
        return _ref_v4
    if not path.exists():
        raise FileNotFoundError(f"{path} not built (needs /root/reference)")
    L = ctypes.CDLL(str(path))
    L.ref_ggml_version.restype = ctypes.c_char_p
    for n in ("ref_quantize_row_q8_0", "ref_quantize_row_q8_0_ref"):
        getattr(L, n).argtypes = [_vp, _vp, _i64]
        getattr(L, n).restype = None
    L.ref_mul_mat.argtypes = [_i32, _vp, _i64, _i64, _vp, _i64, _vp, _i32]
    L.ref_set_rows_f32_f16.argtypes = [_vp, _i64, _i64, _i64, _i64, _vp, _i64, _vp, _i32]
    L.ref_flash_attn_ext_f16.argtypes = [_vp, _i64, _i64, _i64, _vp, _vp, _i64, _i64, _i64,
                                         _vp, _f32, _vp, _i32]
    L.ref_soft_max_f32.argtypes = [_vp, _i64, _i64, _vp, _f32, _vp, _i32]
    L.ref_mm_create.restype = _vp
    L.ref_mm_create.argtypes = [_i32, _vp, _i64, _i64, _i64]
    L.ref_mlp_create.restype = _vp
    L.ref_mlp_create.argtypes = [_i32, _vp, _vp, _i64, _i64, _i64]
    L.ref_graph_run.argtypes = [_vp, _vp, _vp, _i32]
    L.ref_graph_free.argtypes = [_vp]
    L.ref_graph_free.restype = None
    L.ref_swiglu.argtypes = [_vp, _i64, _i64, _vp]
    L.ref_rms_norm.argtypes = [_vp, _i64, _i64, _f32, _vp]
    L.ref_rope.argtypes = [_vp, _i64, _i64, _i64, _vp, _i32, _i32, _f32, _vp]
    L.ref_get_rows.argtypes = [_i32, _vp, _i64, _i64, _vp, _i64, _vp]
    L.ref_argmax.argtypes = [_vp, _i64, _i64, _vp]
    L.ref_llama_create.restype = _vp
    L.ref_llama_create.argtypes = [_vp, _i32, _f32, _f32, _vp, _vp, _vp, _vp]
    L.ref_llama_step.argtypes = [_vp, _vp, _i64, _i64, _i64, _vp, _vp, _vp, _i32]
    L.ref_llama_set_bias.argtypes = [_vp, _i64, _i32, _vp, _i64]
    L.ref_llama_free.argtypes = [_vp]
    L.ref_llama_free.restype = None
    L.ref_rt_last_error.restype = ctypes.c_char_p
    L.ref_rt_load.restype = _vp
    L.ref_rt_load.argtypes = [ctypes.c_char_p]
    L.ref_rt_free.argtypes = [_vp]
    L.ref_rt_free.restype = None
    L.ref_rt_describe.restype = _i64
    L.ref_rt_describe.argtypes = [_vp, ctypes.c_char_p, _i64]
    L.ref_rt_init_kv.argtypes = [_vp, _i64]
    L.ref_rt_reset_kv.argtypes = [_vp]
    L.ref_rt_run.argtypes = [_vp, ctypes.POINTER(ctypes.c_char_p), _vp, _i32, _vp, ctypes.POINTER(_vp), _vp,
                             _i32, _i32]
    L.ref_rt_output.restype = _i64
    L.ref_rt_output.argtypes = [_vp, ctypes.c_uint32, _vp, _vp, _i64]
    L.ref_init()
    if variant == "v4":
        _ref_v4 = L
    return L


# ----------------------------------------------------------------- numpy API

def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def fp32_to_fp16_bits(x) -> np.ndarray:
    x = _c(x, np.float32)
    y = np.empty(x.shape, np.uint16)
    lib().or_fp32_to_fp16_row(_ptr(x), _ptr(y), x.size)
    return y


def quantize_row_q8_0(x, impl: str = "oracle") -> np.ndarray:
    """x86 activation quantizer on each row of x ([..., K]); returns uint8 [..., K/32*34]."""
    x = _c(x, np.float32)
    K = x.shape[-1]
    y = np.empty(x.shape[:-1] + (K // 32 * 34,), np.uint8)
    f = lib().or_quantize_row_q8_0 if impl == "oracle" else ref().ref_quantize_row_q8_0
    f(_ptr(x), _ptr(y), x.size)
    return y


def quantize_row_q8_0_ref(x, impl: str = "oracle") -> np.ndarray:
    """ggml's scalar reference quantizer quantize_row_q8_0_ref (ggml-quants.c:276-299):
    d = amax/127, q = roundf(x * (1/d)) (halves away from zero, unlike the x86 path's
    round-to-nearest-even). Not on the GPU path; kept as the textbook statement the x86
    quantizer is compared with."""
    x = _c(x, np.float32)
    K = x.shape[-1]
    y = np.empty(x.shape[:-1] + (K // 32 * 34,), np.uint8)
    f = lib().or_quantize_row_q8_0_ref if impl == "oracle" else ref().ref_quantize_row_q8_0_ref
    f(_ptr(x), _ptr(y), x.size)
    return y


def quantize_weights(w, wtype: int) -> np.ndarray:
    """ggmlc's Python weight quantizer semantics; w [N, K] -> uint8 [N, K/32*block]."""
    w = _c(w, np.float32)
    N, K = w.shape
    y = np.empty((N, K // 32 * BLOCK_BYTES[wtype]), np.uint8)
    f = lib().or_quantize_q8_0_py if wtype == Q8_0 else lib().or_quantize_q4_0_py
    f(_ptr(w), _ptr(y), w.size)
    return y


def dequantize(wq, wtype: int, K: int) -> np.ndarray:
    wq = _c(wq, np.uint8)
    N = wq.size // (K // 32 * BLOCK_BYTES[wtype])
    y = np.empty((N, K), np.float32)
    f = lib().or_dequantize_row_q8_0 if wtype == Q8_0 else lib().or_dequantize_row_q4_0
    f(_ptr(wq), _ptr(y), N * K)
    return y


def mul_mat(wq, wtype: int, K: int, x, impl: str = "oracle", n_threads: int = 8) -> np.ndarray:
    """Y[M, N] = ggml_mul_mat(W[N rows of K], X[M, K])."""
    wq = _c(wq, np.uint8)
    x = _c(x, np.float32).reshape(-1, K)
    M = x.shape[0]
    N = wq.size // (K // 32 * BLOCK_BYTES[wtype])
    y = np.empty((M, N), np.float32)
    if impl == "oracle":
        r = lib().or_mul_mat(wtype, _ptr(wq), K, N, _ptr(x), M, _ptr(y), n_threads)
    else:
        r = ref().ref_mul_mat(wtype, _ptr(wq), K, N, _ptr(x), M, _ptr(y), n_threads)
    if r != 0:
        raise RuntimeError("mul_mat failed")
    return y


def set_rows_f32_f16(cache: np.ndarray, src, idx, impl: str = "oracle") -> np.ndarray:
    """cache uint16 [B, H, max_ctx, hd] (ggml [hd, max_ctx, H, B]) updated in a copy."""
    out = np.array(cache, dtype=np.uint16, copy=True, order="C")
    B, H, max_ctx, hd = out.shape
    src = _c(src, np.float32)
    s = src.shape[-2]
    idx = _c(idx, np.int64)
    if impl == "oracle":
        r = lib().or_set_rows_f32_f16(_ptr(out), hd, max_ctx, H, B, _ptr(src), s, _ptr(idx))
    else:
        r = ref().ref_set_rows_f32_f16(_ptr(out), hd, max_ctx, H, B, _ptr(src), s, _ptr(idx), 1)
    if r != 0:
        raise ValueError("set_rows: index out of range")
    return out


def flash_attn_ext_f16(q, kc, vc, n_kv: int, mask=None, scale: float | None = None,
                       impl: str = "oracle", mode: int = 0, n_threads: int = 1) -> np.ndarray:
    """q fp32 [Hq, s, hd]; kc/vc uint16 [Hkv, max_ctx, hd]; mask uint16 [s, n_kv] or None.

    Returns fp32 [s, Hq, hd] (the op's permuted output)."""
    q = _c(q, np.float32)
    Hq, s, hd = q.shape
    kc = _c(kc, np.uint16)
    vc = _c(vc, np.uint16)
    Hkv, max_ctx, _ = kc.shape
    if scale is None:
        scale = 1.0 / float(np.sqrt(np.float32(hd)))
    m = None if mask is None else _c(mask, np.uint16)
    out = np.empty((s, Hq, hd), np.float32)
    if impl == "oracle":
        r = lib().or_flash_attn_ext_f16(_ptr(q), hd, s, Hq, _ptr(kc), _ptr(vc), max_ctx, Hkv, n_kv,
                                        _ptr(m), scale, _ptr(out), mode, n_threads)
    else:
        r = ref().ref_flash_attn_ext_f16(_ptr(q), hd, s, Hq, _ptr(kc), _ptr(vc), max_ctx, Hkv, n_kv,
                                         _ptr(m), scale, _ptr(out), n_threads)
    if r != 0:
        raise RuntimeError("flash_attn_ext failed")
    return out


def soft_max_f32(x, mask=None, scale: float = 1.0, impl: str = "oracle") -> np.ndarray:
    x = _c(x, np.float32)
    nrows, ncols = x.shape
    m = None if mask is None else _c(mask, np.uint16)
    y = np.empty_like(x)
    if impl == "oracle":
        lib().or_soft_max_f32(_ptr(x), ncols, nrows, _ptr(m), scale, _ptr(y))
    else:
        ref().ref_soft_max_f32(_ptr(x), ncols, nrows, _ptr(m), scale, _ptr(y), 1)
    return y


def pad_kv_len(n_kv: int, max_ctx: int, n_pad: int = 256) -> int:
    return int(lib().or_pad_kv_len(n_kv, max_ctx, n_pad))


def causal_mask_f16(pos: int, s_q: int, s_kv: int) -> np.ndarray:
    m = np.empty((s_q, s_kv), np.uint16)
    lib().or_fill_causal_mask_f16(_ptr(m), pos, s_q, s_kv)
    return m


def n_cpu_threads() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        return os.cpu_count() or 1


class RefGraph:
    """A persistent one-input graph on the reference ggml CPU backend (timing only)."""

    def __init__(self, handle, x_shape, y_shape, keep):
        self.h = handle
        self.x_shape = x_shape
        self.y_shape = y_shape
        self._keep = keep  # weight buffers referenced until creation copied them

    def run(self, x: np.ndarray, n_threads: int) -> np.ndarray:
        x = _c(x, np.float32)
        y = np.empty(self.y_shape, np.float32)
        if ref().ref_graph_run(self.h, _ptr(x), _ptr(y), n_threads) != 0:
            raise RuntimeError("ref graph run failed")
        return y

    def close(self):
        if self.h:
            ref().ref_graph_free(self.h)
            self.h = None

    def __del__(self):  # pragma: no cover
        try:
            self.close()
        except Exception:
            pass


def ref_mm_graph(wq: np.ndarray, wtype: int, K: int, M: int) -> RefGraph:
    wq = _c(wq, np.uint8)
    N = wq.size // (K // 32 * BLOCK_BYTES[wtype])
    h = ref().ref_mm_create(wtype, _ptr(wq), K, N, M)
    if not h:
        raise RuntimeError("ref_mm_create failed")
    return RefGraph(h, (M, K), (M, N), None)


def ref_mlp_graph(w_gate_up: np.ndarray, w_down: np.ndarray, wtype: int, K: int, F: int, M: int) -> RefGraph:
    a = _c(w_gate_up, np.uint8)
    b = _c(w_down, np.uint8)
    h = ref().ref_mlp_create(wtype, _ptr(a), _ptr(b), K, F, M)
    if not h:
        raise RuntimeError("ref_mlp_create failed")
    return RefGraph(h, (M, K), (M, K), None)


def ref_swiglu(a) -> np.ndarray:
    a = _c(a, np.float32)
    nrows, n2 = a.shape
    y = np.empty((nrows, n2 // 2), np.float32)
    ref().ref_swiglu(_ptr(a), n2 // 2, nrows, _ptr(y))
    return y


def ref_rms_norm(x, eps: float) -> np.ndarray:
    x = _c(x, np.float32)
    y = np.empty_like(x)
    ref().ref_rms_norm(_ptr(x), x.shape[-1], x.size // x.shape[-1], eps, _ptr(y))
    return y


def ref_rope(x, pos, n_dims: int, mode: int = 2, freq_base: float = 10000.0) -> np.ndarray:
    """x fp32 [seq, heads, hd] (ggml [hd, heads, seq]), pos int32 [seq]."""
    x = _c(x, np.float32)
    p = _c(pos, np.int32)
    seq, heads, hd = x.shape
    y = np.empty_like(x)
    ref().ref_rope(_ptr(x), hd, heads, seq, _ptr(p), n_dims, mode, freq_base, _ptr(y))
    return y


def ref_get_rows(table: np.ndarray, wtype: int, n_embd: int, ids) -> np.ndarray:
    t = _c(table, np.uint8 if wtype in BLOCK_BYTES else (np.float16 if wtype == 1 else np.float32))
    ids = _c(ids, np.int32)
    if wtype in BLOCK_BYTES:
        rows = t.size // (n_embd // 32 * BLOCK_BYTES[wtype])
    else:
        rows = t.size // n_embd
    y = np.empty((ids.size, n_embd), np.float32)
    ref().ref_get_rows(wtype, _ptr(t), n_embd, rows, _ptr(ids), ids.size, _ptr(y))
    return y


def ref_argmax(x) -> np.ndarray:
    x = _c(x, np.float32)
    out = np.empty(x.shape[0], np.int32)
    ref().ref_argmax(_ptr(x), x.shape[1], x.shape[0], _ptr(out))
    return out


class RefLlama:
    """The reference ggml CPU backend running ggmlc's LLaMA decoder graph
    (ref_driver.cpp ref_llama_*): persistent F16 KV caches held here, weights
    referenced in place (the caller keeps the arrays alive).

    cfg needs n_layer, n_embd, n_head, n_head_kv, head_dim, n_ff, n_vocab, qtype,
    rms_eps, rope_base; weights = (embed, lm_head, [(qkv, o, gate_up, down), ...])
    as uint8 GGUF block bytes. A layer tuple may carry four more entries, the fp32 biases
    of the same projections (None where a projection has none): the MUL_MAT node's
    bias ADD (executor.cpp:2436-2445)."""

    def __init__(self, cfg, weights, max_ctx: int, n_threads: int = 8, variant: str = "v3"):
        embed, lm_head, layers = weights
        self._R = ref(variant)
        self.cfg, self.max_ctx, self.n_threads = cfg, max_ctx, n_threads
        self._w = [_c(embed, np.uint8), _c(lm_head, np.uint8)] + [_c(m, np.uint8) for L in layers for m in L[:4]]
        self.kc = [np.zeros((cfg.n_head_kv, max_ctx, cfg.head_dim), np.uint16) for _ in layers]
        self.vc = [np.zeros_like(k) for k in self.kc]
        dims = np.array([cfg.n_layer, cfg.n_embd, cfg.n_head, cfg.n_head_kv, cfg.head_dim, cfg.n_ff,
                         cfg.n_vocab, max_ctx], np.int64)
        lw = (_vp * (4 * len(layers)))(*[a.ctypes.data for a in self._w[2:]])
        kv = (_vp * (2 * len(layers)))(*[a.ctypes.data for pair in zip(self.kc, self.vc) for a in pair])
        self.h = self._R.ref_llama_create(_ptr(dims), cfg.qtype, cfg.rms_eps, cfg.rope_base, _ptr(self._w[0]),
                                        _ptr(self._w[1]), lw, kv)
        if not self.h:
            raise RuntimeError("ref_llama_create failed")
        self._b = []
        for li, L in enumerate(layers):
            for which, b in enumerate(L[4:8]):
                if b is None:
                    continue
                b = _c(b, np.float32)
                self._b.append(b)
                if self._R.ref_llama_set_bias(self.h, li, which, _ptr(b), b.size) != 0:
                    raise RuntimeError("ref_llama_set_bias failed")
        self.pos = 0

    def step(self, ids):
        """Run the tokens at the current position; returns (last-token logits, argmax)."""
        ids = _c(ids, np.int32)
        s = ids.size
        n_kv = pad_kv_len(self.pos + s, self.max_ctx)
        mask = causal_mask_f16(self.pos, s, n_kv)
        logits = np.empty(self.cfg.n_vocab, np.float32)
        nxt = np.zeros(1, np.int32)
        if self._R.ref_llama_step(self.h, _ptr(ids), s, self.pos, n_kv, _ptr(mask), _ptr(logits), _ptr(nxt),
                                self.n_threads) != 0:
            raise RuntimeError("ref_llama_step failed")
        self.pos += s
        return logits, int(nxt[0])

    def __del__(self):
        if getattr(self, "h", None):
            self._R.ref_llama_free(self.h)
            self.h = None



class RefRuntime:
    """ggmlc's own runtime (ref_runtime.cpp over the reference's loader.cpp and
    executor.cpp) on the CPU: load a .gguf with the reference loader, run it with
    the reference executor (prepare(symbols) -> set_input -> run, the calls of
    python/ggmlc/runtime/runner.py:97-214)."""

    def __init__(self, path, max_ctx: int | None = None, n_threads: int = 8):
        self.h = ref().ref_rt_load(str(path).encode())
        if not self.h:
            raise RuntimeError("reference loader: " + ref().ref_rt_last_error().decode())
        self.n_threads = n_threads
        if max_ctx is not None and ref().ref_rt_init_kv(self.h, max_ctx) != 0:
            raise RuntimeError("reference init_kv_cache: " + ref().ref_rt_last_error().decode())

    def describe(self) -> list[str]:
        """The loaded graph as the reference loader sees it (ref_rt_describe lines)."""
        n = ref().ref_rt_describe(self.h, None, 0)
        buf = ctypes.create_string_buffer(int(n))
        ref().ref_rt_describe(self.h, buf, n)
        return buf.value.decode().splitlines()

    def reset_kv(self) -> None:
        ref().ref_rt_reset_kv(self.h)

    def run(self, inputs: dict, symbols: dict | None = None) -> None:
        """inputs: tensor id -> numpy array (raw bytes are passed)."""
        symbols = symbols or {}
        names = (ctypes.c_char_p * max(1, len(symbols)))(*[k.encode() for k in symbols])
        vals = np.array(list(symbols.values()) or [0], np.int64)
        arrs = [np.ascontiguousarray(a) for a in inputs.values()]
        tids = np.array(list(inputs.keys()) or [0], np.uint32)
        datas = (_vp * max(1, len(arrs)))(*[a.ctypes.data for a in arrs])
        sizes = np.array([a.nbytes for a in arrs] or [0], np.int64)
        if ref().ref_rt_run(self.h, names, vals.ctypes.data, len(symbols), tids.ctypes.data, datas,
                            sizes.ctypes.data, len(arrs), self.n_threads) != 0:
            raise RuntimeError("reference executor: " + ref().ref_rt_last_error().decode())

    def output(self, tid: int, dtype=np.float32) -> np.ndarray:
        """Output tensor bytes as a C-order array of shape reversed(ne)."""
        ne = np.zeros(4, np.int64)
        n = ref().ref_rt_output(self.h, tid, ne.ctypes.data, None, 0)
        if n < 0:
            raise RuntimeError("reference output: " + ref().ref_rt_last_error().decode())
        out = np.empty(int(n), np.uint8)
        ref().ref_rt_output(self.h, tid, ne.ctypes.data, out.ctypes.data, n)
        return out.view(dtype).reshape([int(d) for d in ne[::-1]])

    def __del__(self):
        if getattr(self, "h", None):
            ref().ref_rt_free(self.h)
            self.h = None
