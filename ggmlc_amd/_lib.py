"""ctypes binding of libgq.so (the C ABI declared in include/gq.h).

The library is loaded from this package directory. There is no fallback: if
libgq.so is missing or cannot be loaded, every op raises.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libgq.so"

# enum gq_type (ggml type ids)
F32, F16, Q4_0, Q8_0, I32, I64 = 0, 1, 2, 8, 26, 27
BLOCK_BYTES = {Q8_0: 34, Q4_0: 18}

GQ_OK = 0
GQ_OPT_ATTN_SEPARATE_MERGE = 1
GQ_OPT_GEMM_I8_RING = 2
GQ_ATTN_SCRATCH_BYTES = 16 << 20  # gq_flash_attn_ext_noalloc's static scratch per device
_ERR_NAMES = {-1: "GQ_ERR_INVALID", -2: "GQ_ERR_UNSUPPORTED", -3: "GQ_ERR_WORKSPACE", -4: "GQ_ERR_DEVICE"}


class GQError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"{_ERR_NAMES.get(code, code)}: {msg}")
        self.code = code


class gq_tensor(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("type", ctypes.c_int32),
        ("pad_", ctypes.c_int32),
        ("ne", ctypes.c_int64 * 4),
        ("nb", ctypes.c_size_t * 4),
    ]


class gq_rope_kv_epilogue(ctypes.Structure):
    _fields_ = [
        ("n_head", ctypes.c_int32),
        ("n_head_kv", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("pos", ctypes.POINTER(gq_tensor)),
        ("n_dims", ctypes.c_int32),
        ("mode", ctypes.c_int32),
        ("freq_base", ctypes.c_float),
        ("freq_scale", ctypes.c_float),
        ("attn_factor", ctypes.c_float),
        ("kv_idx", ctypes.POINTER(gq_tensor)),
        ("q_out", ctypes.POINTER(gq_tensor)),
        ("k_cache", ctypes.POINTER(gq_tensor)),
        ("v_cache", ctypes.POINTER(gq_tensor)),
        ("n_bad", ctypes.c_void_p),
        ("rope_cache", ctypes.POINTER(gq_tensor)),
    ]


class gq_exec_profile(ctypes.Structure):
    _fields_ = [
        ("prepare_ms", ctypes.c_double),
        ("set_decode_pos_ms", ctypes.c_double),
        ("set_chunk_pos_ms", ctypes.c_double),
        ("mask_fill_ms", ctypes.c_double),
        ("run_ms", ctypes.c_double),
        ("n_prepare", ctypes.c_int32),
        ("n_set_decode_pos", ctypes.c_int32),
        ("n_set_chunk_pos", ctypes.c_int32),
        ("n_run", ctypes.c_int32),
    ]


class gq_mul_mat_fusion(ctypes.Structure):
    _fields_ = [
        ("rms_norm", ctypes.c_int32),
        ("rms_eps", ctypes.c_float),
        ("swiglu", ctypes.c_int32),
        ("add", ctypes.POINTER(gq_tensor)),
        ("b_add", ctypes.POINTER(gq_tensor)),
        ("b_sum", ctypes.POINTER(gq_tensor)),
        ("rope_kv", ctypes.POINTER(gq_rope_kv_epilogue)),
        ("b_swiglu", ctypes.c_int32),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_size_t),
        ("bias", ctypes.POINTER(gq_tensor)),
        ("out_q8", ctypes.c_void_p),
        ("b_q8", ctypes.c_void_p),
        ("int8", ctypes.c_int32),
        ("out_halves", ctypes.c_int32),
        ("b_add_halves", ctypes.c_int32),
    ]


_P = ctypes.POINTER(gq_tensor)
_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_f32 = ctypes.c_float

# name -> (restype, argtypes); exactly the entry points of include/gq.h
SIGNATURES = {
    "gq_abi_version": (ctypes.c_int, []),
    "gq_last_error": (ctypes.c_char_p, []),
    "gq_init": (ctypes.c_int, []),
    "gq_set_option": (ctypes.c_int, [ctypes.c_int, _i64]),
    "gq_quantize_row_q8_0": (ctypes.c_int, [_vp, _vp, _i64, _vp]),
    "gq_quantize_weights": (ctypes.c_int, [ctypes.c_int, _vp, _vp, _i64, _vp]),
    "gq_mul_mat_workspace_size": (ctypes.c_size_t, [_P, _P]),
    "gq_mul_mat": (ctypes.c_int, [_P, _P, _P, _vp, ctypes.c_size_t, _vp]),
    "gq_mul_mat_fused": (ctypes.c_int, [_P, _P, _P, ctypes.POINTER(gq_mul_mat_fusion), _vp]),
    "gq_rope_cache": (ctypes.c_int, [_P, ctypes.c_int, _f32, _f32, _f32, _P, _vp]),
    "gq_set_rows": (ctypes.c_int, [_P, _P, _P, _vp, _vp]),
    "gq_flash_attn_ext_workspace_size": (ctypes.c_size_t, [_P, _P]),
    "gq_flash_attn_ext": (ctypes.c_int, [_P, _P, _P, _P, _f32, _f32, _f32, _P, _vp, ctypes.c_size_t, _vp]),
    "gq_flash_attn_ext_noalloc": (ctypes.c_int, [_P, _P, _P, _P, _f32, _f32, _f32, _P, _vp]),
    "gq_attn_reset_counters": (ctypes.c_int, [_vp]),
    "gq_soft_max": (ctypes.c_int, [_P, _P, _f32, _f32, _P, _vp]),
    "gq_swiglu": (ctypes.c_int, [_P, _P, _P, ctypes.c_int, _vp]),
    "gq_rms_norm": (ctypes.c_int, [_P, _f32, _P, _vp]),
    "gq_rope_ext": (ctypes.c_int, [_P, _P, ctypes.c_int, ctypes.c_int, ctypes.c_int, _f32, _f32, _f32, _f32, _f32,
                                   _f32, _P, _vp]),
    "gq_rope_kv_store": (ctypes.c_int, [_P, _P, _P, _P, ctypes.c_int, ctypes.c_int, _f32, _f32, _f32, _P, _P, _P,
                                        _P, _vp, _vp]),
    "gq_add": (ctypes.c_int, [_P, _P, _P, _vp]),
    "gq_get_rows": (ctypes.c_int, [_P, _P, _P, _vp]),
    "gq_argmax": (ctypes.c_int, [_P, _P, _vp]),
    "gq_kv_step_inputs": (ctypes.c_int, [_vp, _i64, _vp, _vp, _P, _vp]),
    "gq_kv_advance": (ctypes.c_int, [_vp, _i64, _vp]),
    "gq_mul_mat_fused_workspace_size": (ctypes.c_size_t, [_P, _P, ctypes.POINTER(gq_mul_mat_fusion)]),
    "gq_mul_mat_fused_halves": (ctypes.c_int, [_P, _P, ctypes.POINTER(gq_mul_mat_fusion)]),
    "gq_flash_attn_paged_workspace_size": (ctypes.c_size_t, [_P, _P, _i64, _i64]),
    "gq_flash_attn_paged": (ctypes.c_int, [_P, _P, _P, _P, _P, _i64, _i64, _f32, _P, _vp, ctypes.c_size_t, _vp]),
    "gq_flash_attn_paged_q8": (ctypes.c_int, [_P, _P, _P, _P, _P, _i64, _i64, _f32, _P, _vp, _vp, ctypes.c_size_t,
                                              _vp]),
    "gq_q8_rows_bytes": (ctypes.c_size_t, [_i64]),
    "gq_paged_step_inputs": (ctypes.c_int, [_vp, _i64, _P, _i64, _i64, _vp, _vp, _vp]),
    "gq_paged_advance": (ctypes.c_int, [_vp, _vp, _i64, _vp]),
    "gq_kv_pages_copy": (ctypes.c_int, [_P, _P, _vp, _i64, _i64, _i64, _i64, ctypes.c_int, _vp]),
    "gq_exec_available_devices": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_size_t, ctypes.POINTER(ctypes.c_size_t)]),
    "gq_exec_create": (ctypes.c_int, [_vp, ctypes.c_size_t, ctypes.c_char_p, ctypes.POINTER(_vp)]),
    "gq_exec_free": (None, [_vp]),
    "gq_exec_describe": (ctypes.c_int, [_vp, ctypes.c_char_p, ctypes.c_size_t, ctypes.POINTER(ctypes.c_size_t)]),
    "gq_exec_inspect": (ctypes.c_int, [_vp, ctypes.c_size_t, ctypes.c_char_p, ctypes.c_size_t,
                                       ctypes.POINTER(ctypes.c_size_t)]),
    "gq_exec_prepare": (ctypes.c_int, [_vp, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(_i64), _i64]),
    "gq_exec_set_input": (ctypes.c_int, [_vp, ctypes.c_uint32, _vp, ctypes.c_size_t]),
    "gq_exec_set_input_by_name": (ctypes.c_int, [_vp, ctypes.c_char_p, _vp, ctypes.c_size_t]),
    "gq_exec_run": (ctypes.c_int, [_vp]),
    "gq_exec_synchronize": (ctypes.c_int, [_vp]),
    "gq_exec_get_tensor_shape": (ctypes.c_int, [_vp, ctypes.c_uint32, ctypes.POINTER(_i64)]),
    "gq_exec_get_output": (ctypes.c_int, [_vp, ctypes.c_uint32, _vp, ctypes.c_size_t,
                                          ctypes.POINTER(ctypes.c_size_t)]),
    "gq_exec_init_kv_cache": (ctypes.c_int, [_vp, _i64]),
    "gq_exec_reset_kv_cache": (ctypes.c_int, [_vp]),
    "gq_exec_has_kv_cache": (ctypes.c_int, [_vp]),
    "gq_exec_set_logits_last_only": (ctypes.c_int, [_vp, ctypes.c_int]),
    "gq_exec_logits_last_only": (ctypes.c_int, [_vp]),
    "gq_exec_set_enable_graphs": (ctypes.c_int, [_vp, ctypes.c_int]),
    "gq_exec_position": (_i64, [_vp]),
    "gq_exec_set_tokens_per_page": (ctypes.c_int, [_vp, _i64]),
    "gq_exec_get_tokens_per_page": (_i64, [_vp]),
    "gq_exec_init_paged_kv_cache": (ctypes.c_int, [_vp, _i64, _i64]),
    "gq_exec_is_paged_kv_cache_enabled": (ctypes.c_int, [_vp]),
    "gq_exec_paged_kv_alloc_slot": (ctypes.c_int, [_vp, _i64]),
    "gq_exec_paged_kv_free_slot": (ctypes.c_int, [_vp, _i64]),
    "gq_exec_is_paged_slot_allocated": (ctypes.c_int, [_vp, _i64]),
    "gq_exec_paged_kv_ensure_tokens": (ctypes.c_int, [_vp, _i64, _i64]),
    "gq_exec_paged_kv_map_existing_pages": (ctypes.c_int, [_vp, _i64, _i64, ctypes.POINTER(ctypes.c_int32), _i64]),
    "gq_exec_paged_kv_extract_page": (ctypes.c_int, [_vp, _i64, _i64, ctypes.POINTER(ctypes.c_int32)]),
    "gq_exec_paged_page_retain": (ctypes.c_int, [_vp, ctypes.c_int32]),
    "gq_exec_paged_page_release": (ctypes.c_int, [_vp, ctypes.c_int32]),
    "gq_exec_get_paged_active_vram_bytes": (ctypes.c_size_t, [_vp]),
    "gq_exec_paged_slot_position": (ctypes.c_int, [_vp, _i64, ctypes.POINTER(_i64)]),
    "gq_exec_paged_set_slot_position": (ctypes.c_int, [_vp, _i64, _i64]),
    "gq_exec_set_enable_profile": (ctypes.c_int, [_vp, ctypes.c_int]),
    "gq_exec_reset_profile": (ctypes.c_int, [_vp]),
    "gq_exec_get_profile": (ctypes.c_int, [_vp, ctypes.POINTER(gq_exec_profile)]),
    "gq_exec_runtime_graph_summary": (ctypes.c_int, [_vp, ctypes.c_char_p, ctypes.c_size_t,
                                                     ctypes.POINTER(ctypes.c_size_t)]),
    "gq_exec_runtime_mul_mat_shape_summary": (ctypes.c_int, [_vp, ctypes.c_char_p, ctypes.c_size_t,
                                                             ctypes.POINTER(ctypes.c_size_t)]),
}

_lib = None


def load() -> ctypes.CDLL:
    """Load libgq.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is not built; run `python -m ggmlc_amd.build` (or __graft_entry__.build())"
            )
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def check(rc: int) -> None:
    if rc != GQ_OK:
        raise GQError(rc, load().gq_last_error().decode(errors="replace"))


def make_tensor(ptr: int, gtype: int, ne, nb) -> gq_tensor:
    t = gq_tensor()
    t.data = ptr
    t.type = gtype
    ne = list(ne) + [1] * (4 - len(ne))
    nb = list(nb)
    while len(nb) < 4:
        nb.append(nb[-1] * ne[len(nb) - 1])
    for i in range(4):
        t.ne[i] = int(ne[i])
        t.nb[i] = int(nb[i])
    return t
