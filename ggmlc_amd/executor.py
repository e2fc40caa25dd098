"""ggmlc's ModelExecutor surface (runtime/include/ggmlc/executor.h:25-289 as bound at
runtime/bindings/python_bindings.cpp:137-216) over libgq's executor handle
(`gq_exec_*` in include/gq.h): no torch on this path.

    ex = ModelExecutor(open("model.gguf", "rb").read(), device="gpu")
    ex.init_kv_cache(2048)
    ex.prepare({"s": len(ids), "pos": 0})
    ex.set_input_by_id(ex.inputs[0], np.asarray(ids, np.int32))
    ex.run()
    logits = np.frombuffer(ex.get_output_bytes(ex.outputs[0]), np.float32)

Errors raise ggmlc_amd.GQError (a RuntimeError), and a rejected call leaves the
executor usable, as the reference's std::runtime_error / std::invalid_argument do.

The paged-KV methods of the reference executor (`init_paged_kv_cache`, `paged_kv_*`,
`set_tokens_per_page`, `get_paged_active_vram_bytes`, executor.cpp:634-920) are native
here too: with the paged cache on, `prepare({"s": n, "slot": i, "pos": p})` is a prompt
step of slot i and `prepare({"b": B, "s": 1})` one decode token for slots [0, B), each at
its own position — the protocol of the reference's C++ scheduler
(batch_scheduler.cpp:190-194, 318-321). Page handles are int32 page ids.
"""

from __future__ import annotations

import ctypes
import json

import numpy as np

from . import _lib
from ._lib import GQError, check


def available() -> bool:
    """libgq.so with the executor entry points is built."""
    try:
        return hasattr(_lib.load(), "gq_exec_create")
    except RuntimeError:
        return False


def get_available_devices() -> list[str]:
    """ModelExecutor::get_available_devices: the visible GPUs as "cuda:N"."""
    L = _lib.load()
    need = ctypes.c_size_t(0)
    check(L.gq_exec_available_devices(None, 0, ctypes.byref(need)))
    out = ctypes.create_string_buffer(need.value)
    check(L.gq_exec_available_devices(out, need.value, None))
    return list(json.loads(out.value.decode()))


def inspect(model_bytes: bytes) -> dict:
    """The description gq_exec_describe gives, from the file alone (no device)."""
    L = _lib.load()
    buf = ctypes.create_string_buffer(bytes(model_bytes), len(model_bytes))
    need = ctypes.c_size_t(0)
    check(L.gq_exec_inspect(buf, len(model_bytes), None, 0, ctypes.byref(need)))
    out = ctypes.create_string_buffer(need.value)
    check(L.gq_exec_inspect(buf, len(model_bytes), out, need.value, None))
    return json.loads(out.value.decode())


class ModelExecutor:
    """The executor handle: one per thread, as in the reference."""

    def __init__(self, model_bytes: bytes, device: str = "auto"):
        self._L = _lib.load()
        h = ctypes.c_void_p()
        data = bytes(model_bytes)
        check(self._L.gq_exec_create(data, len(data), str(device).encode(), ctypes.byref(h)))
        self._h = h
        d = self.describe()
        self.device = d["device"]
        self.name = d["name"]
        self.inputs = list(d["inputs"])
        self.outputs = list(d["outputs"])
        self.parameters = list(d["parameters"])
        self.symbol_table = list(d["symbol_table"])
        self.tensor_names = {int(k): v for k, v in d["names"].items()}
        self.config = d["config"]

    def describe(self) -> dict:
        need = ctypes.c_size_t(0)
        check(self._L.gq_exec_describe(self._h, None, 0, ctypes.byref(need)))
        out = ctypes.create_string_buffer(need.value)
        check(self._L.gq_exec_describe(self._h, out, need.value, None))
        return json.loads(out.value.decode())

    def close(self) -> None:
        if getattr(self, "_h", None):
            self._L.gq_exec_free(self._h)
            self._h = None

    def __del__(self):
        self.close()

    # -- the reference's methods ---------------------------------------------------
    def prepare(self, symbols: dict[str, int] | None = None, enable_arena_reuse: bool = True) -> None:
        syms = dict(symbols or {})
        names = (ctypes.c_char_p * len(syms))(*[k.encode() for k in syms])
        vals = (ctypes.c_int64 * len(syms))(*[int(v) for v in syms.values()])
        check(self._L.gq_exec_prepare(self._h, names, vals, len(syms)))

    def set_input_by_id(self, tensor_id: int, array) -> None:
        a = np.ascontiguousarray(array)
        check(self._L.gq_exec_set_input(self._h, int(tensor_id), a.ctypes.data, a.nbytes))

    def set_input_by_name(self, name: str, array) -> None:
        a = np.ascontiguousarray(array)
        check(self._L.gq_exec_set_input_by_name(self._h, name.encode(), a.ctypes.data, a.nbytes))

    def run(self, n_threads: int = 1) -> None:
        check(self._L.gq_exec_run(self._h))

    def synchronize(self) -> None:
        check(self._L.gq_exec_synchronize(self._h))

    def get_tensor_shape(self, tensor_id: int) -> list[int]:
        ne = (ctypes.c_int64 * 4)()
        check(self._L.gq_exec_get_tensor_shape(self._h, int(tensor_id), ne))
        return list(ne)

    def get_tensor_size_bytes(self, tensor_id: int) -> int:
        n = ctypes.c_size_t(0)
        check(self._L.gq_exec_get_output(self._h, int(tensor_id), None, 0, ctypes.byref(n)))
        return int(n.value)

    def get_output_bytes(self, tensor_id: int) -> bytes:
        n = self.get_tensor_size_bytes(tensor_id)
        buf = ctypes.create_string_buffer(n)
        check(self._L.gq_exec_get_output(self._h, int(tensor_id), buf, n, None))
        return buf.raw

    def get_output(self, tensor_id: int) -> np.ndarray:
        """The output as float32 [rows, n_vocab] (rows = tokens)."""
        ne = self.get_tensor_shape(tensor_id)
        return np.frombuffer(self.get_output_bytes(tensor_id), np.float32).reshape(ne[1], ne[0])

    def init_kv_cache(self, max_ctx: int = 2048) -> None:
        check(self._L.gq_exec_init_kv_cache(self._h, int(max_ctx)))

    def reset_kv_cache(self) -> None:
        check(self._L.gq_exec_reset_kv_cache(self._h))

    def has_kv_cache(self) -> bool:
        return bool(self._L.gq_exec_has_kv_cache(self._h))

    def set_logits_last_only(self, enable: bool) -> None:
        check(self._L.gq_exec_set_logits_last_only(self._h, 1 if enable else 0))

    def logits_last_only(self) -> bool:
        return bool(self._L.gq_exec_logits_last_only(self._h))

    def set_enable_cuda_graph(self, enable: bool) -> None:
        check(self._L.gq_exec_set_enable_graphs(self._h, 1 if enable else 0))

    @property
    def position(self) -> int:
        return int(self._L.gq_exec_position(self._h))

    # -- paged KV (executor.h:73-93) ---------------------------------------------------
    def set_tokens_per_page(self, n: int) -> None:
        check(self._L.gq_exec_set_tokens_per_page(self._h, int(n)))

    def get_tokens_per_page(self) -> int:
        return int(self._L.gq_exec_get_tokens_per_page(self._h))

    def init_paged_kv_cache(self, max_batch: int = 8, max_ctx: int = 2048) -> None:
        check(self._L.gq_exec_init_paged_kv_cache(self._h, int(max_batch), int(max_ctx)))

    def is_paged_kv_cache_enabled(self) -> bool:
        return bool(self._L.gq_exec_is_paged_kv_cache_enabled(self._h))

    def paged_kv_alloc_slot(self, slot_id: int, prefix_hash: str = "") -> None:
        check(self._L.gq_exec_paged_kv_alloc_slot(self._h, int(slot_id)))

    def paged_kv_free_slot(self, slot_id: int) -> None:
        check(self._L.gq_exec_paged_kv_free_slot(self._h, int(slot_id)))

    def is_paged_slot_allocated(self, slot_id: int) -> bool:
        return bool(self._L.gq_exec_is_paged_slot_allocated(self._h, int(slot_id)))

    def paged_kv_ensure_tokens(self, slot_id: int, total_tokens: int) -> None:
        check(self._L.gq_exec_paged_kv_ensure_tokens(self._h, int(slot_id), int(total_tokens)))

    def paged_kv_map_existing_pages(self, slot_id: int, start_page_idx: int, pages) -> None:
        ids = np.ascontiguousarray(np.asarray(pages, np.int32))
        ptr = ids.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))
        check(self._L.gq_exec_paged_kv_map_existing_pages(self._h, int(slot_id), int(start_page_idx), ptr, ids.size))

    def paged_kv_extract_page_handles(self, slot_id: int, page_idx: int) -> int:
        page = ctypes.c_int32(0)
        check(self._L.gq_exec_paged_kv_extract_page(self._h, int(slot_id), int(page_idx), ctypes.byref(page)))
        return int(page.value)

    def paged_page_retain(self, page: int) -> None:
        check(self._L.gq_exec_paged_page_retain(self._h, int(page)))

    def paged_page_release(self, page: int) -> None:
        check(self._L.gq_exec_paged_page_release(self._h, int(page)))

    def get_paged_active_vram_bytes(self) -> int:
        return int(self._L.gq_exec_get_paged_active_vram_bytes(self._h))

    def paged_slot_position(self, slot_id: int) -> int:
        p = ctypes.c_int64(0)
        check(self._L.gq_exec_paged_slot_position(self._h, int(slot_id), ctypes.byref(p)))
        return int(p.value)

    def paged_set_slot_position(self, slot_id: int, pos: int) -> None:
        check(self._L.gq_exec_paged_set_slot_position(self._h, int(slot_id), int(pos)))

    # -- profiling (executor.h:101-118) ----------------------------------------------
    def set_enable_profile(self, enable: bool) -> None:
        check(self._L.gq_exec_set_enable_profile(self._h, 1 if enable else 0))

    def reset_profile(self) -> None:
        check(self._L.gq_exec_reset_profile(self._h))

    def get_profile(self) -> dict:
        p = _lib.gq_exec_profile()
        check(self._L.gq_exec_get_profile(self._h, ctypes.byref(p)))
        return {name: getattr(p, name) for name, _ in p._fields_}

    def _json(self, fn) -> dict:
        need = ctypes.c_size_t(0)
        check(fn(self._h, None, 0, ctypes.byref(need)))
        out = ctypes.create_string_buffer(need.value)
        check(fn(self._h, out, need.value, None))
        return json.loads(out.value.decode())

    def runtime_graph_summary(self) -> dict:
        return self._json(self._L.gq_exec_runtime_graph_summary)

    def runtime_mul_mat_shape_summary(self) -> dict:
        return self._json(self._L.gq_exec_runtime_mul_mat_shape_summary)


__all__ = ["ModelExecutor", "inspect", "available", "get_available_devices", "GQError"]
