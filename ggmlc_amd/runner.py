"""The runner surface of ggmlc (`python/ggmlc/runtime/runner.py:34-334`) over this
package's MI355X path: load a compiled ggmlc .gguf and run it on the GPU.

    runner = load("model.gguf", device="gpu")      # "gpu", "cuda", "cuda:N" or "auto"
    runner.init_kv_cache(2048)
    logits = runner(ids[None, :], symbols={"pos": 0, "s": len(ids)})   # [s, vocab]
    logits = runner(np.array([[tok]]), symbols={"pos": len(ids), "s": 1})

The file is read with :mod:`ggmlc_amd.gguf` and its `ggmlc.graph_spec` with
:mod:`ggmlc_amd.graph_spec`. The graph is matched against the LLaMA-family decoder
layout ggmlc's runtime executes (:func:`ggmlc_amd.llama_gguf.llama_graph`: embedding
GET_ROWS, per layer RMS_NORM -> fused QKV MUL_MAT -> VIEW/RESHAPE -> ROPE (NEOX) ->
FLASH_ATTN_EXT -> output MUL_MAT -> ADD, RMS_NORM -> fused gate|up MUL_MAT -> GLU
SWIGLU -> down MUL_MAT -> ADD, final RMS_NORM -> lm_head MUL_MAT), with separate
q/k/v projections also accepted (their quantized rows are concatenated, which is
exact). The weights are the file's bytes, uploaded once; every op runs on libgq
(`model.Decoder`). Graphs outside that layout raise `NotImplementedError` naming
the first node that does not fit: there is no CPU path.

Semantics kept from the reference runtime: symbols `s` and `pos`; the KV cache is
runtime state (`init_kv_cache`, `reset_kv_cache`, executor.cpp:498-620) written at
rows pos..pos+s-1; outputs are all s rows of logits, shaped like `get_outputs`
(rank max(2, input rank)); RMS_NORM's `eps` attribute is read as an integer, as
executor.cpp:2024 reads it (absent: 1e-5).
"""

from __future__ import annotations

import math
from pathlib import Path
from typing import Any

import numpy as np

from .gguf import GGUFReader
from .graph_spec import INPUT, OPS, Graph

_QUANT = {2, 8}  # Q4_0, Q8_0


def get_available_devices() -> list[str]:
    """Devices this runtime executes on (runner.py:34-38; executor.cpp:184): the visible
    GPUs, from libgq's executor."""
    from .executor import get_available_devices as devs

    return devs()


class _Match:
    """Decoder hyper-parameters and weight names read off a graph."""

    def __init__(self):
        self.layers: list[dict[str, Any]] = []


def _fail(node, why: str):
    raise NotImplementedError(f"graph node {node.id} ({node.op} '{node.name}'): {why}")


def match_llama(g: Graph, reader: GGUFReader) -> _Match:
    """Read the LLaMA decoder layout off graph g (see the module docstring)."""
    prod = {}
    cons: dict[int, list] = {}
    for n in g.nodes:
        for o in n.outputs:
            prod[o] = n
        for i in n.inputs:
            cons.setdefault(i, []).append(n)
    T = g.tensors
    m = _Match()
    ins = [t for t in g.inputs if T[t].storage == INPUT]
    if len(ins) != 1 or T[ins[0]].type not in (26, 27):
        raise NotImplementedError("expected one integer input (token ids)")
    m.input_tid = ins[0]
    if len(g.outputs) != 1:
        raise NotImplementedError("expected one output (logits)")
    m.output_tid = g.outputs[0]

    def only(nodes, op, what, node):
        sel = [n for n in nodes if n.opcode == OPS[op]]
        if len(sel) != 1:
            _fail(node, f"expected one {op} consumer ({what}), found {len(sel)}")
        return sel[0]

    def weight(tid, node):
        t = T[tid]
        if t.type not in _QUANT or t.name not in reader.tensors:
            _fail(node, f"weight '{t.name}' must be a Q8_0/Q4_0 tensor stored in the file")
        ne = reader.tensors[t.name].ne
        return t.name, t.type, int(ne[0]), int(ne[1])

    def bias_of(node, n):
        """the MUL_MAT node's bias input (executor.cpp:2436-2445): an F32 [n] tensor in the file"""
        if len(node.inputs) < 3:
            return None
        if len(node.inputs) > 3:
            _fail(node, "MUL_MAT with more than three inputs")
        t = T[node.inputs[2]]
        if t.type != 0 or t.name not in reader.tensors:
            _fail(node, f"bias '{t.name}' must be an F32 tensor stored in the file")
        ne = [int(v) for v in reader.tensors[t.name].ne if int(v) != 1] or [1]
        if ne != [n]:
            _fail(node, f"bias '{t.name}' must hold {n} values")
        return t.name

    def rms_eps(node):
        if len(node.inputs) != 1:
            _fail(node, "RMS_NORM with a weight input (expected the weight baked into the next MUL_MAT)")
        return float(node.attr_int("eps")) if node.has("eps") else 1e-5

    gr = [n for n in g.nodes if n.opcode == OPS["GET_ROWS"] and m.input_tid in n.inputs]
    if len(gr) != 1:
        raise NotImplementedError("expected the token ids to feed one GET_ROWS (embedding)")
    emb = gr[0]
    m.embed, m.embed_type, m.n_embd, m.n_vocab = weight(emb.inputs[0], emb)
    x = emb.outputs[0]
    eps = []
    ropes = []
    while True:
        norm = only(cons.get(x, []), "RMS_NORM", "next norm", prod.get(x, emb))
        eps.append(rms_eps(norm))
        h = norm.outputs[0]
        mms = [n for n in cons.get(h, []) if n.opcode == OPS["MUL_MAT"]]
        if len(mms) == 1 and mms[0].outputs[0] == m.output_tid:  # final norm -> lm_head
            m.lm_head, m.lm_type, k, n = weight(mms[0].inputs[0], mms[0])
            if k != m.n_embd or n != m.n_vocab:
                _fail(mms[0], "lm_head shape")
            if len(mms[0].inputs) > 2:
                _fail(mms[0], "an output head with a bias is not mapped")
            break
        L: dict[str, Any] = {}
        # q, k, v: RESHAPE [hd, H, s] of either VIEWs of one fused product or three products
        if len(mms) == 1:
            L["qkv"] = [weight(mms[0].inputs[0], mms[0])]
            views = [n for n in cons.get(mms[0].outputs[0], []) if n.opcode == OPS["VIEW"]]
            if len(views) != 3:
                _fail(mms[0], "fused QKV product must feed three VIEWs")
            views.sort(key=lambda n: n.attr_int("start"))
            if any(v.attr_int("ggml_dim") != 0 or v.attr_int("step", 1) != 1 for v in views):
                _fail(views[0], "QKV views must slice ne[0]")
            srcs = views
        elif len(mms) == 3:
            srcs = mms
            L["qkv"] = None
        else:
            _fail(norm, f"expected 1 (fused) or 3 QKV products, found {len(mms)}")
        # each head tensor: RESHAPE [hd, H, s] -> (ROPE for q, k) -> PERMUTE -> FLASH_ATTN_EXT input i
        paths = []
        for sn in srcs:
            r = only(cons.get(sn.outputs[0], []), "RESHAPE", "head reshape", sn)
            ne = T[r.outputs[0]].ne
            nxt = cons.get(r.outputs[0], [])
            rope = nxt[0] if len(nxt) == 1 and nxt[0].opcode == OPS["ROPE"] else None
            src = rope or r
            pm = only(cons.get(src.outputs[0], []), "PERMUTE", "attention permute", src)
            fa = only(cons.get(pm.outputs[0], []), "FLASH_ATTN_EXT", "attention", pm)
            paths.append((fa.inputs.index(pm.outputs[0]), sn, ne[0].evaluate({"s": 1}), ne[1].evaluate({"s": 1}),
                          rope, fa))
        paths.sort(key=lambda t: t[0])
        if [t[0] for t in paths] != [0, 1, 2] or len({t[5].id for t in paths}) != 1:
            _fail(srcs[0], "q, k, v must be the inputs 0, 1, 2 of one attention node")
        if paths[0][4] is None or paths[1][4] is None or paths[2][4] is not None:
            _fail(srcs[0], "rope must apply to q and k only")
        hd = paths[0][2]
        if any(t[2] != hd for t in paths):
            _fail(srcs[0], "q, k, v head sizes differ")
        n_head, n_head_kv = paths[0][3], paths[1][3]
        if paths[2][3] != n_head_kv:
            _fail(srcs[2], "k and v head counts differ")
        if L["qkv"] is None:  # three products, concatenated in q | k | v order
            L["qkv"] = [weight(t[1].inputs[0], t[1]) for t in paths]
            L["qkv_b"] = [bias_of(t[1], t[3] * hd) for t in paths]
            if any(b is None for b in L["qkv_b"]):
                if any(b is not None for b in L["qkv_b"]):
                    _fail(srcs[0], "biases on some of q, k, v only")
                L["qkv_b"] = None
        else:
            w0 = L["qkv"][0]
            if w0[3] != (n_head + 2 * n_head_kv) * hd or [t[1].attr_int("start") for t in paths] != \
                    [0, n_head * hd, (n_head + n_head_kv) * hd]:
                _fail(srcs[0], "fused QKV rows are not q | k | v")
            b0 = bias_of(mms[0], w0[3])
            L["qkv_b"] = [b0] if b0 is not None else None
        rq, rk = paths[0][4], paths[1][4]
        for rn in (rq, rk):
            if rn.attr_int("mode", 2) != 2 or rn.attr_int("n_dims", hd) != hd:
                _fail(rn, "only NEOX rope over the whole head is mapped")
            if rn.attr_float("ext_factor", 0.0) != 0.0 or rn.attr_float("freq_scale", 1.0) != 1.0:
                _fail(rn, "rope scaling is not mapped")
            ropes.append(rn.attr_float("freq_base", 10000.0))
        fa = paths[0][5]
        scale = fa.attr_float("scale", 1.0 / math.sqrt(hd))
        if abs(scale - 1.0 / math.sqrt(hd)) > 1e-7 * scale or fa.attr_float("max_bias", 0.0) or \
                fa.attr_float("logit_softcap", 0.0):
            _fail(fa, "attention scale must be 1/sqrt(head_dim), no ALiBi/softcap")
        if not fa.attr_int("fused_transpose"):
            _fail(fa, "expected the fused-transpose attention output [hd, H, s]")
        a2 = only(cons.get(fa.outputs[0], []), "RESHAPE", "attention output reshape", fa)
        o = only(cons.get(a2.outputs[0], []), "MUL_MAT", "output projection", a2)
        L["o"] = weight(o.inputs[0], o)
        L["o_b"] = bias_of(o, L["o"][3])
        add1 = only(cons.get(o.outputs[0], []), "ADD", "residual", o)
        if x not in add1.inputs:
            _fail(add1, "residual must add the layer input")
        x1 = add1.outputs[0]
        norm2 = only(cons.get(x1, []), "RMS_NORM", "ffn norm", add1)
        eps.append(rms_eps(norm2))
        gu = only(cons.get(norm2.outputs[0], []), "MUL_MAT", "gate|up projection", norm2)
        L["gate_up"] = weight(gu.inputs[0], gu)
        L["gate_up_b"] = bias_of(gu, L["gate_up"][3])
        glu = only(cons.get(gu.outputs[0], []), "GLU", "SWIGLU", gu)
        if glu.attr_int("op", 2) != 2 or glu.attr_int("swapped", 0) != 0:
            _fail(glu, "only SWIGLU is mapped")
        dn = only(cons.get(glu.outputs[0], []), "MUL_MAT", "down projection", glu)
        L["down"] = weight(dn.inputs[0], dn)
        L["down_b"] = bias_of(dn, L["down"][3])
        add2 = only(cons.get(dn.outputs[0], []), "ADD", "residual", dn)
        if x1 not in add2.inputs:
            _fail(add2, "residual must add the attention block's output")
        L.update(hd=hd, n_head=n_head, n_head_kv=n_head_kv, n_ff=L["gate_up"][3] // 2)
        m.layers.append(L)
        x = add2.outputs[0]
    if not m.layers:
        raise NotImplementedError("no decoder layer found")
    first = m.layers[0]
    for k in ("hd", "n_head", "n_head_kv", "n_ff"):
        if any(L[k] != first[k] for L in m.layers):
            raise NotImplementedError(f"layers differ in {k}")
    if len(set(eps)) != 1 or len(set(ropes)) != 1:
        raise NotImplementedError("layers differ in RMS_NORM eps or rope base")
    m.head_dim, m.n_head, m.n_head_kv, m.n_ff = first["hd"], first["n_head"], first["n_head_kv"], first["n_ff"]
    m.rms_eps, m.rope_base = eps[0], ropes[0]
    return m


class ModelRunner:
    """ggmlc's ModelRunner (runner.py:48-316) on the MI355X path: runs go through libgq's
    executor handle (`executor.ModelExecutor`, the C ABI gq_exec_*: GGUF and graph parsing,
    the decoder and its per-bucket HIP graphs in C++, no torch); `executor` also serves
    the paged-KV surface the continuous-batching scheduler drives."""

    def __init__(self, model_source: str | Path | bytes, n_threads: int = 1, device: str = "auto"):
        from .executor import ModelExecutor

        if isinstance(model_source, (str, Path)):
            p = Path(model_source)
            if not p.exists():
                raise FileNotFoundError(f"Model file not found: {p}")
            raw = p.read_bytes()
        elif isinstance(model_source, (bytes, bytearray, memoryview)):
            raw = bytes(model_source)
        else:
            raise TypeError(f"Expected file path or bytes, got {type(model_source)}")
        reader = GGUFReader(raw)
        if "ggmlc.graph_spec" not in reader.metadata:
            raise ValueError("GGUF metadata missing 'ggmlc.graph_spec'")
        self.n_threads = n_threads
        self.graph = Graph.from_json(reader.metadata["ggmlc.graph_spec"])
        self.name = self.graph.name
        self.symbol_table = list(self.graph.symbol_table)
        self.inputs = list(self.graph.inputs)
        self.outputs = list(self.graph.outputs)
        self.parameters = list(self.graph.parameters)
        self.tensor_info = dict(self.graph.tensors)
        self.input_name_to_id = {self.graph.tensors[t].name: t for t in self.inputs}

        dev = str(device)
        if dev in ("auto", "gpu", "cuda"):
            dev = "cuda:0"
        elif dev.startswith("gpu:"):
            dev = "cuda:" + dev[4:]
        if not dev.startswith("cuda"):
            raise ValueError(f"device {device!r}: this runtime executes on the GPU only ('gpu[:N]', 'cuda[:N]', "
                             "'auto')")
        m = match_llama(self.graph, reader)
        self.match = m
        self._reader = reader
        qt = {m.embed_type, m.lm_type} | {w[1] for L in m.layers for k in ("o", "gate_up", "down")
                                             for w in [L[k]]} | {w[1] for L in m.layers for w in L["qkv"]}
        from .model import LlamaConfig

        self.cfg = LlamaConfig(self.name, len(m.layers), m.n_embd, m.n_head, m.n_head_kv, m.head_dim, m.n_ff,
                               m.n_vocab, m.embed_type if len(qt) == 1 else -1,
                               tied_embeddings=m.lm_head == m.embed, rms_eps=m.rms_eps, rope_base=m.rope_base,
                               qkv_bias=m.layers[0]["qkv_b"] is not None)
        try:
            native = ModelExecutor(raw, dev)
        except RuntimeError as e:  # no GPU, or a device index past the visible ones
            raise RuntimeError(f"no usable GPU for device {device!r}: {e}") from e
        self.device = native.device
        self._weights = None
        self.executor = PagedExecutor(self, native)

    @property
    def weights(self):
        """The model as device tensors for the batched decoder (built on first use)."""
        if self._weights is None:
            self._weights = self._build_weights()
        return self._weights

    @property
    def _dev(self):
        import torch

        return torch.device(self.device)

    def _build_weights(self):
        import torch

        from . import ops
        from .model import LayerWeights, ModelWeights

        m, reader = self.match, self._reader
        cache: dict[str, ops.QWeight] = {}

        def upload(names_types) -> ops.QWeight:
            key = "|".join(n for n, *_ in names_types)
            if key not in cache:
                parts = [reader.tensor_array(n) for n, *_ in names_types]
                types = {t for _, t, *_ in names_types}
                if len(types) != 1:
                    raise NotImplementedError("q/k/v weights of different types")
                host = np.concatenate(parts, axis=0) if len(parts) > 1 else parts[0]
                dev_t = torch.from_numpy(np.array(host, copy=True)).to(self._dev)
                cache[key] = ops.QWeight(dev_t, types.pop(), names_types[0][2])
            return cache[key]

        def upload_bias(names) -> torch.Tensor | None:
            if not names:
                return None
            host = np.concatenate([np.asarray(reader.tensor_array(n), np.float32).reshape(-1) for n in names])
            return torch.from_numpy(host).to(self._dev)

        layers = [LayerWeights(qkv=upload(L["qkv"]), o=upload([L["o"]]), gate_up=upload([L["gate_up"]]),
                               down=upload([L["down"]]), qkv_b=upload_bias(L["qkv_b"]),
                               o_b=upload_bias([L["o_b"]] if L["o_b"] else None),
                               gate_up_b=upload_bias([L["gate_up_b"]] if L["gate_up_b"] else None),
                               down_b=upload_bias([L["down_b"]] if L["down_b"] else None)) for L in m.layers]
        embed = upload([(m.embed, m.embed_type, m.n_embd)])
        lm = upload([(m.lm_head, m.lm_type, m.n_embd)])
        return ModelWeights(self.cfg, embed, lm, layers)

    # -- KV cache (runner.py:304-316) -------------------------------------------------
    def init_kv_cache(self, max_ctx: int = 2048) -> None:
        self.executor.native.init_kv_cache(int(max_ctx))

    def reset_kv_cache(self) -> None:
        self.executor.native.reset_kv_cache()

    def has_kv_cache(self) -> bool:
        return self.executor.native.has_kv_cache()

    # -- run --------------------------------------------------------------------------
    def __call__(self, *args: np.ndarray, symbols: dict[str, int] | None = None, n_threads: int | None = None,
                 enable_arena_reuse: bool = True, **kwargs: np.ndarray):
        """Token ids (positional or by input name) -> logits of every token (of the last
        one with executor.set_logits_last_only(True)), shaped like the reference's
        get_outputs: [s, vocab] for a rank-2 input."""
        if len(args) == 1 and isinstance(args[0], dict) and not kwargs:
            kwargs, args = args[0], ()
        if args:
            ids = args[0]
        elif kwargs:
            name = next(iter(kwargs))
            if name not in self.input_name_to_id and len(kwargs) > 1:
                raise ValueError(f"unknown input {name!r}")
            ids = kwargs[name]
        else:
            raise ValueError("no input ids")
        ids = np.asarray(ids)
        rank = ids.ndim
        flat = np.ascontiguousarray(ids.reshape(-1).astype(np.int32))
        s = int(flat.size)
        syms = dict(symbols or {})
        if "s" in syms and int(syms["s"]) != s:
            raise ValueError(f"symbol s = {syms['s']} but {s} input ids")
        ex = self.executor.native
        syms["s"] = s
        if not ex.has_kv_cache():
            syms["pos"] = 0
        ex.prepare(syms, enable_arena_reuse)
        ex.set_input_by_id(self.inputs[0], flat)
        ex.run()
        logits = ex.get_output(self.outputs[0])
        self._last = (logits, dict(syms))
        rows = logits.shape[0]
        return logits.reshape([1, 1, rows, self.cfg.n_vocab][-max(2, rank):])

    def get_outputs(self, input_ndim: int = 2):
        logits = self._last[0]
        return logits.reshape([1, 1, logits.shape[0], self.cfg.n_vocab][-max(2, input_ndim):])

    def run_benchmark(self, runs: int = 5, n_threads: int | None = None) -> list[float]:
        """Latency (ms) of the last call's step, replayed `runs` times at its position."""
        import time

        if not hasattr(self, "_last"):
            raise RuntimeError("call the runner once before benchmarking")
        ex = self.executor.native
        syms = self._last[1]
        ids = np.zeros(int(syms["s"]), np.int32)
        out = []
        for _ in range(runs):
            ex.prepare(syms)
            ex.set_input_by_id(self.inputs[0], ids)
            t0 = time.perf_counter()
            ex.run()
            out.append((time.perf_counter() - t0) * 1e3)
        return out


class PagedExecutor:
    """The paged-KV surface of the reference executor (`ModelExecutor.init_paged_kv_cache`,
    `paged_kv_*`, `get_paged_active_vram_bytes`, `set_tokens_per_page`: executor.cpp:634-920,
    python_bindings.cpp:196-201) over `paged.BatchDecoder`; what
    `batching.ContinuousBatchScheduler(runner.executor, ...)` drives.

    Pages hold `tokens_per_page` KV rows of every layer (default 128, a power of two >= 64)
    in one pool sized at `init_paged_kv_cache` for max_batch sequences of max_ctx rows;
    `configure_vmm_pool` is accepted for the reference's signature and changes nothing
    (the pool is allocated once, there is no warm pool of mapped pages)."""

    def __init__(self, runner: "ModelRunner", native=None):
        self._runner = runner
        self.native = native  # executor.ModelExecutor: the handle the runner's calls go through
        self._tpp = 128
        self.batch = None

    def __getattr__(self, name):
        # the reference executor's other methods (prepare, set_input_by_id, run,
        # get_output_bytes, get_tensor_shape, set_logits_last_only, ...) are the native handle's
        native = self.__dict__.get("native")
        if native is None:
            raise AttributeError(name)
        return getattr(native, name)

    # -- setup ------------------------------------------------------------------------
    def set_tokens_per_page(self, n: int) -> None:
        if self.batch is not None:
            raise RuntimeError("tokens_per_page must be set before init_paged_kv_cache")
        if n < 64 or n & (n - 1):
            raise ValueError("tokens_per_page must be a power of two >= 64")
        self._tpp = int(n)

    @property
    def tokens_per_page(self) -> int:
        return self._tpp

    def get_tokens_per_page(self) -> int:
        return self._tpp

    def configure_vmm_pool(self, max_warm_pages: int = 0, prealloc_pages: int = 0) -> None:
        pass

    def init_paged_kv_cache(self, max_batch: int = 8, max_ctx: int = 2048) -> None:
        from .paged import BatchDecoder

        if self.batch is None:
            self.batch = BatchDecoder(self._runner.weights, int(max_batch), int(max_ctx), page_size=self._tpp,
                                      device=self._runner._dev)

    def is_paged_kv_cache_enabled(self) -> bool:
        return self.batch is not None

    def paged_decoder(self, max_batch: int = 8):
        """The batched decoder (created with max_batch slots of 2048 rows if not yet)."""
        if self.batch is None:
            self.init_paged_kv_cache(max_batch, 2048)
        return self.batch

    # -- slots ------------------------------------------------------------------------
    def _kv(self):
        if self.batch is None:
            raise RuntimeError("init_paged_kv_cache first")
        return self.batch.kv

    def paged_kv_alloc_slot(self, slot_id: int, prefix_hash: str = "") -> None:
        self._kv().alloc_slot(slot_id)

    def paged_kv_free_slot(self, slot_id: int) -> None:
        self._kv().free_slot(slot_id)

    def paged_kv_ensure_tokens(self, slot_id: int, total_tokens: int) -> None:
        self._kv().ensure_tokens(slot_id, int(total_tokens))

    def is_paged_slot_allocated(self, slot_id: int) -> bool:
        return self.batch is not None and self.batch.kv.active[slot_id]

    def get_paged_active_vram_bytes(self) -> int:
        return 0 if self.batch is None else self.batch.kv.active_bytes()


def load(model_source: str | Path | bytes, n_threads: int = 1, device: str = "auto") -> ModelRunner:
    """runner.py:319-334"""
    return ModelRunner(model_source, n_threads=n_threads, device=device)
