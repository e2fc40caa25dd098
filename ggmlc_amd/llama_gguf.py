"""LLaMA-family decoders as ggmlc .gguf files (the "compile -> .gguf" step for the
decoder shapes of this path).

`llama_graph` lays out the execution graph the way ggmlc's runtime executes it
(`runtime/src/executor.cpp:1738-2810`), for one sequence of `s` tokens:

    x = GET_ROWS(tok_embd, input_ids)                              [E, s]
    per layer:
      qkv = MUL_MAT(attn_qkv, RMS_NORM(x))                         [(Hq+2Hkv)hd, s]
      q, k, v = VIEW(qkv) at 0, Hq*hd, (Hq+Hkv)*hd  -> RESHAPE     [hd, H, s]
      q, k = ROPE(q|k, rope_arange) (NEOX, n_dims = hd)
      a = FLASH_ATTN_EXT(PERMUTE q, PERMUTE k, PERMUTE v)          [hd, Hq, s] (fused_transpose)
      x = ADD(x, MUL_MAT(attn_output, RESHAPE a))
      x = ADD(x, MUL_MAT(ffn_down, GLU(MUL_MAT(ffn_gate_up, RMS_NORM(x)))))
    logits = MUL_MAT(output, RMS_NORM(x))                          [V, s]

The fused QKV and gate|up projections and the weightless RMS_NORM are ggmlc's
compile-time fusions (horizontal QKV / gate-up fusion, RMS weight bake). Positions
come from the constant `rope_arange` (0..max_pos-1), which the runtime views at
`pos` for each step (executor.cpp:2857-2866); the KV cache, the causal mask and the
`(s, n_kv)` buckets are runtime state (`init_kv_cache`), not part of the file.
"""

from __future__ import annotations

import math
from pathlib import Path

import numpy as np

from .gguf import GGUFWriter
from .graph_spec import ACTIVATION, CONSTANT, INPUT, OUTPUT, PARAMETER, Dim, Graph

F32, I32 = 0, 26
GLU_SWIGLU = 2  # enum ggml_glu_op
ROPE_NEOX = 2


def llama_graph(cfg, max_pos: int, wtypes: dict[str, int] | None = None, fused_qkv: bool = True,
                biases: frozenset = frozenset()) -> Graph:
    """The execution graph of `cfg` (a model.LlamaConfig); wtypes maps a weight name
    to its ggml type (default cfg.qtype). fused_qkv=False emits three projections
    (attn_q, attn_k, attn_v) instead of the fused one and its VIEWs. biases names the
    projections ("qkv", "o", "gate_up", "down") whose MUL_MAT takes an F32 bias as its
    third input, as ggmlc's lowering of a Linear with bias emits it
    (dialect/ggml/lowering.py:462-475; fused q | k | v biases concatenated like the
    weight rows, transforms/fusion.py:1347-1390)."""
    g = Graph(name=cfg.name, symbol_table=["s"])
    s = Dim.symbol("s")
    E, hd, Hq, Hkv, F, V = cfg.n_embd, cfg.head_dim, cfg.n_head, cfg.n_head_kv, cfg.n_ff, cfg.n_vocab
    wt = lambda name: (wtypes or {}).get(name, cfg.qtype)  # noqa: E731

    def act(name, ne):
        return g.add_tensor(name, F32, ne, ACTIVATION)

    def bias(name, n, which):
        return [g.add_tensor(name, F32, [n], PARAMETER, role="parameter")] if which in biases else []

    ids = g.add_tensor("input_ids", I32, [s, 1], INPUT)
    embd = g.add_tensor("tok_embd", wt("tok_embd"), [E, V], PARAMETER, role="parameter")
    pos = g.add_tensor("rope_arange", I32, [s], CONSTANT, role="constant")
    x = g.add_node("GET_ROWS", [embd, ids], act("inp_embd", [E, s, 1, 1]))
    nq = (Hq + 2 * Hkv) * hd
    # RMS_NORM's eps as the PyTorch importer records it; the runtime's default needs none
    eps = {} if float(cfg.rms_eps) == 1e-5 else {"eps": float(cfg.rms_eps)}
    for li in range(cfg.n_layer):
        p = f"blk.{li}."
        if fused_qkv:
            w_qkv = g.add_tensor(p + "attn_qkv", wt("attn_qkv"), [E, nq], PARAMETER, role="parameter")
        else:
            w_sep = {nm: g.add_tensor(p + "attn_" + nm, wt("attn_" + nm), [E, H * hd], PARAMETER, role="parameter")
                     for nm, H in (("q", Hq), ("k", Hkv), ("v", Hkv))}
        w_o = g.add_tensor(p + "attn_output", wt("attn_output"), [Hq * hd, E], PARAMETER, role="parameter")
        w_gu = g.add_tensor(p + "ffn_gate_up", wt("ffn_gate_up"), [E, 2 * F], PARAMETER, role="parameter")
        w_d = g.add_tensor(p + "ffn_down", wt("ffn_down"), [F, E], PARAMETER, role="parameter")
        h = g.add_node("RMS_NORM", [x], act(p + "attn_norm", [E, s]), **eps)
        if fused_qkv:
            qkv = g.add_node("MUL_MAT", [w_qkv, h] + bias(p + "attn_qkv.bias", nq, "qkv"), act(p + "qkv", [nq, s]))
        heads = {}
        for nm, H, start in (("q", Hq, 0), ("k", Hkv, Hq * hd), ("v", Hkv, (Hq + Hkv) * hd)):
            if fused_qkv:
                src = g.add_node("VIEW", [qkv], act(p + nm + "_view", [H * hd, s]), ggml_dim=0, start=start)
            else:
                src = g.add_node("MUL_MAT", [w_sep[nm], h] + bias(p + "attn_" + nm + ".bias", H * hd, "qkv"),
                                 act(p + nm + "_proj", [H * hd, s]))
            heads[nm] = g.add_node("RESHAPE", [src], act(p + nm + "_3d", [hd, H, s]))
        for nm in ("q", "k"):
            heads[nm] = g.add_node("ROPE", [heads[nm], pos], act(p + nm + "_rope", [hd, Hq if nm == "q" else Hkv, s]),
                                   n_dims=hd, mode=ROPE_NEOX, freq_base=float(cfg.rope_base))
        perm = {}
        for nm, H in (("q", Hq), ("k", Hkv), ("v", Hkv)):
            perm[nm] = g.add_node("PERMUTE", [heads[nm]], act(p + nm + "_perm", [hd, s, H]),
                                  axis0=0, axis1=2, axis2=1, axis3=3)
        a = g.add_node("FLASH_ATTN_EXT", [perm["q"], perm["k"], perm["v"]], act(p + "attn", [hd, Hq, s]),
                       scale=1.0 / math.sqrt(hd), fused_transpose=1, is_causal=1)
        a2 = g.add_node("RESHAPE", [a], act(p + "attn_2d", [Hq * hd, s]))
        o = g.add_node("MUL_MAT", [w_o, a2] + bias(p + "attn_output.bias", E, "o"), act(p + "attn_out", [E, s]))
        x = g.add_node("ADD", [x, o], act(p + "ffn_inp", [E, s]))
        h2 = g.add_node("RMS_NORM", [x], act(p + "ffn_norm", [E, s]), **eps)
        gu = g.add_node("MUL_MAT", [w_gu, h2] + bias(p + "ffn_gate_up.bias", 2 * F, "gate_up"),
                        act(p + "ffn_gate_up_out", [2 * F, s]))
        sw = g.add_node("GLU", [gu], act(p + "ffn_act", [F, s]), op=GLU_SWIGLU)
        d = g.add_node("MUL_MAT", [w_d, sw] + bias(p + "ffn_down.bias", E, "down"), act(p + "ffn_out", [E, s]))
        x = g.add_node("ADD", [x, d], act(p + "l_out", [E, s]))
    hf = g.add_node("RMS_NORM", [x], act("result_norm", [E, s]), **eps)
    w_lm = embd if cfg.tied_embeddings else g.add_tensor("output", wt("output"), [E, V], PARAMETER,
                                                          role="parameter")
    logits = g.add_tensor("logits", F32, [V, s], OUTPUT)
    g.add_node("MUL_MAT", [w_lm, hf], logits)
    g.outputs.append(logits)
    g.metadata = {"max_pos": int(max_pos)}
    return g


def write_llama_gguf(path: str | Path, cfg, weights, max_pos: int = 4096, fused_qkv: bool = True) -> Path:
    """Write cfg's decoder with host weights = (embed, lm_head, [(qkv, o, gate_up, down), ...])
    (uint8 GGUF block rows, as model.ModelWeights holds them) to a .gguf file. A layer
    tuple may carry the four projections' fp32 biases after them (None where absent;
    model.host_weights), written as F32 tensors feeding the MUL_MATs' third input."""
    embed, lm_head, layers = weights
    names = ("qkv", "o", "gate_up", "down")
    biases = frozenset(nm for nm, b in zip(names, layers[0][4:8]) if b is not None) if layers else frozenset()
    for L in layers:
        if frozenset(nm for nm, b in zip(names, L[4:8]) if b is not None) != biases:
            raise ValueError("every layer must carry the same projection biases")
    g = llama_graph(cfg, max_pos, fused_qkv=fused_qkv, biases=biases)
    w = GGUFWriter()
    w.add_string("general.architecture", "ggmlc")
    w.add_string("general.name", g.name)
    w.add_string("ggmlc.version", "1.0.0")
    w.add_string_array("ggmlc.symbol_table", g.symbol_table)
    w.add_string("ggmlc.graph_spec", g.to_json())
    data = {"tok_embd": embed, "output": lm_head, "rope_arange": np.arange(max_pos, dtype=np.int32)}
    qd, kvd = cfg.n_head * cfg.head_dim, cfg.n_head_kv * cfg.head_dim
    for li, L in enumerate(layers):
        for nm, arr in zip(("attn_qkv", "attn_output", "ffn_gate_up", "ffn_down"), L):
            data[f"blk.{li}.{nm}"] = arr
        qkv = np.asarray(L[0])  # rows q | k | v: the separate projections are row slices
        data[f"blk.{li}.attn_q"], data[f"blk.{li}.attn_k"], data[f"blk.{li}.attn_v"] = \
            qkv[:qd], qkv[qd:qd + kvd], qkv[qd + kvd:]
        for nm, b in zip(("attn_qkv", "attn_output", "ffn_gate_up", "ffn_down"), L[4:8]):
            if b is not None:
                data[f"blk.{li}.{nm}.bias"] = np.asarray(b, np.float32)
        if L[4:5] and L[4] is not None:
            bq = np.asarray(L[4], np.float32)
            data[f"blk.{li}.attn_q.bias"], data[f"blk.{li}.attn_k.bias"], data[f"blk.{li}.attn_v.bias"] = \
                bq[:qd], bq[qd:qd + kvd], bq[qd + kvd:]
    for tid in sorted(g.tensors):
        t = g.tensors[tid]
        if t.name not in data:
            continue
        arr = np.ascontiguousarray(data[t.name])
        if t.name == "rope_arange":
            ne = [max_pos]
        elif t.name.endswith(".bias"):
            ne = [arr.size]
        else:
            ne = [d.evaluate({}) for d in t.ne[:2]]
        w.add_tensor(t.name, ne + [1] * (4 - len(ne)), t.type, arr.view(np.uint8).reshape(-1))
    return w.write_file(path)
