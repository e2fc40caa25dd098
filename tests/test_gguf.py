"""GGUF v3 + ggmlc.graph_spec (CPU): the writer/reader round trip, the file as the
reference's own loader reads it (oracle/_ref: runtime/src/loader.cpp over ggml's
gguf.cpp), symbolic dimensions, and the LLaMA graph run by the reference's own
executor against the reference ggml decoder graph (oracle.RefLlama)."""

from __future__ import annotations

import numpy as np
import pytest

import oracle as O
from ggmlc_amd import gguf
from ggmlc_amd.graph_spec import Dim, Graph, OPS
from ggmlc_amd.llama_gguf import llama_graph, write_llama_gguf
from ggmlc_amd.model import LlamaConfig
from ggmlc_amd.runner import match_llama

needs_ref = pytest.mark.skipif(not O.ref_available(), reason="reference build (oracle/_ref) absent")


def _tiny(qtype=O.Q8_0, tied=False):
    return LlamaConfig("tiny", 2, 256, 4, 2, 64, 512, 512, qtype, tied_embeddings=tied)


def _weights(c, seed=7):
    rng = np.random.default_rng(seed)

    def q(n, k):
        return O.quantize_weights((rng.standard_normal((n, k)) * 0.02).astype(np.float32), c.qtype)

    layers = [(q(c.q_dim + 2 * c.kv_dim, c.n_embd), q(c.n_embd, c.q_dim), q(2 * c.n_ff, c.n_embd),
               q(c.n_embd, c.n_ff)) for _ in range(c.n_layer)]
    embed = q(c.n_vocab, c.n_embd)
    return embed, embed if c.tied_embeddings else q(c.n_vocab, c.n_embd), layers


def test_gguf_round_trip(tmp_path):
    w = gguf.GGUFWriter()
    w.add_string("general.architecture", "ggmlc")
    w.add_uint32("u32", 7)
    w.add_int32("i32", -3)
    w.add_float32("f32", 0.5)
    w.add_bool("flag", True)
    w.add_string_array("syms", ["s", "pos", "ünï"])
    w.add_float_array("fa", [1.0, 2.5])
    w.add(("u64"), gguf.UINT64, 2 ** 40)
    w.add("i8arr", gguf.ARRAY, [1, -2, 3], gguf.INT8)
    rng = np.random.default_rng(0)
    a = rng.standard_normal((3, 5)).astype(np.float32)
    q = O.quantize_weights((rng.standard_normal((4, 64)) * 0.02).astype(np.float32), O.Q4_0)
    ids = np.arange(11, dtype=np.int32)
    w.add_tensor("a", [5, 3], 0, a.tobytes())
    w.add_tensor("q4", [64, 4], 2, q.tobytes())
    w.add_tensor("ids", [11], 26, ids.tobytes())
    p = w.write_file(tmp_path / "x.gguf")
    assert p.stat().st_size % 32 == 0
    for src in (p, p.read_bytes()):
        r = gguf.GGUFReader(src)
        assert r.version == 3 and r.alignment == 32
        assert r.metadata["u32"] == 7 and r.metadata["i32"] == -3 and r.metadata["f32"] == 0.5
        assert r.metadata["flag"] is True and r.metadata["syms"] == ["s", "pos", "ünï"]
        assert r.metadata["fa"] == [1.0, 2.5] and r.metadata["u64"] == 2 ** 40 and r.metadata["i8arr"] == [1, -2, 3]
        assert r.value_types["syms"] == (gguf.ARRAY, gguf.STRING)
        assert list(r.tensors) == ["a", "q4", "ids"]
        assert all(t.offset % 32 == 0 for t in r.tensors.values())
        assert np.array_equal(r.tensor_array("a"), a)
        assert np.array_equal(r.tensor_array("q4"), q)
        assert np.array_equal(r.tensor_array("ids"), ids)
    with pytest.raises(ValueError):
        gguf.GGUFReader(b"GGUX" + bytes(40))
    with pytest.raises(ValueError):
        w.add_tensor("bad", [64, 4], 2, q.tobytes()[:-1])


def test_dim_expressions_follow_int64_semantics():
    s, p = Dim.symbol("s"), Dim.symbol("pos")
    env = {"s": 7, "pos": -9}
    assert (s * 4 + 1).evaluate(env) == 29
    assert (p // 2).evaluate(env) == -4               # C++ truncates toward zero (Python's -9 // 2 is -5)
    assert (s.ceildiv(4)).evaluate(env) == 2
    assert ((s - 10).ceildiv(4)).evaluate(env) == 0  # (-3 + 3) / 4
    d = ((s * 3) // (p + 10)).ceildiv(2)
    assert Dim.from_json(d.to_json()) == d and d.evaluate(env) == 11
    assert Dim.from_json({"type": "bogus"}).evaluate({}) == 1  # unknown -> static 1, as the loader
    assert d.free_symbols() == {"s", "pos"}
    with pytest.raises(KeyError):
        s.evaluate({})
    with pytest.raises(ZeroDivisionError):
        (s // (s - 7)).evaluate(env)


def test_graph_json_round_trip():
    g = llama_graph(_tiny(), 1024)
    h = Graph.from_json(g.to_json())
    assert h.to_json() == g.to_json()
    assert h.symbol_table == ["s"] and len(h.nodes) == len(g.nodes)
    shapes = h.shapes({"s": 5})
    logits = h.outputs[0]
    assert shapes[logits] == [512, 5, 1, 1]
    assert {n.op for n in h.nodes} == {"GET_ROWS", "RMS_NORM", "MUL_MAT", "VIEW", "RESHAPE", "ROPE", "PERMUTE",
                                      "FLASH_ATTN_EXT", "ADD", "GLU"}


def _describe(g: Graph, r: gguf.GGUFReader, syms) -> list[str]:
    """What ref_rt_describe prints, computed from our own reader and graph."""
    def dim(d):
        if d.kind == "static":
            return str(d.val)
        if d.kind == "symbol":
            return d.name if d.name in syms else "?"
        return f"({d.kind} {dim(d.left)} {dim(d.right)})"

    out = [f"S {x}" for x in g.symbol_table]
    out += [f"I {t}" for t in g.inputs] + [f"O {t}" for t in g.outputs] + [f"P {t}" for t in g.parameters]
    for tid in sorted(g.tensors):
        t = g.tensors[tid]
        size = r.tensors[t.name].nbytes if t.name in r.tensors else 0
        out.append(f"T {tid} {t.name} {t.type} {t.storage} " + " ".join(dim(d) for d in t.ne) + f" {size}")
    for n in g.nodes:
        attrs = "".join(f"{k}={n.attr_int(k)}:{float(n.attr_float(k)):.9g};" for k in sorted(n.attributes))
        out.append(f"N {n.id} {n.opcode} {n.name or '-'} {','.join(map(str, n.inputs))} "
                   f"{','.join(map(str, n.outputs))} {attrs}")
    out += [f"M {k} {v}" for k, v in sorted(r.metadata.items()) if isinstance(v, str) and k != "ggmlc.graph_spec"]
    return out


@needs_ref
@pytest.mark.parametrize("fused_qkv", [True, False])
def test_reference_loader_reads_our_file(tmp_path, fused_qkv):
    """The reference loader (ggml gguf.cpp + runtime loader.cpp) sees exactly the
    graph, tensors, sizes, attributes and metadata our reader and graph model see."""
    c = _tiny()
    p = write_llama_gguf(tmp_path / "m.gguf", c, _weights(c), max_pos=1024, fused_qkv=fused_qkv)
    r = gguf.GGUFReader(p)
    g = Graph.from_json(r.metadata["ggmlc.graph_spec"])
    ref = O.RefRuntime(p).describe()
    ours = _describe(g, r, set(g.symbol_table))
    # float attributes print through %.9g in C; compare those numerically, the rest as text
    assert len(ref) == len(ours)
    for a, b in zip(ref, ours):
        if a.startswith("N "):
            ha, ta = a.rsplit(" ", 1)
            hb, tb = b.rsplit(" ", 1)
            assert ha == hb
            fa = dict(kv.split("=") for kv in ta.split(";") if kv)
            fb = dict(kv.split("=") for kv in tb.split(";") if kv)
            assert fa.keys() == fb.keys()
            for k in fa:
                ia, xa = fa[k].split(":")
                ib, xb = fb[k].split(":")
                assert ia == ib and float(xa) == pytest.approx(float(xb), rel=1e-8), (k, a, b)
        else:
            assert a == b


@needs_ref
@pytest.mark.parametrize("qtype,tied,fused_qkv,bias", [(O.Q8_0, False, True, False), (O.Q4_0, True, False, False),
                                                       (O.Q8_0, True, True, True), (O.Q8_0, False, False, True)])
def test_reference_runtime_runs_our_llama_file(tmp_path, qtype, tied, fused_qkv, bias):
    """The reference's own executor running our .gguf (prefill of 37 tokens, then
    decode steps with the KV cache, symbols s/pos) gives the bits of the reference
    ggml decoder graph (oracle.RefLlama) on the same weights: the file's graph is the
    decoder, projection biases (q | k | v, and o / gate_up / down) included."""
    c = _tiny(qtype, tied)
    w = _weights(c)
    if bias:
        rng = np.random.default_rng(11)
        nq, E, F = c.q_dim + 2 * c.kv_dim, c.n_embd, c.n_ff
        w = (w[0], w[1], [tuple(L) + tuple((rng.standard_normal(n) * 0.3).astype(np.float32)
                                            for n in (nq, E, 2 * F, E)) for L in w[2]])
    p = write_llama_gguf(tmp_path / "m.gguf", c, w, max_pos=1024, fused_qkv=fused_qkv)
    g = Graph.from_json(gguf.GGUFReader(p).metadata["ggmlc.graph_spec"])
    rt = O.RefRuntime(p, max_ctx=512, n_threads=8)
    rl = O.RefLlama(c, w, 512, n_threads=8)
    toks = np.random.default_rng(3).integers(0, c.n_vocab, 37).astype(np.int32)
    rt.run({g.inputs[0]: toks.reshape(1, -1)}, {"s": 37, "pos": 0})
    got = rt.output(g.outputs[0]).reshape(37, c.n_vocab)
    want, nxt = rl.step(toks)
    assert np.array_equal(got[-1], want)
    for i in range(3):
        rt.run({g.inputs[0]: np.array([[nxt]], np.int32)}, {"s": 1, "pos": 37 + i})
        got = rt.output(g.outputs[0]).reshape(-1)
        want, nxt = rl.step(np.array([nxt], np.int32))
        assert np.array_equal(got, want)


@pytest.mark.parametrize("fused_qkv", [True, False])
def test_graph_maps_onto_the_decoder(tmp_path, fused_qkv):
    """The runner's matcher reads the decoder's shape, weights and attributes off the
    file's graph; separate q/k/v projections map onto the fused rows."""
    c = LlamaConfig("m", 3, 960, 15, 5, 64, 2560, 1024, O.Q8_0, tied_embeddings=True, rope_base=50000.0)
    rng = np.random.default_rng(1)

    def q(n, k):
        return O.quantize_weights((rng.standard_normal((n, k)) * 0.02).astype(np.float32), c.qtype)

    layers = [(q(c.q_dim + 2 * c.kv_dim, c.n_embd), q(c.n_embd, c.q_dim), q(2 * c.n_ff, c.n_embd),
               q(c.n_embd, c.n_ff)) for _ in range(c.n_layer)]
    emb = q(c.n_vocab, c.n_embd)
    p = write_llama_gguf(tmp_path / "m.gguf", c, (emb, emb, layers), max_pos=256, fused_qkv=fused_qkv)
    r = gguf.GGUFReader(p)
    m = match_llama(Graph.from_json(r.metadata["ggmlc.graph_spec"]), r)
    assert (len(m.layers), m.n_embd, m.n_head, m.n_head_kv, m.head_dim, m.n_ff, m.n_vocab) == \
           (3, 960, 15, 5, 64, 2560, 1024)
    assert m.rope_base == 50000.0 and m.rms_eps == 1e-5 and m.lm_head == m.embed
    for L, host in zip(m.layers, layers):
        rows = np.concatenate([r.tensor_array(n) for n, *_ in L["qkv"]])
        assert np.array_equal(rows, host[0])
        assert len(L["qkv"]) == (1 if fused_qkv else 3)
        assert np.array_equal(r.tensor_array(L["down"][0]), host[3])


def test_matcher_rejects_other_graphs():
    c = _tiny()
    g = llama_graph(c, 64)
    w = gguf.GGUFWriter()
    data = {}
    rng = np.random.default_rng(0)
    for t in g.tensors.values():
        if t.storage == 1:
            ne = [d.evaluate({}) for d in t.ne[:2]]
            data[t.name] = (ne, t.type, rng.integers(0, 255, gguf.tensor_nbytes(t.type, ne), dtype=np.uint8))
    for name, (ne, ty, b) in data.items():
        w.add_tensor(name, ne + [1, 1], ty, b.tobytes())
    r = gguf.GGUFReader(w.to_bytes())
    # a rope mode the decoder does not map
    for n in g.nodes:
        if n.op == "ROPE":
            n.attributes["mode"] = 0
    with pytest.raises(NotImplementedError, match="NEOX"):
        match_llama(g, r)
    g2 = llama_graph(c, 64)
    g2.nodes = [n for n in g2.nodes if n.op != "GLU"]
    with pytest.raises(NotImplementedError):
        match_llama(g2, r)
    assert OPS["FLASH_ATTN_EXT"] == 74 and OPS["GLU"] == 100  # ggml 0.20.2 enum ggml_op


@pytest.mark.parametrize("fused_qkv,bias,tied", [(True, False, True), (False, False, False), (True, True, True),
                                                 (False, True, False)])
def test_native_executor_reads_the_file_like_the_python_reader(tmp_path, fused_qkv, bias, tied):
    """libgq's executor parser (GGUF v3 + graph_spec JSON + the decoder matcher, C++,
    gq_exec_inspect: no device) reports the graph surface, the matched weights and the
    hyper-parameters the Python reader and matcher report for the same file."""
    from ggmlc_amd.executor import inspect

    c = LlamaConfig("m", 3, 960, 15, 5, 64, 2560, 1024, O.Q8_0, tied_embeddings=tied, rope_base=50000.0,
                    rms_eps=1e-6)
    rng = np.random.default_rng(5)

    def q(n, k):
        return O.quantize_weights((rng.standard_normal((n, k)) * 0.02).astype(np.float32), c.qtype)

    nq = c.q_dim + 2 * c.kv_dim
    layers = [(q(nq, c.n_embd), q(c.n_embd, c.q_dim), q(2 * c.n_ff, c.n_embd), q(c.n_embd, c.n_ff))
              + (((rng.standard_normal(nq) * 0.1).astype(np.float32), None,
                  (rng.standard_normal(2 * c.n_ff) * 0.1).astype(np.float32), None) if bias else ())
              for _ in range(c.n_layer)]
    emb = q(c.n_vocab, c.n_embd)
    p = write_llama_gguf(tmp_path / "m.gguf", c, (emb, emb if tied else q(c.n_vocab, c.n_embd), layers),
                         max_pos=256, fused_qkv=fused_qkv)
    raw = p.read_bytes()
    d = inspect(raw)
    r = gguf.GGUFReader(p)
    g = Graph.from_json(r.metadata["ggmlc.graph_spec"])
    m = match_llama(g, r)
    cfg = d["config"]
    assert (cfg["n_layer"], cfg["n_embd"], cfg["n_head"], cfg["n_head_kv"], cfg["head_dim"], cfg["n_ff"],
            cfg["n_vocab"]) == (len(m.layers), m.n_embd, m.n_head, m.n_head_kv, m.head_dim, m.n_ff, m.n_vocab)
    assert cfg["rope_base"] == m.rope_base and cfg["rms_eps"] == pytest.approx(m.rms_eps)
    assert cfg["tied"] == (m.lm_head == m.embed) and cfg["qkv_bias"] == bias
    assert d["inputs"] == g.inputs and d["outputs"] == g.outputs and d["symbol_table"] == g.symbol_table
    assert d["embed"] == m.embed and d["lm_head"] == m.lm_head
    for Ln, Lp in zip(d["layers"], m.layers):
        assert Ln["qkv"]["names"] == [n for n, *_ in Lp["qkv"]]
        assert Ln["qkv"]["bias"] == (list(Lp["qkv_b"]) if Lp["qkv_b"] else [])
        assert Ln["gate_up"]["bias"] == ([Lp["gate_up_b"]] if Lp["gate_up_b"] else [])
        assert Ln["down"]["names"] == [Lp["down"][0]] and Ln["o"]["bias"] == []
        assert (Ln["qkv"]["K"], Ln["qkv"]["N"]) == (c.n_embd, nq)


def test_native_executor_rejects_bad_files(tmp_path):
    from ggmlc_amd import _lib
    from ggmlc_amd.executor import inspect

    c = _tiny()
    p = write_llama_gguf(tmp_path / "m.gguf", c, _weights(c), max_pos=64)
    raw = p.read_bytes()
    with pytest.raises(_lib.GQError, match="magic"):
        inspect(b"XXXX" + raw[4:])
    with pytest.raises(_lib.GQError, match="truncated|past the end"):
        inspect(raw[: len(raw) // 2])
    # a graph the decoder layout does not cover is refused, naming the node
    g = Graph.from_json(gguf.GGUFReader(p).metadata["ggmlc.graph_spec"])
    for n in g.nodes:
        if n.op == "ROPE":
            n.attributes["mode"] = 0
    w = gguf.GGUFWriter()
    w.add_string("ggmlc.graph_spec", g.to_json())
    rd = gguf.GGUFReader(p)
    for name in rd.tensor_order:
        t = rd.tensors[name]
        w.add_tensor(name, list(t.ne) + [1] * (4 - len(t.ne)), t.ggml_type, bytes(rd.tensor_bytes(name)))
    with pytest.raises(_lib.GQError, match="NEOX") as e:
        inspect(w.to_bytes())
    assert e.value.code == -2  # GQ_ERR_UNSUPPORTED


def _one_tensor_gguf(ne, ggml_type=8, offset=0, data=b""):
    """A GGUF v3 file holding one tensor info with the raw dims ne (u64 each)."""
    import struct

    name = b"w"
    head = b"GGUF" + struct.pack("<IQQ", 3, 1, 0)
    info = struct.pack("<Q", len(name)) + name + struct.pack("<I", len(ne))
    info += b"".join(struct.pack("<Q", d & (2**64 - 1)) for d in ne)
    info += struct.pack("<IQ", ggml_type, offset)
    raw = head + info
    return raw + b"\0" * (-len(raw) % 32) + data


@pytest.mark.parametrize("ne,what", [
    ([32, -1], "negative dimension"),
    ([-32, 4], "negative dimension"),
    ([2**40, 2**40], "element count"),                # 2^80 elements
    ([32, 2**31, 2**31, 4], "element count"),          # 2^69
    ([2**62, 4], "element count"),
    ([32, 2**59], "element count"),                   # 2^64 elements
    ([32, 2**56], "past the end"),                    # 2.4e18 bytes: no wrap, far past the file
    ([64, 1], "past the end"),                        # two blocks declared, one present
    ([2**61, 2, 1, 1, 28], "byte size"),              # F64: 2^62 elements of 8 bytes, past 2^64
])
def test_native_gguf_rejects_bad_dimensions(ne, what):
    """gq_exec's GGUF reader refuses negative dims, element counts past int64 and byte sizes
    that wrap (the reference's gguf.cpp:682-735 refuses the same), before any size is
    used; a tensor whose bytes run past the file is refused with overflow-free checks."""
    from ggmlc_amd import _lib
    from ggmlc_amd.executor import inspect

    ggml_type = 8  # Q8_0, or the fifth entry
    if len(ne) == 5:
        ne, ggml_type = ne[:4], ne[4]
    with pytest.raises(_lib.GQError, match=what):
        inspect(_one_tensor_gguf(ne, ggml_type, data=b"\x01" * 34))


@needs_ref
@pytest.mark.skipif(not O.ref_v4_usable(), reason="AVX-512 reference build absent or host lacks AVX-512 VNNI")
@pytest.mark.parametrize("qtype", [O.Q8_0, O.Q4_0])
def test_reference_avx512_build_agrees_with_v3_build(qtype):
    """The AVX-512 build of the reference (bench.py's CPU baseline on hosts that have
    the instructions) computes the decoder of the x86-64-v3 build. The int block sums
    are exact in both; the fp32 accumulation of ggml's 16-lane AVX-512 paths is ordered
    differently from its 8-lane AVX2 ones for Q4_0 (Q8_0 gives the same bits), which a
    random-init model amplifies to a few 1e-5 in the logits' cosine, the order of the
    reference's own prefill-vs-token-by-token spread at this depth."""
    c = _tiny(qtype, False)
    w = _weights(c)
    toks = np.random.default_rng(8).integers(0, c.n_vocab, 29).astype(np.int32)
    a, b = O.RefLlama(c, w, 256, n_threads=4), O.RefLlama(c, w, 256, n_threads=4, variant="v4")
    la, na = a.step(toks)
    lb, _ = b.step(toks)
    for _ in range(3):
        cos = float(la @ lb / np.linalg.norm(la) / np.linalg.norm(lb))
        assert cos > 0.9999 and np.abs(la - lb).max() <= 3e-2 * np.abs(la).max(), cos
        t = np.array([na], np.int32)  # both decode the v3 build's token
        la, na = a.step(t)
        lb, _ = b.step(t)
