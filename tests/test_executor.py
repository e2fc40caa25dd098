"""libgq's executor handle (include/gq.h gq_exec_*, ggmlc_amd.executor.ModelExecutor):
the reference executor's surface in C++ over this library's kernels, no torch.

* against ggmlc's own runtime running the same .gguf on the CPU (oracle.RefRuntime:
  the reference loader.cpp + executor.cpp): prefill and decode steps with the KV cache,
  at the bars of tests/test_runner.py; LLaMA and Qwen2 (q/k/v biases) layouts;
* HIP-graph replay gives the bits of eager execution, call after call;
* logits_last_only (executor.cpp:2396-2410), tensor shapes, reset_kv_cache, runs
  without a KV cache, and rejected calls that leave the handle usable.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle as O
from ggmlc_amd.model import LlamaConfig

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not O.ref_available(), reason="needs oracle/_ref")]


def _cos(a, b):
    a, b = np.asarray(a, np.float64).ravel(), np.asarray(b, np.float64).ravel()
    return float(a @ b / np.linalg.norm(a) / np.linalg.norm(b))


def _model(tmp_path, kind="tiny", fused_qkv=True):
    from ggmlc_amd.llama_gguf import write_llama_gguf

    if kind == "qwen":
        c = LlamaConfig("tiny-qwen", 2, 256, 12, 2, 128, 512, 512, O.Q8_0, rope_base=1e6, qkv_bias=True)
    else:
        c = LlamaConfig("tiny", 2, 256, 4, 2, 64, 512, 512, O.Q8_0 if kind == "tiny" else O.Q4_0)
    rng = np.random.default_rng(17)

    def q(n, k):
        return O.quantize_weights((rng.standard_normal((n, k)) * 0.02).astype(np.float32), c.qtype)

    nq = c.q_dim + 2 * c.kv_dim
    layers = [(q(nq, c.n_embd), q(c.n_embd, c.q_dim), q(2 * c.n_ff, c.n_embd), q(c.n_embd, c.n_ff))
              + (((rng.standard_normal(nq) * 0.3).astype(np.float32), None, None, None) if c.qkv_bias else ())
              for _ in range(c.n_layer)]
    emb = q(c.n_vocab, c.n_embd)
    p = write_llama_gguf(tmp_path / f"{kind}.gguf", c, (emb, q(c.n_vocab, c.n_embd), layers), max_pos=1024,
                         fused_qkv=fused_qkv)
    return c, p


def _run(ex, ids, pos):
    ex.prepare({"s": len(ids), "pos": pos})
    ex.set_input_by_id(ex.inputs[0], np.asarray(ids, np.int32))
    ex.run()
    return ex.get_output(ex.outputs[0]).copy()


@pytest.mark.parametrize("kind,fused_qkv", [("tiny", True), ("tiny_q4", False), ("qwen", True)])
def test_executor_matches_reference_runtime(tmp_path, kind, fused_qkv):
    from ggmlc_amd.executor import ModelExecutor

    c, p = _model(tmp_path, kind, fused_qkv)
    ex = ModelExecutor(p.read_bytes(), "gpu")
    assert ex.device == "cuda:0" and ex.config["n_layer"] == 2 and ex.config["qkv_bias"] == c.qkv_bias
    ex.init_kv_cache(512)
    assert ex.has_kv_cache()
    ref = O.RefRuntime(p, max_ctx=512, n_threads=8)
    tid_in, tid_out = ex.inputs[0], ex.outputs[0]
    prompt = np.random.default_rng(3).integers(0, c.n_vocab, 37).astype(np.int32)
    got = _run(ex, prompt, 0)
    assert ex.get_tensor_shape(tid_out) == [c.n_vocab, 37, 1, 1] and got.shape == (37, c.n_vocab)
    ref.run({tid_in: prompt[None, :]}, {"s": 37, "pos": 0})
    want = ref.output(tid_out).reshape(37, c.n_vocab)
    cos = [_cos(got[i], want[i]) for i in range(37)]
    print(kind, "prefill min cos", min(cos), "last", cos[-1])
    assert cos[-1] >= 0.9999 and min(cos) >= 0.9999 - 1e-4
    tok = int(np.argmax(want[-1]))
    for i in range(4):  # decode steps: the s = 1 bucket's graph replays from the second on
        got = _run(ex, [tok], 37 + i)
        ref.run({tid_in: np.array([[tok]], np.int32)}, {"s": 1, "pos": 37 + i})
        want = ref.output(tid_out).reshape(-1)
        assert _cos(got[0], want) >= 0.9999, (i, _cos(got[0], want))
        tok = int(np.argmax(want))
    assert ex.position == 41


def test_executor_graph_replay_is_bit_identical_to_eager(tmp_path):
    from ggmlc_amd.executor import ModelExecutor

    c, p = _model(tmp_path, "qwen")
    outs = []
    for graphs in (False, True):
        ex = ModelExecutor(p.read_bytes(), "gpu")
        ex.set_enable_cuda_graph(graphs)
        ex.init_kv_cache(512)
        prompt = np.random.default_rng(4).integers(0, c.n_vocab, 23).astype(np.int32)
        seq = [_run(ex, prompt, 0)]
        for i in range(5):  # runs 2.. of the s = 1 bucket replay its graph
            seq.append(_run(ex, [int(np.argmax(seq[-1][-1]))], 23 + i))
        seq.append(_run(ex, prompt[:7], 28))  # a second prompt-sized bucket (GEMM path)
        outs.append(seq)
    for a, b in zip(*outs):
        assert np.array_equal(a, b)


def test_executor_logits_last_only_and_state(tmp_path):
    from ggmlc_amd.executor import ModelExecutor

    c, p = _model(tmp_path)
    ex = ModelExecutor(p.read_bytes(), "gpu")
    prompt = np.random.default_rng(5).integers(0, c.n_vocab, 19).astype(np.int32)
    no_cache = _run(ex, prompt, 0)  # without a KV cache: a scratch cache for the call
    assert not ex.has_kv_cache()
    ex.init_kv_cache(256)
    full = _run(ex, prompt, 0)
    assert np.array_equal(full, no_cache)
    ex.reset_kv_cache()
    assert ex.position == 0
    ex.set_logits_last_only(True)
    assert ex.logits_last_only()
    last = _run(ex, prompt, 0)
    assert last.shape == (1, c.n_vocab) and ex.get_tensor_shape(ex.outputs[0]) == [c.n_vocab, 1, 1, 1]
    # one row through the GEMV against 19 through the GEMM: the same exact block products
    assert np.abs(last[0] - full[-1]).max() <= 1e-5 * np.abs(full[-1]).max()
    assert int(np.argmax(last[0])) == int(np.argmax(full[-1]))


def test_executor_rejected_calls_leave_it_usable(tmp_path):
    from ggmlc_amd import GQError
    from ggmlc_amd.executor import ModelExecutor, get_available_devices

    assert get_available_devices()[0] == "cuda:0"
    c, p = _model(tmp_path)
    with pytest.raises(GQError, match="GPU only"):
        ModelExecutor(p.read_bytes(), "cpu")
    ex = ModelExecutor(p.read_bytes(), "auto")
    ex.init_kv_cache(256)
    with pytest.raises(GQError, match="prepare"):
        ex.set_input_by_id(ex.inputs[0], np.zeros(3, np.int32))
    with pytest.raises(GQError, match="exceeds the KV cache"):
        ex.prepare({"s": 10, "pos": 250})
    with pytest.raises(GQError, match="unknown symbol"):
        ex.prepare({"s": 1, "bogus": 3})
    ex.prepare({"s": 2, "pos": 0})
    with pytest.raises(GQError, match="bytes"):
        ex.set_input_by_id(ex.inputs[0], np.zeros(3, np.int32))
    ex.set_input_by_id(ex.inputs[0], np.array([1, c.n_vocab], np.int32))
    with pytest.raises(GQError, match="vocabulary"):
        ex.run()
    with pytest.raises(GQError, match="no output"):
        ex.get_output_bytes(ex.outputs[0])
    ex.set_input_by_name("input_ids", np.array([1, 2], np.int32))
    ex.run()
    out = ex.get_output(ex.outputs[0])
    assert out.shape == (2, c.n_vocab) and np.isfinite(out).all()
