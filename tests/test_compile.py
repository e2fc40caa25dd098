"""The compile path (ggmlc_amd.compile): PyTorch LLaMA-family module -> fused, baked,
quantized .gguf (LlamaForCausalLM and Qwen2ForCausalLM, whose q/k/v biases ride on the
fused QKV MUL_MAT's third input).

* the host quantizer gives the bytes of the oracle's restatement of quantize.py
  (itself pinned by tests/test_oracle.py), ties and zero blocks included;
* a compiled random-init transformers LlamaForCausalLM (with non-trivial RMSNorm
  gammas, tied and untied heads, eps 1e-5 and 1e-6) has the fused layout, and its
  baked weights dequantize to W * gamma within the quantization step;
* ggmlc's own runtime (oracle.RefRuntime: the reference loader + executor) running
  the compiled file reproduces the module's float32 logits up to the weight
  quantization (bars below the values measured on these shapes, 0.9997 for Q8_0 and 0.967 for
  Q4_0: cosine >= 0.999 and >= 0.95), and the GPU runner matches that runtime at the
  end-to-end bar (0.9999).
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle as O


def _cos(a, b):
    a, b = np.asarray(a, np.float64).ravel(), np.asarray(b, np.float64).ravel()
    return float(a @ b / np.linalg.norm(a) / np.linalg.norm(b))


def test_host_quantizer_matches_oracle():
    from ggmlc_amd.compile import quantize_rows

    rng = np.random.default_rng(0)
    w = (rng.standard_normal((37, 256)) * 0.02).astype(np.float32)
    w[0] = 0.0                                           # zero blocks: d = 0
    w[1, :32] = np.arange(32, dtype=np.float32) - 15.5   # ties at half steps
    w[2, :32] = 127.0                                    # q = 127 everywhere
    w[3, :32] = -8.0 * np.arange(1, 33, dtype=np.float32) / 32  # Q4_0 signed max at the end
    w[4] = rng.standard_normal(256).astype(np.float32) * 1e4
    for qt in (O.Q8_0, O.Q4_0):
        assert np.array_equal(quantize_rows(w, qt), O.quantize_weights(w, qt)), qt


def _hf_llama(tied: bool, eps: float, seed: int = 0):
    import torch
    from transformers import LlamaConfig, LlamaForCausalLM

    cfg = LlamaConfig(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=1024,
                      rms_norm_eps=eps, rope_theta=10000.0, tie_word_embeddings=tied)
    torch.manual_seed(seed)
    m = LlamaForCausalLM(cfg).eval()
    with torch.no_grad():  # RMSNorm gammas away from 1, so the bake is visible
        for mod in m.modules():
            if type(mod).__name__.endswith("RMSNorm"):
                mod.weight.copy_(1.0 + 0.2 * torch.randn_like(mod.weight))
    return m


def _hf_qwen2(tied: bool, seed: int = 0):
    """A random-init transformers Qwen2ForCausalLM: the LLaMA layout plus q/k/v biases
    (made non-zero here: the module initialises them to zero)."""
    import torch
    from transformers import Qwen2Config, Qwen2ForCausalLM

    cfg = Qwen2Config(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=1024,
                      rms_norm_eps=1e-6, rope_theta=1000000.0, tie_word_embeddings=tied)
    torch.manual_seed(seed)
    m = Qwen2ForCausalLM(cfg).eval()
    with torch.no_grad():
        for mod in m.modules():
            if type(mod).__name__.endswith("RMSNorm"):
                mod.weight.copy_(1.0 + 0.2 * torch.randn_like(mod.weight))
        for L in m.model.layers:
            for lin in (L.self_attn.q_proj, L.self_attn.k_proj, L.self_attn.v_proj):
                lin.bias.copy_(0.5 * torch.randn_like(lin.bias))
    return m


def test_compiled_qwen2_biases(tmp_path):
    """q/k/v biases land concatenated (q | k | v, fp32, unbaked) on the fused QKV MUL_MAT's
    third input, and the runner's matcher reads them back."""
    from ggmlc_amd.compile import compile_llama
    from ggmlc_amd.gguf import GGUFReader
    from ggmlc_amd.graph_spec import OPS, Graph
    from ggmlc_amd.runner import match_llama

    m = _hf_qwen2(tied=True)
    p = compile_llama(m, tmp_path / "q.gguf", quantize="q8_0", max_pos=512)
    r = GGUFReader(p)
    g = Graph.from_json(r.metadata["ggmlc.graph_spec"])
    mt = match_llama(g, r)
    assert mt.rope_base == 1e6 and mt.layers[0]["o_b"] is None and mt.layers[0]["down_b"] is None
    for li, L in enumerate(m.model.layers):
        (name,) = mt.layers[li]["qkv_b"]
        want = np.concatenate([lin.bias.detach().numpy() for lin in
                               (L.self_attn.q_proj, L.self_attn.k_proj, L.self_attn.v_proj)])
        assert np.array_equal(r.tensor_array(name), want.astype(np.float32))
    mm3 = [n for n in g.nodes if n.opcode == OPS["MUL_MAT"] and len(n.inputs) == 3]
    assert len(mm3) == 2  # one fused QKV product per layer


def test_compiled_layout_and_bake(tmp_path):
    from ggmlc_amd.compile import compile_llama
    from ggmlc_amd.gguf import GGUFReader
    from ggmlc_amd.graph_spec import Graph
    from ggmlc_amd.runner import match_llama

    m = _hf_llama(tied=False, eps=1e-5)
    p = compile_llama(m, tmp_path / "m.gguf", quantize="q8_0", max_pos=512)
    r = GGUFReader(p)
    g = Graph.from_json(r.metadata["ggmlc.graph_spec"])
    mt = match_llama(g, r)
    assert (mt.n_embd, mt.n_head, mt.n_head_kv, mt.head_dim, mt.n_ff, mt.n_vocab) == (256, 4, 2, 64, 512, 512)
    assert list(r.tensors["blk.0.attn_qkv"].ne[:2]) == [256, 512]
    assert list(r.tensors["blk.1.ffn_gate_up"].ne[:2]) == [256, 1024]
    L = m.model.layers[1]
    g1 = L.input_layernorm.weight.detach().numpy()
    want = np.concatenate([L.self_attn.q_proj.weight.detach().numpy(), L.self_attn.k_proj.weight.detach().numpy(),
                           L.self_attn.v_proj.weight.detach().numpy()]) * g1[None, :]
    got = O.dequantize(r.tensor_array("blk.1.attn_qkv"), O.Q8_0, 256)
    # half a quantization step per block, plus the fp16 rounding of the block scale (|q| <= 127)
    step = np.abs(want).reshape(-1, 32).max(1) / 127.0
    assert np.all(np.abs(got - want).reshape(-1, 32) <= (0.5 + 127 * 2.0 ** -11) * step[:, None] * 1.001)
    gf = m.model.norm.weight.detach().numpy()
    head = O.dequantize(r.tensor_array("output"), O.Q8_0, 256)
    assert _cos(head, m.lm_head.weight.detach().numpy() * gf[None, :]) > 0.9999


@pytest.mark.skipif(not O.ref_available(), reason="needs oracle/_ref")
@pytest.mark.parametrize("quant,tied,eps,bar", [("q8_0", False, 1e-5, 0.999), ("q8_0", True, 1e-6, 0.999),
                                                 ("q4_0", False, 1e-5, 0.95), ("qwen2", True, 1e-6, 0.999)])
def test_reference_runtime_runs_the_compiled_module(tmp_path, quant, tied, eps, bar):
    import torch

    from ggmlc_amd.compile import compile_llama

    if quant == "qwen2":  # q/k/v biases through the reference executor's bias ADD
        m, quant = _hf_qwen2(tied=tied, seed=1), "q8_0"
    else:
        m = _hf_llama(tied=tied, eps=eps, seed=1)
    p = compile_llama(m, tmp_path / "m.gguf", quantize=quant, max_pos=512)
    ids = np.random.default_rng(2).integers(0, 512, 29).astype(np.int32)
    with torch.no_grad():
        want = m(torch.from_numpy(ids[None, :]).long()).logits[0].numpy()
    from ggmlc_amd.gguf import GGUFReader
    from ggmlc_amd.graph_spec import Graph

    g = Graph.from_json(GGUFReader(p).metadata["ggmlc.graph_spec"])
    tid_in, tid_out = g.inputs[0], g.outputs[0]
    rt = O.RefRuntime(p, max_ctx=256, n_threads=8)
    rt.run({tid_in: ids[None, :]}, {"s": 29, "pos": 0})
    got = rt.output(tid_out).reshape(29, 512)
    cs = [_cos(got[i], want[i]) for i in range(29)]
    print(quant, tied, eps, "min cos vs module", min(cs))
    assert min(cs) >= bar


@pytest.mark.gpu
@pytest.mark.skipif(not O.ref_available(), reason="needs oracle/_ref")
@pytest.mark.parametrize("family", ["llama", "qwen2"])
def test_gpu_runner_runs_the_compiled_module(tmp_path, family):
    import torch

    from ggmlc_amd import runner as R
    from ggmlc_amd.compile import compile_llama

    m = _hf_llama(tied=False, eps=1e-5, seed=3) if family == "llama" else _hf_qwen2(tied=True, seed=3)
    p = compile_llama(m, tmp_path / "m.gguf", quantize="q8_0", max_pos=512)
    ids = np.random.default_rng(4).integers(0, 512, 33).astype(np.int32)
    run = R.load(p, device="gpu")
    run.init_kv_cache(256)
    got = run(ids[None, :], symbols={"pos": 0, "s": 33})
    rt = O.RefRuntime(p, max_ctx=256, n_threads=8)
    rt.run({run.inputs[0]: ids[None, :]}, {"s": 33, "pos": 0})
    ref = rt.output(run.outputs[0]).reshape(33, 512)
    with torch.no_grad():
        want = m(torch.from_numpy(ids[None, :]).long()).logits[0].numpy()
    assert _cos(got[-1], ref[-1]) >= 0.9999
    assert min(_cos(got[i], ref[i]) for i in range(33)) >= 0.9999 - 1e-4
    assert min(_cos(got[i], want[i]) for i in range(33)) >= 0.999
