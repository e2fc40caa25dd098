"""The runner surface (ggmlc_amd.runner: load / ModelRunner over a .gguf) on the GPU,
against ggmlc's own runtime running the same file on the CPU (oracle.RefRuntime:
the reference's loader.cpp + executor.cpp built from its sources).

Bars: the whole-model bars of tests/test_model.py (the quantized pipeline's noise
floor keeps end-to-end cosine near 0.99995, see test_noise_floor_of_quantized_pipeline):
cosine >= 0.9999 for the last prompt row and each decode step on the tiny models, >= 0.9995
at SmolLM2 layer shapes; every one of the 37 prompt rows within 1e-4 of that bar (the
minimum over 37 rows samples the tail of the floor)."""

from __future__ import annotations

import numpy as np
import pytest

import oracle as O
from ggmlc_amd.model import SMOLLM2_360M, LlamaConfig

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not O.ref_available(), reason="needs oracle/_ref")]


def _cos(a, b):
    a, b = np.asarray(a, np.float64).ravel(), np.asarray(b, np.float64).ravel()
    return float(a @ b / np.linalg.norm(a) / np.linalg.norm(b))


def _weights(c, seed=7):
    rng = np.random.default_rng(seed)

    def q(n, k):
        return O.quantize_weights((rng.standard_normal((n, k)) * 0.02).astype(np.float32), c.qtype)

    layers = [(q(c.q_dim + 2 * c.kv_dim, c.n_embd), q(c.n_embd, c.q_dim), q(2 * c.n_ff, c.n_embd),
               q(c.n_embd, c.n_ff)) for _ in range(c.n_layer)]
    embed = q(c.n_vocab, c.n_embd)
    return embed, embed if c.tied_embeddings else q(c.n_vocab, c.n_embd), layers


@pytest.mark.parametrize("shape,fused_qkv", [("tiny_q8", True), ("tiny_q4", False), ("smollm2", True),
                                             ("qwen_bias", True), ("qwen_bias", False)])
def test_runner_matches_reference_runtime(tmp_path, shape, fused_qkv):
    from dataclasses import replace

    from ggmlc_amd import runner as R
    from ggmlc_amd.llama_gguf import write_llama_gguf

    if shape == "smollm2":
        c, bar = replace(SMOLLM2_360M, n_layer=2, n_vocab=4096), 0.9995
    elif shape == "qwen_bias":  # the Qwen2 layout: GQA 6, q/k/v biases, rope base 1e6
        c, bar = LlamaConfig("tiny-qwen", 2, 256, 12, 2, 128, 512, 512, O.Q8_0, rope_base=1e6, qkv_bias=True), 0.9999
    else:
        c, bar = LlamaConfig("tiny", 2, 256, 4, 2, 64, 512, 512, O.Q8_0 if shape == "tiny_q8" else O.Q4_0), 0.9999
    w = _weights(c)
    if c.qkv_bias:
        rng = np.random.default_rng(12)
        w = (w[0], w[1], [tuple(L) + ((rng.standard_normal(c.q_dim + 2 * c.kv_dim) * 0.3).astype(np.float32),
                                      None, None, None) for L in w[2]])
    p = write_llama_gguf(tmp_path / "m.gguf", c, w, max_pos=1024, fused_qkv=fused_qkv)
    with pytest.raises(ValueError, match="GPU only"):
        R.load(p, device="cpu")
    run = R.load(p, device="gpu")
    assert run.device == "cuda:0" and run.cfg.n_layer == 2 and run.cfg.head_dim == c.head_dim
    run.init_kv_cache(512)
    assert run.has_kv_cache()
    ref = O.RefRuntime(p, max_ctx=512, n_threads=8)
    tid_in, tid_out = run.inputs[0], run.outputs[0]
    prompt = np.random.default_rng(3).integers(0, c.n_vocab, 37).astype(np.int32)[None, :]

    got = run(prompt, symbols={"pos": 0, "s": 37})
    ref.run({tid_in: prompt}, {"s": 37, "pos": 0})
    want = ref.output(tid_out).reshape(37, c.n_vocab)
    assert got.shape == (37, c.n_vocab)
    cos = [_cos(got[i], want[i]) for i in range(37)]
    print(shape, "prefill min cos", min(cos), "last", cos[-1])
    assert cos[-1] >= bar  # the row a generator samples from, at the end-to-end bar
    assert min(cos) >= bar - 1e-4  # all 37 rows: the minimum samples the noise floor's tail
    tok = int(np.argmax(want[-1]))
    for i in range(3):
        ids = np.array([[tok]], np.int32)
        got = run(ids, symbols={"pos": 37 + i, "s": 1})
        ref.run({tid_in: ids}, {"s": 1, "pos": 37 + i})
        want = ref.output(tid_out).reshape(-1)
        print(shape, "decode", i, _cos(got, want))
        assert got.shape == (1, c.n_vocab) and _cos(got, want) >= bar
        tok = int(np.argmax(want))

    # no KV cache: the whole sequence from position 0 gives the prefill's bits
    run2 = R.load(p, device="auto")
    assert not run2.has_kv_cache()
    full = run2(prompt)
    run.reset_kv_cache()
    again = run(prompt, symbols={"pos": 0, "s": 37})
    assert np.array_equal(full, again)


def test_runner_rejects_missing_or_bad_files(tmp_path):
    from ggmlc_amd import runner as R

    with pytest.raises(FileNotFoundError):
        R.load(tmp_path / "none.gguf")
    with pytest.raises(ValueError, match="GGUF"):
        R.load(b"not a gguf file at all.........................")
    assert R.get_available_devices()[0] == "cuda:0"


def test_runner_executor_drives_the_scheduler(tmp_path):
    """`ContinuousBatchScheduler(runner.executor, ...)` as the reference's tests call it
    (tests/e2e/test_prefix_caching.py): tokens_per_page set before the paged cache, two
    requests sharing a one-page prefix, the ids generated for each request checked
    against the reference executor running the same file on that request alone."""
    from ggmlc_amd import runner as R
    from ggmlc_amd.batching import ContinuousBatchScheduler
    from ggmlc_amd.llama_gguf import write_llama_gguf

    c = LlamaConfig("tiny", 2, 256, 4, 2, 64, 512, 512, O.Q8_0)
    p = write_llama_gguf(tmp_path / "m.gguf", c, _weights(c), max_pos=1024)
    run = R.load(p, device="gpu")
    ex = run.executor
    ex.set_tokens_per_page(128)
    assert ex.tokens_per_page == 128 and not ex.is_paged_kv_cache_enabled()
    ex.configure_vmm_pool(max_warm_pages=32, prealloc_pages=8)
    ex.init_paged_kv_cache(4, 512)
    sched = ContinuousBatchScheduler(ex, max_batch_size=4, eos_token_id=-1)
    rng = np.random.default_rng(8)
    shared = rng.integers(0, c.n_vocab, 128).tolist()
    prompts = [shared + rng.integers(0, c.n_vocab, 9).tolist(), shared + rng.integers(0, c.n_vocab, 3).tolist()]
    rids = [sched.add_request(prompts[0], max_new_tokens=5)]
    sched.step()
    rids.append(sched.add_request(prompts[1], max_new_tokens=5))
    while sched.has_work():
        sched.step()
    assert sched.total_prefix_cache_hits == 1
    assert ex.get_paged_active_vram_bytes() == ex.batch.kv.page_bytes  # the cached prefix page
    tid_in, tid_out = run.inputs[0], run.outputs[0]
    for rid, prompt in zip(rids, prompts):
        r = sched.get_request(rid)
        assert r.finished and len(r.generated_tokens) == 5
        ref = O.RefRuntime(p, max_ctx=512, n_threads=8)
        ref.run({tid_in: np.array([prompt], np.int32)}, {"s": len(prompt), "pos": 0})
        want = ref.output(tid_out).reshape(len(prompt), c.n_vocab)[-1]
        for j, tok in enumerate(r.generated_tokens):
            top = float(want.max())
            assert tok == int(np.argmax(want)) or top - float(want[tok]) <= 0.02 * float(want.std()), (rid, j)
            ref.run({tid_in: np.array([[tok]], np.int32)}, {"s": 1, "pos": len(prompt) + j})
            want = ref.output(tid_out).reshape(-1)
