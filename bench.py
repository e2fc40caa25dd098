#!/usr/bin/env python3
"""Benchmark of the quantized hot path on one MI355X (gfx950).

Workload: a LLaMA-7B-shape decoder (32 layers, hidden
4096, 32 heads MHA, head_dim 128, FFN 11008, vocab 32000), random-init weights
N(0, 0.02) quantized to Q4_0 on the device, F16 KV cache, batch 1. A 1024-token
uniform-random prompt runs in ubatches of 512 (pp512 = the first ubatch, pp1024 =
both), then greedy decode; the first decode token is untimed (ggmlc_bench.cpp
methodology, runtime/tools/ggmlc_bench.cpp:295-560).

* step      = one greedy decode token through the whole model (embedding ->
              32 layers -> lm_head -> argmax), replayed from the (1, n_kv) bucket's
              HIP graph whose input is its own previous output; value = tg tokens/s
              over exactly --steps tokens (tg128 by default).
* roofline  = the decode GEMV, the dominant kernel of the step: the 129 fused GEMV
              launches of one decode token exactly as the timed step issues them
              (qkv with ADD + RMS_NORM + ROPE + SET_ROWS, o, gate_up with ADD +
              RMS_NORM + SWIGLU, down, lm_head with ADD + RMS_NORM), same buffers and
              weights, captured back to back in one graph and timed with HIP events on
              the launch stream; achieved = their algorithmic bytes (weights + the fp32
              activations read + the outputs written) / their time.
* roofline_prefill_gemm = the 128 prefill GEMMs (M = 512) of one ubatch, same way.
* gemv_c1_q8_0 = configs[0], the Q8_0 Linear 4096 -> 4096 GEMV (16 rotating copies).
* mlp_c2_q4_0 = configs[1], the SwiGLU MLP block 4096 -> 11008 -> 4096 (Q4_0) at
              M = 1, 8, 128, 512 tokens (4 rotating weight copies, 304 MB).
* smollm2_c3 = configs[2], the SmolLM2-360M-shape decoder (Q8_0): pp512, then tg128.
* c5_batched_decode = configs[4]: a Qwen2.5-1.5B-shape decoder (Q8_0, tied embeddings)
              over the paged KV pool; 16 sequences with contexts uniform in [256, 4096],
              half of them sharing a 512-token prefix (its pages computed once), then 64
              batched decode steps at B = 1, 2, 4, 8, 16, every sequence at its own
              position; tokens/s = B * steps / time (graph replays chained on the device).
* cpu_baseline = the reference's own ggml CPU backend (oracle/_ref, built from the
              reference sources, AVX-512 build where the host has it) running the same
              decoder graph on the same weights with the host's cores: pp512, then decode
              tokens at the GPU's context (~1030), and a 1-thread decode sample.

Weights (3.7 GB) far exceed the 256 MB Infinity Cache, so every decode token
streams them from HBM. Inputs are resident before timing.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "pp512 & tg128 tokens/sec (1 GPU, Q8_0/Q4_0); GEMV HBM GB/s as % of peak"
HBM_PEAK_GBS = 8000.0
FP16_MFMA_PEAK_TFLOPS = 2500.0
UBATCH = 512
CPU_SHARE = 16  # host cores one GPU's job may use on the GPU boxes


def parse():
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=128, help="timed decode tokens (tg128)")
    p.add_argument("--warmup", type=int, default=2, help="untimed decode tokens before the timed ones")
    p.add_argument("--prompt", type=int, default=1024, help="prompt tokens (multiple of 512)")
    p.add_argument("--pp-reps", type=int, default=5)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--cpu-seconds", type=float, default=10.0, help="decode budget of the CPU sample")
    p.add_argument("--c1-launches", type=int, default=400)
    p.add_argument("--no-sweep", action="store_true", help="skip the Q8_0 decode GEMV size sweep")
    p.add_argument("--no-c2", action="store_true", help="skip the configs[1] MLP M-sweep")
    p.add_argument("--no-c3", action="store_true", help="skip the configs[2] SmolLM2-360M decoder")
    p.add_argument("--c5-steps", type=int, default=64, help="timed batched decode steps per batch size")
    p.add_argument("--no-c5", action="store_true", help="skip the configs[4] continuous-batching decode")
    p.add_argument("--c5-only", action="store_true", help="run only the configs[4] measurement (profiling)")
    p.add_argument("--c3-only", action="store_true", help="run only the configs[2] measurement (profiling)")
    p.add_argument("--c5-batches", default="1,2,4,8,16", help="configs[4] batch sizes")
    p.add_argument("--roofline-only", action="store_true",
                   help="only the configs[3] decoder (pp, tg) and the step-GEMV roofline graph: the workload of "
                        "the rocprofv3 --kernel-trace --stats summary behind roofline")
    p.add_argument("--traffic-probe", action="store_true",
                   help="only launch one token's fused decode GEMVs and a 256 MiB device copy, eagerly, 3 times "
                        "each (the workload of the rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs behind "
                        "roofline.traffic)")
    p.add_argument("--attn-probe", action="store_true",
                   help="only launch the configs[3] decode attention at its tg context over 16 K/V copies "
                        "(cold in the Infinity Cache), eagerly, 3 rounds, then a 256 MiB device copy 3 times "
                        "(the workload of the rocprofv3 --pmc runs behind the decode attention summary)")
    p.add_argument("--attn-stamps", action="store_true",
                   help="with --attn-probe: run the same launches through libgqbench's timestamped build of "
                        "the attention and print the per-wave event times")
    p.add_argument("--i8-probe", action="store_true",
                   help="only measure the configs[4] gate|up product on the int8 path (M = 16, K = 1536, SWIGLU "
                        "and the quantized rows): launch time against the row count (workgroups per CU), "
                        "per-wave event times from libgqbench's timestamped build, and a streaming read of "
                        "14 MiB against its workgroup count")
    p.add_argument("--gemm-probe", action="store_true",
                   help="only launch one ubatch's 128 prefill GEMMs (M = 512) eagerly, 3 times (the workload of "
                        "the rocprofv3 --pmc MFMA counter runs)")
    return p.parse_args()


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _ev():
    import torch

    return torch.cuda.Event(enable_timing=True)


def time_graph(fn, reps: int, warm: int = 1) -> float:
    """ms per replay of a HIP graph of fn(), timed with events on the replay stream."""
    import torch

    fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    for _ in range(warm):
        g.replay()
    torch.cuda.synchronize()
    e0, e1 = _ev(), _ev()
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    del g
    return e0.elapsed_time(e1) / reps


def main() -> int:
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (every GPU box here has one; "
              "run with --gpus 1)", file=sys.stderr)
        return 2
    if args.prompt % UBATCH or args.prompt <= 0:
        print("bench.py: --prompt must be a positive multiple of 512", file=sys.stderr)
        return 2

    import torch

    from ggmlc_amd import _lib, ops
    from ggmlc_amd.model import LLAMA_7B, random_weights

    torch.cuda.set_device(0)
    _lib.check(_lib.load().gq_init())
    dev = torch.device("cuda", 0)
    batches = tuple(int(b) for b in args.c5_batches.split(","))
    if args.c5_only:
        print(json.dumps({"c5_batched_decode": bench_c5(dev, args.c5_steps, batches)}), flush=True)
        return 0
    if args.attn_probe:
        return attn_probe(dev, args.attn_stamps)
    if args.c3_only:
        print(json.dumps({"smollm2_c3": bench_c3(dev, args.pp_reps)}), flush=True)
        return 0
    if args.i8_probe:
        print(json.dumps({"i8_probe": i8_probe(dev)}), flush=True)
        return 0
    cfg = LLAMA_7B

    log(f"building {cfg.name} Q4_0 weights on device")
    w = random_weights(cfg, dev, seed=1234)
    torch.cuda.synchronize()
    if args.traffic_probe:
        return traffic_probe(w, dev)
    if args.gemm_probe:
        return gemm_probe(w, dev)

    r7, dec = bench_decoder(w, dev, args.prompt, args.steps, args.warmup, args.pp_reps)
    ws = ops.Workspace(dev)
    ws.get(1 << 20)

    # ---- roofline: the fused GEMVs of the timed decode step, one graph, HIP events
    run_gemvs, gemv_bytes = step_gemv_launches(dec)
    R = 20
    gemv_ms_token = time_graph(run_gemvs, R, warm=3)
    n_gemv = len(gemv_bytes)
    gemv_bytes_token = sum(gemv_bytes)
    gemv_gbs = gemv_bytes_token / (gemv_ms_token * 1e-3) / 1e9
    weights_token = w.decode_bytes
    # the same launches as plain streaming reads of the same weight buffers: the
    # ceiling a kernel that only reads its weights reaches at these per-launch sizes
    probe_ms_token = time_probe_launches(step_weight_buffers(w))
    log(f"step GEMVs: {gemv_ms_token * 1e3:.1f} us/token, {gemv_gbs:.0f} GB/s "
        f"({gemv_gbs / HBM_PEAK_GBS:.1%}), same-size read {probe_ms_token * 1e3:.1f} us")
    roofline = {
        "kernel": "k_gemv_grp<Q4_0, M=1> fused: the 129 GEMV launches of one timed decode step (qkv + "
                  "ADD/RMS_NORM/ROPE/SET_ROWS, o, gate_up + ADD/RMS_NORM/SWIGLU, down x 32; lm_head + ADD/RMS_NORM)",
        "bound": "hbm",
        "achieved": round(gemv_gbs, 1),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(gemv_gbs / HBM_PEAK_GBS, 4),
        "traffic": load_traffic("k_gemv_grp<Q4_0, M=1> fused step mix"),
        "traffic_source": "not measured in this run: HBM bytes per launch from two rocprofv3 --pmc passes "
                          "(FETCH_SIZE, WRITE_SIZE, scaled by a 256 MiB copy) over an eager replay of the same "
                          "129 launches (bench.py --traffic-probe), profiles/gemv_traffic.json",
        "bytes_per_launch": round(gemv_bytes_token / n_gemv),
        "weight_bytes_per_launch": round(weights_token / n_gemv),
        "us_per_launch": round(gemv_ms_token * 1e3 / n_gemv, 3),
        "launches_per_token": n_gemv,
        "gemv_ms_per_token": round(gemv_ms_token, 4),
        "gemv_share_of_step": round(gemv_ms_token / r7["ms_per_token"], 4),
        "read_probe_same_launches_ms": round(probe_ms_token, 4),
        "frac_of_same_size_read": round(probe_ms_token / gemv_ms_token, 4),
    }
    if args.roofline_only:
        print(json.dumps({"configs[3]": r7, "roofline": roofline}), flush=True)
        return 0

    # ---- prefill GEMM rate: the 128 GEMMs of one ubatch (M = 512)
    gemm_ubatch, gemm_flops = prefill_gemms(w, dev, ws)
    gemm_ms = time_graph(gemm_ubatch, 3)
    gemm_tflops = gemm_flops / (gemm_ms * 1e-3) / 1e12
    del gemm_ubatch
    log(f"prefill GEMMs: {gemm_ms:.3f} ms/ubatch, {gemm_tflops:.0f} TFLOP/s")

    c1 = bench_c1(dev, ws, args.c1_launches)
    sweep = [] if args.no_sweep else gemv_sweep_q8_0(dev, ws)
    read_gbs, copy_gbs = measured_ceilings(dev)

    result = {
        "metric": METRIC,
        "value": r7["tg_tok_s"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": r7["ms_per_token"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_0 weights x q8_0 activations: int8 dot4 with exact int32 block sums (decode); exact "
                 "fp16 hi+lo block products on f16 MFMA (prefill); exact int32 block sums on int8 MFMA "
                 "(5..16 rows); f32 accumulate; f16 KV",
        "data": "synthetic (random-init weights N(0,0.02) -> Q4_0; uniform-random prompt ids)",
        "config": {
            "workload": f"configs[3] {cfg.name} decoder, Q4_0, batch 1: pp{args.prompt} (ubatch 512) then "
                        f"greedy decode; value = tg{args.steps} tokens/s",
            "global_batch": 1,
            "seq_len": args.prompt,
            "parallelism": "single GPU",
            "weight_bytes": w.nbytes,
        },
        "tg_tok_s": r7["tg_tok_s"],
        "pp512_tok_s": r7["pp512_tok_s"],
        f"pp{args.prompt}_tok_s": r7[f"pp{args.prompt}_tok_s"],
        "decode_weight_GBps": r7["decode_weight_GBps"],
        "decode_weight_plus_kv_GBps": r7["decode_weight_plus_kv_GBps"],
        "roofline": roofline,
        "roofline_prefill_gemm": {
            "kernel": "k_gemm_ws<Q4_0>: the 128 GEMMs of one 512-token ubatch (activation quantize excluded); "
                      "each exact block product takes two f16 MFMAs (hi, lo) per 32 K",
            "bound": "mfma",
            "achieved": round(gemm_tflops, 1),
            "peak": FP16_MFMA_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(gemm_tflops / FP16_MFMA_PEAK_TFLOPS, 4),
            "mfma_tflops_issued": round(2 * gemm_tflops, 1),
            "ms_per_ubatch": round(gemm_ms, 3),
        },
        "gemv_c1_q8_0": c1,
        "gemv_sweep_q8_0": sweep,
        "measured_read_GBps": round(read_gbs, 1),
        "measured_copy_GBps": round(copy_gbs, 1),
        "wall_s_timed": r7["wall_s_timed"],
    }

    del dec, run_gemvs
    torch.cuda.empty_cache()
    if not args.no_c2:
        log("configs[1]: SwiGLU MLP block, M sweep")
        result["mlp_c2_q4_0"] = bench_c2(dev, ws)
    if not args.no_c3:
        log("configs[2]: SmolLM2-360M-shape decoder")
        result["smollm2_c3"] = bench_c3(dev, args.pp_reps)
        torch.cuda.empty_cache()
    if not args.no_c5:
        log("configs[4]: batched paged decode")
        result["c5_batched_decode"] = bench_c5(dev, args.c5_steps, batches)
    if not args.no_cpu:
        log("cpu baseline")
        result["cpu_baseline"] = cpu_baseline(w, cfg, args.cpu_seconds, ctx=args.prompt)
    print(json.dumps(result), flush=True)
    return 0


def bench_c3(dev, pp_reps: int) -> dict:
    """the SmolLM2-360M-shape decoder (Q8_0): pp512 and tg128, plus its step
    GEMVs replayed as one graph."""
    from ggmlc_amd.model import SMOLLM2_360M, random_weights

    w3 = random_weights(SMOLLM2_360M, dev, seed=360)
    r3, d3 = bench_decoder(w3, dev, 512, 128, 2, pp_reps)
    run3, bytes3 = step_gemv_launches(d3)
    ms3 = time_graph(run3, 20, warm=3)
    r3["step_gemvs"] = {"launches": len(bytes3), "us_per_launch": round(ms3 * 1e3 / len(bytes3), 3),
                        "achieved_GBps": round(sum(bytes3) / (ms3 * 1e-3) / 1e9, 1),
                        "ms_per_token": round(ms3, 4)}
    r3["published_context"] = {"pp512_tok_s": 9900, "tg32_tok_s": 160.6,
                               "hardware": "NVIDIA RTX 4050 Laptop (reference README.md:243, "
                                           "docs/benchmarks/ggmlc_vs_llama_cpp.md:121,150)"}
    return r3


def bench_decoder(w, dev, prompt_len: int, steps: int, warmup: int, pp_reps: int):
    """pp (per 512-token ubatch graph) and tg (graph replays chained on the device) of
    one decoder at batch 1; returns (figures, the Decoder)."""
    import numpy as np
    import torch

    from ggmlc_amd.model import Decoder, pad_kv_len

    cfg = w.cfg
    n_ctx = prompt_len + warmup + steps
    max_ctx = pad_kv_len(n_ctx, 1 << 30)
    dec = Decoder(w, max_ctx, dev)
    log(f"{cfg.name}: weights {w.nbytes / 1e9:.3f} GB, KV cache "
        f"{2 * cfg.n_layer * cfg.kv_dim * max_ctx * 2 / 1e9:.3f} GB (max_ctx {max_ctx})")

    # ---- prefill graphs: one per ubatch bucket, reading its slice of the prompt
    gen = torch.Generator(device=dev)
    gen.manual_seed(99)
    prompt = torch.randint(0, cfg.n_vocab, (prompt_len,), generator=gen, device=dev, dtype=torch.int32)
    n_ub = prompt_len // UBATCH
    pp_graphs = []
    for u in range(n_ub):
        dec.reset(u * UBATCH)
        pp_graphs.append(dec.capture(UBATCH, pad_kv_len((u + 1) * UBATCH, max_ctx),
                                     ids=prompt[u * UBATCH:(u + 1) * UBATCH]))
    b_pp = dec._buffers(UBATCH)

    # ---- decode graphs: (1, n_kv) buckets; each reads the s=1 bucket's "next" and
    # overwrites it with the new token, so replays generate without host work
    _, next1 = dec.decode_buffers()
    tg_graphs = {}
    for i in range(warmup + steps):
        n_kv = pad_kv_len(prompt_len + i + 1, max_ctx)
        if n_kv not in tg_graphs:
            dec.reset(prompt_len + i)
            tg_graphs[n_kv] = dec.capture(1, n_kv, ids=next1)
    torch.cuda.synchronize()

    def prefill():
        dec.reset(0)
        for g in pp_graphs:
            g.replay()

    log(f"prefill: {n_ub} ubatch(es) of {UBATCH}, {pp_reps} reps")
    prefill()
    torch.cuda.synchronize()
    t_first, t_all = [], []
    for _ in range(pp_reps):
        dec.reset(0)
        es = [_ev() for _ in range(n_ub + 1)]
        es[0].record()
        for u, g in enumerate(pp_graphs):
            g.replay()
            es[u + 1].record()
        torch.cuda.synchronize()
        t_first.append(es[0].elapsed_time(es[1]))
        t_all.append(es[0].elapsed_time(es[-1]))
    pp512_tok_s = UBATCH * 1000.0 / float(np.median(t_first))
    ppN_tok_s = prompt_len * 1000.0 / float(np.median(t_all))
    log(f"pp512 {pp512_tok_s:.0f} tok/s, pp{prompt_len} {ppN_tok_s:.0f} tok/s")

    # ---- tg: the prompt's KV is in the cache (last prefill rep); decode from its token
    prefill()
    next1.copy_(b_pp["next"])
    torch.cuda.synchronize()
    if int(dec.pos[0]) != prompt_len:
        raise RuntimeError("device position after prefill is wrong")
    pos = prompt_len
    for i in range(warmup):
        tg_graphs[pad_kv_len(pos + 1, max_ctx)].replay()
        pos += 1
    torch.cuda.synchronize()
    log(f"decode: {warmup} warmup + {steps} timed tokens (graph replay)")
    e0, e1 = _ev(), _ev()
    t0 = time.perf_counter()
    e0.record()
    for i in range(steps):
        tg_graphs[pad_kv_len(pos + 1, max_ctx)].replay()
        pos += 1
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = e0.elapsed_time(e1) / steps
    tg_tok_s = 1000.0 / ms_step
    logits = dec._buffers(1)["logits"]
    if int(dec.pos[0]) != pos or not bool(torch.isfinite(logits).all()):
        raise RuntimeError("decode produced a wrong position or non-finite logits")
    # valid K+V rows read by the tokens, on average over the timed ones
    kv_bytes = 2 * cfg.n_layer * cfg.kv_dim * 2 * (pos - steps / 2)
    log(f"tg {tg_tok_s:.1f} tok/s ({ms_step:.3f} ms/token)")
    out = {
        "model": f"{cfg.name}, {'Q4_0' if cfg.qtype == 2 else 'Q8_0'}, batch 1",
        "pp512_tok_s": round(pp512_tok_s, 1),
        f"pp{prompt_len}_tok_s": round(ppN_tok_s, 1),
        "tg_tok_s": round(tg_tok_s, 2),
        "tg_steps": steps,
        "ms_per_token": round(ms_step, 5),
        "decode_context": [prompt_len + warmup + 1, pos],
        "decode_weight_GBps": round(w.decode_bytes / (ms_step * 1e-3) / 1e9, 1),
        "decode_weight_plus_kv_GBps": round((w.decode_bytes + kv_bytes) / (ms_step * 1e-3) / 1e9, 1),
        "wall_s_timed": round(wall, 3),
    }
    del pp_graphs, tg_graphs
    dec.graphs.clear()
    return out, dec


def step_gemv_launches(dec):
    """The fused GEMV launches of one decode step of `dec` (model.forward's fused path
    at s = 1, on the s = 1 bucket's buffers, KV cache and weights), without the other
    kernels of the step; returns (issue(), algorithmic bytes of each launch)."""
    from ggmlc_amd import ops

    w, c, b = dec.w, dec.cfg, dec._buffers(1)
    qd, kvd = c.q_dim, c.kv_dim
    f32 = 4

    def rope_kv(li):
        return ops.RopeKv(c.n_head, c.n_head_kv, c.head_dim, b["pos_ids"], c.head_dim, 2, c.rope_base,
                          b["kv_idx"], b["q"], dec.k_cache[li], dec.v_cache[li], cache=b["rope_cs"])

    def bias(t):
        return 0 if t is None else t.numel() * f32

    nbytes = []
    for li, L in enumerate(w.layers):
        x_io = c.n_embd * f32 * (3 if li else 1)  # x (+ the pending residual, + the new x)
        nbytes.append(L.qkv.nbytes + x_io + bias(L.qkv_b) + qd * f32 + 2 * kvd * 2)
        nbytes.append(L.o.nbytes + qd * f32 + c.n_embd * f32 + bias(L.o_b))
        nbytes.append(L.gate_up.nbytes + 3 * c.n_embd * f32 + c.n_ff * f32 + bias(L.gate_up_b))
        nbytes.append(L.down.nbytes + c.n_ff * f32 + c.n_embd * f32 + bias(L.down_b))
    nbytes.append(w.lm_head.nbytes + 2 * c.n_embd * f32 + c.n_vocab * f32)

    def issue():
        x = b["x"]
        other = {id(b["x"]): b["x_alt"], id(b["x_alt"]): b["x"]}
        pending = None
        for li, L in enumerate(w.layers):
            nx = other[id(x)] if pending is not None else None
            ops.mul_mat_fused(L.qkv, x, rms_eps=c.rms_eps, x_add=pending, x_sum=nx, rope_kv=rope_kv(li),
                              bias=L.qkv_b)
            x = nx if nx is not None else x
            o = ops.mul_mat_fused(L.o, b["attn"].view(1, qd), out=b["proj"], bias=L.o_b)
            nx = other[id(x)]
            a = ops.mul_mat_fused(L.gate_up, x, out=b["act"], rms_eps=c.rms_eps, swiglu=True, x_add=o, x_sum=nx,
                                  bias=L.gate_up_b)
            x = nx
            pending = ops.mul_mat_fused(L.down, a, out=b["proj"], bias=L.down_b)
        ops.mul_mat_fused(w.lm_head, x, out=b["logits"], rms_eps=c.rms_eps, x_add=pending)

    return issue, nbytes


def step_weight_buffers(w) -> list:
    """The weight buffers of one decode step, in launch order."""
    bufs = []
    for L in w.layers:
        bufs += [L.qkv.data, L.o.data, L.gate_up.data, L.down.data]
    bufs.append(w.lm_head.data)
    return bufs


def prefill_gemms(w, dev, ws):
    """The 128 GEMMs of one 512-token ubatch (fp32 N(0,1) activations); returns
    (issue(), flops)."""
    import torch

    from ggmlc_amd import ops

    cfg = w.cfg
    gen = torch.Generator(device=dev)
    gen.manual_seed(77)
    xs = {k: torch.randn((UBATCH, k), generator=gen, device=dev) for k in (cfg.n_embd, cfg.q_dim, cfg.n_ff)}
    gmats = []
    for L in w.layers:
        gmats += [(L.qkv, xs[cfg.n_embd]), (L.o, xs[cfg.q_dim]), (L.gate_up, xs[cfg.n_embd]), (L.down, xs[cfg.n_ff])]
    gout = {n: torch.empty((UBATCH, n), device=dev) for n in {m.N for m, _ in gmats}}
    ws.get(max(ops.mul_mat_workspace_size(m, UBATCH) for m, _ in gmats))

    def issue():
        for m, x in gmats:
            ops.mul_mat(m, x, out=gout[m.N], ws=ws)

    return issue, sum(2.0 * UBATCH * m.N * m.K for m, _ in gmats)


def bench_c1(dev, ws, launches: int) -> dict:
    """Linear 4096 -> 4096, Q8_0, M = 1 (17.8 MB per launch), 16 rotating
    weight copies (285 MB > the 256 MB Infinity Cache)."""
    import torch

    from ggmlc_amd import ops

    g = torch.Generator(device=dev)
    g.manual_seed(7)
    c1 = []
    for _ in range(16):
        t = torch.randn((4096, 4096), generator=g, device=dev) * 0.02
        c1.append(ops.quantize_weights(t, ops.Q8_0))
        del t
    x1 = torch.randn((1, 4096), generator=g, device=dev)
    out1 = torch.empty((1, 4096), device=dev)

    def loop():
        for i in range(launches):
            ops.mul_mat(c1[i % 16], x1, out=out1, ws=ws)

    ms = time_graph(loop, 3) / launches
    nbytes = c1[0].nbytes + 4096 * 4 + 4096 * 4
    gbs = nbytes / (ms * 1e-3) / 1e9
    probe_ms = time_probe_launches([c1[i % 16].data for i in range(launches)]) / launches
    log(f"configs[0] Q8_0 GEMV: {ms * 1e3:.2f} us, {gbs:.0f} GB/s")
    return {
        "kernel": "k_gemv_grp<Q8_0, M=1> (configs[0] Linear 4096->4096)",
        "achieved_GBps": round(gbs, 1),
        "frac_of_peak": round(gbs / HBM_PEAK_GBS, 4),
        "us_per_launch": round(ms * 1e3, 3),
        "bytes_per_launch": nbytes,
        "read_probe_same_size_us": round(probe_ms * 1e3, 3),
        "frac_of_same_size_read": round(probe_ms / ms, 4),
    }


def bench_c2(dev, ws, Ms=(1, 8, 128, 512), copies: int = 4, blocks: int = 16) -> dict:
    """the SwiGLU MLP block (gate/up 4096 -> 11008 as one fused 4096 ->
    22016 MUL_MAT, SWIGLU, down 11008 -> 4096), Q4_0, at M tokens; `copies` weight sets
    rotate so every block streams its weights from HBM. Up to 4 rows: gate_up GEMV with
    SWIGLU in its epilogue, then the down GEMV; more rows: the gate_up GEMM, then the
    down GEMM with SWIGLU in its activation prologue."""
    import torch

    from ggmlc_amd import ops

    H, F = 4096, 11008
    g = torch.Generator(device=dev)
    g.manual_seed(1101)
    sets = []
    for _ in range(copies):
        t = torch.randn((2 * F, H), generator=g, device=dev) * 0.02
        gu = ops.quantize_weights(t, ops.Q4_0)
        t = torch.randn((H, F), generator=g, device=dev) * 0.02
        dn = ops.quantize_weights(t, ops.Q4_0)
        del t
        sets.append((gu, dn))
    wbytes = sets[0][0].nbytes + sets[0][1].nbytes
    out = {"shape": "gate/up 4096->11008 (fused 4096->22016), SWIGLU, down 11008->4096, Q4_0",
           "weight_bytes": wbytes, "weight_copies": copies, "M": {}}
    for M in Ms:
        x = torch.randn((M, H), generator=g, device=dev)
        act = torch.empty((M, F), device=dev)
        gu_out = torch.empty((M, 2 * F), device=dev)
        y = torch.empty((M, H), device=dev)
        ws.get(max(ops.mul_mat_workspace_size(m, M) for s in sets for m in s))

        def block(gu, dn):
            if M <= 4:
                a = ops.mul_mat_fused(gu, x, out=act, swiglu=True)
                ops.mul_mat(dn, a, out=y, ws=ws)
            else:
                ops.mul_mat(gu, x, out=gu_out, ws=ws)
                ops.mul_mat_fused(dn, gu_out, out=y, x_swiglu=True, ws=ws)

        def loop():
            for i in range(blocks):
                block(*sets[i % copies])

        ms = time_graph(loop, 5 if M <= 128 else 3) / blocks
        flops = 2.0 * M * (2 * F * H + H * F)
        nbytes = wbytes + 4 * M * (H + F + H)
        path = "GEMV (v_dot4)" if M <= 4 else ("int8 MFMA GEMM" if M <= 16 else "fp16 MFMA GEMM (exact hi + lo products)")
        row = {"path": path, "us_per_block": round(ms * 1e3, 3),
               "tok_s": round(M * 1000.0 / ms, 1), "achieved_GBps": round(nbytes / (ms * 1e-3) / 1e9, 1),
               "frac_of_hbm_peak": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
               "achieved_TFLOPs": round(flops / (ms * 1e-3) / 1e12, 2),
               "frac_of_f16_mfma_peak": round(flops / (ms * 1e-3) / 1e12 / FP16_MFMA_PEAK_TFLOPS, 4)}
        out["M"][str(M)] = row
        log(f"  M={M}: {ms * 1e3:.1f} us/block, {row['achieved_GBps']} GB/s, {row['achieved_TFLOPs']} TFLOP/s")
        del x, act, gu_out, y
    del sets
    torch.cuda.empty_cache()
    return out


def measured_ceilings(dev) -> tuple[float, float]:
    """Streaming-read probe (the GEMV's 16-byte nontemporal load pattern) and device
    copy GB/s over 1 GiB: measured ceilings next to the datasheet peak."""
    import torch

    from ggmlc_amd import _lib

    big = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    Lib = _probe_lib()
    stream = torch.cuda.current_stream()

    def probe():
        _probe_check(Lib.gqbench_stream_read(big.data_ptr(), big.numel(), sink.data_ptr(), stream.cuda_stream))

    probe(), probe()
    torch.cuda.synchronize()
    e0, e1 = _ev(), _ev()
    e0.record()
    for _ in range(10):
        probe()
    e1.record()
    torch.cuda.synchronize()
    read_gbs = big.numel() * 10 / (e0.elapsed_time(e1) * 1e-3) / 1e9
    big2 = torch.empty_like(big)
    big2.copy_(big)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(10):
        big2.copy_(big)
    e1.record()
    torch.cuda.synchronize()
    copy_gbs = 2 * big.numel() * 10 / (e0.elapsed_time(e1) * 1e-3) / 1e9
    del big, big2
    torch.cuda.empty_cache()
    return read_gbs, copy_gbs


def bench_c5(dev, steps: int, batches=(1, 2, 4, 8, 16)) -> dict:
    """continuous-batching decode over the paged KV cache (see the module doc)."""
    import numpy as np
    import torch

    from ggmlc_amd.model import QWEN25_1_5B, random_weights
    from ggmlc_amd.paged import BatchDecoder

    cfg, Bmax, P, PREFIX = QWEN25_1_5B, 16, 128, 512
    w = random_weights(cfg, dev, seed=4242)
    rng = np.random.default_rng(4242)
    ctx = rng.integers(256, 4097, Bmax)
    # the even sequences share the prefix, so their contexts are drawn above it
    ctx[0::2] = np.where(ctx[0::2] > PREFIX, ctx[0::2], rng.integers(PREFIX + 1, 4097, Bmax // 2))
    prefix = rng.integers(0, cfg.n_vocab, PREFIX).astype(np.int32)
    prompts = []
    for b in range(Bmax):
        t = rng.integers(0, cfg.n_vocab, int(ctx[b])).astype(np.int32)
        if b % 2 == 0:  # 50% of the sequences open with the shared prefix
            t[:PREFIX] = prefix
        prompts.append(t)
    max_ctx = 4096 + 2 * steps + 8
    bd = BatchDecoder(w, max_batch=Bmax, max_ctx=max_ctx, page_size=P)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    first = np.zeros(Bmax, np.int32)
    for b in range(Bmax):
        bd.kv.alloc_slot(b)
        start = 0
        if b % 2 == 0 and b > 0:  # the prefix pages of sequence 0, shared
            bd.kv.map_existing_pages(b, 0, bd.kv.pages[0][:PREFIX // P])
            start = PREFIX
        bd.kv.ensure_tokens(b, len(prompts[b]) + 2 * steps + 4)
        first[b] = int(torch.argmax(bd.prefill(b, prompts[b], start)))
    torch.cuda.synchronize()
    prefill_s = time.perf_counter() - t0
    n_prefill = int(sum(len(t) for t in prompts)) - (Bmax // 2 - 1) * PREFIX
    kv_token = 2 * cfg.n_layer * cfg.n_head_kv * cfg.head_dim * 2  # bytes of K+V per cached token
    out = {"model": f"{cfg.name} Q8_0, tied embeddings", "weight_bytes": w.decode_bytes,
           "contexts": [int(c) for c in ctx], "shared_prefix": PREFIX, "page_tokens": P,
           "prefill_tokens_computed": n_prefill, "prefill_s": round(prefill_s, 3), "steps": steps, "B": {}}
    e0, e1 = _ev(), _ev()
    for B in batches:
        b = bd._buffers(B)

        def run(n):
            for _ in range(n):
                L = bd.ctx_bucket(int(bd.pos_host[:B].max()) + 1)
                bd.capture(B, L).replay()
                b["ids"].copy_(b["next"])
                bd.pos_host[:B] += 1

        for phase in ("warm", "timed"):  # the warm pass captures every graph the timed pass replays
            for i in range(B):
                bd.set_pos(i, len(prompts[i]))
            b["ids"].copy_(torch.from_numpy(first[:B]).to(dev))
            torch.cuda.synchronize()
            if phase == "timed":
                e0.record()
            run(steps)
            if phase == "timed":
                e1.record()
            torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / steps
        kv = sum(len(prompts[i]) + steps / 2 for i in range(B)) * kv_token
        out["B"][str(B)] = {"tok_s": round(B * 1000.0 / ms, 1), "ms_per_step": round(ms, 4),
                            "GBps_weights_plus_kv": round((w.decode_bytes + kv) / (ms * 1e-3) / 1e9, 1)}
        log(f"  B={B}: {B * 1000.0 / ms:.0f} tok/s, {ms:.3f} ms/step")
    del bd, w
    torch.cuda.empty_cache()
    return out


# (N, K) of the Q8_0 decode GEMV sweep: configs[0], the LLaMA-7B layer and lm_head
# shapes, the SmolLM2-360M K = 960 projections and tied head, and the Qwen2.5-1.5B tied
# lm_head (248 MB, the largest single weight here)
SWEEP_SHAPES = ((4096, 4096), (4096, 11008), (12288, 4096), (22016, 4096), (32000, 4096),
                (1600, 960), (5120, 960), (960, 2560), (49152, 960), (151936, 1536))


def gemv_sweep_q8_0(dev, ws, min_launches: int = 96, reps: int = 3) -> list:
    """Q8_0 GEMV (M = 1) over SWEEP_SHAPES: achieved GB/s (weight + x + y bytes per
    launch) as a fraction of the HBM peak and of a streaming read of the same buffers.
    Each shape rotates over enough weight copies (>= 512 MB together, each read once per
    replay) that no launch finds its weight in the 256 MB Infinity Cache; launches run
    back to back in one graph, as the decode GEMVs of a token do."""
    import torch

    from ggmlc_amd import ops

    g = torch.Generator(device=dev)
    g.manual_seed(11)
    rows = []
    for N, K in SWEEP_SHAPES:
        wbytes = N * (K // 32) * ops.BLOCK_BYTES[ops.Q8_0]
        ncopy = max(2, min(400, -(-(512 << 20) // wbytes)))
        launches = max(min_launches, ncopy)
        ws_ = []
        for _ in range(ncopy):
            t = torch.randn((N, K), generator=g, device=dev) * 0.02
            ws_.append(ops.quantize_weights(t, ops.Q8_0))
            del t
        x = torch.randn((1, K), generator=g, device=dev)
        y = torch.empty((1, N), device=dev)

        def loop():
            for i in range(launches):
                ops.mul_mat(ws_[i % ncopy], x, out=y, ws=ws)

        ms = time_graph(loop, reps) / launches
        nbytes = wbytes + 4 * K + 4 * N
        gbs = nbytes / (ms * 1e-3) / 1e9
        probe_ms = time_probe_launches([ws_[i % ncopy].data for i in range(launches)]) / launches
        rows.append({
            "N": N, "K": K, "bytes_per_launch": nbytes, "weight_copies": ncopy,
            "us_per_launch": round(ms * 1e3, 3), "achieved_GBps": round(gbs, 1),
            "frac_of_peak": round(gbs / HBM_PEAK_GBS, 4),
            "frac_of_same_size_read": round(probe_ms / ms, 4),
        })
        log(f"sweep q8_0 N={N} K={K}: {ms * 1e3:.2f} us, {gbs:.0f} GB/s ({gbs / HBM_PEAK_GBS:.1%} of peak)")
        del ws_
    return rows


_PROBE = None


def _probe_lib():
    """libgqbench.so: the streaming-read probe (a measurement aid outside libgq's ABI)."""
    global _PROBE
    if _PROBE is None:
        import ctypes

        path = ROOT / "ggmlc_amd" / "libgqbench.so"
        if not path.exists():
            raise RuntimeError(f"{path} is not built; run `python -m ggmlc_amd.build`")
        lib = ctypes.CDLL(str(path))
        lib.gqbench_stream_read.restype = ctypes.c_int
        lib.gqbench_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_void_p]
        _PROBE = lib
    return _PROBE


def _probe_check(rc: int) -> None:
    if rc != 0:
        raise RuntimeError(f"streaming-read probe: HIP error {rc}")


def time_probe_launches(bufs, reps: int = 5) -> float:
    """ms for one pass of streaming-read probes, one launch per buffer (each read once,
    whole), captured in a graph and timed like the GEMV graphs."""
    import torch

    Lib = _probe_lib()
    sink = torch.zeros(4, dtype=torch.int32, device=bufs[0].device)

    def run():
        st = torch.cuda.current_stream().cuda_stream  # the capture stream inside the graph
        for b in bufs:
            _probe_check(Lib.gqbench_stream_read(b.data_ptr(), b.numel() // 16 * 16, sink.data_ptr(), st))

    return time_graph(run, reps)


def traffic_probe(w, dev) -> int:
    """Eager launches for the PMC runs (per-dispatch counters do not survive graph
    replay under the profiler): 3 x one decode step's fused GEMVs, then 3 x a 256 MiB
    device copy whose FETCH_SIZE / WRITE_SIZE calibrate the counters (256 MiB each way)."""
    import torch

    from ggmlc_amd.model import Decoder

    dec = Decoder(w, 256, dev)
    b = dec._buffers(1)
    b["x"].normal_(), b["x_alt"].normal_(), b["attn"].normal_()
    b["pos_ids"].fill_(100), b["kv_idx"].fill_(100)
    issue, nbytes = step_gemv_launches(dec)
    for _ in range(3):
        issue()
    a = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
    c = torch.empty_like(a)
    for _ in range(3):
        c.copy_(a)
    torch.cuda.synchronize()
    log(f"traffic probe: {3 * len(nbytes)} fused GEMV launches ({sum(nbytes) / len(nbytes):.0f} algorithmic "
        f"bytes per launch), 3 copies of {a.numel()} bytes")
    return 0


ATTN_EVENTS = ("start", "loads issued", "first K row in registers", "rows accumulated", "partial stored",
               "arrival counted", "merge written", "end")


def attn_probe(dev, stamps: bool) -> int:
    """The decode attention of the configs[3] step at its tg context: 32 heads of 128,
    the query at position 1099, the 1280-row KV bucket (mask 0 up to the position, -32768
    after it, as the step builds it), over 16 K/V copies (336 MB, more than the 256 MB
    Infinity Cache, so each launch reads its rows from HBM as in the step). Without
    stamps: the product launches eagerly (3 rounds of 16) and 3 x 256 MiB device copies
    that calibrate FETCH_SIZE / WRITE_SIZE. With stamps: 2 rounds through libgqbench's
    timestamped build (same source and launch plan), the second round's per-wave event
    times summarised (µs from the launch's first wave start; s_memrealtime at 100 MHz)."""
    import ctypes

    import numpy as np
    import torch

    from ggmlc_amd import ops

    Hq = Hkv = 32
    D, pos, n_kv, copies = 128, 1099, 1280, 16
    gen = torch.Generator(device=dev).manual_seed(7)
    ks = [torch.randn((Hkv, n_kv, D), device=dev, generator=gen).half() for _ in range(copies)]
    vs = [torch.randn((Hkv, n_kv, D), device=dev, generator=gen).half() for _ in range(copies)]
    q = torch.randn((Hq, 1, D), device=dev, generator=gen)
    mask = torch.zeros((1, n_kv), dtype=torch.float16, device=dev)
    mask[0, pos + 1:] = -32768.0
    out = torch.empty((1, Hq, D), device=dev)
    ws = ops.Workspace(dev)
    scale = 1.0 / float(np.sqrt(D))
    if not stamps:
        for _ in range(3):
            for i in range(copies):
                ops.flash_attn_ext(q, ks[i], vs[i], mask, scale, out=out, ws=ws)
        a = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
        c = torch.empty_like(a)
        for _ in range(3):
            c.copy_(a)
        torch.cuda.synchronize()
        log(f"attention probe: {3 * copies} decode attention launches (Hq {Hq}, D {D}, n_kv {n_kv}, valid rows "
            f"{pos + 1}, {2 * Hkv * n_kv * D * 2} K/V bytes each), 3 copies of {a.numel()} bytes")
        return 0

    lib = _probe_lib()
    vp, i64 = ctypes.c_void_p, ctypes.c_int64
    lib.gqbench_attn_stamped.restype = ctypes.c_int
    lib.gqbench_attn_stamped.argtypes = [vp, i64, i64, i64, i64, vp, vp, i64, i64, vp, ctypes.c_float, vp, vp,
                                         ctypes.c_size_t, vp]
    lib.gqbench_attn_stamp_slots.restype = ctypes.c_int
    lib.gqbench_attn_stamps_take.restype = ctypes.c_int
    lib.gqbench_attn_stamps_take.argtypes = [vp]
    lib.gqbench_attn_last_error.restype = ctypes.c_char_p
    host = np.zeros(lib.gqbench_attn_stamp_slots(), dtype=np.uint64)
    wbytes = 16 << 20
    wsp = ws.get(wbytes)[0]

    def take():
        if lib.gqbench_attn_stamps_take(host.ctypes.data) != 0:
            raise RuntimeError(lib.gqbench_attn_last_error().decode())
        return host.copy()

    take()
    runs = []
    for r in range(2):
        for i in range(copies):
            rc = lib.gqbench_attn_stamped(q.data_ptr(), D, 1, Hq, Hkv, ks[i].data_ptr(), vs[i].data_ptr(), n_kv,
                                          n_kv * D * 2, mask.data_ptr(), scale, out.data_ptr(), wsp, wbytes,
                                          torch.cuda.current_stream().cuda_stream)
            if rc != 0:
                raise RuntimeError(lib.gqbench_attn_last_error().decode())
            torch.cuda.synchronize()
            st = take()
            if r == 1:
                runs.append(st.reshape(-1, 8))
    stamped = out.clone()
    ref = ops.flash_attn_ext(q, ks[-1], vs[-1], mask, scale)  # libgq on the last launch's copy
    torch.cuda.synchronize()
    summary = {"waves": None, "events_us": {}}
    per_event = {e: [] for e in range(8)}
    spans, waves = [], []
    for st in runs:
        live = st[st[:, 0] != 0].astype(np.int64)
        waves.append(len(live))
        t0 = live[:, 0].min()
        spans.append((live[:, 7].max() - t0) / 100.0)
        for e in range(8):
            v = live[:, e]
            per_event[e].extend(((v[v != 0] - t0) / 100.0).tolist())
    summary["waves"] = int(np.median(waves))
    summary["launch_span_us_median"] = round(float(np.median(spans)), 2)
    for e, name in enumerate(ATTN_EVENTS):
        v = np.asarray(per_event[e])
        if v.size:
            summary["events_us"][name] = {"waves": int(v.size // len(runs)),
                                          **{f"p{p}": round(float(np.percentile(v, p)), 2) for p in (0, 10, 50, 90, 100)}}
    summary["bits_equal_to_libgq"] = bool(torch.equal(stamped, ref))
    print(json.dumps({"attn_stamps": summary}), flush=True)
    return 0


I8_EVENTS = ["wave start", "activation and weight loads issued", "activation in LDS",
             "first weight step arrived", "steps accumulated", "K parts added", "quantized rows' barrier passed",
             "end"]


def i8_probe(dev) -> dict:
    """The configs[4] gate|up product on the int8 path (16 rows, K = 1536, Q8_0, SWIGLU and
    the down projection's quantized rows; one workgroup of 8 waves per 64 weight rows):
    * launch time against N (graphs of 64 launches over weight copies totalling >= 600 MB),
      at and around 256 workgroups (one per CU) and the configs' 17920 rows (280);
    * per-wave event times (µs from the launch's first wave start; s_memrealtime at 100 MHz)
      of 16 cold launches through libgqbench's timestamped build (same source and launch
      plan), second of two rounds, at N = 17920 and 16384, with a bit check against libgq;
    * a streaming read of 14 MiB (the configs[4] down weights) against its workgroup count,
      256 threads each, over 32 buffers."""
    import ctypes

    import numpy as np
    import torch

    from ggmlc_amd import ops

    K, M = 1536, 16
    gen = torch.Generator(device=dev).manual_seed(5)
    x = torch.randn((M, K), generator=gen, device=dev)
    out = {"shape": "gate|up N x 1536 (Q8_0), 16 rows, SWIGLU + quantized rows", "launch_us": {}, "timeline": {},
           "read_14MiB": {}}
    for N in (8192, 12288, 16384, 16448, 17920, 20480, 32768, 49152):
        copies = max(2, int(600e6 // (N * K * 34 // 32)))
        wts = [ops.quantize_weights(torch.randn((N, K), generator=gen, device=dev) * 0.02, ops.Q8_0)
               for _ in range(copies)]
        q8 = torch.empty((ops.q8_rows_bytes(N // 2),), dtype=torch.uint8, device=dev)
        y = torch.empty((M, N // 2), device=dev)

        def loop():
            for i in range(64):
                ops.mul_mat_fused(wts[i % copies], x, out=y, swiglu=True, out_q8=q8)

        us = time_graph(loop, 5) / 64 * 1e3
        mb = N * K * 34 / 32 / 1e6
        out["launch_us"][str(N)] = {"workgroups": N // 64, "us": round(us, 2), "MB": round(mb, 1),
                                    "TBps": round(mb / us, 2)}
        log(f"  gate|up N={N}: {N // 64} workgroups, {us:.2f} us, {mb / us:.2f} TB/s")
        del wts
        torch.cuda.empty_cache()

    lib = _probe_lib()
    vp, i64 = ctypes.c_void_p, ctypes.c_int64
    lib.gqbench_gemm_i8_glu_stamped.restype = ctypes.c_int
    lib.gqbench_gemm_i8_glu_stamped.argtypes = [ctypes.c_int, vp, i64, i64, vp, i64, vp, i64, vp, vp]
    lib.gqbench_gemm_stamp_slots.restype = ctypes.c_int
    lib.gqbench_gemm_stamps_take.restype = ctypes.c_int
    lib.gqbench_gemm_stamps_take.argtypes = [vp]
    lib.gqbench_gemm_last_error.restype = ctypes.c_char_p
    lib.gqbench_stream_read_grid.restype = ctypes.c_int
    lib.gqbench_stream_read_grid.argtypes = [vp, ctypes.c_size_t, ctypes.c_int, vp, vp]
    host = np.zeros(lib.gqbench_gemm_stamp_slots(), dtype=np.uint64)
    stream = torch.cuda.current_stream().cuda_stream

    def take():
        if lib.gqbench_gemm_stamps_take(host.ctypes.data) != 0:
            raise RuntimeError(lib.gqbench_gemm_last_error().decode())
        return host.copy()

    # the activation in act_prep_i8's layout for K = 1536: the quantized SWIGLU rows of a
    # 3072-row product
    w0 = ops.quantize_weights(torch.randn((2 * K, 256), generator=gen, device=dev) * 0.05, ops.Q8_0)
    act = torch.empty((ops.q8_rows_bytes(K),), dtype=torch.uint8, device=dev)
    ops.mul_mat_fused(w0, torch.randn((M, 256), generator=gen, device=dev), swiglu=True, out_q8=act, no_out=True)
    copies = 16
    for N in (17920, 16384):
        wts = [ops.quantize_weights(torch.randn((N, K), generator=gen, device=dev) * 0.02, ops.Q8_0)
               for _ in range(copies)]
        q8 = torch.empty((ops.q8_rows_bytes(N // 2),), dtype=torch.uint8, device=dev)
        y = torch.empty((M, N // 2), device=dev)
        take()
        runs = []
        for r in range(2):
            for i in range(copies):
                rc = lib.gqbench_gemm_i8_glu_stamped(ops.Q8_0, wts[i].data.data_ptr(), N, K, act.data_ptr(), M,
                                                     y.data_ptr(), N // 2, q8.data_ptr(), stream)
                if rc != 0:
                    raise RuntimeError(lib.gqbench_gemm_last_error().decode())
                torch.cuda.synchronize()
                st = take()
                if r == 1:
                    runs.append(st.reshape(-1, 8))
        q8r = torch.empty_like(q8)
        yr = ops.mul_mat_fused(wts[-1], torch.zeros((M, K), device=dev), swiglu=True, out_q8=q8r, x_q8=act)
        torch.cuda.synchronize()
        per = {e: [] for e in range(8)}
        spans, nw = [], []
        for st in runs:
            live = st[st[:, 0] != 0].astype(np.int64)
            nw.append(len(live))
            t0 = live[:, 0].min()
            spans.append((live[:, 7].max() - t0) / 100.0)
            for e in range(8):
                v = live[:, e]
                per[e].extend(((v[v != 0] - t0) / 100.0).tolist())
        tl = {"workgroups": N // 64, "waves": int(np.median(nw)), "launch_span_us_median": round(float(np.median(spans)), 2),
              "bits_equal_to_libgq": bool(torch.equal(y, yr) and torch.equal(q8, q8r)), "events_us": {}}
        for e, name in enumerate(I8_EVENTS):
            v = np.asarray(per[e])
            if v.size:
                tl["events_us"][name] = {f"p{p}": round(float(np.percentile(v, p)), 2) for p in (0, 10, 50, 90, 100)}
        out["timeline"][str(N)] = tl
        log(f"  gate|up N={N} timeline: span {tl['launch_span_us_median']} us, bits {tl['bits_equal_to_libgq']}")
        del wts
        torch.cuda.empty_cache()

    nbytes, nbuf = 14 << 20, 32
    bufs = [torch.ones(nbytes, dtype=torch.uint8, device=dev) for _ in range(nbuf)]
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    for grid in (96, 128, 192, 256, 384, 512, 1024, 2048):
        best = float("inf")
        for _ in range(5):
            e0, e1 = _ev(), _ev()
            e0.record()
            for b in bufs:
                rc = lib.gqbench_stream_read_grid(b.data_ptr(), nbytes, grid, sink.data_ptr(), stream)
                if rc != 0:
                    raise RuntimeError(f"stream read probe: HIP error {rc}")
            e1.record()
            torch.cuda.synchronize()
            best = min(best, e0.elapsed_time(e1) * 1e3 / nbuf)
        out["read_14MiB"][str(grid)] = {"us": round(best, 2), "TBps": round(nbytes / best / 1e6, 2),
                                        "GBps_per_workgroup": round(nbytes / best / 1e3 / grid, 1)}
        log(f"  read 14 MiB with {grid} workgroups: {best:.2f} us")
    del bufs
    torch.cuda.empty_cache()
    return out


def gemm_probe(w, dev) -> int:
    """Eager launches for the MFMA counter runs: 3 x one ubatch's 128 prefill GEMMs."""
    import torch

    from ggmlc_amd import ops

    ws = ops.Workspace(dev)
    issue, flops = prefill_gemms(w, dev, ws)
    for _ in range(3):
        issue()
    torch.cuda.synchronize()
    log(f"gemm probe: 3 x 128 GEMMs, {flops / 1e12:.3f} TFLOP per ubatch")
    return 0


def load_traffic(kernel: str) -> float | None:
    """HBM bytes per launch of `kernel` measured by the PMC runs and summarised in
    profiles/gemv_traffic.json (null when absent)."""
    f = ROOT / "profiles" / "gemv_traffic.json"
    if not f.exists():
        return None
    d = json.loads(f.read_text()).get(kernel)
    return None if d is None else float(d["hbm_bytes_per_launch"])


def cpu_identity() -> dict:
    """Host CPU model (lscpu's "Model name", else /proc/cpuinfo's), its family / model /
    stepping, sockets and cores, and the ISA extensions ggml's x86 kernels use."""
    import subprocess

    model, flags, extra = "unknown", set(), {}
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name") and model == "unknown":
                model = line.split(":", 1)[1].strip()
            elif line.startswith("flags") and not flags:
                flags = set(line.split(":", 1)[1].split())
    except OSError:
        pass
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            k, _, v = line.partition(":")
            k, v = k.strip(), v.strip()
            if k == "Model name" and v:
                model = v
            elif k in ("CPU family", "Model", "Stepping", "Socket(s)", "Core(s) per socket", "Thread(s) per core",
                       "Vendor ID", "BIOS Model name"):
                extra[k] = v
    except (OSError, subprocess.SubprocessError):
        pass
    isa = [f for f in ("avx2", "fma", "f16c", "avx512f", "avx512bw", "avx512vl", "avx512_vnni", "avx512_bf16",
                       "avx_vnni", "amx_int8", "amx_bf16") if f in flags]
    return {"cpu_model": model, "cpu_lscpu": extra, "isa": isa}


def cpu_baseline(w, cfg, seconds: float, ctx: int = 1024) -> dict:
    """The reference ggml CPU backend running the same decoder on the same weights:
    pp512 (one ubatch from position 0), then greedy decode tokens at the GPU's decode
    context for ~`seconds` on CPU_SHARE threads, then a few at 1 thread. The cache rows
    between 512 and `ctx` are not computed on the CPU (it would cost minutes): they hold
    zeros, and a decode token at position ctx reads them all the same (the work of
    attention depends on n_kv, not on the values)."""
    import numpy as np

    import oracle as O
    from ggmlc_amd.model import host_weights, pad_kv_len

    cores = min(CPU_SHARE, O.n_cpu_threads())
    ident = cpu_identity()
    host = host_weights(w)
    prompt = np.random.default_rng(5).integers(0, cfg.n_vocab, UBATCH).astype(np.int32)
    if O.ref_available():
        variant = "v4" if O.ref_v4_usable() else "v3"
        max_ctx = pad_kv_len(ctx + 64, 1 << 30)
        rl = O.RefLlama(cfg, host, max_ctx, n_threads=cores, variant=variant)
        t0 = time.perf_counter()
        _, tok = rl.step(prompt)
        pp_s = time.perf_counter() - t0
        rl.pos = ctx
        rl.step([tok])  # first decode token untimed
        n, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < seconds and rl.pos < ctx + 48:
            _, tok = rl.step([tok])
            n += 1
        dt = (time.perf_counter() - t0) / n
        rl.n_threads = 1
        n1, t0 = 0, time.perf_counter()
        while (n1 < 2 or time.perf_counter() - t0 < seconds / 3) and rl.pos < ctx + 60:
            _, tok = rl.step([tok])
            n1 += 1
        dt1 = (time.perf_counter() - t0) / n1
        del rl
        isa = "x86-64-v4 + AVX-512 VNNI" if variant == "v4" else "x86-64-v3 (AVX2 + FMA + F16C)"
        return {"value": round(1.0 / dt, 3), "unit": "tokens/s", "cores": cores, "kind": "reference",
                "sample": f"ggml CPU backend built from the reference sources for {isa} ({cores} threads) on the "
                          f"same {cfg.name} Q4_0 weights: one 512-token prefill ubatch, then {n} timed greedy "
                          f"decode tokens at context {ctx + 1}..{ctx + 1 + n}; then {n1} tokens at 1 thread",
                "ms_per_step": round(dt * 1e3, 2), "pp512_tok_s": round(UBATCH / pp_s, 2),
                "one_thread_tok_s": round(1.0 / dt1, 4), "one_thread_ms_per_step": round(dt1 * 1e3, 1),
                "build": f"oracle/_ref{'/v4' if variant == 'v4' else ''}/libggmlref.so ({isa})", **ident}
    # no reference build: the C restatement's MUL_MATs of one decode token (the bulk of its work)
    x = np.random.default_rng(6).standard_normal((1, cfg.n_ff)).astype(np.float32)
    mats = [(m, cfg.n_embd if i != 3 else cfg.n_ff) for L in host[2] for i, m in enumerate(L[:4])]
    mats.append((host[1], cfg.n_embd))
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds and n < 20:
        for m, K in mats:
            O.mul_mat(m, cfg.qtype, K, x[:, :K], n_threads=cores)
        n += 1
    dt = (time.perf_counter() - t0) / n
    return {"value": round(1.0 / dt, 3), "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": f"{n} decode tokens' MUL_MATs (the {len(mats)} GEMVs) through the C restatement",
            "ms_per_step": round(dt * 1e3, 2), **ident}


if __name__ == "__main__":
    sys.exit(main())
