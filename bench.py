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
* roofline  = the decode GEMV (k_gemv_grp<Q4_0, M=1>), the dominant kernel: the
              129 GEMV launches of one decode token (qkv, o, gate_up, down per layer,
              lm_head) captured in one graph with the model's own weights and timed
              with HIP events on the launch stream; achieved = their algorithmic bytes
              (weights + fp32 x + fp32 y) / their time. rocprofv3's average for
              k_gemv_grp<Q4_0> over this command covers the same launch mix.
* roofline_prefill_gemm = the 128 prefill GEMMs (M = 512) of one ubatch, same way.
* gemv_c1_q8_0 = configs[0], the Q8_0 Linear 4096 -> 4096 GEMV (16 rotating copies).
* c5_batched_decode = configs[4]: a Qwen2.5-1.5B-shape decoder (Q8_0, tied embeddings)
              over the paged KV pool; 16 sequences with contexts uniform in [256, 4096],
              half of them sharing a 512-token prefix (its pages computed once), then 64
              batched decode steps at B = 1, 2, 4, 8, 16, every sequence at its own
              position; tokens/s = B * steps / time (graph replays chained on the device).
* cpu_baseline = the reference's own ggml CPU backend (oracle/_ref, built from the
              reference sources) running the same decoder graph on the same weights
              with the host's cores: pp512 then decode tokens for a bounded sample.

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
    p.add_argument("--c5-steps", type=int, default=64, help="timed batched decode steps per batch size")
    p.add_argument("--no-c5", action="store_true", help="skip the configs[4] continuous-batching decode")
    p.add_argument("--c5-only", action="store_true", help="run only the configs[4] measurement (profiling)")
    p.add_argument("--c5-batches", default="1,2,4,8,16", help="configs[4] batch sizes")
    p.add_argument("--traffic-probe", action="store_true",
                   help="only launch one token's decode GEMVs and a 256 MiB device copy, eagerly, 3 times each "
                        "(the workload of the rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs behind roofline.traffic)")
    return p.parse_args()


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def main() -> int:
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (every GPU box here has one; "
              "run with --gpus 1)", file=sys.stderr)
        return 2
    if args.prompt % UBATCH or args.prompt <= 0:
        print("bench.py: --prompt must be a positive multiple of 512", file=sys.stderr)
        return 2

    import numpy as np
    import torch

    from ggmlc_amd import _lib, ops
    from ggmlc_amd.model import LLAMA_7B, Decoder, pad_kv_len, random_weights

    torch.cuda.set_device(0)
    _lib.check(_lib.load().gq_init())
    dev = torch.device("cuda", 0)
    batches = tuple(int(b) for b in args.c5_batches.split(","))
    if args.c5_only:
        print(json.dumps({"c5_batched_decode": bench_c5(dev, args.c5_steps, batches)}), flush=True)
        return 0
    cfg = LLAMA_7B
    stream = torch.cuda.current_stream()

    log(f"building {cfg.name} Q4_0 weights on device")
    w = random_weights(cfg, dev, seed=1234)
    torch.cuda.synchronize()
    if args.traffic_probe:
        return traffic_probe(w, cfg, dev)
    n_ctx = args.prompt + args.warmup + args.steps
    max_ctx = pad_kv_len(n_ctx, 1 << 30)
    dec = Decoder(w, max_ctx, dev)
    log(f"weights {w.nbytes / 1e9:.3f} GB, KV cache {2 * cfg.n_layer * cfg.kv_dim * max_ctx * 2 / 1e9:.3f} GB "
        f"(max_ctx {max_ctx})")

    ev = lambda: torch.cuda.Event(enable_timing=True)  # noqa: E731

    # ---- prefill graphs: one per ubatch bucket, reading its slice of the prompt
    gen = torch.Generator(device=dev)
    gen.manual_seed(99)
    prompt = torch.randint(0, cfg.n_vocab, (args.prompt,), generator=gen, device=dev, dtype=torch.int32)
    n_ub = args.prompt // UBATCH
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
    for i in range(args.warmup + args.steps):
        n_kv = pad_kv_len(args.prompt + i + 1, max_ctx)
        if n_kv not in tg_graphs:
            dec.reset(args.prompt + i)
            tg_graphs[n_kv] = dec.capture(1, n_kv, ids=next1)
    torch.cuda.synchronize()

    def prefill():
        dec.reset(0)
        for g in pp_graphs:
            g.replay()

    # ---- pp: time each ubatch (pp512 = the first, ppN = all)
    log(f"prefill: {n_ub} ubatch(es) of {UBATCH}, {args.pp_reps} reps")
    prefill()
    torch.cuda.synchronize()
    t_first, t_all = [], []
    for _ in range(args.pp_reps):
        dec.reset(0)
        es = [ev() for _ in range(n_ub + 1)]
        es[0].record()
        for u, g in enumerate(pp_graphs):
            g.replay()
            es[u + 1].record()
        torch.cuda.synchronize()
        t_first.append(es[0].elapsed_time(es[1]))
        t_all.append(es[0].elapsed_time(es[-1]))
    pp512_tok_s = UBATCH * 1000.0 / float(np.median(t_first))
    ppN_tok_s = args.prompt * 1000.0 / float(np.median(t_all))
    log(f"pp512 {pp512_tok_s:.0f} tok/s, pp{args.prompt} {ppN_tok_s:.0f} tok/s")

    # ---- tg: the prompt's KV is in the cache (last prefill rep); decode from its token
    prefill()
    next1.copy_(b_pp["next"])
    torch.cuda.synchronize()
    if int(dec.pos[0]) != args.prompt:
        raise RuntimeError("device position after prefill is wrong")
    tokens = []
    pos = args.prompt
    for i in range(args.warmup):
        tg_graphs[pad_kv_len(pos + 1, max_ctx)].replay()
        pos += 1
    torch.cuda.synchronize()
    log(f"decode: {args.warmup} warmup + {args.steps} timed tokens (graph replay)")
    e0, e1 = ev(), ev()
    t0 = time.perf_counter()
    e0.record()
    for i in range(args.steps):
        tg_graphs[pad_kv_len(pos + 1, max_ctx)].replay()
        pos += 1
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = e0.elapsed_time(e1) / args.steps
    tg_tok_s = 1000.0 / ms_step
    logits = dec._buffers(1)["logits"]
    if int(dec.pos[0]) != pos or not bool(torch.isfinite(logits).all()):
        raise RuntimeError("decode produced a wrong position or non-finite logits")
    tokens.append(int(next1[0]))
    kv_bytes_last = 2 * cfg.n_layer * cfg.kv_dim * 2 * pos  # valid K+V rows read by the last token
    log(f"tg {tg_tok_s:.1f} tok/s ({ms_step:.3f} ms/token)")

    # ---- roofline: the 129 decode GEMVs of one token, one graph, HIP events
    mats, outs = decode_gemvs(w, cfg, dev, gen)
    ws = ops.Workspace(dev)
    ws.get(1 << 20)

    def gemv_token():
        for (m, x), o in zip(mats, outs):
            ops.mul_mat(m, x, out=o, ws=ws)

    gemv_token()
    torch.cuda.synchronize()
    gg = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gg):
        gemv_token()
    for _ in range(3):
        gg.replay()
    torch.cuda.synchronize()
    R = 20
    e0.record()
    for _ in range(R):
        gg.replay()
    e1.record()
    torch.cuda.synchronize()
    gemv_ms_token = e0.elapsed_time(e1) / R
    gemv_bytes_token = sum(m.nbytes + m.K * 4 + m.N * 4 for m, _ in mats)
    n_gemv = len(mats)
    gemv_gbs = gemv_bytes_token / (gemv_ms_token * 1e-3) / 1e9
    del gg
    # the same launches as plain streaming reads of the same weight buffers: the
    # ceiling a kernel that only reads its weights reaches at these per-launch sizes
    probe_ms_token = time_probe_launches([m.data for m, _ in mats], e0, e1)

    # ---- prefill GEMM rate: the 128 GEMMs of one ubatch (M = 512)
    xs = {k: torch.randn((UBATCH, k), generator=gen, device=dev) for k in (cfg.n_embd, cfg.q_dim, cfg.n_ff)}
    gmats = []
    for L in w.layers:
        gmats += [(L.qkv, xs[cfg.n_embd]), (L.o, xs[cfg.q_dim]), (L.gate_up, xs[cfg.n_embd]), (L.down, xs[cfg.n_ff])]
    gout = {n: torch.empty((UBATCH, n), device=dev) for n in {m.N for m, _ in gmats}}
    ws.get(max(ops.mul_mat_workspace_size(m, UBATCH) for m, _ in gmats))

    def gemm_ubatch():
        for m, x in gmats:
            ops.mul_mat(m, x, out=gout[m.N], ws=ws)

    gemm_ubatch()
    torch.cuda.synchronize()
    gm = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gm):
        gemm_ubatch()
    gm.replay()
    torch.cuda.synchronize()
    e0.record()
    for _ in range(3):
        gm.replay()
    e1.record()
    torch.cuda.synchronize()
    gemm_ms = e0.elapsed_time(e1) / 3
    gemm_flops = sum(2.0 * UBATCH * m.N * m.K for m, _ in gmats)
    gemm_tflops = gemm_flops / (gemm_ms * 1e-3) / 1e12
    del gm, gout, xs

    # ---- Linear 4096 -> 4096, Q8_0, M = 1 (17.8 MB per launch)
    gc1 = torch.Generator(device=dev)
    gc1.manual_seed(7)
    c1 = []
    for _ in range(16):  # 16 x 17.8 MB = 285 MB > Infinity Cache
        t = torch.randn((4096, 4096), generator=gc1, device=dev) * 0.02
        c1.append(ops.quantize_weights(t, ops.Q8_0))
        del t
    x1 = torch.randn((1, 4096), generator=gc1, device=dev)
    out1 = torch.empty((1, 4096), device=dev)
    Lc = args.c1_launches

    def c1_loop():
        for i in range(Lc):
            ops.mul_mat(c1[i % 16], x1, out=out1, ws=ws)

    c1_loop()
    torch.cuda.synchronize()
    gq = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gq):
        c1_loop()
    gq.replay()
    torch.cuda.synchronize()
    e0.record()
    for _ in range(3):
        gq.replay()
    e1.record()
    torch.cuda.synchronize()
    c1_ms = e0.elapsed_time(e1) / (3 * Lc)
    c1_bytes = c1[0].nbytes + 4096 * 4 + 4096 * 4
    c1_gbs = c1_bytes / (c1_ms * 1e-3) / 1e9
    c1_probe_ms = time_probe_launches([c1[i % 16].data for i in range(Lc)], e0, e1) / Lc
    del gq, c1
    sweep = [] if args.no_sweep else gemv_sweep_q8_0(dev, ws, e0, e1)

    # ---- measured ceilings next to the datasheet peak: the streaming-read probe
    # (the GEMV's 16-byte nontemporal load pattern) and a device copy
    big = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    Lib = _lib.load()

    def probe():
        _lib.check(Lib.gq_probe_stream_read(big.data_ptr(), big.numel(), sink.data_ptr(), stream.cuda_stream))

    probe(), probe()
    torch.cuda.synchronize()
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

    decode_bytes = w.decode_bytes
    result = {
        "metric": METRIC,
        "value": round(tg_tok_s, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_0 weights x q8_0 activations, int8 dot, f32 accum (prefill: f16 MFMA); f16 KV",
        "data": "synthetic (random-init weights N(0,0.02) -> Q4_0; uniform-random prompt ids)",
        "config": {
            "workload": f"configs[3] {cfg.name} decoder, Q4_0, batch 1: pp{args.prompt} (ubatch 512) then "
                        f"greedy decode; value = tg{args.steps} tokens/s",
            "global_batch": 1,
            "seq_len": args.prompt,
            "parallelism": "single GPU",
            "weight_bytes": w.nbytes,
        },
        "tg_tok_s": round(tg_tok_s, 2),
        "pp512_tok_s": round(pp512_tok_s, 1),
        f"pp{args.prompt}_tok_s": round(ppN_tok_s, 1),
        "decode_weight_GBps": round(decode_bytes / (ms_step * 1e-3) / 1e9, 1),
        "decode_weight_plus_kv_GBps": round((decode_bytes + kv_bytes_last) / (ms_step * 1e-3) / 1e9, 1),
        "roofline": {
            "kernel": "k_gemv_grp<Q4_0, M=1>: the 129 decode GEMVs of one token (qkv, o, gate_up, down x 32, lm_head)",
            "bound": "hbm",
            "achieved": round(gemv_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(gemv_gbs / HBM_PEAK_GBS, 4),
            "traffic": load_traffic("k_gemv_grp<Q4_0, M=1> decode mix"),
            "bytes_per_launch": round(gemv_bytes_token / n_gemv),
            "us_per_launch": round(gemv_ms_token * 1e3 / n_gemv, 3),
            "launches_per_token": n_gemv,
            "gemv_ms_per_token": round(gemv_ms_token, 4),
            "read_probe_same_launches_ms": round(probe_ms_token, 4),
            "frac_of_same_size_read": round(probe_ms_token / gemv_ms_token, 4),
        },
        "roofline_prefill_gemm": {
            "kernel": "k_gemm<Q4_0>: the 128 GEMMs of one 512-token ubatch (activation quantize excluded)",
            "bound": "mfma",
            "achieved": round(gemm_tflops, 1),
            "peak": FP16_MFMA_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(gemm_tflops / FP16_MFMA_PEAK_TFLOPS, 4),
            "ms_per_ubatch": round(gemm_ms, 3),
        },
        "gemv_c1_q8_0": {
            "kernel": "k_gemv_grp<Q8_0, M=1> (configs[0] Linear 4096->4096)",
            "achieved_GBps": round(c1_gbs, 1),
            "frac_of_peak": round(c1_gbs / HBM_PEAK_GBS, 4),
            "us_per_launch": round(c1_ms * 1e3, 3),
            "bytes_per_launch": c1_bytes,
            "read_probe_same_size_us": round(c1_probe_ms * 1e3, 3),
            "frac_of_same_size_read": round(c1_probe_ms / c1_ms, 4),
        },
        "gemv_sweep_q8_0": sweep,
        "measured_read_GBps": round(read_gbs, 1),
        "measured_copy_GBps": round(copy_gbs, 1),
        "wall_s_timed": round(wall, 3),
    }
    log(f"gemv {gemv_gbs:.0f} GB/s, gemm {gemm_tflops:.0f} TFLOP/s, c1 {c1_gbs:.0f} GB/s, read {read_gbs:.0f} GB/s")

    if not args.no_c5:
        del dec, pp_graphs, tg_graphs
        torch.cuda.empty_cache()
        log("configs[4]: batched paged decode")
        result["c5_batched_decode"] = bench_c5(dev, args.c5_steps, batches)
    if not args.no_cpu:
        log("cpu baseline")
        result["cpu_baseline"] = cpu_baseline(w, cfg, args.cpu_seconds)
    print(json.dumps(result), flush=True)
    return 0


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
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
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
# shapes, and the Qwen2.5-1.5B tied lm_head (248 MB, the largest single weight here)
SWEEP_SHAPES = ((4096, 4096), (4096, 11008), (12288, 4096), (22016, 4096), (32000, 4096), (151936, 1536))


def gemv_sweep_q8_0(dev, ws, e0, e1, launches: int = 96, reps: int = 3) -> list:
    """Q8_0 GEMV (M = 1) over SWEEP_SHAPES: achieved GB/s (weight + x + y bytes per
    launch) as a fraction of the HBM peak and of a streaming read of the same buffers.
    Each shape rotates over enough weight copies (>= 512 MB together) that no launch
    finds its weight in the 256 MB Infinity Cache; launches run back to back in one
    graph, as the decode GEMVs of a token do."""
    import torch

    from ggmlc_amd import ops

    g = torch.Generator(device=dev)
    g.manual_seed(11)
    rows = []
    for N, K in SWEEP_SHAPES:
        wbytes = N * (K // 32) * ops.BLOCK_BYTES[ops.Q8_0]
        ncopy = max(2, min(16, -(-(512 << 20) // wbytes)))
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

        loop()
        torch.cuda.synchronize()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            loop()
        gr.replay()
        torch.cuda.synchronize()
        e0.record()
        for _ in range(reps):
            gr.replay()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / (reps * launches)
        nbytes = wbytes + 4 * K + 4 * N
        gbs = nbytes / (ms * 1e-3) / 1e9
        probe_ms = time_probe_launches([ws_[i % ncopy].data for i in range(launches)], e0, e1) / launches
        rows.append({
            "N": N, "K": K, "bytes_per_launch": nbytes, "weight_copies": ncopy,
            "us_per_launch": round(ms * 1e3, 3), "achieved_GBps": round(gbs, 1),
            "frac_of_peak": round(gbs / HBM_PEAK_GBS, 4),
            "frac_of_same_size_read": round(probe_ms / ms, 4),
        })
        log(f"sweep q8_0 N={N} K={K}: {ms * 1e3:.2f} us, {gbs:.0f} GB/s ({gbs / HBM_PEAK_GBS:.1%} of peak)")
        del gr, ws_
    return rows


def time_probe_launches(bufs, e0, e1, reps: int = 5) -> float:
    """ms for one pass of streaming-read probes, one launch per buffer (each read once,
    whole), captured in a graph and timed like the GEMV graphs."""
    import torch

    from ggmlc_amd import _lib

    Lib = _lib.load()
    sink = torch.zeros(4, dtype=torch.int32, device=bufs[0].device)

    def run():
        st = torch.cuda.current_stream().cuda_stream  # the capture stream inside the graph
        for b in bufs:
            _lib.check(Lib.gq_probe_stream_read(b.data_ptr(), b.numel() // 16 * 16, sink.data_ptr(), st))

    run()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run()
    g.replay()
    torch.cuda.synchronize()
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


def decode_gemvs(w, cfg, dev, gen):
    """The 129 decode GEMVs of one token (qkv, o, gate_up, down per layer; lm_head)
    with activations of the right widths."""
    import torch

    x_h = torch.randn((1, cfg.n_embd), generator=gen, device=dev)
    x_f = torch.randn((1, cfg.n_ff), generator=gen, device=dev)
    mats = []
    for L in w.layers:
        mats += [(L.qkv, x_h), (L.o, x_h), (L.gate_up, x_h), (L.down, x_f)]
    mats.append((w.lm_head, x_h))
    outs = [torch.empty((1, m.N), device=dev) for m, _ in mats]
    return mats, outs


def traffic_probe(w, cfg, dev) -> int:
    """Eager launches for the PMC runs (per-dispatch counters do not survive graph
    replay under the profiler): 3 x the decode GEMV mix, then 3 x a 256 MiB device copy
    whose FETCH_SIZE / WRITE_SIZE calibrate the counters (256 MiB each way)."""
    import torch

    from ggmlc_amd import ops

    gen = torch.Generator(device=dev)
    gen.manual_seed(5)
    mats, outs = decode_gemvs(w, cfg, dev, gen)
    for _ in range(3):
        for (m, x), o in zip(mats, outs):
            ops.mul_mat(m, x, out=o)
    a = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    log(f"traffic probe: {3 * len(mats)} GEMV launches, 3 copies of {a.numel()} bytes")
    return 0


def load_traffic(kernel: str) -> float | None:
    """HBM bytes per launch of `kernel` measured by the PMC runs and summarised in
    profiles/gemv_traffic.json (null when absent)."""
    f = ROOT / "profiles" / "gemv_traffic.json"
    if not f.exists():
        return None
    d = json.loads(f.read_text()).get(kernel)
    return None if d is None else float(d["hbm_bytes_per_launch"])


def cpu_baseline(w, cfg, seconds: float) -> dict:
    """The reference ggml CPU backend running the same decoder on the same weights:
    pp512 (one ubatch from position 0), then greedy decode tokens for ~`seconds`."""
    import numpy as np

    import oracle as O
    from ggmlc_amd.model import host_weights

    cores = O.n_cpu_threads()
    host = host_weights(w)
    prompt = np.random.default_rng(5).integers(0, cfg.n_vocab, UBATCH).astype(np.int32)
    if O.ref_available():
        rl = O.RefLlama(cfg, host, 1024, n_threads=cores)
        t0 = time.perf_counter()
        _, tok = rl.step(prompt)
        pp_s = time.perf_counter() - t0
        rl.step([tok])  # first decode token untimed
        n, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < seconds and rl.pos < 1024:
            _, tok = rl.step([tok])
            n += 1
        dt = (time.perf_counter() - t0) / n
        del rl
        return {"value": round(1.0 / dt, 3), "unit": "tokens/s", "cores": cores, "kind": "reference",
                "sample": f"ggml CPU backend ({cores} threads) on the same {cfg.name} Q4_0 weights: one 512-token "
                          f"prefill ubatch, then {n} timed greedy decode tokens at context ~{UBATCH}",
                "ms_per_step": round(dt * 1e3, 2), "pp512_tok_s": round(UBATCH / pp_s, 2)}
    # no reference build: the C restatement's MUL_MATs of one decode token (the bulk of its work)
    x = np.random.default_rng(6).standard_normal((1, cfg.n_ff)).astype(np.float32)
    mats = [(m, cfg.n_embd if i != 3 else cfg.n_ff) for L in host[2] for i, m in enumerate(L)]
    mats.append((host[1], cfg.n_embd))
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds and n < 20:
        for m, K in mats:
            O.mul_mat(m, cfg.qtype, K, x[:, :K], n_threads=cores)
        n += 1
    dt = (time.perf_counter() - t0) / n
    return {"value": round(1.0 / dt, 3), "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": f"{n} decode tokens' MUL_MATs (the {len(mats)} GEMVs) through the C restatement",
            "ms_per_step": round(dt * 1e3, 2)}


if __name__ == "__main__":
    sys.exit(main())
