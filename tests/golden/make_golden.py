"""Write the golden vectors for the hot path from the reference's compiled ggml.

Run in the build container (needs oracle/_ref/libggmlref.so, i.e. /root/reference):

    python tests/golden/make_golden.py

Every expected output here is produced by the reference's own ggml 0.20.2 CPU
backend (oracle/_ref, built by oracle/Makefile from the reference sources) on
seeded inputs; inputs are stored next to the outputs. Weight bytes are made by
the oracle's restatement of ggmlc's Python quantizer (they are inputs: CPU and
GPU read the same bytes). The reference itself holds no golden vectors.
"""

from __future__ import annotations

import json
import platform
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

import oracle as O  # noqa: E402

OUT = Path(__file__).resolve().parent


def f16(a):
    return np.asarray(a, np.float32).astype(np.float16).view(np.uint16)


def main() -> None:
    R = O.ref()
    rng = np.random.default_rng(20260101)
    manifest = {"ggml": R.ref_ggml_version().decode(), "host": platform.processor() or platform.machine(),
                "seed": 20260101, "files": {}}

    # ---- quantize_row_q8_0 (x86 runtime quantizer), edge blocks included
    X = rng.standard_normal((12, 1024)).astype(np.float32)
    X[1] *= 1e-3
    X[2] *= 300.0
    X[3, :32] = 0.0                                   # all-zero block -> d = 0, q = 0
    X[3, 32:64] = 0.5                                 # constant block -> q = 127
    X[3, 64:96] = np.linspace(-1, 1, 32)              # +-amax -> +-127
    X[4, :32] = np.arange(32, dtype=np.float32) - 15.5  # halves against id
    X[5, :32] = 1e-30                                 # tiny amax, d underflows fp16
    X[6, :32] = 7e4                                   # amax/127 above fp16 max? (551) no: fine
    X[7] = np.round(X[7] * 8) / 8                     # many exact ties x*id = k + 0.5
    q = O.quantize_row_q8_0(X, impl="ref")
    np.savez_compressed(OUT / "quantize_q8_0.npz", x=X, q=q)
    manifest["files"]["quantize_q8_0.npz"] = "x fp32 [12,1024] -> q uint8 [12, 32*34] (ggml x86 quantize_row_q8_0)"

    # ---- mul_mat Q8_0 / Q4_0: GEMV (M=1) and GEMM (M=2,5,16), K in {256, 960, 1024}
    cases = []
    for wt, name in ((O.Q8_0, "q8_0"), (O.Q4_0, "q4_0")):
        for K, N, M in ((1024, 96, 1), (1024, 64, 5), (960, 40, 1), (256, 48, 16), (512, 33, 3)):
            W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
            wq = O.quantize_weights(W, wt)
            Xm = rng.standard_normal((M, K)).astype(np.float32)
            Y = O.mul_mat(wq, wt, K, Xm, impl="ref", n_threads=1)
            fn = f"mul_mat_{name}_K{K}_N{N}_M{M}.npz"
            np.savez_compressed(OUT / fn, w=wq, x=Xm, y=Y, wtype=np.int32(wt), K=np.int64(K))
            cases.append(fn)
    manifest["files"]["mul_mat_*"] = "w uint8 quantized [N, K/32*bb], x fp32 [M,K] -> y fp32 [M,N] (ggml_mul_mat, 1 thread)"

    # ---- python weight quantizer bytes for a fixed small tensor (self-check input)
    # ---- set_rows F32 -> F16 into a padded cache
    B, H, ctx, hd, s = 1, 5, 96, 64, 9
    cache = f16(rng.standard_normal((B, H, ctx, hd)))
    src = (rng.standard_normal((B, H, s, hd)) * 4).astype(np.float32)
    src[0, 0, 0, :8] = [0.0, -0.0, 65504.0, 65520.0, 1e-8, -3e-5, 6.1e-5, 2.0 ** -25]
    idx = np.array([40, 41, 42, 43, 44, 45, 46, 47, 95], np.int64)
    out = O.set_rows_f32_f16(cache, src, idx, impl="ref")
    np.savez_compressed(OUT / "set_rows_f32_f16.npz", cache=cache, src=src, idx=idx, out=out)
    manifest["files"]["set_rows_f32_f16.npz"] = "cache uint16 [1,5,96,64], src fp32 [1,5,9,64], idx i64 [9] -> out"

    # ---- flash_attn_ext (F16 K/V cache views + causal mask), decode and prefill
    fa = []
    for (Hq, Hkv, hd, n_kv, s, pos, nt) in ((15, 5, 64, 256, 1, 200, 1), (6, 1, 128, 512, 1, 300, 4),
                                            (4, 2, 128, 256, 4, 100, 1), (4, 2, 64, 256, 64, 150, 1)):
        ctx = n_kv + 16  # cache rows beyond the active n_kv view exercise the row stride
        kc = f16(rng.standard_normal((Hkv, ctx, hd)))
        vc = f16(rng.standard_normal((Hkv, ctx, hd)))
        qq = rng.standard_normal((Hq, s, hd)).astype(np.float32)
        mask = O.causal_mask_f16(pos, s, n_kv)
        o = O.flash_attn_ext_f16(qq, kc, vc, n_kv, mask, impl="ref", n_threads=nt)
        fn = f"flash_attn_Hq{Hq}_Hkv{Hkv}_hd{hd}_nkv{n_kv}_s{s}.npz"
        np.savez_compressed(OUT / fn, q=qq, kc=kc, vc=vc, mask=mask, out=o, n_kv=np.int64(n_kv),
                            n_threads=np.int32(nt))
        fa.append(fn)
    manifest["files"]["flash_attn_*"] = ("q fp32 [Hq,s,hd], kc/vc uint16 [Hkv,n_kv+16,hd], mask uint16 [s,n_kv] -> "
                                         "out fp32 [s,Hq,hd] (ggml_flash_attn_ext, scale 1/sqrt(hd))")

    # ---- soft_max with mask and scale
    xs = (rng.standard_normal((16, 300)) * 3).astype(np.float32)
    ms = O.causal_mask_f16(250, 16, 300)
    ys = O.soft_max_f32(xs, ms, 0.125, impl="ref")
    np.savez_compressed(OUT / "soft_max_f32.npz", x=xs, mask=ms, y=ys, scale=np.float32(0.125))
    manifest["files"]["soft_max_f32.npz"] = "x fp32 [16,300], mask uint16 [16,300], scale 0.125 -> y"

    # ---- decoder ops around the path (one ggml node each)
    a = (rng.standard_normal((5, 2 * 96)) * 3).astype(np.float32)
    np.savez_compressed(OUT / "swiglu.npz", a=a, y=O.ref_swiglu(a))
    xr = (rng.standard_normal((7, 960)) * 2).astype(np.float32)
    np.savez_compressed(OUT / "rms_norm.npz", x=xr, eps=np.float32(1e-5), y=O.ref_rms_norm(xr, 1e-5))
    for mode, name in ((2, "neox"), (0, "normal")):
        xq = rng.standard_normal((6, 5, 64)).astype(np.float32)     # [seq, heads, hd]
        pos = np.array([0, 1, 17, 255, 1000, 4095], np.int32)
        np.savez_compressed(OUT / f"rope_{name}.npz", x=xq, pos=pos, n_dims=np.int32(64), mode=np.int32(mode),
                            freq_base=np.float32(10000.0), y=O.ref_rope(xq, pos, 64, mode, 10000.0))
    for wt, name in ((O.Q8_0, "q8_0"), (O.Q4_0, "q4_0")):
        tab = O.quantize_weights((rng.standard_normal((50, 960)) * 0.02).astype(np.float32), wt)
        ids = np.array([0, 49, 7, 7, 23], np.int32)
        np.savez_compressed(OUT / f"get_rows_{name}.npz", table=tab, wtype=np.int32(wt), n_embd=np.int64(960), ids=ids,
                            y=O.ref_get_rows(tab, wt, 960, ids))
    xa = rng.standard_normal((4, 1000)).astype(np.float32)
    xa[2, 10] = xa[2, 500] = 99.0  # tie: first index wins
    np.savez_compressed(OUT / "argmax.npz", x=xa, y=O.ref_argmax(xa))
    manifest["files"]["decoder ops"] = ("swiglu / rms_norm / rope_{neox,normal} / get_rows_{q8_0,q4_0} / argmax: "
                                        "one ggml node each on the CPU backend")

    config_attention(manifest)
    (OUT / "MANIFEST.json").write_text(json.dumps(manifest, indent=1) + "\n")
    print("wrote", len(list(OUT.glob("*.npz"))), "fixtures")


# decode attention at the BASELINE configs' shapes: (name, Hq, Hkv, hd, pos) with s = 1 and
# n_kv = pad_kv_len(pos + 1); pos is the last decode position of each config's run
CFG_ATTN = (
    ("smollm2_gqa3", 15, 5, 64, 639),      # configs[2]: 512-token prompt + 128 steps -> n_kv 768
    ("llama7b_mha", 32, 32, 128, 1279),    # configs[3]: 1024 + 128 (+ margin) -> n_kv 1280
    ("qwen_gqa6_3k", 12, 2, 128, 3071),    # configs[4]: contexts up to 4096
    ("qwen_gqa6_4k", 12, 2, 128, 4095),
)
CFG_THREADS = (1, 4, 16)


def cfg_attn_inputs(seed: int, Hq: int, Hkv: int, hd: int, pos: int):
    """Seeded inputs of a config-shape attention fixture (regenerated by the tests; the
    fixture stores their sha256 so a different generator is caught)."""
    rng = np.random.default_rng(seed)
    n_kv = O.pad_kv_len(pos + 1, 1 << 20)
    kc = f16(rng.standard_normal((Hkv, n_kv, hd)))
    vc = f16(rng.standard_normal((Hkv, n_kv, hd)))
    q = rng.standard_normal((Hq, 1, hd)).astype(np.float32)
    mask = O.causal_mask_f16(pos, 1, n_kv)
    return q, kc, vc, mask, n_kv


def inputs_digest(*arrays) -> str:
    import hashlib

    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def config_attention(manifest: dict) -> None:
    """ggml's decode attention at the configs' shapes, at 1, 4 and 16 threads: its
    split-KV chunking (ops.cpp:9179-9209) and fp16 V accumulator make the output depend
    on the thread count, and these fixtures record by how much."""
    for i, (name, Hq, Hkv, hd, pos) in enumerate(CFG_ATTN):
        seed = 777000 + i
        q, kc, vc, mask, n_kv = cfg_attn_inputs(seed, Hq, Hkv, hd, pos)
        outs = {f"out_t{t}": O.flash_attn_ext_f16(q, kc, vc, n_kv, mask, impl="ref", n_threads=t)
                for t in CFG_THREADS}
        np.savez_compressed(OUT / f"cfg_attn_{name}.npz", seed=np.int64(seed), Hq=np.int64(Hq), Hkv=np.int64(Hkv),
                            hd=np.int64(hd), pos=np.int64(pos), n_kv=np.int64(n_kv),
                            digest=np.array(inputs_digest(q, kc, vc, mask)), **outs)
    manifest["files"]["cfg_attn_*"] = ("decode attention at the configs' shapes: inputs regenerated from `seed` "
                                       "(cfg_attn_inputs, checked against `digest`), outputs of ggml_flash_attn_ext "
                                       "at 1, 4 and 16 threads (out_t1, out_t4, out_t16)")


if __name__ == "__main__":
    if sys.argv[1:] == ["--config-attention"]:
        man = json.loads((OUT / "MANIFEST.json").read_text())
        config_attention(man)
        (OUT / "MANIFEST.json").write_text(json.dumps(man, indent=1) + "\n")
    else:
        main()
