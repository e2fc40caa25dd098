"""LLaMA-style decoder executed over libgq, the way ggmlc's executor runs it.

Per layer, the graph ggmlc compiles for a LLaMA block (runtime/src/executor.cpp
:1738-2810 after python/ggmlc/transforms/fusion.py:1224-1546 fuses Q/K/V and
gate/up and bakes the RMSNorm weight into the following Linear):

    h = RMS_NORM(x) ; qkv = MUL_MAT(Wqkv, h) ; q, k = ROPE_NEOX(q, k)
    SET_ROWS(Kcache, k), SET_ROWS(Vcache, v)          # persistent KV, rows pos..pos+s-1
    a = FLASH_ATTN_EXT(q, K[:, :n_kv], V[:, :n_kv], mask[n_kv, s], 1/sqrt(hd))
    x = x + MUL_MAT(Wo, a)
    x = x + MUL_MAT(Wdown, SWIGLU(MUL_MAT(Wgate_up, RMS_NORM(x))))

then RMS_NORM -> MUL_MAT(lm_head) on the last token only (logits_last_only,
executor.cpp:2396-2410) -> ARGMAX for greedy decoding. n_kv follows
pad_kv_len (executor.cpp:58-64): max(256, roundup(pos + s, 256)) capped at max_ctx.

Every op is one libgq call on device tensors. ROPE(q), ROPE(k) and the two
SET_ROWS run as one launch (gq_rope_kv_store); decode steps (s <= 4) also fuse the
residual ADD and RMS_NORM into the following MUL_MAT, ROPE + SET_ROWS into the QKV
projection's epilogue and SWIGLU into gate_up (gq_mul_mat_fused). The fusions are
bit-identical to the separate ops. A whole step
(embedding to the argmax of the next token, plus pos += s) can be captured as one
HIP graph per (s, n_kv) bucket and replayed without host work.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

from . import ops


@dataclass
class LlamaConfig:
    name: str
    n_layer: int
    n_embd: int
    n_head: int
    n_head_kv: int
    head_dim: int
    n_ff: int
    n_vocab: int
    qtype: int
    tied_embeddings: bool = False
    rms_eps: float = 1e-5
    rope_base: float = 10000.0
    qkv_bias: bool = False  # q/k/v projections carry biases (the Qwen2 family)

    @property
    def q_dim(self) -> int:
        return self.n_head * self.head_dim

    @property
    def kv_dim(self) -> int:
        return self.n_head_kv * self.head_dim


# BASELINE.json configs[2] and configs[3]
SMOLLM2_360M = LlamaConfig("smollm2-360m-shape", 32, 960, 15, 5, 64, 2560, 49152, ops.Q8_0, tied_embeddings=True)
LLAMA_7B = LlamaConfig("llama-7b-shape", 32, 4096, 32, 32, 128, 11008, 32000, ops.Q4_0)
# the Qwen2 architecture, q/k/v biases included
QWEN25_1_5B = LlamaConfig("qwen2.5-1.5b-shape", 28, 1536, 12, 2, 128, 8960, 151936, ops.Q8_0, tied_embeddings=True,
                          qkv_bias=True)


class _Recorder:
    """Collects (name, layer, copy) of op outputs when a trace list is given."""

    def __init__(self, trace: list | None):
        self.trace = trace

    def __call__(self, name, li, t):
        if self.trace is not None:
            self.trace.append((name, li, t.detach().clone()))


def pad_kv_len(n: int, max_ctx: int, n_pad: int = 256) -> int:
    """executor.cpp:58-64"""
    n = max(n, 1)
    if n_pad <= 1:
        return min(n, max_ctx)
    return min(max(n_pad, ((n + n_pad - 1) // n_pad) * n_pad), max_ctx)


@dataclass
class LayerWeights:
    qkv: ops.QWeight
    o: ops.QWeight
    gate_up: ops.QWeight
    down: ops.QWeight
    # the MUL_MAT nodes' bias inputs (fp32 [N] device tensors, e.g. Qwen2's q/k/v biases,
    # concatenated q | k | v like the weight rows): ADD(MUL_MAT(W, x), bias)
    qkv_b: torch.Tensor | None = None
    o_b: torch.Tensor | None = None
    gate_up_b: torch.Tensor | None = None
    down_b: torch.Tensor | None = None


@dataclass
class ModelWeights:
    cfg: LlamaConfig
    embed: ops.QWeight
    lm_head: ops.QWeight
    layers: list[LayerWeights] = field(default_factory=list)

    @property
    def nbytes(self) -> int:
        n = self.embed.nbytes + (0 if self.cfg.tied_embeddings else self.lm_head.nbytes)
        for L in self.layers:
            n += L.qkv.nbytes + L.o.nbytes + L.gate_up.nbytes + L.down.nbytes
        return n

    @property
    def decode_bytes(self) -> int:
        """weight bytes one decode token streams (the embedding row is negligible)"""
        n = self.lm_head.nbytes
        for L in self.layers:
            n += L.qkv.nbytes + L.o.nbytes + L.gate_up.nbytes + L.down.nbytes
        return n


def random_weights(cfg: LlamaConfig, device, seed: int = 0, std: float = 0.02, bias_std: float = 0.1) -> ModelWeights:
    """Random-init weights N(0, std) quantized on the device with ggmlc's quantizer
    (quantize.py semantics). RMSNorm weights are 1 at init, so the fused graph's
    baked-in gamma leaves the Linear weights unchanged. With cfg.qkv_bias the fused
    q | k | v projection gets an fp32 bias N(0, bias_std) (the quantizer keeps 1-d
    parameters in fp32)."""
    g = torch.Generator(device=device)
    g.manual_seed(seed)

    def q(n, k):
        w = torch.randn((n, k), generator=g, device=device) * std
        out = ops.quantize_weights(w, cfg.qtype)
        del w
        return out

    embed = q(cfg.n_vocab, cfg.n_embd)
    lm_head = embed if cfg.tied_embeddings else q(cfg.n_vocab, cfg.n_embd)
    layers = []
    for _ in range(cfg.n_layer):
        layers.append(LayerWeights(
            qkv=q(cfg.q_dim + 2 * cfg.kv_dim, cfg.n_embd),
            o=q(cfg.n_embd, cfg.q_dim),
            gate_up=q(2 * cfg.n_ff, cfg.n_embd),
            down=q(cfg.n_embd, cfg.n_ff),
            qkv_b=(torch.randn(cfg.q_dim + 2 * cfg.kv_dim, generator=g, device=device) * bias_std
                   if cfg.qkv_bias else None),
        ))
    return ModelWeights(cfg, embed, lm_head, layers)


def host_weights(w: ModelWeights) -> tuple:
    """(embed, lm_head, [(qkv, o, gate_up, down, qkv_b, o_b, gate_up_b, down_b), ...]) on the
    host: the GGUF block bytes (uint8) and the fp32 biases (None where absent)."""
    def np_(t):
        return None if t is None else t.cpu().numpy()

    return (np_(w.embed.data), np_(w.lm_head.data),
            [tuple(np_(m.data) for m in (L.qkv, L.o, L.gate_up, L.down)) +
             tuple(np_(b) for b in (L.qkv_b, L.o_b, L.gate_up_b, L.down_b)) for L in w.layers])


def _linear(wt: ops.QWeight, bias: torch.Tensor | None, x: torch.Tensor, out: torch.Tensor, ws) -> torch.Tensor:
    """MUL_MAT(W, x) (+ bias: the node's ADD, executor.cpp:2436-2445) as separate ops"""
    y = ops.mul_mat(wt, x, out=out, ws=ws)
    return ops.add(y, bias, out=y) if bias is not None else y


def q8_chain_ok(w: ModelWeights) -> bool:
    """Whether every product of a layer can take the int8 path with the quantized-row
    handoffs (K % 256 == 0, 16-byte aligned weights, gate|up rows % 64, QKV rows % 16,
    a power-of-two head_dim >= 16): see forward's q8 mode."""
    c = w.cfg
    hd = c.head_dim
    if hd < 16 or hd & (hd - 1):
        return False
    for L in w.layers:
        for wt in (L.qkv, L.o, L.gate_up, L.down):
            if wt.K % 256 or wt.data.data_ptr() % 16:
                return False
        if L.gate_up.N % 64 or L.qkv.N % 16:
            return False
    return True


def forward(w: ModelWeights, s: int, b: dict, ids: torch.Tensor, k_cache: list, v_cache: list, attend, fused: bool,
            rec, ws: ops.Workspace, out: torch.Tensor, r0: int, q8: bool = False) -> torch.Tensor:
    """The layer stack of one step over s rows: embedding -> layers -> RMS_NORM -> lm_head
    logits of rows [r0, s) into `out`. b holds the step's buffers, with pos_ids (int32 [s])
    and kv_idx (int64 [s]) already filled: row i is rotated at pos_ids[i] and its K/V rows
    are stored at row kv_idx[i] of k_cache[l] / v_cache[l] ([1, Hkv, rows, hd] fp16).
    attend(l, q) returns the attention output [s, Hq, hd] of layer l for the rotated q
    ([1, s, Hq, hd]); the caller picks what the rows attend to (one sequence's cache with
    its causal mask, or each row its own sequence's pages).
    q8 (up to 16 rows, not fused, q8_chain_ok, attend(l, q, out_q8) writing the rows
    quantized): every product on the int8 path, with ROPE + SET_ROWS in the QKV product's
    epilogue, the attention's split merge quantizing the o projection's input, and
    gate_up's epilogue writing SWIGLU's rows quantized for down — the quantize steps of
    the unfused ops moved into their producers (bit-identical), 3 launches fewer per
    layer; o and down, where the int8 path takes K in two halves (narrow products), leave
    the halves' sums for the next prologue's ADD to add (bit-identical too)."""
    c = w.cfg
    qd, kvd = c.q_dim, c.kv_dim
    # more than 4 rows without a trace: the GEMM path with ADD / RMS_NORM / SWIGLU fused
    # into the prologue that quantizes each GEMM's activation (bit-identical as well)
    q8 = q8 and not fused and rec.trace is None and s <= 16
    pro = not fused and rec.trace is None and (s > 4 or q8)
    if fused or q8:  # the rope (cos, sin) table of this step's positions, shared by all layers
        ops.rope_cache(b["pos_ids"], c.head_dim, c.rope_base, out=b["rope_cs"])
    x = b["x"]
    ops.get_rows(w.embed, ids, out=x)
    # fused path: the residual ADD after O and after down is done by the next GEMV's
    # prologue (x_next = x + proj, stored for the following ADD), alternating buffers
    other = {id(b["x"]): b["x_alt"], id(b["x_alt"]): b["x"]}
    pending = None  # proj still to be added to x
    pend_halves = False  # pending holds a product's two halves of K ([2, s, n_embd])
    for li, L in enumerate(w.layers):
        if fused:  # ADD + RMS_NORM + QKV + ROPE x2 + SET_ROWS x2 in one launch (bit-identical)
            nx = other[id(x)] if pending is not None else None
            ops.mul_mat_fused(L.qkv, x, rms_eps=c.rms_eps, x_add=pending, x_sum=nx, rope_kv=ops.RopeKv(
                c.n_head, c.n_head_kv, c.head_dim, b["pos_ids"], c.head_dim, 2, c.rope_base, b["kv_idx"],
                b["q"], k_cache[li], v_cache[li], cache=b["rope_cs"]), bias=L.qkv_b)
            x = nx if nx is not None else x
            q = b["q"]
        elif q8:  # ADD + RMS_NORM in the prologue, ROPE + SET_ROWS in the epilogue
            nx = other[id(x)] if pending is not None else None
            ops.mul_mat_fused(L.qkv, x, rms_eps=c.rms_eps, x_add=pending, x_sum=nx, ws=ws, bias=L.qkv_b, int8=True,
                              rope_kv=ops.RopeKv(c.n_head, c.n_head_kv, c.head_dim, b["pos_ids"], c.head_dim, 2,
                                                 c.rope_base, b["kv_idx"], b["q"], k_cache[li], v_cache[li],
                                                 cache=b["rope_cs"]), x_add_halves=pend_halves)
            x = nx if nx is not None else x
            q = b["q"]
        else:
            if pro:  # ADD + RMS_NORM in the QKV GEMM's prologue
                nx = other[id(x)] if pending is not None else None
                qkv = ops.mul_mat_fused(L.qkv, x, out=b["qkv"], rms_eps=c.rms_eps, x_add=pending, x_sum=nx, ws=ws,
                                        bias=L.qkv_b)
                x = nx if nx is not None else x
            else:
                rec("x_in", li, x)
                h = ops.rms_norm(x, c.rms_eps, out=b["h"])
                rec("h1", li, h)
                qkv = _linear(L.qkv, L.qkv_b, h, b["qkv"], ws)
                rec("qkv", li, qkv)
            # views of the fused projection (ggml VIEW/RESHAPE, executor.cpp:75-113)
            qv = qkv[:, :qd].view(1, s, c.n_head, c.head_dim)
            kv = qkv[:, qd:qd + kvd].view(1, s, c.n_head_kv, c.head_dim)
            vv = qkv[:, qd + kvd:].view(1, s, c.n_head_kv, c.head_dim)
            if rec.trace is None:  # ROPE x2 + SET_ROWS x2 in one launch (bit-identical)
                q = ops.rope_kv_store(qv, kv, vv, b["pos_ids"], c.head_dim, 2, c.rope_base, b["kv_idx"], b["q"],
                                      k_cache[li], v_cache[li])
            else:
                q = ops.rope_ext(qv, b["pos_ids"], c.head_dim, 2, c.rope_base, out=b["q"])
                k = ops.rope_ext(kv, b["pos_ids"], c.head_dim, 2, c.rope_base, out=b["k"])
                # [1, s, H, hd] -> ggml src [hd, s, H, 1] for SET_ROWS
                ops.set_rows(k_cache[li], k.permute(0, 2, 1, 3), b["kv_idx"])
                ops.set_rows(v_cache[li], vv.permute(0, 2, 1, 3), b["kv_idx"])
                rec("q", li, q), rec("k", li, k), rec("kc", li, k_cache[li]), rec("vc", li, v_cache[li])
        if q8:
            attend(li, q, b["q8_o"])
        else:
            attend(li, q)
        rec("attn", li, b["attn"])
        if q8:  # o from the merge's quantized rows; SWIGLU's rows quantized for down; o and
            # down in two halves of K where the int8 path splits them
            av = b["attn"].view(s, qd)
            oh = ops.mul_mat_halves(L.o, av, L.o_b, int8=True)
            o = ops.mul_mat_fused(L.o, av, out=b["proj2"] if oh else b["proj"], x_q8=b["q8_o"], ws=ws, bias=L.o_b,
                                  int8=True, out_halves=oh)
            nx = other[id(x)]
            ops.mul_mat_fused(L.gate_up, x, rms_eps=c.rms_eps, x_add=o, x_sum=nx, swiglu=True, out_q8=b["q8_d"],
                              no_out=True, ws=ws, bias=L.gate_up_b, int8=True, x_add_halves=oh)
            x = nx
            pend_halves = ops.mul_mat_halves(L.down, b["act"], L.down_b, int8=True)
            pending = ops.mul_mat_fused(L.down, b["act"], out=b["proj2"] if pend_halves else b["proj"],
                                        x_q8=b["q8_d"], ws=ws, bias=L.down_b, int8=True, out_halves=pend_halves)
        elif fused:
            o = ops.mul_mat_fused(L.o, b["attn"].view(s, qd), out=b["proj"], bias=L.o_b)
            nx = other[id(x)]
            a = ops.mul_mat_fused(L.gate_up, x, out=b["act"], rms_eps=c.rms_eps, swiglu=True, x_add=o, x_sum=nx,
                                  bias=L.gate_up_b)
            x = nx
            pending = ops.mul_mat_fused(L.down, a, out=b["proj"], bias=L.down_b)
        elif pro:  # ADD + RMS_NORM before gate_up, SWIGLU before down, in their prologues
            o = _linear(L.o, L.o_b, b["attn"].view(s, qd), b["proj"], ws)
            nx = other[id(x)]
            gu = ops.mul_mat_fused(L.gate_up, x, out=b["gu"], rms_eps=c.rms_eps, x_add=o, x_sum=nx, ws=ws,
                                   bias=L.gate_up_b)
            x = nx
            pending = ops.mul_mat_fused(L.down, gu, out=b["proj"], x_swiglu=True, ws=ws, bias=L.down_b)
        else:
            o = _linear(L.o, L.o_b, b["attn"].view(s, qd), b["proj"], ws)
            ops.add(x, o, out=x)
            rec("x_mid", li, x)
            h = ops.rms_norm(x, c.rms_eps, out=b["h"])
            rec("h2", li, h)
            gu = _linear(L.gate_up, L.gate_up_b, h, b["gu"], ws)
            rec("gu", li, gu)
            a = ops.swiglu(gu, out=b["act"])
            rec("act", li, a)
            d = _linear(L.down, L.down_b, a, b["proj"], ws)
            ops.add(x, d, out=x)
        rec("x_out", li, x)
    if fused or pro:
        head8 = q8 and w.lm_head.K % 256 == 0 and w.lm_head.data.data_ptr() % 16 == 0
        if pend_halves and not head8 and s - r0 <= 4:  # the GEMV path adds one tensor: the halves' sum first
            pending, pend_halves = ops.add(pending[0], pending[1], out=b["proj"]), False
        if pending is not None:
            pending = pending[:, r0:] if pend_halves else pending[r0:]
        return ops.mul_mat_fused(w.lm_head, x[r0:], out=out, rms_eps=c.rms_eps, x_add=pending, ws=ws, int8=head8,
                                 x_add_halves=pend_halves)
    h = ops.rms_norm(x[r0:], c.rms_eps, out=b["h"][:s - r0])
    rec("hf", -1, h)
    return ops.mul_mat(w.lm_head, h, out=out, ws=ws)


class Decoder:
    """Executor for one sequence with a persistent F16 KV cache of max_ctx rows."""

    def __init__(self, w: ModelWeights, max_ctx: int, device, n_pad: int = 256):
        self.w = w
        self.cfg = cfg = w.cfg
        self.dev = device
        self.max_ctx = max_ctx
        self.n_pad = n_pad
        self.k_cache = [torch.zeros((1, cfg.n_head_kv, max_ctx, cfg.head_dim), dtype=torch.float16, device=device)
                        for _ in range(cfg.n_layer)]
        self.v_cache = [torch.zeros_like(k) for k in self.k_cache]
        self.pos = torch.zeros(1, dtype=torch.int32, device=device)  # device-resident position
        self.ws = ops.Workspace(device)
        self._bufs: dict[int, dict[str, torch.Tensor]] = {}
        self.graphs: dict[tuple[int, int], torch.cuda.CUDAGraph] = {}

    # -- state ---------------------------------------------------------------
    def reset(self, pos: int = 0) -> None:
        """Rewind the position (the cache rows past it are rewritten before use)."""
        self.pos.fill_(pos)

    def _buffers(self, s: int) -> dict[str, torch.Tensor]:
        if s not in self._bufs:
            c, d = self.cfg, self.dev
            f32 = dict(dtype=torch.float32, device=d)
            self._bufs[s] = {
                "ids": torch.zeros(s, dtype=torch.int32, device=d),
                "x": torch.empty((s, c.n_embd), **f32),
                "x_alt": torch.empty((s, c.n_embd), **f32),
                "h": torch.empty((s, c.n_embd), **f32),
                "qkv": torch.empty((s, c.q_dim + 2 * c.kv_dim), **f32),
                "q": torch.empty((1, s, c.n_head, c.head_dim), **f32),
                "k": torch.empty((1, s, c.n_head_kv, c.head_dim), **f32),
                "attn": torch.empty((s, c.n_head, c.head_dim), **f32),
                "proj": torch.empty((s, c.n_embd), **f32),
                "proj2": torch.empty((2, s, c.n_embd), **f32),  # a product's two halves of K
                "gu": torch.empty((s, 2 * c.n_ff), **f32),
                "act": torch.empty((s, c.n_ff), **f32),
                "logits": torch.empty((1, c.n_vocab), **f32),
                "next": torch.zeros(1, dtype=torch.int32, device=d),
                "pos_ids": torch.zeros(s, dtype=torch.int32, device=d),
                "kv_idx": torch.zeros(s, dtype=torch.int64, device=d),
                "rope_cs": torch.zeros((s, c.head_dim), dtype=torch.float32, device=d),
                "mask": torch.zeros((s, self.max_ctx), dtype=torch.float16, device=d),
            }
        return self._bufs[s]

    # -- one step -------------------------------------------------------------
    def step(self, s: int, n_kv: int, ids: torch.Tensor | None = None, advance: bool = True,
             trace: list | None = None, fused: bool | None = None, logits_all: bool = False) -> torch.Tensor:
        """Run s tokens (ids int32 [s], default: this bucket's ids buffer) at the device
        position; returns the argmax of the last token's logits (device int32 [1]).

        fused (default: s <= 4 without a trace): run ADD -> RMS_NORM -> MUL_MAT (-> ROPE
        + SET_ROWS for QKV, -> SWIGLU for gate_up) as single GEMV launches
        (gq_mul_mat_fused, bit-identical).
        trace (eager only): receives (name, layer, copy) of every op's output, so a
        checker can recompute each op from the inputs this step actually used.
        logits_all: compute the logits of all s tokens into this bucket's "logits_all"
        buffer [s, vocab] (the graph output of the reference runtime), not only the last."""
        c, b, ws = self.cfg, self._buffers(s), self.ws
        if fused is None:
            fused = s <= 4 and trace is None

        rec = _Recorder(trace)

        if n_kv > self.max_ctx:
            raise ValueError("n_kv exceeds the KV cache")
        ids = b["ids"] if ids is None else ids
        self.ws.get(self._ws_need(s))
        mask = b["mask"][:, :n_kv]
        ops.kv_step_inputs(self.pos, s, b["pos_ids"], b["kv_idx"], mask)
        rec("pos", -1, self.pos)
        scale = 1.0 / math.sqrt(c.head_dim)

        def attend(li, q):
            return ops.flash_attn_ext(q[0].permute(1, 0, 2), self.k_cache[li][0, :, :n_kv],
                                      self.v_cache[li][0, :, :n_kv], mask, scale, out=b["attn"], ws=ws)

        r0 = 0 if logits_all else s - 1  # first row that gets logits
        if logits_all:
            if "logits_all" not in b:
                b["logits_all"] = torch.empty((s, c.n_vocab), dtype=torch.float32, device=self.dev)
            out = b["logits_all"]
            self.ws.get(ops.mul_mat_workspace_size(self.w.lm_head, s))
        else:
            out = b["logits"]
        logits = forward(self.w, s, b, ids, self.k_cache, self.v_cache, attend, fused, rec, ws, out, r0)
        ops.argmax(logits[s - 1 - r0:], out=b["next"])
        rec("logits", -1, logits), rec("next", -1, b["next"])
        if advance:
            ops.kv_advance(self.pos, s)
        return b["next"]

    # -- graphs -----------------------------------------------------------------
    def capture(self, s: int, n_kv: int, ids: torch.Tensor | None = None) -> torch.cuda.CUDAGraph:
        """HIP graph of one step for the (s, n_kv) bucket (ids: the input buffer the
        graph reads; for decode pass the graph's own "next" buffer to chain tokens)."""
        key = (s, n_kv)
        if key in self.graphs:
            return self.graphs[key]
        self.ws.get(self._ws_need(s))
        saved = self.pos.clone()
        self.step(s, n_kv, ids)  # warm-up (kernel attributes, occupancy caches)
        torch.cuda.synchronize()
        self.pos.copy_(saved)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self.step(s, n_kv, ids)
        torch.cuda.synchronize()
        self.pos.copy_(saved)
        self.graphs[key] = g
        return g

    def _ws_need(self, s: int) -> int:
        """Largest workspace any op of an s-token step can ask for (attention's split
        plan depends on n_kv, not monotonically: every bucket size is checked)."""
        c, L = self.cfg, self.w.layers[0]
        need = [ops.mul_mat_workspace_size(wt, s) for wt in (L.qkv, L.o, L.gate_up, L.down)]
        need.append(ops.mul_mat_workspace_size(self.w.lm_head, 1))
        for n_kv in sorted(set(list(range(256, self.max_ctx + 1, 256)) + [self.max_ctx])):
            need.append(ops.flash_attn_workspace_size(c.head_dim, s, c.n_head, c.n_head_kv, n_kv))
        return max(need)

    def decode_buffers(self) -> tuple[torch.Tensor, torch.Tensor]:
        """(ids, next) of the s = 1 bucket: chaining next -> ids makes replays generate."""
        b = self._buffers(1)
        return b["ids"], b["next"]
