"""The compile path for LLaMA-family PyTorch modules: module -> fused, baked, quantized
weights -> a ggmlc .gguf the runner (and ggmlc's own runtime) executes.

What ggmlc's compiler does for these modules (python/ggmlc/compiler.py:32-247 driving
transforms/fusion.py and transforms/affine_bake.py, then quantization/quantize.py),
restated for the decoders this package runs, with the same results:

* horizontal fusion: q, k, v projections -> one QKV MUL_MAT (rows q | k | v), gate and
  up -> one gate|up MUL_MAT (rows gate | up; GLU SWIGLU takes the first half as the
  gate), rows concatenated (fusion.py:21-41);
* RMS bake: each RMSNorm's gamma scales the input columns of the Linear that consumes
  it, W'[j, k] = W[j, k] * gamma[k] in float32 (affine_bake.py:413-416), leaving a
  weightless RMS_NORM; the final norm bakes into the output head unless that weight
  is tied to the embedding (not exclusive): a tied head with gamma != 1 is written as
  its own baked tensor, a tied head with gamma == 1 stays tied;
* uniform quantization policies "q8_0" / "q4_0" (quantization/policies.py Q8_0_POLICY,
  Q4_0_POLICY): every 2-D weight, embedding included, in that type, with
  quantize.py's float32 numpy arithmetic (:10-47 Q8_0, :65-107 Q4_0);
* RMS_NORM carries the module's eps as an attribute, as the PyTorch importer writes it
  (frontend/pytorch/importer.py:1041-1053), except the runtime's default 1e-5.

* Linear biases stay fp32 and feed the MUL_MAT node's third input (dialect/ggml/
  lowering.py:462-475), those of a fused group concatenated like its rows (the Qwen2
  family's q/k/v biases).

Supported: LlamaForCausalLM-shaped modules (model.embed_tokens, model.layers[i].
{input_layernorm, self_attn.{q,k,v,o}_proj, post_attention_layernorm,
mlp.{gate,up,down}_proj}, model.norm, lm_head), Qwen2ForCausalLM included, with the
default rotary embedding (NEOX pairs over the whole head); anything else raises
NotImplementedError naming what does not fit.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np

from .llama_gguf import write_llama_gguf
from .model import LlamaConfig

Q8_0, Q4_0 = 8, 2
_POLICIES = {"q8_0": Q8_0, "q4_0": Q4_0}


def quantize_rows(w: np.ndarray, qtype: int) -> np.ndarray:
    """Rows of a float32 [N, K] matrix (K % 32 == 0) -> uint8 [N, K/32 * block bytes]
    GGUF blocks with quantize.py's steps: Q8_0 d = fp16(amax / 127), q = rne(x * (1/d));
    Q4_0 d = fp16(signed_max / -8), q = clip(rne(x / d) + 8, 0, 15), elements 0-15 in the
    low nibbles and 16-31 in the high ones."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    N, K = w.shape
    if K % 32:
        raise ValueError("rows must hold whole 32-element blocks")
    blk = w.reshape(-1, 32)
    nbk = blk.shape[0]
    if qtype == Q8_0:
        amax = np.abs(blk).max(axis=1)
        d = np.where(amax > 0, amax / np.float32(127.0), np.float32(0.0)).astype(np.float32)
        inv = (np.float32(1.0) / np.where(d != 0, d, np.float32(1.0))).astype(np.float32)
        q = np.clip(np.round(blk * inv[:, None]), -128, 127).astype(np.int8).view(np.uint8)
        out = np.empty((nbk, 34), np.uint8)
        out[:, :2] = d.astype(np.float16).view(np.uint8).reshape(nbk, 2)
        out[:, 2:] = q
    elif qtype == Q4_0:
        i = np.abs(blk).argmax(axis=1)
        smax = blk[np.arange(nbk), i]
        d = np.where(smax != 0, smax / np.float32(-8.0), np.float32(0.0)).astype(np.float32)
        safe = np.where(d != 0, d, np.float32(1.0)).astype(np.float32)
        q = np.where(d[:, None] != 0, np.clip(np.round(blk / safe[:, None]) + 8, 0, 15), 8).astype(np.uint8)
        out = np.empty((nbk, 18), np.uint8)
        out[:, :2] = d.astype(np.float16).view(np.uint8).reshape(nbk, 2)
        out[:, 2:] = (q[:, :16] & 0x0F) | ((q[:, 16:] & 0x0F) << 4)
    else:
        raise ValueError("qtype must be Q8_0 or Q4_0")
    return out.reshape(N, -1)


def _f32(t) -> np.ndarray:
    return t.detach().to("cpu").float().numpy()


def _need(cond: bool, what: str) -> None:
    if not cond:
        raise NotImplementedError(f"compile: {what}")


def llama_config_of(model, qtype: int, name: str | None = None) -> LlamaConfig:
    """The decoder hyper-parameters of a LlamaForCausalLM-shaped module."""
    c = model.config
    H = int(c.num_attention_heads)
    hd = int(getattr(c, "head_dim", None) or c.hidden_size // H)
    rs = getattr(c, "rope_scaling", None)
    _need(rs is None or (isinstance(rs, dict) and rs.get("rope_type", rs.get("type", "default")) == "default"),
          f"rope scaling {rs!r} (only the default rotary embedding)")
    _need(getattr(c, "partial_rotary_factor", 1.0) in (None, 1.0), "partial rotary embedding")
    sw = getattr(c, "sliding_window", None)
    _need(sw is None or getattr(c, "use_sliding_window", True) is False or sw >= c.max_position_embeddings,
          "sliding-window attention")
    rp = getattr(c, "rope_parameters", None)  # newer transformers keep rope_theta here
    theta = getattr(c, "rope_theta", None)
    if theta is None and isinstance(rp, dict):
        theta = rp.get("rope_theta")
    return LlamaConfig(name or getattr(c, "name_or_path", "") or "model", int(c.num_hidden_layers),
                       int(c.hidden_size), H, int(getattr(c, "num_key_value_heads", None) or H), hd,
                       int(c.intermediate_size), int(c.vocab_size), qtype,
                       tied_embeddings=bool(getattr(c, "tie_word_embeddings", False)),
                       rms_eps=float(c.rms_norm_eps), rope_base=float(theta if theta is not None else 10000.0))


def compile_llama(model, path: str | Path, quantize: str = "q8_0", max_pos: int | None = None,
                  name: str | None = None) -> Path:
    """Fuse, bake and quantize a LlamaForCausalLM-shaped module and write a ggmlc .gguf."""
    if quantize not in _POLICIES:
        raise ValueError(f"quantize must be one of {sorted(_POLICIES)}")
    qt = _POLICIES[quantize]
    cfg = llama_config_of(model, qt, name)
    body = model.model
    layers = []

    def biases(lins, what):
        """the fp32 biases of a fused group, concatenated like the rows (fusion.py:1347-1390)"""
        bs = [getattr(lin, "bias", None) for lin in lins]
        if all(b is None for b in bs):
            return None
        _need(all(b is not None for b in bs), f"{what}: biases on some projections of a fused group only")
        return np.concatenate([_f32(b) for b in bs]).astype(np.float32)

    for li, L in enumerate(body.layers):
        at, mlp = L.self_attn, L.mlp
        g1, g2 = _f32(L.input_layernorm.weight), _f32(L.post_attention_layernorm.weight)
        qkv = np.concatenate([_f32(at.q_proj.weight), _f32(at.k_proj.weight), _f32(at.v_proj.weight)], axis=0)
        gu = np.concatenate([_f32(mlp.gate_proj.weight), _f32(mlp.up_proj.weight)], axis=0)
        _need(qkv.shape == (cfg.q_dim + 2 * cfg.kv_dim, cfg.n_embd), f"layer {li}: q/k/v shapes")
        _need(gu.shape == (2 * cfg.n_ff, cfg.n_embd), f"layer {li}: gate/up shapes")
        # the RMS bake scales W's input columns only: a bias is added after the product
        layers.append((quantize_rows(qkv * g1[None, :], qt), quantize_rows(_f32(at.o_proj.weight), qt),
                       quantize_rows(gu * g2[None, :], qt), quantize_rows(_f32(mlp.down_proj.weight), qt),
                       biases((at.q_proj, at.k_proj, at.v_proj), f"layer {li} q/k/v"),
                       biases((at.o_proj,), f"layer {li} o"),
                       biases((mlp.gate_proj, mlp.up_proj), f"layer {li} gate/up"),
                       biases((mlp.down_proj,), f"layer {li} down")))
    cfg.qkv_bias = layers[0][4] is not None if layers else False
    _need(getattr(model.lm_head, "bias", None) is None, "an output head with a bias")
    emb = _f32(body.embed_tokens.weight)
    gf = _f32(body.norm.weight)
    embed_q = quantize_rows(emb, qt)
    head = _f32(model.lm_head.weight)
    tied = cfg.tied_embeddings or model.lm_head.weight.data_ptr() == body.embed_tokens.weight.data_ptr()
    if tied and np.all(gf == 1.0):
        lm_q = embed_q
    else:  # an exclusive head (or a tied one that needs the final gamma) gets its own baked copy
        lm_q = quantize_rows(head * gf[None, :], qt)
        tied = False
    cfg.tied_embeddings = tied
    if max_pos is None:
        max_pos = int(getattr(model.config, "max_position_embeddings", 4096))
    return write_llama_gguf(path, cfg, (embed_q, lm_q, layers), max_pos=max_pos)
