"""Seeded synthetic XTR-base-shaped models (no network, no real weights).

The reference loads `assets/xtr.gguf` converted from google/xtr-base-en
(downloadweights.py:13-46, tools/quantize-tool).  Those weights are not available
offline, so tests and benchmarks build random-init models of the same architecture
and tensor names (src/quantized_t5.rs:216-221,323-355,514-516,582-590,640-690):

  encoder.embed_tokens.weight                             [vocab, d_model]  F32 N(0,1)
  encoder.block.{i}.layer.0.SelfAttention.{q,k,v}.weight  [inner, d_model]  Q4_K N(0,0.02^2)
  encoder.block.{i}.layer.0.SelfAttention.o.weight        [d_model, inner]  Q4_K
  encoder.block.0.layer.0.SelfAttention.relative_attention_bias.weight [buckets, heads] F32
  encoder.block.{i}.layer.{0,1}.layer_norm.weight         [d_model]         F32
  encoder.block.{i}.layer.1.DenseReluDense.{wi_0,wi_1}.weight [d_ff, d_model] Q4_K
  encoder.block.{i}.layer.1.DenseReluDense.wo.weight      [d_model, d_ff]   Q4_K
  encoder.final_layer_norm.weight                         [d_model]         F32
  linear.weight                                           [128, d_model]    Q4_K

Q4_K tensors are quantized by `quantize.quantize_q4k`, the quantize tool's scale/min search.
The benchmark configurations keep the embedding table F32; `emb_format="q4k"` gives the
quantize tool's own layout (tools/quantize-tool/src/main.rs:17-22: every rank-2 tensor whose
second dimension is a multiple of 256 is Q4_K, the embedding table included).
`layout="hybrid"` stores q/k/v/o/wo as F32 (the `hybrid-dequant` feature's dense weights)
and keeps wi_0/wi_1/linear Q4_K.  Every tensor draws from its own generator
seeded by (seed, crc32(name)), so any subset is reproducible on any host.
"""
from __future__ import annotations

import json
import zlib

import numpy as np

from .gguf import GGML_F32, GGML_Q4_K, Tensor, write_gguf
from .quantize import quantize_q4k

XTR_BASE = {
    "vocab_size": 32128,
    "d_model": 768,
    "d_kv": 64,
    "d_ff": 2048,
    "num_layers": 12,
    "num_decoder_layers": 12,
    "num_heads": 12,
    "relative_attention_num_buckets": 32,
    "relative_attention_max_distance": 128,
    "dropout_rate": 0.1,
    "layer_norm_epsilon": 1e-6,
    "initializer_factor": 1.0,
    "feed_forward_proj": "gated-gelu",
    "tie_word_embeddings": False,
    "is_encoder_decoder": True,
    "pad_token_id": 0,
    "eos_token_id": 1,
    "decoder_start_token_id": 0,
    "proj_dim": 128,
}


def small_config(**over) -> dict:
    """A reduced T5 (same structure, small dims) for fast oracle-side tests."""
    cfg = dict(XTR_BASE)
    cfg.update(vocab_size=1000, d_model=256, d_ff=512, num_layers=2, num_heads=4)
    cfg.update(over)
    return cfg


def _rng(seed: int, name: str) -> np.random.Generator:
    return np.random.default_rng([seed, zlib.crc32(name.encode())])


def _normal(seed: int, name: str, shape, std: float) -> np.ndarray:
    return (_rng(seed, name).standard_normal(shape, dtype=np.float32) * np.float32(std)).astype(np.float32)


def make_model(cfg: dict = XTR_BASE, seed: int = 0, layout: str = "q4k", emb_format: str = "f32",
               norm_jitter: float = 0.1, bias_std: float | None = None,
               std_over: dict | None = None) -> bytes:
    """Build a GGUF image of a random-init encoder.

    layout: "q4k" (every linear Q4_K) or "hybrid" (q/k/v/o/wo F32, wi_0/wi_1/linear Q4_K).
    emb_format: "f32" or "q4k" for the embedding table.
    norm_jitter: RMSNorm weights are 1 + jitter * N(0,1) (0 gives the all-ones init).
    std_over: {name fragment: std} for the linears whose tensor name contains the fragment
    (default std 0.02), e.g. {"DenseReluDense.wo": 20.0} for a residual stream that grows
    by orders of magnitude in one FFN.
    """
    if layout not in ("q4k", "hybrid"):
        raise ValueError("layout must be 'q4k' or 'hybrid'")
    D, F, H, dk = cfg["d_model"], cfg["d_ff"], cfg["num_heads"], cfg["d_kv"]
    inner = H * dk
    V, NB, P = cfg["vocab_size"], cfg["relative_attention_num_buckets"], cfg.get("proj_dim", 128)
    gated = cfg.get("feed_forward_proj", "gated-gelu").startswith("gated")
    bias_std = bias_std if bias_std is not None else D ** -0.5
    ts: list[Tensor] = []

    def dense(name, rows, cols, quant: bool, std=0.02):
        for frag, v in (std_over or {}).items():
            if frag in name:
                std = v
        w = _normal(seed, name, (rows, cols), std)
        if quant:
            ts.append(Tensor(name, GGML_Q4_K, (rows, cols), quantize_q4k(w).tobytes()))
        else:
            ts.append(Tensor(name, GGML_F32, (rows, cols), w.tobytes()))

    def vec(name, n):
        v = np.ones(n, np.float32)
        if norm_jitter:
            v += _normal(seed, name, (n,), norm_jitter)
        ts.append(Tensor(name, GGML_F32, (n,), v.astype(np.float32).tobytes()))

    dense("encoder.embed_tokens.weight", V, D, emb_format == "q4k", std=1.0)
    q_attn = layout == "q4k"
    for i in range(cfg["num_layers"]):
        p = f"encoder.block.{i}.layer."
        for m in ("q", "k", "v"):
            dense(p + f"0.SelfAttention.{m}.weight", inner, D, q_attn)
        dense(p + "0.SelfAttention.o.weight", D, inner, q_attn)
        if i == 0:
            name = p + "0.SelfAttention.relative_attention_bias.weight"
            ts.append(Tensor(name, GGML_F32, (NB, H), _normal(seed, name, (NB, H), bias_std).tobytes()))
        vec(p + "0.layer_norm.weight", D)
        if gated:
            dense(p + "1.DenseReluDense.wi_0.weight", F, D, True)
            dense(p + "1.DenseReluDense.wi_1.weight", F, D, True)
        else:
            dense(p + "1.DenseReluDense.wi.weight", F, D, True)
        dense(p + "1.DenseReluDense.wo.weight", D, F, q_attn)
        vec(p + "1.layer_norm.weight", D)
    vec("encoder.final_layer_norm.weight", D)
    dense("linear.weight", P, D, True)
    return write_gguf(ts)


def config_json(cfg: dict = XTR_BASE) -> bytes:
    """config.json bytes as the reference's serde `Config` reads them (src/quantized_t5.rs:90-115)."""
    return json.dumps({k: v for k, v in cfg.items() if k != "proj_dim"}, indent=2).encode()


def ragged_batch(n_seqs: int, lo: int, hi: int, vocab: int, seed: int):
    """Token ids of a ragged batch: lengths uniform in [lo, hi], ids uniform in [1, vocab).

    Returns (ids uint32 [T], cu_seqlens int32 [n_seqs + 1])."""
    rng = np.random.default_rng(seed)
    lens = rng.integers(lo, hi + 1, size=n_seqs)
    cu = np.zeros(n_seqs + 1, np.int32)
    cu[1:] = np.cumsum(lens)
    ids = rng.integers(1, vocab, size=int(cu[-1])).astype(np.uint32)
    return ids, cu
