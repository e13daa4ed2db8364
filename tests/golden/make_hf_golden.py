"""Writes tests/golden/hf_t5_small.npz: an independent check of the CPU oracle.

HuggingFace `transformers` T5EncoderModel (local T5Config, never `from_pretrained`) is
loaded with the dequantized weights of a seeded small synthetic model (witchcraft_amd.synth)
and run on a few sequences one at a time, as the reference's Embedder runs them
(src/embedder.rs:40-41).  The reference itself is Rust + candle and cannot run here; HF's
T5 is the published implementation candle's T5 follows (src/quantized_t5.rs:16).

Q4_K tensors are dequantized here by a vectorised numpy restatement of the GGML block
closed form, independent of oracle/t5_oracle.c.

Stored: config, seed, sha256 of the GGUF image (the test regenerates the model and
checks it is byte-identical), token ids, per-sequence projected outputs [L, 128],
hidden states entering each block for one sequence, and HF's bucket table.

Run:  python tests/golden/make_hf_golden.py
"""
from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from witchcraft_amd import gguf, synth  # noqa: E402

SEED = 1234
CFG = synth.small_config(vocab_size=512, d_model=256, d_ff=512, num_layers=2, num_heads=4)
LENGTHS = [9, 40, 100]


def dequant_q4k_np(raw: bytes, rows: int, cols: int) -> np.ndarray:
    b = np.frombuffer(raw, np.uint8).reshape(-1, 144)
    d = b[:, 0:2].copy().view(np.float16).astype(np.float32)[:, 0]
    dmin = b[:, 2:4].copy().view(np.float16).astype(np.float32)[:, 0]
    s = b[:, 4:16].astype(np.int32)
    sc = np.empty((b.shape[0], 8), np.int32)
    mn = np.empty((b.shape[0], 8), np.int32)
    sc[:, :4] = s[:, 0:4] & 63
    mn[:, :4] = s[:, 4:8] & 63
    sc[:, 4:] = (s[:, 8:12] & 15) | ((s[:, 0:4] >> 6) << 4)
    mn[:, 4:] = (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)
    qs = b[:, 16:].reshape(-1, 4, 32)
    q = np.empty((b.shape[0], 8, 32), np.float32)
    q[:, 0::2, :] = qs & 15
    q[:, 1::2, :] = qs >> 4
    scale = (d[:, None] * sc.astype(np.float32)).astype(np.float32)
    off = (dmin[:, None] * mn.astype(np.float32)).astype(np.float32)
    y = (scale[:, :, None] * q - off[:, :, None]).astype(np.float32)
    return y.reshape(rows, cols)


def tensor_f32(t: gguf.Tensor) -> np.ndarray:
    if t.ggml_type == gguf.GGML_Q4_K:
        return dequant_q4k_np(t.data, t.shape[0], t.shape[1])
    return np.frombuffer(t.data, np.float32).reshape(t.shape).copy()


def main() -> None:
    import torch
    from transformers import T5Config, T5EncoderModel
    from transformers.models.t5.modeling_t5 import T5Attention

    img = synth.make_model(CFG, seed=SEED)
    sha = hashlib.sha256(img).hexdigest()
    ts = gguf.read_gguf(img)
    hf_cfg = T5Config(
        vocab_size=CFG["vocab_size"], d_model=CFG["d_model"], d_kv=CFG["d_kv"], d_ff=CFG["d_ff"],
        num_layers=CFG["num_layers"], num_heads=CFG["num_heads"],
        relative_attention_num_buckets=CFG["relative_attention_num_buckets"],
        relative_attention_max_distance=CFG["relative_attention_max_distance"],
        dropout_rate=0.0, layer_norm_epsilon=CFG["layer_norm_epsilon"],
        feed_forward_proj="gated-gelu", is_encoder_decoder=False, use_cache=False)
    model = T5EncoderModel(hf_cfg).eval().float()
    sd = model.state_dict()
    new_sd = {}
    for k in sd:
        src = "encoder.embed_tokens.weight" if k in ("shared.weight", "encoder.embed_tokens.weight") else k
        if src not in ts:
            raise KeyError(f"no tensor for {k}")
        new_sd[k] = torch.from_numpy(tensor_f32(ts[src]).reshape(sd[k].shape))
    model.load_state_dict(new_sd)
    proj = tensor_f32(ts["linear.weight"]).astype(np.float64)

    rng = np.random.default_rng(SEED + 1)
    ids_all, cu, outs = [], [0], []
    hidden = None
    with torch.no_grad():
        for n, L in enumerate(LENGTHS):
            ids = rng.integers(1, CFG["vocab_size"], size=L).astype(np.uint32)
            r = model(input_ids=torch.from_numpy(ids.astype(np.int64))[None], output_hidden_states=True)
            last = r.last_hidden_state[0].double().numpy()
            outs.append((last @ proj.T).astype(np.float32))
            ids_all.append(ids)
            cu.append(cu[-1] + L)
            if n == 1:
                hidden = np.stack([h[0].numpy() for h in r.hidden_states[:-1]]).astype(np.float32)
        rp = torch.arange(-2047, 2048)[None, :]
        buckets = T5Attention._relative_position_bucket(
            rp, bidirectional=True, num_buckets=CFG["relative_attention_num_buckets"],
            max_distance=CFG["relative_attention_max_distance"]).numpy()[0].astype(np.int32)
    out_path = Path(__file__).resolve().parent / "hf_t5_small.npz"
    np.savez_compressed(
        out_path, config=json.dumps(CFG), seed=SEED, gguf_sha256=sha,
        ids=np.concatenate(ids_all), cu_seqlens=np.array(cu, np.int32),
        out=np.concatenate(outs), hidden_seq1=hidden, hf_buckets_by_delta=buckets)
    print(f"wrote {out_path} ({out_path.stat().st_size} bytes), gguf sha256 {sha}")


if __name__ == "__main__":
    main()
