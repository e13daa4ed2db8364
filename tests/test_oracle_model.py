"""Pins the oracle's encoder forward (CPU only).

- against HuggingFace transformers' T5EncoderModel run on the same dequantized weights
  (tests/golden/hf_t5_small.npz, written by tests/golden/make_hf_golden.py);
- against a brute-force float64 numpy restatement on a tiny model (materialised
  [H, L, L] bias, exact softmax), which catches dropped terms (bias, residual, norm
  weight, gating) that a smaller tolerance on real shapes would hide;
- the hybrid-dequant variants against the default path (the reference's own
  compare-backends threshold for vanilla vs hybrid is cosine >= 0.99,
  tools/compare-backends/src/main.rs:446).
"""
import hashlib
import json
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle as orc
from witchcraft_amd import gguf, synth

GOLDEN = Path(__file__).resolve().parent / "golden"


def cosine_rows(a, b):
    return (a * b).sum(1) / (np.linalg.norm(a, axis=1) * np.linalg.norm(b, axis=1))


@pytest.fixture(scope="module")
def hf_golden():
    z = np.load(GOLDEN / "hf_t5_small.npz")
    cfg = json.loads(str(z["config"]))
    img = synth.make_model(cfg, seed=int(z["seed"]))
    assert hashlib.sha256(img).hexdigest() == str(z["gguf_sha256"]), "synthetic model drifted"
    return z, cfg, img


def test_oracle_matches_hf_t5(hf_golden):
    z, cfg, img = hf_golden
    m = orc.OracleModel(img, cfg)
    cu, ids = z["cu_seqlens"], z["ids"]
    for b in range(len(cu) - 1):
        got = m.forward(ids[cu[b]:cu[b + 1]])
        ref = z["out"][cu[b]:cu[b + 1]]
        assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max()
        assert cosine_rows(got, ref).min() > 0.999999


def test_oracle_hidden_states_match_hf(hf_golden):
    z, cfg, img = hf_golden
    m = orc.OracleModel(img, cfg)
    cu, ids = z["cu_seqlens"], z["ids"]
    seq = ids[cu[1]:cu[2]]
    for layer in range(cfg["num_layers"]):
        h = m.hidden(seq, layer)
        ref = z["hidden_seq1"][layer]
        assert np.abs(h - ref).max() <= 1e-5 * np.abs(ref).max()


def _deq(t):
    if t.ggml_type == gguf.GGML_Q4_K:
        return orc.q4k_dequant(np.frombuffer(t.data, np.uint8)).reshape(t.shape).astype(np.float64)
    return np.frombuffer(t.data, np.float32).reshape(t.shape).astype(np.float64)


def brute_force_forward(img: bytes, cfg: dict, ids: np.ndarray) -> np.ndarray:
    """Float64 restatement of src/quantized_t5.rs:598-701 with everything materialised."""
    ts = gguf.read_gguf(img)
    W = {k: _deq(v) for k, v in ts.items()}
    H, dk, eps = cfg["num_heads"], cfg["d_kv"], cfg["layer_norm_epsilon"]
    L = ids.size

    def norm(x, w):
        return x / np.sqrt((x * x).mean(1, keepdims=True) + eps) * w

    rb = W["encoder.block.0.layer.0.SelfAttention.relative_attention_bias.weight"]
    bias = np.empty((H, L, L))
    for i in range(L):
        for j in range(L):
            bias[:, i, j] = rb[orc.rel_bucket(i, j, cfg["relative_attention_num_buckets"],
                                              cfg["relative_attention_max_distance"])]
    x = W["encoder.embed_tokens.weight"][ids]
    for l in range(cfg["num_layers"]):
        p = f"encoder.block.{l}.layer."
        xn = norm(x, W[p + "0.layer_norm.weight"])
        q = xn @ W[p + "0.SelfAttention.q.weight"].T
        k = xn @ W[p + "0.SelfAttention.k.weight"].T
        v = xn @ W[p + "0.SelfAttention.v.weight"].T
        o = np.empty_like(q)
        for h in range(H):
            sl = slice(h * dk, (h + 1) * dk)
            s = q[:, sl] @ k[:, sl].T + bias[h]
            s = np.exp(s - s.max(1, keepdims=True))
            o[:, sl] = (s / s.sum(1, keepdims=True)) @ v[:, sl]
        x = x + o @ W[p + "0.SelfAttention.o.weight"].T
        xn = norm(x, W[p + "1.layer_norm.weight"])
        g = xn @ W[p + "1.DenseReluDense.wi_0.weight"].T
        u = xn @ W[p + "1.DenseReluDense.wi_1.weight"].T
        gelu = 0.5 * g * (1 + np.tanh(np.sqrt(2 / np.pi) * (g + 0.044715 * g ** 3)))
        x = x + (gelu * u) @ W[p + "1.DenseReluDense.wo.weight"].T
    x = norm(x, W["encoder.final_layer_norm.weight"])
    return x @ W["linear.weight"].T


def test_oracle_matches_float64_brute_force():
    cfg = synth.small_config(vocab_size=300, d_model=256, d_ff=256, num_layers=2, num_heads=4)
    img = synth.make_model(cfg, seed=11, norm_jitter=0.3, bias_std=0.5)
    m = orc.OracleModel(img, cfg)
    ids = np.random.default_rng(2).integers(1, 300, size=70).astype(np.uint32)
    got = m.forward(ids).astype(np.float64)
    ref = brute_force_forward(img, cfg, ids)
    assert np.abs(got - ref).max() <= 2e-6 * np.abs(ref).max()


def test_layer_and_ffn_hooks_consistent():
    cfg = synth.small_config()
    img = synth.make_model(cfg, seed=3)
    m = orc.OracleModel(img, cfg)
    ids = np.random.default_rng(4).integers(1, cfg["vocab_size"], size=33).astype(np.uint32)
    x0 = m.hidden(ids, 0)
    x1 = m.layer(0, x0)
    assert np.allclose(x1, m.hidden(ids, 1), rtol=0, atol=1e-6)
    x2 = m.layer(1, x1)
    assert np.allclose(m.final(x2), m.forward(ids), rtol=0, atol=1e-5)
    # the FFN hook is T5DenseGatedActDense alone: no norm, no residual
    ts = gguf.read_gguf(img)
    xin = np.random.default_rng(5).standard_normal((16, cfg["d_model"])).astype(np.float32)
    W0, W1, Wo = (_deq(ts[f"encoder.block.0.layer.1.DenseReluDense.{n}.weight"]) for n in ("wi_0", "wi_1", "wo"))
    g, u = xin @ W0.T, xin @ W1.T
    ref = (0.5 * g * (1 + np.tanh(np.sqrt(2 / np.pi) * (g + 0.044715 * g ** 3))) * u) @ Wo.T
    assert np.allclose(m.ffn(0, xin), ref, rtol=1e-5, atol=1e-5)


def test_hybrid_variants_close_to_default():
    cfg = synth.small_config()
    img = synth.make_model(cfg, seed=8)
    ids = np.random.default_rng(9).integers(1, cfg["vocab_size"], size=48).astype(np.uint32)
    ref = orc.OracleModel(img, cfg).forward(ids)
    for variant in (orc.VARIANT_HYBRID, orc.VARIANT_HYBRID_BF16):
        got = orc.OracleModel(img, cfg, variant).forward(ids)
        assert cosine_rows(got, ref).min() >= 0.99
        assert not np.array_equal(got, ref)


def test_embedder_windows_and_filter():
    cfg = synth.small_config()
    img = synth.make_model(cfg, seed=12)
    m = orc.OracleModel(img, cfg)
    ids = np.random.default_rng(13).integers(1, cfg["vocab_size"], size=150).astype(np.uint32)
    # one window: equals normalised forward rows with norm >= 1
    out, kept = m.embed_ids(ids, max_len=2048, stride=256)
    full = m.forward(ids)
    n = np.linalg.norm(full, axis=1)
    assert np.array_equal(kept, np.nonzero(n >= 1.0)[0])
    assert np.allclose(out, full[kept] / n[kept, None], atol=1e-6)
    # overlapping windows: [0,64), [48,112), [96,150) -> overlaps summed
    out2, kept2 = m.embed_ids(ids, max_len=64, stride=16)
    acc = np.zeros_like(full)
    for s, e in [(0, 64), (48, 112), (96, 150)]:
        acc[s:e] += m.forward(ids[s:e])
    n2 = np.linalg.norm(acc, axis=1)
    assert np.array_equal(kept2, np.nonzero(n2 >= 1.0)[0])
    assert np.allclose(out2, acc[kept2] / n2[kept2, None], atol=1e-5)


def test_missing_tensor_is_an_error():
    cfg = synth.small_config()
    ts = gguf.read_gguf(synth.make_model(cfg, seed=1))
    del ts["encoder.final_layer_norm.weight"]
    with pytest.raises(ValueError, match="missing tensor"):
        orc.OracleModel(gguf.write_gguf(list(ts.values())), cfg)


def test_torch_cpu_port_matches_oracle():
    """The torch-CPU f32 restatement that bench.py times as the strong-BLAS CPU baseline computes
    the same encoder as the C oracle (float64 accumulation): f32 rounding only."""
    from oracle.torch_port import TorchCpuEncoder
    cfg = synth.small_config()
    img = synth.make_model(cfg, seed=17)
    port = TorchCpuEncoder(img, cfg, threads=2)
    ora = orc.OracleModel(img, cfg)
    for L in (1, 37, 200):
        ids = np.random.default_rng(L).integers(1, cfg["vocab_size"], size=L).astype(np.uint32)
        a, b = port.forward(ids), ora.forward(ids)
        assert a.shape == b.shape == (L, 128)
        assert np.linalg.norm(a - b) / np.linalg.norm(b) <= 1e-5, L
    ora.close()
