"""torch-CPU f32 restatement of the reference's default `t5-quantized` CPU encoder.

TEST INFRASTRUCTURE ONLY: imported by tests/ and by bench.py's cpu_baseline leg, never by the
witchcraft_amd product path.  It exists to time the reference's CPU numerics on a strong BLAS:
the C oracle (t5_oracle.c) is the parity checker and keeps float64 accumulation; this port runs
the same f32 algorithm through torch's multithreaded CPU GEMMs, as candle's `gemm` crate does
for the reference (src/quantized_t5.rs:39-49 dequantizes every Q4_K weight to f32 at load).

Per sequence, exactly as the reference runs it ([1, L], src/embedder.rs:40-41):
  embedding gather                                   src/quantized_t5.rs:659,687
  12 x T5Block                                       :598-627
    T5LayerNorm  x / sqrt(mean(x^2) + eps) * w       :162-173
    q, k, v; scores Q K^T (no 1/sqrt(d) scale)       :383-426
    + relative-position bias of block 0              :439-491
    softmax, . V, o projection, + residual           :496-501, fast_add :291
    T5LayerNorm, gelu_tanh(x W0^T) * (x W1^T) . Wo^T :231-252, + residual
  final T5LayerNorm, 768 -> 128 projection           :669, :698-701
Q4_K weights are dequantized by the C oracle's bit-exact dequantizer (orc.q4k_dequant).
"""
from __future__ import annotations

import numpy as np

from . import oracle as orc


def _read_tensors(gguf: bytes) -> dict:
    """name -> float32 array of every tensor of a GGUF image (Q4_K dequantized)."""
    import struct
    off = 4
    ver, n_t, n_kv = struct.unpack_from("<IQQ", gguf, off)
    off += 20
    if gguf[:4] != b"GGUF" or ver != 3 or n_kv:
        raise ValueError("expected a GGUF v3 image without metadata")
    infos = []
    for _ in range(n_t):
        (ln,) = struct.unpack_from("<Q", gguf, off)
        off += 8
        name = gguf[off:off + ln].decode()
        off += ln
        (nd,) = struct.unpack_from("<I", gguf, off)
        off += 4
        dims = struct.unpack_from(f"<{nd}Q", gguf, off)
        off += 8 * nd
        typ, toff = struct.unpack_from("<IQ", gguf, off)
        off += 12
        infos.append((name, tuple(reversed(dims)), typ, toff))
    base = (off + 31) // 32 * 32
    out = {}
    for name, shape, typ, toff in infos:
        ne = int(np.prod(shape))
        start = base + toff
        if typ == 0:
            a = np.frombuffer(gguf, np.float32, ne, start)
        elif typ == 1:
            a = np.frombuffer(gguf, np.float16, ne, start).astype(np.float32)
        elif typ == 12:
            a = orc.q4k_dequant(np.frombuffer(gguf, np.uint8, ne // 256 * 144, start))
        else:
            raise ValueError(f"{name}: unsupported GGML type {typ}")
        out[name] = a.reshape(shape).copy()
    return out


class TorchCpuEncoder:
    """The default CPU encoder in torch f32, one [1, L] sequence per call."""

    def __init__(self, gguf: bytes, cfg: dict, threads: int | None = None):
        import torch
        self.torch = torch
        if threads:
            torch.set_num_threads(int(threads))
        w = {k: torch.from_numpy(v) for k, v in _read_tensors(gguf).items()}
        self.cfg = cfg
        self.H, self.dk = cfg["num_heads"], cfg["d_kv"]
        self.eps = float(cfg["layer_norm_epsilon"])
        emb = "shared.weight" if "shared.weight" in w else "encoder.embed_tokens.weight"
        self.emb = w[emb]
        self.rel = w["encoder.block.0.layer.0.SelfAttention.relative_attention_bias.weight"]  # [buckets, H]
        self.layers = []
        for i in range(cfg["num_layers"]):
            p = f"encoder.block.{i}.layer."
            self.layers.append({
                "ln0": w[p + "0.layer_norm.weight"], "ln1": w[p + "1.layer_norm.weight"],
                "q": w[p + "0.SelfAttention.q.weight"], "k": w[p + "0.SelfAttention.k.weight"],
                "v": w[p + "0.SelfAttention.v.weight"], "o": w[p + "0.SelfAttention.o.weight"],
                "wi0": w[p + "1.DenseReluDense.wi_0.weight"], "wi1": w[p + "1.DenseReluDense.wi_1.weight"],
                "wo": w[p + "1.DenseReluDense.wo.weight"],
            })
        self.final_ln = w["encoder.final_layer_norm.weight"]
        self.proj = w["linear.weight"]
        self._bias_cache = {}

    def _bias(self, L: int):
        """[H, L, L] relative-position bias, buckets from the oracle's bucket function."""
        b = self._bias_cache.get(L)
        if b is None:
            nb, md = self.cfg["relative_attention_num_buckets"], self.cfg["relative_attention_max_distance"]
            bucket = np.empty((L, L), np.int64)
            by_delta = {}
            for i in range(L):
                for j in range(L):
                    d = j - i
                    if d not in by_delta:
                        by_delta[d] = orc.rel_bucket(i, j, nb, md)
                    bucket[i, j] = by_delta[d]
            b = self.rel[self.torch.from_numpy(bucket)].permute(2, 0, 1).contiguous()
            self._bias_cache[L] = b
        return b

    def _norm(self, x, w):
        var = (x * x).mean(-1, keepdim=True)
        return x / self.torch.sqrt(var + self.eps) * w

    def forward(self, ids: np.ndarray) -> np.ndarray:
        """[L] token ids -> [L, proj_dim] f32, un-normalised (T5EncoderModel::forward)."""
        torch = self.torch
        F = torch.nn.functional
        L = int(ids.size)
        with torch.inference_mode():
            x = self.emb[torch.from_numpy(np.asarray(ids, np.int64))]
            bias = self._bias(L)
            for ly in self.layers:
                h = self._norm(x, ly["ln0"])
                q = (h @ ly["q"].T).view(L, self.H, self.dk).transpose(0, 1)
                k = (h @ ly["k"].T).view(L, self.H, self.dk).transpose(0, 1)
                v = (h @ ly["v"].T).view(L, self.H, self.dk).transpose(0, 1)
                s = torch.matmul(q, k.transpose(1, 2)) + bias
                a = torch.matmul(torch.softmax(s, dim=-1), v).transpose(0, 1).reshape(L, self.H * self.dk)
                x = x + a @ ly["o"].T
                h = self._norm(x, ly["ln1"])
                g = F.gelu(h @ ly["wi0"].T, approximate="tanh") * (h @ ly["wi1"].T)
                x = x + g @ ly["wo"].T
            x = self._norm(x, self.final_ln)
            return (x @ self.proj.T).numpy()
