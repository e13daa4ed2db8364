"""Python face of the `t5-hip` backend, mirroring the reference's `t5_encoder` contract.

Reference interface (module aliased as `t5_encoder`, src/lib.rs:10-21; used by
src/embedder.rs:1,17-18,24-25,41):

    T5ModelBuilder::load(assets) -> (T5ModelBuilder, Tokenizer)     src/quantized_t5.rs:713-729
    T5ModelBuilder::build_encoder(&Device, assets) -> T5EncoderModel :731-749
    T5EncoderModel::forward(&Tensor[B, L] u32) -> Tensor[B, L, 128] :698-701 (un-normalised)
    T5EncoderModel::device() -> &Device                              :703-705
    Embedder::new(&Device, assets) / Embedder::embed(&str)          src/embedder.rs:16-103

Everything here calls libt5hip.so through ctypes; no numerics are done in Python.
"""
from __future__ import annotations

import ctypes as C
import json
from pathlib import Path

import numpy as np

from . import _lib
from ._lib import T5HConfig, T5HKernelStat, check, lib


def config_from_json(data: bytes | str | dict, max_seq_len: int = 2048) -> T5HConfig:
    """Parse config.json the way the reference's serde `Config` does (src/quantized_t5.rs:90-144).

    `feed_forward_proj`: "gated-gelu" -> gated NewGelu (candle
    deserialize_feed_forward_proj_activation, :105-106); "relu" -> T5DenseActDense."""
    d = data if isinstance(data, dict) else json.loads(data)
    for key in ("vocab_size", "d_model", "d_kv", "d_ff", "num_layers", "num_heads",
                "relative_attention_num_buckets", "layer_norm_epsilon"):
        if key not in d:
            raise ValueError(f"config.json: missing field `{key}`")
    ffp = d.get("feed_forward_proj", "relu")
    if ffp not in ("gated-gelu", "relu"):
        raise ValueError(f"config.json: unsupported feed_forward_proj {ffp!r}")
    c = T5HConfig()
    c.vocab_size = d["vocab_size"]
    c.d_model = d["d_model"]
    c.d_kv = d["d_kv"]
    c.d_ff = d["d_ff"]
    c.num_layers = d["num_layers"]
    c.num_heads = d["num_heads"]
    c.relative_attention_num_buckets = d["relative_attention_num_buckets"]
    c.relative_attention_max_distance = d.get("relative_attention_max_distance", 128)
    c.layer_norm_epsilon = d["layer_norm_epsilon"]
    c.feed_forward_gated = 1 if ffp == "gated-gelu" else 0
    c.proj_dim = d.get("proj_dim", 128)
    c.max_seq_len = max_seq_len
    return c


class T5EncoderModel:
    """A model handle on one GPU (owns its weights, workspace and HIP stream)."""

    def __init__(self, gguf: bytes, cfg: T5HConfig, hip_device: int = 0):
        self.cfg = cfg
        self._buf = np.frombuffer(gguf, np.uint8)
        h = C.c_void_p()
        check(lib.t5h_create(np.ascontiguousarray(self._buf), self._buf.size, C.byref(cfg),
                             hip_device, C.byref(h)))
        self._buf = None  # borrowed only during create
        self._h = h

    @classmethod
    def from_gguf(cls, gguf: bytes, cfg: dict | T5HConfig, hip_device: int = 0, max_seq_len: int = 2048):
        c = cfg if isinstance(cfg, T5HConfig) else config_from_json(cfg, max_seq_len)
        return cls(gguf, c, hip_device)

    def close(self) -> None:
        if getattr(self, "_h", None):
            lib.t5h_destroy(self._h)
            self._h = None

    def __del__(self):
        self.close()

    @property
    def handle(self) -> C.c_void_p:
        return self._h

    def device(self) -> str:
        """Inputs and outputs live on the host, as with the reference's CPU device."""
        return "cpu"

    # ---- encoding ----
    def forward(self, input_ids: np.ndarray) -> np.ndarray:
        """[B, L] u32 -> [B, L, proj] f32 un-normalised; each row is one full-length
        sequence, exactly as the reference treats a [B, L] input (no padding mask)."""
        ids = np.ascontiguousarray(input_ids, np.uint32)
        if ids.ndim != 2:
            raise ValueError("expected a [batch, seq_len] array of token ids")
        B, L = ids.shape
        cu = (np.arange(B + 1, dtype=np.int32) * L).astype(np.int32)
        out, _ = self.encode_packed(ids.reshape(-1), cu)
        return out.reshape(B, L, -1)

    def encode_packed(self, ids: np.ndarray, cu_seqlens: np.ndarray, normalize: bool = False):
        """Ragged batch: ids [T], cu_seqlens [B+1] -> (out [T, proj], norms [T])."""
        ids = np.ascontiguousarray(ids, np.uint32).reshape(-1)
        cu = np.ascontiguousarray(cu_seqlens, np.int32).reshape(-1)
        T = int(cu[-1]) if cu.size else 0
        out = np.empty((T, self.cfg.proj_dim), np.float32)
        norms = np.empty(T, np.float32)
        fn = lib.t5h_encode_normalized if normalize else lib.t5h_encode
        check(fn(self._h, ids, cu, cu.size - 1, out, norms.ctypes.data_as(C.c_void_p)))
        return out, norms

    def encode_device(self, d_ids: int, cu_seqlens: np.ndarray, d_out: int, d_norm: int | None = None):
        """Asynchronous encode of device-resident ids into device-resident outputs."""
        cu = np.ascontiguousarray(cu_seqlens, np.int32)
        check(lib.t5h_encode_device(self._h, C.c_void_p(d_ids), cu, cu.size - 1, C.c_void_p(d_out),
                                    C.c_void_p(d_norm) if d_norm else None))

    def encode_device_noalloc(self, d_ids: int, cu_seqlens: np.ndarray, d_out: int, d_norm: int | None = None):
        """encode_device on the library's fixed per-GPU scratch array: allocates nothing."""
        cu = np.ascontiguousarray(cu_seqlens, np.int32)
        check(lib.t5h_encode_device_noalloc(self._h, C.c_void_p(d_ids), cu, cu.size - 1, C.c_void_p(d_out),
                                            C.c_void_p(d_norm) if d_norm else None))

    def synchronize(self) -> None:
        check(lib.t5h_synchronize(self._h))

    def stream(self) -> int:
        return int(lib.t5h_stream(self._h) or 0)

    def embed_ids(self, ids: np.ndarray, max_len: int = 2048, stride: int = 256):
        """Embedder::embed on token ids (src/embedder.rs:27-101): -> ([n_kept, proj], kept)."""
        ids = np.ascontiguousarray(ids, np.uint32).reshape(-1)
        out = np.empty((ids.size, self.cfg.proj_dim), np.float32)
        kept = np.empty(ids.size, np.int32)
        nk = C.c_int32(0)
        check(lib.t5h_embed_ids(self._h, ids, ids.size, max_len, stride, out, kept, C.byref(nk)))
        return out[: nk.value], kept[: nk.value]

    def embed_batch(self, docs, max_len: int = 2048, stride: int = 256):
        """Embedder::embed on several token-id documents in one packed encode
        (src/embedder.rs:22-103 per document) -> [(rows [n_kept, proj], kept positions)]."""
        docs = [np.ascontiguousarray(d, np.uint32).reshape(-1) for d in docs]
        offs = np.zeros(len(docs) + 1, np.int32)
        offs[1:] = np.cumsum([d.size for d in docs])
        ids = np.concatenate(docs) if docs else np.zeros(0, np.uint32)
        out = np.empty((ids.size, self.cfg.proj_dim), np.float32)
        kept = np.empty(ids.size, np.int32)
        koff = np.zeros(len(docs) + 1, np.int32)
        check(lib.t5h_embed_batch(self._h, ids, offs, len(docs), max_len, stride, out, kept, koff))
        return [(out[koff[d]:koff[d + 1]], kept[koff[d]:koff[d + 1]]) for d in range(len(docs))]

    def set_numerics(self, mode: int) -> None:
        """T5H_NUMERICS_DEFAULT (t5-quantized), T5H_NUMERICS_HYBRID (hybrid-dequant: Q8_K x Q4_K
        integer dot products for wi_0 / wi_1 and the projection, Pade gelu) or
        T5H_NUMERICS_HYBRID_BF16 (hybrid-dequant + fbgemm: the same, with q/k/v/o/wo truncated to
        bf16)."""
        check(lib.t5h_set_numerics(self._h, int(mode)))

    # ---- test hooks ----
    def layer_forward(self, layer: int, x: np.ndarray, cu_seqlens: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        cu = np.ascontiguousarray(cu_seqlens, np.int32)
        y = np.empty_like(x)
        check(lib.t5h_layer_forward(self._h, layer, x, cu, cu.size - 1, y))
        return y

    def ffn_block(self, layer: int, x: np.ndarray, mode: int = 0) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty_like(x)
        check(lib.t5h_ffn_block(self._h, layer, x, x.shape[0], y, mode))
        return y

    # ---- profiling ----
    def set_profiling(self, on: bool) -> None:
        check(lib.t5h_set_profiling(self._h, 1 if on else 0))

    def kernel_stats(self) -> dict:
        arr = (T5HKernelStat * 32)()
        n = lib.t5h_kernel_stats(self._h, arr, 32)
        if n < 0:
            check(n)
        return {arr[i].name.decode(): dict(kind=i, launches=arr[i].launches, total_ms=arr[i].total_ms,
                                           flops=arr[i].flops, bytes=arr[i].bytes)
                for i in range(min(n, 32))}

    def replay_kernel(self, kind: int, reps: int = 20) -> float:
        """Average microseconds of `reps` back-to-back relaunches of kernel class `kind` (its
        kernel_stats()[name]["kind"]) from the last profiled forward."""
        us = C.c_double()
        check(lib.t5h_replay_kernel(self._h, kind, reps, C.byref(us)))
        return us.value


class T5ModelBuilder:
    """T5ModelBuilder::load / build_encoder (src/quantized_t5.rs:708-750)."""

    def __init__(self, config: T5HConfig):
        self.config = config

    @staticmethod
    def load(assets: str | Path):
        assets = Path(assets)
        try:
            cfg_bytes = (assets / "config.json").read_bytes()
        except OSError as e:
            raise FileNotFoundError("failed to get bytes for CONFIG") from e
        config = config_from_json(cfg_bytes)
        tokenizer = None
        tok = assets / "tokenizer.json"
        if tok.exists():
            from tokenizers import Tokenizer  # the reference's tokenizer, when assets carry one
            tokenizer = Tokenizer.from_file(str(tok))
        return T5ModelBuilder(config), tokenizer

    def build_encoder(self, device: int | str, assets: str | Path) -> T5EncoderModel:
        try:
            model_bytes = (Path(assets) / "xtr.gguf").read_bytes()
        except OSError as e:
            raise FileNotFoundError("failed to get bytes for MODEL") from e
        dev = device if isinstance(device, int) else 0
        return T5EncoderModel(model_bytes, self.config, dev)


def attention_work(cu_seqlens: np.ndarray, heads: int) -> np.ndarray:
    """The attention work list the encoder uploads for a batch: [n, 4] int32 items (sequence
    start, length, first query, head), one per workgroup of 64 queries (sequences of at most 128
    tokens) or 128 (longer ones), length 0 for the padding of the 8 per-XCD lists; item i runs
    on XCD i % 8.  Host only."""
    cu = np.ascontiguousarray(cu_seqlens, np.int32).reshape(-1)
    B = cu.size - 1
    cap = heads * (int(cu[-1]) // 64 + 2 * B + 8) + 8 * 64 + 64 if B > 0 else 64
    items = np.zeros(cap * 4, np.int32)
    n = C.c_int32(0)
    check(lib.t5h_attention_work(cu, B, heads, items, cap, C.byref(n)))
    return items[: 4 * n.value].reshape(-1, 4)


def q8k_quantize(x: np.ndarray, hip_device: int = 0) -> np.ndarray:
    """BlockQ8K::from_float on the GPU (src/fused_matmul.rs:36-41): f32 [rows, cols]
    (cols % 256 == 0) -> uint8 [rows, cols / 256 * 292]."""
    x = np.ascontiguousarray(x, np.float32)
    rows, cols = x.shape
    out = np.empty((rows, cols // 256 * 292), np.uint8)
    check(lib.t5h_q8k_quantize(hip_device, x, rows, cols, out))
    return out


def q4k_q8k_matmul(w: np.ndarray, x8: np.ndarray, K: int, hip_device: int = 0) -> np.ndarray:
    """out[t, n] = BlockQ4K::vec_dot(w[n], x8[t]) on the GPU: Q4_K rows [N, K/256*144] and
    Q8_K rows [T, K/256*292] -> f32 [T, N]."""
    w = np.ascontiguousarray(w, np.uint8).reshape(-1, K // 256 * 144)
    x8 = np.ascontiguousarray(x8, np.uint8).reshape(-1, K // 256 * 292)
    out = np.empty((x8.shape[0], w.shape[0]), np.float32)
    check(lib.t5h_q4k_q8k_matmul(hip_device, w, w.shape[0], x8, x8.shape[0], K, out))
    return out


class Embedder:
    """Embedder::new / embed (src/embedder.rs:10-103) over the HIP encoder."""

    MAX_LEN = 2048
    STRIDE = 256

    def __init__(self, device: int | str, assets: str | Path):
        builder, self.tokenizer = T5ModelBuilder.load(assets)
        self.model = builder.build_encoder(device, assets)

    def embed_ids(self, ids: np.ndarray):
        out, kept = self.model.embed_ids(ids, self.MAX_LEN, self.STRIDE)
        return out[None], kept

    def embed(self, text: str):
        if self.tokenizer is None:
            raise RuntimeError("assets carry no tokenizer.json")
        enc = self.tokenizer.encode(text, add_special_tokens=True)
        out, kept = self.embed_ids(np.asarray(enc.ids, np.uint32))
        offsets = [enc.offsets[i] for i in kept]
        return out, offsets
