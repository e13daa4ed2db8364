"""ctypes front end of the CPU oracle (t5_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, as the checker -- never by the witchcraft_amd product path.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent

VARIANT_DEFAULT = 0       # t5-quantized CPU: Q4_K dequantized to f32 at load
VARIANT_HYBRID = 1        # hybrid-dequant: Q4_K x Q8_K wi_0/wi_1/linear, Pade gelu
VARIANT_HYBRID_BF16 = 2   # hybrid-dequant + fbgemm: bf16-truncated q/k/v/o/wo


class OrcConfig(C.Structure):
    _fields_ = [
        ("vocab_size", C.c_int32), ("d_model", C.c_int32), ("d_kv", C.c_int32),
        ("d_ff", C.c_int32), ("num_layers", C.c_int32), ("num_heads", C.c_int32),
        ("num_buckets", C.c_int32), ("max_distance", C.c_int32), ("eps", C.c_float),
        ("gated", C.c_int32), ("proj_dim", C.c_int32),
    ]


def _cpu_has_avx512() -> bool:
    try:
        flags = Path("/proc/cpuinfo").read_text()
    except OSError:
        return False
    return all(f in flags for f in ("avx512f", "avx512bw", "avx512vl", "avx512dq"))


def _load() -> C.CDLL:
    names = ["liboracle_v4.so", "liboracle_v3.so"] if _cpu_has_avx512() else ["liboracle_v3.so"]
    for n in names:
        p = _HERE / n
        if p.exists():
            lib = C.CDLL(str(p))
            break
    else:
        raise RuntimeError(f"oracle library not built in {_HERE} (run `make -C oracle`)")
    f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
    u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
    u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
    i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
    lib.orc_set_threads.argtypes = [C.c_int]
    lib.orc_max_threads.restype = C.c_int
    lib.orc_f16_to_f32.argtypes = [C.c_uint16]
    lib.orc_f16_to_f32.restype = C.c_float
    lib.orc_q4k_dequant.argtypes = [u8p, C.c_size_t, f32p]
    lib.orc_q8k_quantize.argtypes = [f32p, C.c_size_t, u8p]
    lib.orc_q4k_q8k_vec_dot.argtypes = [C.c_size_t, u8p, u8p]
    lib.orc_q4k_q8k_vec_dot.restype = C.c_float
    lib.orc_bf16_trunc.argtypes = [C.c_float]
    lib.orc_bf16_trunc.restype = C.c_float
    lib.orc_rel_bucket.argtypes = [C.c_uint32] * 4
    lib.orc_rel_bucket.restype = C.c_uint32
    for fn in ("orc_gelu_tanh", "orc_fast_tanh", "orc_gelu_pade"):
        getattr(lib, fn).argtypes = [C.c_float]
        getattr(lib, fn).restype = C.c_float
    lib.orc_rmsnorm.argtypes = [f32p, f32p, C.c_int, C.c_int, C.c_float, f32p, C.c_int]
    lib.orc_softmax_rows.argtypes = [f32p, C.c_int, C.c_int]
    lib.orc_linear.argtypes = [f32p, f32p, C.c_int, C.c_int, C.c_int, f32p, C.c_int]
    lib.orc_matmul_t.argtypes = [f32p, C.c_int, f32p, C.c_int, C.c_int, C.c_int, f32p, C.c_int]
    lib.orc_matmul_argmax.argtypes = [f32p, C.c_int, f32p, C.c_int, C.c_int, C.c_int,
                                      np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS"), C.c_int]
    lib.orc_model_from_gguf.argtypes = [u8p, C.c_size_t, C.POINTER(OrcConfig), C.c_int,
                                        C.c_char_p, C.c_size_t]
    lib.orc_model_from_gguf.restype = C.c_void_p
    lib.orc_model_free.argtypes = [C.c_void_p]
    lib.orc_encoder_forward.argtypes = [C.c_void_p, u32p, C.c_int, f32p, C.c_int]
    lib.orc_encoder_hidden.argtypes = [C.c_void_p, u32p, C.c_int, C.c_int, f32p, C.c_int]
    lib.orc_layer_forward.argtypes = [C.c_void_p, C.c_int, f32p, C.c_int, f32p, C.c_int]
    lib.orc_ffn_dense.argtypes = [C.c_void_p, C.c_int, f32p, C.c_int, f32p, C.c_int]
    lib.orc_final.argtypes = [C.c_void_p, f32p, C.c_int, f32p, C.c_int]
    lib.orc_position_bias.argtypes = [C.c_void_p, C.c_int, f32p]
    lib.orc_embed_ids.argtypes = [C.c_void_p, u32p, C.c_int, C.c_int, C.c_int, f32p, i32p, C.c_int]
    # embedding codecs (codec_oracle.c)
    lib.orc_compand_q4.argtypes = [C.c_float]
    lib.orc_compand_q4.restype = C.c_uint8
    lib.orc_q4_dequant_table.argtypes = [f32p]
    lib.orc_residual_encode.argtypes = [f32p, f32p, u32p, C.c_int, C.c_int, u8p]
    lib.orc_residual_decode.argtypes = [u8p, C.c_int, C.c_int, f32p, f32p]
    lib.orc_ladder_mismatches.argtypes = [f32p, C.POINTER(C.c_uint32)]
    lib.orc_ladder_mismatches.restype = C.c_uint64
    lib.orc_haar_forward.argtypes = [f32p, C.c_int]
    lib.orc_haar_inverse.argtypes = [f32p, C.c_int]
    lib.orc_scale_histogram.argtypes = [u32p, C.c_int, C.c_int,
                                        np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")]
    lib.orc_embeddings_to_packed.argtypes = [f32p, C.c_int, C.c_int, u8p, C.c_size_t]
    lib.orc_embeddings_to_packed.restype = C.c_long
    lib.orc_embeddings_from_packed.argtypes = [u8p, C.c_size_t, C.c_int, f32p, C.c_size_t]
    lib.orc_embeddings_from_packed.restype = C.c_long
    return lib


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        _lib = _load()
    return _lib


def set_threads(n: int) -> int:
    """Sets the OpenMP thread count of the oracle's parallel loops; returns the count they
    will use, as the OpenMP runtime reports it."""
    lib().orc_set_threads(int(n))
    return int(lib().orc_max_threads())


# ---- block codecs / scalar ops ------------------------------------------------------

def q4k_dequant(blocks: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(blocks, dtype=np.uint8).reshape(-1)
    assert b.size % 144 == 0
    n = b.size // 144
    out = np.empty(n * 256, np.float32)
    lib().orc_q4k_dequant(b, n, out)
    return out


def q8k_quantize(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    out = np.empty(x.size // 256 * 292, np.uint8)
    lib().orc_q8k_quantize(x, x.size, out)
    return out


def q4k_q8k_vec_dot(n: int, q4k: np.ndarray, q8k: np.ndarray) -> float:
    return float(lib().orc_q4k_q8k_vec_dot(n, np.ascontiguousarray(q4k, np.uint8).reshape(-1),
                                           np.ascontiguousarray(q8k, np.uint8).reshape(-1)))


def rel_bucket(i: int, j: int, num_buckets: int = 32, max_distance: int = 128) -> int:
    return int(lib().orc_rel_bucket(i, j, num_buckets, max_distance))


def gelu_tanh(x: float) -> float:
    return float(lib().orc_gelu_tanh(x))


def gelu_pade(x: float) -> float:
    return float(lib().orc_gelu_pade(x))


def fast_tanh(x: float) -> float:
    return float(lib().orc_fast_tanh(x))


def bf16_trunc(x: float) -> float:
    return float(lib().orc_bf16_trunc(x))


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float = 1e-6, acc64: bool = True) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    lib().orc_rmsnorm(x, np.ascontiguousarray(w, np.float32), x.shape[0], x.shape[1], eps, out, int(acc64))
    return out


def softmax_rows(s: np.ndarray) -> np.ndarray:
    s = np.array(s, np.float32, order="C")
    lib().orc_softmax_rows(s, s.shape[0], s.shape[1])
    return s


def linear(x: np.ndarray, w: np.ndarray, acc64: bool = True) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    y = np.empty((x.shape[0], w.shape[0]), np.float32)
    lib().orc_linear(x, w, x.shape[0], w.shape[0], x.shape[1], y, int(acc64))
    return y


# ---- model ------------------------------------------------------------------------

def matmul_t(a: np.ndarray, b: np.ndarray, bf16_b: bool = False, acc64: bool = True) -> np.ndarray:
    """C = A . B^T (src/fast_ops.rs:98-116); bf16_b truncates B first (fbgemm build)."""
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    c = np.empty((a.shape[0], b.shape[0]), np.float32)
    lib().orc_matmul_t(a, a.shape[0], b, b.shape[0], a.shape[1], int(bf16_b), c, int(acc64))
    return c


def matmul_argmax(a: np.ndarray, b: np.ndarray, bf16_b: bool = False, acc64: bool = True) -> np.ndarray:
    """First argmax_j of A[i] . B[j] per row (src/lib.rs:187-208)."""
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    out = np.empty(a.shape[0], np.uint32)
    lib().orc_matmul_argmax(a, a.shape[0], b, b.shape[0], a.shape[1], int(bf16_b), out, int(acc64))
    return out


def make_config(cfg: dict) -> OrcConfig:
    return OrcConfig(
        vocab_size=cfg["vocab_size"], d_model=cfg["d_model"], d_kv=cfg["d_kv"], d_ff=cfg["d_ff"],
        num_layers=cfg["num_layers"], num_heads=cfg["num_heads"],
        num_buckets=cfg["relative_attention_num_buckets"],
        max_distance=cfg.get("relative_attention_max_distance", 128),
        eps=cfg.get("layer_norm_epsilon", 1e-6),
        gated=1 if cfg.get("feed_forward_proj", "gated-gelu").startswith("gated") else 0,
        proj_dim=cfg.get("proj_dim", 128))


class OracleModel:
    """The reference encoder restated on the CPU, loaded from GGUF bytes."""

    def __init__(self, gguf: bytes, cfg: dict, variant: int = VARIANT_DEFAULT):
        self.cfg = dict(cfg)
        self._c = make_config(cfg)
        self._buf = np.frombuffer(gguf, np.uint8)
        err = C.create_string_buffer(512)
        h = lib().orc_model_from_gguf(np.ascontiguousarray(self._buf), self._buf.size,
                                      C.byref(self._c), variant, err, 512)
        if not h:
            raise ValueError(err.value.decode())
        self._h = h
        self.D = cfg["d_model"]
        self.P = cfg.get("proj_dim", 128)

    def close(self):
        if getattr(self, "_h", None):
            lib().orc_model_free(self._h)
            self._h = None

    __del__ = close

    def forward(self, ids: np.ndarray, acc64: bool = True) -> np.ndarray:
        """T5EncoderModel::forward on one [1, L] sequence -> [L, proj_dim] un-normalised."""
        ids = np.ascontiguousarray(ids, np.uint32).reshape(-1)
        out = np.empty((ids.size, self.P), np.float32)
        rc = lib().orc_encoder_forward(self._h, ids, ids.size, out, int(acc64))
        if rc:
            raise ValueError(f"oracle forward failed ({rc})")
        return out

    def hidden(self, ids: np.ndarray, upto: int, acc64: bool = True) -> np.ndarray:
        ids = np.ascontiguousarray(ids, np.uint32).reshape(-1)
        x = np.empty((ids.size, self.D), np.float32)
        rc = lib().orc_encoder_hidden(self._h, ids, ids.size, upto, x, int(acc64))
        if rc:
            raise ValueError(f"oracle hidden failed ({rc})")
        return x

    def layer(self, layer: int, x: np.ndarray, acc64: bool = True) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty_like(x)
        rc = lib().orc_layer_forward(self._h, layer, x, x.shape[0], y, int(acc64))
        if rc:
            raise ValueError(f"oracle layer failed ({rc})")
        return y

    def ffn(self, layer: int, x: np.ndarray, acc64: bool = True) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty_like(x)
        rc = lib().orc_ffn_dense(self._h, layer, x, x.shape[0], y, int(acc64))
        if rc:
            raise ValueError(f"oracle ffn failed ({rc})")
        return y

    def final(self, x: np.ndarray, acc64: bool = True) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty((x.shape[0], self.P), np.float32)
        lib().orc_final(self._h, x, x.shape[0], out, int(acc64))
        return out

    def position_bias(self, L: int) -> np.ndarray:
        H = self.cfg["num_heads"]
        b = np.empty((H, L, L), np.float32)
        lib().orc_position_bias(self._h, L, b)
        return b

    def embed_ids(self, ids: np.ndarray, max_len: int = 2048, stride: int = 256,
                  acc64: bool = True):
        """Embedder::embed after tokenisation -> (normalised [n_kept, P], kept indices)."""
        ids = np.ascontiguousarray(ids, np.uint32).reshape(-1)
        out = np.empty((ids.size, self.P), np.float32)
        kept = np.empty(ids.size, np.int32)
        nk = lib().orc_embed_ids(self._h, ids, ids.size, max_len, stride, out, kept, int(acc64))
        if nk < 0:
            raise ValueError("all token embeddings below minimum norm threshold")
        return out[:nk], kept[:nk]


# ---- embedding codecs (codec_oracle.c) -------------------------------------------------

def compand_q4(x: float) -> int:
    """compand().quantize(4) of one f32 value (packops.rs:136-162)."""
    return int(lib().orc_compand_q4(float(np.float32(x))))


def q4_dequant_table() -> np.ndarray:
    """make_q4_dequant_table (packops.rs:14-25)."""
    t = np.empty(16, np.float32)
    lib().orc_q4_dequant_table(t)
    return t


def residual_encode(emb: np.ndarray, centers: np.ndarray, assign: np.ndarray) -> np.ndarray:
    """residual.compand().quantize(4).to_q4_bytes() per row (src/lib.rs:1375-1376)."""
    emb = np.ascontiguousarray(emb, np.float32)
    N, D = emb.shape
    out = np.empty((N, D // 2), np.uint8)
    lib().orc_residual_encode(emb, np.ascontiguousarray(centers, np.float32),
                              np.ascontiguousarray(assign, np.uint32), N, D, out)
    return out


def residual_decode(codes: np.ndarray, D: int, table: np.ndarray | None = None) -> np.ndarray:
    """from_companded_q4_bytes (packops.rs:491-513)."""
    codes = np.ascontiguousarray(codes, np.uint8).reshape(-1)
    N = codes.size * 2 // D
    out = np.empty((N, D), np.float32)
    lib().orc_residual_decode(codes, N, D, q4_dequant_table() if table is None else
                              np.ascontiguousarray(table, np.float32), out)
    return out


def ladder_mismatches(thresholds: np.ndarray) -> tuple[int, int]:
    """Exhaustive check of a 15-step threshold ladder against compand_q4 (all 2^32 f32)."""
    bad = C.c_uint32(0)
    n = lib().orc_ladder_mismatches(np.ascontiguousarray(thresholds, np.float32), C.byref(bad))
    return int(n), int(bad.value)


def haar_forward(x: np.ndarray) -> np.ndarray:
    y = np.array(x, np.float32, copy=True)
    lib().orc_haar_forward(y, y.size)
    return y


def haar_inverse(x: np.ndarray) -> np.ndarray:
    y = np.array(x, np.float32, copy=True)
    lib().orc_haar_inverse(y, y.size)
    return y


def scale_histogram(counts: np.ndarray, log2_scale: int = 12) -> np.ndarray:
    c = np.ascontiguousarray(counts, np.uint32)
    out = np.empty(c.size, np.uint16)
    if lib().orc_scale_histogram(c, c.size, log2_scale, out):
        raise ValueError("scale_histogram: the reference asserts on this input")
    return out


def embeddings_to_packed(x: np.ndarray) -> bytes:
    """embeddings_to_packed (packops.rs:172-301)."""
    x = np.ascontiguousarray(x, np.float32)
    rows, cols = x.shape
    cap = 4 + (rows // 1024 + 1) * (cols + 2 + 4 * 65536 + 2 + 2 * 1024 * cols + 16)
    cap = min(cap, 4 + (rows // 1024 + 1) * (cols + 6 + 4 * 4096) + 2 * rows * cols + 64 * (rows // 1024 + 1))
    out = np.empty(cap, np.uint8)
    n = lib().orc_embeddings_to_packed(x, rows, cols, out, cap)
    if n == -2:
        out = np.empty(4 + (rows // 1024 + 1) * (cols + 6 + 4 * 65536 + 16) + 2 * rows * cols, np.uint8)
        n = lib().orc_embeddings_to_packed(x, rows, cols, out, out.size)
    if n < 0:
        raise ValueError("embeddings_to_packed failed (the reference errors or panics on this input)")
    return out[:n].tobytes()


def embeddings_from_packed(buf: bytes, cols: int = 128) -> np.ndarray:
    """embeddings_from_packed (packops.rs:303-438): rows L2-normalised."""
    b = np.frombuffer(buf, np.uint8).copy()
    if b.size < 4:
        raise ValueError("buffer too short")
    rows = int(np.frombuffer(buf[:4], np.uint32)[0])
    out = np.empty((rows, cols), np.float32)
    n = lib().orc_embeddings_from_packed(b, b.size, cols, out.reshape(-1) if rows else np.empty(1, np.float32), rows)
    if n < 0:
        raise ValueError("malformed packed embeddings")
    return out
