"""Embedding codecs next to the encoder, on the GPU.

Mirrors the reference's ``TensorPackOps`` helpers (src/packops.rs) that Witchcraft applies to
encoder output:
  * ``make_q4_dequant_table()``                 -- packops.rs:14-25
  * ``residual_to_q4_bytes(emb, centers, assign)`` -- ``(emb[i] - center).compand()?.quantize(4)?
    .to_q4_bytes()`` at index build (src/lib.rs:1375-1376), for all rows at once
  * ``from_companded_q4_bytes(codes, cols)``    -- packops.rs:491-513 (search, src/lib.rs:676)
  * ``matmul_t_q4(query, codes)``               -- ``matmul_t(query, from_companded_q4_bytes(..))``
    (src/lib.rs:676-680,734-735) without materialising the f32 residuals
Everything runs in libt5hip.so; there is no CPU fallback.  Shape errors raise ValueError.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._lib import check, lib


def make_q4_dequant_table() -> np.ndarray:
    """The f32 value of each 4-bit residual code (packops.rs:14-25)."""
    t = np.empty(16, np.float32)
    check(lib.t5h_q4_dequant_table(t))
    return t


def q4_compand_thresholds() -> np.ndarray:
    """The 15 exact decision thresholds of compand().quantize(4) the GPU encoder compares against."""
    t = np.empty(15, np.float32)
    check(lib.t5h_q4_compand_thresholds(t))
    return t


def residual_to_q4_bytes(emb: np.ndarray, centers: np.ndarray, assign: np.ndarray,
                         hip_device: int = 0) -> np.ndarray:
    """codes[i] = to_q4_bytes(compand(emb[i] - centers[assign[i]]).quantize(4)), [N, D/2] u8."""
    emb = np.ascontiguousarray(emb, np.float32)
    centers = np.ascontiguousarray(centers, np.float32)
    assign = np.ascontiguousarray(assign, np.uint32)
    if emb.ndim != 2 or centers.ndim != 2 or emb.shape[1] != centers.shape[1] or assign.shape != (emb.shape[0],):
        raise ValueError(f"shapes emb {emb.shape}, centers {centers.shape}, assign {assign.shape} do not match")
    n, d = emb.shape
    out = np.empty((n, d // 2), np.uint8)
    check(lib.t5h_residual_encode(hip_device, emb, n, centers, centers.shape[0], assign, d, out))
    return out


def from_companded_q4_bytes(codes: np.ndarray, cols: int, hip_device: int = 0) -> np.ndarray:
    """Decode [N, cols/2] codes to [N, cols] f32 (packops.rs:491-513)."""
    codes = np.ascontiguousarray(codes, np.uint8).reshape(-1)
    if cols <= 0 or (codes.size * 2) % cols:
        raise ValueError(f"{codes.size} code bytes do not hold rows of {cols} values")
    n = codes.size * 2 // cols
    out = np.empty((n, cols), np.float32)
    check(lib.t5h_residual_decode(hip_device, codes, n, cols, out))
    return out


def matmul_t_q4(a: np.ndarray, codes: np.ndarray, hip_device: int = 0) -> np.ndarray:
    """C[M, N] = A[M, D] . from_companded_q4_bytes(codes[N, D/2])^T in f32."""
    a = np.ascontiguousarray(a, np.float32)
    codes = np.ascontiguousarray(codes, np.uint8)
    if a.ndim != 2 or codes.ndim != 2 or codes.shape[1] * 2 != a.shape[1]:
        raise ValueError(f"matmul_t_q4 shape mismatch: a {a.shape}, codes {codes.shape}")
    m, d = a.shape
    n = codes.shape[0]
    c = np.empty((m, n), np.float32)
    check(lib.t5h_matmul_t_q4(hip_device, a, m, codes, n, d, c))
    return c


def matmul_t_q4_device(d_a: int, m: int, d_codes: int, n: int, d: int, d_c: int, stream: int = 0) -> None:
    """Device-pointer form of matmul_t_q4, enqueued on `stream` (a hipStream_t as int)."""
    check(lib.t5h_matmul_t_q4_device(d_a, m, d_codes, n, d, d_c, stream or None))


def residual_encode_device(d_emb: int, n: int, d_centers: int, k: int, d_assign: int, d: int, d_codes: int,
                           d_bad: int, stream: int = 0) -> None:
    """Device-pointer form of residual_to_q4_bytes; rows assigned past k set *d_bad."""
    check(lib.t5h_residual_encode_device(d_emb, n, d_centers, k, d_assign, d, d_codes, d_bad, stream or None))


# ---- packed chunk embeddings (src/packops.rs:172-438) ------------------------------------

def _rows_of(mats) -> tuple[np.ndarray, np.ndarray, int]:
    mats = [np.ascontiguousarray(m, np.float32) for m in mats]
    cols = mats[0].shape[1] if mats else 128
    for m in mats:
        if m.ndim != 2 or m.shape[1] != cols:
            raise ValueError("every matrix must be 2-D with the same column count")
    ro = np.zeros(len(mats) + 1, np.int32)
    ro[1:] = np.cumsum([m.shape[0] for m in mats])
    x = np.concatenate(mats, 0) if mats and ro[-1] > 0 else np.zeros((1, cols), np.float32)
    return x, ro, cols


def embeddings_to_packed_batch(mats, hip_device: int = 0, timing: bool = False):
    """embeddings_to_packed of each [rows, cols] matrix (src/packops.rs:172-301), in one
    batch on the GPU.  Returns the list of packed byte strings (and the device ms if timing)."""
    x, ro, cols = _rows_of(mats)
    B = len(ro) - 1
    offs = np.zeros(B + 1, np.uint64)
    cap = int(4 * B + (int(ro[-1]) // 1024 + B + 1) * (cols + 4 + 4 * 4096) + 2 * int(ro[-1]) * cols + 64)
    out = np.empty(max(cap, 1), np.uint8)
    ms = C.c_double(0.0)
    check(lib.t5h_embeddings_to_packed(hip_device, x, ro, B, cols, out, cap, offs, C.byref(ms)))
    res = [out[int(offs[b]):int(offs[b + 1])].tobytes() for b in range(B)]
    return (res, ms.value) if timing else res


def embeddings_to_packed(x: np.ndarray, hip_device: int = 0) -> bytes:
    """TensorPackOps::embeddings_to_packed of one [rows, cols] matrix."""
    return embeddings_to_packed_batch([x], hip_device)[0]


def embeddings_from_packed_batch(bufs, cols: int = 128, hip_device: int = 0, timing: bool = False):
    """embeddings_from_packed of each packed buffer (src/packops.rs:303-438): rows
    L2-normalised.  Returns the list of [rows, cols] f32 arrays (and the device ms if timing)."""
    B = len(bufs)
    offs = np.zeros(B + 1, np.uint64)
    offs[1:] = np.cumsum([len(b) for b in bufs])
    buf = np.frombuffer(b"".join(bufs), np.uint8).copy() if offs[-1] else np.zeros(1, np.uint8)
    rows = 0
    for b in bufs:
        if len(b) >= 4:
            rows += int(np.frombuffer(b[:4], np.uint32)[0])
    out = np.empty((max(rows, 1), cols), np.float32)
    ro = np.zeros(B + 1, np.int32)
    ms = C.c_double(0.0)
    check(lib.t5h_embeddings_from_packed(hip_device, buf, offs, B, cols, out, rows, ro, C.byref(ms)))
    res = [out[ro[b]:ro[b + 1]].copy() for b in range(B)]
    return (res, ms.value) if timing else res


def embeddings_from_packed(buf: bytes, cols: int = 128, hip_device: int = 0) -> np.ndarray:
    """TensorPackOps::embeddings_from_packed of one packed buffer."""
    return embeddings_from_packed_batch([buf], cols, hip_device)[0]
