"""Query-side scoring on the GPU, next to the encoder.

Mirrors the reference's CPU scoring helpers:
  * ``matmul_t(a, b)``            -- fast_ops::matmul_t (src/fast_ops.rs:98-116): [M,D] x [N,D]^T
  * ``PackedRight(b).matmul(a)``  -- fast_ops::PackedRight (src/fast_ops.rs:65-95): B kept
    resident (here: in HBM) and reused against many A
  * ``matmul_argmax(a, b)``       -- matmul_argmax_batched (src/lib.rs:187-208): per-row argmax
    of A . B^T, first index on ties (k-means assignment, src/lib.rs:235,1330)

``bf16_b=True`` reproduces the fbgemm build, which truncates B to bf16 before the product
(PackedMatrixBf16::from_transposed, fbgemm-rs/src/bf16.rs:21-31); the default is the f32
candle product.  Everything runs in libt5hip.so; there is no CPU fallback.
Argument checks raise ValueError like the reference's dimension bail (src/fast_ops.rs:104-106).
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._lib import check, lib


def _as_2d_f32(x: np.ndarray, name: str) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    if x.ndim != 2:
        raise ValueError(f"{name} must be 2-D, got shape {x.shape}")
    return x


def _dims(a: np.ndarray, b: np.ndarray) -> tuple[int, int, int]:
    m, d = a.shape
    n, d2 = b.shape
    if d != d2:
        raise ValueError(f"matmul_t dimension mismatch: a is [{m},{d}], b is [{n},{d2}]")
    return m, n, d


def matmul_t(a: np.ndarray, b: np.ndarray, bf16_b: bool = False, hip_device: int = 0) -> np.ndarray:
    """C[M,N] = A[M,D] . B[N,D]^T in f32 on the GPU (host arrays in and out)."""
    a = _as_2d_f32(a, "a")
    b = _as_2d_f32(b, "b")
    m, n, d = _dims(a, b)
    c = np.empty((m, n), np.float32)
    check(lib.t5h_matmul_t(hip_device, a, m, b, n, d, int(bf16_b), c))
    return c


def matmul_argmax(a: np.ndarray, b: np.ndarray, bf16_b: bool = False, hip_device: int = 0) -> np.ndarray:
    """out[i] = argmax_j A[i] . B[j] as u32, smallest j on ties; no [M,N] intermediate."""
    a = _as_2d_f32(a, "a")
    b = _as_2d_f32(b, "b")
    m, n, d = _dims(a, b)
    out = np.empty(m, np.uint32)
    check(lib.t5h_matmul_argmax(hip_device, a, m, b, n, d, int(bf16_b), out))
    return out


def matmul_t_device(d_a: int, m: int, d_b: int, n: int, d: int, d_c: int, bf16_b: bool = False,
                    stream: int = 0) -> None:
    """Asynchronous C = A . B^T on device buffers (raw device addresses) on `stream`."""
    check(lib.t5h_matmul_t_device(C.c_void_p(d_a), m, C.c_void_p(d_b), n, d, int(bf16_b), C.c_void_p(d_c),
                                  C.c_void_p(stream) if stream else None))


def matmul_argmax_device(d_a: int, m: int, d_b: int, n: int, d: int, d_out: int, bf16_b: bool = False,
                         stream: int = 0) -> None:
    """Asynchronous per-row argmax of A . B^T on device buffers on `stream`."""
    check(lib.t5h_matmul_argmax_device(C.c_void_p(d_a), m, C.c_void_p(d_b), n, d, int(bf16_b),
                                       C.c_void_p(d_out), C.c_void_p(stream) if stream else None))


class PackedRight:
    """B[N,D] uploaded once and kept in HBM, for repeated A . B^T (src/fast_ops.rs:55-95).

    Device memory comes from torch (plumbing only: the products run in libt5hip.so).
    """

    def __init__(self, b: np.ndarray, bf16_b: bool = False, device: str = "cuda:0"):
        import torch

        b = _as_2d_f32(b, "b")
        self.n, self.d = b.shape
        self.bf16_b = bool(bf16_b)
        self._torch = torch
        self._dev = torch.device(device)
        self._b = torch.from_numpy(b).to(self._dev)

    def _upload(self, a: np.ndarray):
        a = _as_2d_f32(a, "a")
        _dims(a, np.empty((self.n, self.d), np.float32))
        return self._torch.from_numpy(a).to(self._dev)

    def _stream(self) -> int:
        return int(self._torch.cuda.current_stream(self._dev).cuda_stream)

    def matmul(self, a: np.ndarray) -> np.ndarray:
        """[M,D] -> [M,N] = A . B^T."""
        da = self._upload(a)
        m = da.shape[0]
        dc = self._torch.empty((m, self.n), dtype=self._torch.float32, device=self._dev)
        if m:
            matmul_t_device(da.data_ptr(), m, self._b.data_ptr(), self.n, self.d, dc.data_ptr(), self.bf16_b,
                            self._stream())
        return dc.cpu().numpy()

    def argmax(self, a: np.ndarray) -> np.ndarray:
        """[M,D] -> [M] u32 first argmax of A . B^T."""
        da = self._upload(a)
        m = da.shape[0]
        do = self._torch.empty(m, dtype=self._torch.int32, device=self._dev)
        if m:
            matmul_argmax_device(da.data_ptr(), m, self._b.data_ptr(), self.n, self.d, do.data_ptr(), self.bf16_b,
                                 self._stream())
        return do.cpu().numpy().view(np.uint32)
