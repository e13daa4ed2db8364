"""Q4_K quantizer: f32 rows -> GGML Q4_K super-blocks (the `quantize-tool` step).

Reference: tools/quantize-tool/src/main.rs:12-24 quantizes every rank-2 tensor whose
last dimension is a multiple of 256 to Q4_K (candle `QTensor::quantize`, i.e.
`BlockQ4K::from_float` with GGML's `make_qkx1_quants` scale/min search) and keeps the rest
F32.  `quantize_q4k` runs that search natively (`t5h_quantize_q4k` in libt5hip.so, host
threads, no GPU needed):

    block = {f16 d, f16 dmin, u8 scales[12], u8 qs[128]}          (144 bytes / 256 values)
    value = d * sc_j * q - dmin * m_j   for sub-block j = 0..7 (32 values each),
    (sc_j, m_j) 6-bit, packed as get_scale_min_k4 unpacks them,
    qs[32c + l] = q[64c + l] | q[64c + 32 + l] << 4.

`quantize_q4k_minmax` is a one-pass encoder of the same format (range [min(x, 0), max(x)]
over 15 steps per sub-block), kept as the simple baseline the search is measured against.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

QK_K = 256
BLOCK_BYTES = 144


def quantize_q4k(x: np.ndarray, threads: int = 0) -> np.ndarray:
    """Quantize float rows [..., K] (K % 256 == 0) -> uint8 [..., K // 256 * 144]."""
    from ._lib import check, lib
    x = np.ascontiguousarray(x, dtype=np.float32)
    if x.shape[-1] % QK_K:
        raise ValueError("last dimension must be a multiple of 256")
    out = np.empty(x.size // QK_K * BLOCK_BYTES, np.uint8)
    check(lib.t5h_quantize_q4k(x.reshape(-1), C.c_int64(x.size), out, int(threads)))
    return out.reshape(*x.shape[:-1], (x.shape[-1] // QK_K) * BLOCK_BYTES)


def quantize_q4k_minmax(x: np.ndarray) -> np.ndarray:
    """One-pass Q4_K encoder: per sub-block scale = (max(x, 0) - min(x, 0)) / 15, min = -min(x, 0)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    if x.shape[-1] % QK_K:
        raise ValueError("last dimension must be a multiple of 256")
    lead = x.shape[:-1]
    xb = x.reshape(-1, 8, 32)
    nblk = xb.shape[0]
    mn = np.minimum(xb.min(axis=2), 0.0)
    mx = np.maximum(xb.max(axis=2), 0.0)
    scale = (mx - mn) / 15.0
    mins = -mn
    d = (scale.max(axis=1) / 63.0).astype(np.float16)
    dmin = (mins.max(axis=1) / 63.0).astype(np.float16)
    df = d.astype(np.float32)[:, None]
    dminf = dmin.astype(np.float32)[:, None]
    with np.errstate(divide="ignore", invalid="ignore"):
        sc = np.where(df > 0, np.rint(scale / df), 0).clip(0, 63).astype(np.uint8)
        m = np.where(dminf > 0, np.rint(mins / dminf), 0).clip(0, 63).astype(np.uint8)
        eff_s = (df * sc)[:, :, None]
        eff_m = (dminf * m)[:, :, None]
        q = np.where(eff_s > 0, np.rint((xb + eff_m) / eff_s), 0).clip(0, 15).astype(np.uint8)
    return pack_q4k(d, dmin, sc, m, q).reshape(*lead, (x.shape[-1] // QK_K) * BLOCK_BYTES)


def pack_q4k(d: np.ndarray, dmin: np.ndarray, sc: np.ndarray, m: np.ndarray, q: np.ndarray) -> np.ndarray:
    """Blocks from f16 d, dmin [n], 6-bit sc, m [n, 8] and 4-bit q [n, 8, 32] -> uint8 [n, 144]."""
    nblk = d.shape[0]
    sc = sc.astype(np.uint8)
    m = m.astype(np.uint8)
    scales = np.empty((nblk, 12), np.uint8)
    scales[:, 0:4] = sc[:, 0:4] | ((sc[:, 4:8] >> 4) << 6)
    scales[:, 4:8] = m[:, 0:4] | ((m[:, 4:8] >> 4) << 6)
    scales[:, 8:12] = (sc[:, 4:8] & 15) | ((m[:, 4:8] & 15) << 4)
    q = q.astype(np.uint8)
    qs = (q[:, 0::2, :] | (q[:, 1::2, :] << 4)).reshape(nblk, 128)
    out = np.empty((nblk, BLOCK_BYTES), np.uint8)
    out[:, 0:2] = np.asarray(d, np.float16).view(np.uint8).reshape(nblk, 2)
    out[:, 2:4] = np.asarray(dmin, np.float16).view(np.uint8).reshape(nblk, 2)
    out[:, 4:16] = scales
    out[:, 16:] = qs
    return out


def q4k_nbytes(rows: int, cols: int) -> int:
    return rows * (cols // QK_K) * BLOCK_BYTES
