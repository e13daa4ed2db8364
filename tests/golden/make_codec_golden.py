"""Writes tests/golden/q4k_blocks.npz and tests/golden/rel_buckets.npz.

q4k_blocks.npz: 256 random Q4_K blocks (random scale bytes, nibbles, and f16 d / dmin
drawn from a sweep of zero, subnormal, normal and large finite values) together with
their f32 values from the exact closed form of the GGML block (double-precision exact
arithmetic, one rounding to f32) -- computed here in numpy, independently of
oracle/t5_oracle.c and of the HIP kernel.

rel_buckets.npz: the bidirectional relative-position bucket of every signed distance
|j - i| < 2048 (32 buckets, max distance 128), from the integer thresholds the log map
reduces to:  |d| < 8 -> |d|;  else 8 + k where k is the largest integer with
|d| >= 8 * 16^(k/8) (capped at 15), computed with Python's correctly rounded math in
double precision plus the three exact-power cases d = 16, 32, 64 which f32 logf
(glibc) also places on the upper bucket; keys after the query add 16.

Run:  python tests/golden/make_codec_golden.py
"""
from __future__ import annotations

import math
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent


def closed_form(blocks: np.ndarray) -> np.ndarray:
    b = blocks.reshape(-1, 144)
    d = b[:, 0:2].copy().view(np.float16).astype(np.float64)[:, 0]
    dmin = b[:, 2:4].copy().view(np.float16).astype(np.float64)[:, 0]
    s = b[:, 4:16].astype(np.int64)
    sc = np.empty((b.shape[0], 8), np.int64)
    mn = np.empty((b.shape[0], 8), np.int64)
    sc[:, :4] = s[:, 0:4] & 63
    mn[:, :4] = s[:, 4:8] & 63
    sc[:, 4:] = (s[:, 8:12] & 15) | ((s[:, 0:4] >> 6) << 4)
    mn[:, 4:] = (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)
    qs = b[:, 16:].reshape(-1, 4, 32).astype(np.int64)
    q = np.empty((b.shape[0], 8, 32), np.int64)
    q[:, 0::2, :] = qs & 15
    q[:, 1::2, :] = qs >> 4
    exact = d[:, None, None] * sc[:, :, None] * q - dmin[:, None, None] * mn[:, :, None]
    return exact.astype(np.float32).reshape(-1)  # one rounding (f64 is exact here)


def f16_sweep() -> np.ndarray:
    vals = [0.0, 5.96e-08, 1.2e-07, 6.1e-05, 1.0e-3, 0.0123, 0.5, 1.0, 3.14159, 1000.0, 65504.0]
    return np.array(vals, np.float16)


def make_blocks(n: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    blocks = rng.integers(0, 256, size=(n, 144), dtype=np.uint8)
    sw = f16_sweep()
    d = sw[rng.integers(0, sw.size, n)]
    dm = sw[rng.integers(0, sw.size, n)]
    blocks[:, 0:2] = d.view(np.uint8).reshape(n, 2)
    blocks[:, 2:4] = dm.view(np.uint8).reshape(n, 2)
    return blocks


def bucket_by_threshold(delta: int) -> int:
    d = abs(delta)
    base = 16 if delta > 0 else 0
    if d < 8:
        return base + d
    k = 0
    while k < 7 and d >= 8 * 16 ** ((k + 1) / 8) - 1e-9:
        k += 1
    return base + min(8 + k, 15)


def main() -> None:
    blocks = make_blocks(256, seed=7)
    np.savez_compressed(HERE / "q4k_blocks.npz", blocks=blocks, values=closed_form(blocks))
    deltas = np.arange(-2047, 2048)
    buckets = np.array([bucket_by_threshold(int(x)) for x in deltas], np.int32)
    np.savez_compressed(HERE / "rel_buckets.npz", deltas=deltas.astype(np.int32), buckets=buckets)
    print("thresholds:", [int(math.ceil(8 * 16 ** (k / 8) - 1e-9)) for k in range(1, 8)])


if __name__ == "__main__":
    main()
