"""Scalar restatement of the reference quantize tool's Q4_K block encoder.

TEST INFRASTRUCTURE ONLY: imported by tests/ as the checker of `t5h_quantize_q4k`; never by
the witchcraft_amd product path.

Reference: tools/quantize-tool/src/main.rs:12-24 calls candle's `QTensor::quantize(_, Q4K)`
(candle-core at git rev 0.9.2-alpha.2, a dependency absent from the reference tree), which
is `BlockQ4K::from_float`: candle's port of GGML's `quantize_row_q4_K_reference` with
`make_qkx1_quants(n = 32, nmax = 15, ntry = 5)` as GGML published them (k_quants.c).  Written
here from that published algorithm, one np.float32 operation at a time so that every
intermediate is rounded to f32 in the order the Rust code evaluates it; pure-Python loops, for
a few hundred blocks at most.

Parity of the candle bytes themselves is unpinned (candle is not importable here and the
reference holds no quantized fixture); this restatement is pinned by closed forms in the tests
(exactly representable blocks come back unchanged, constant sub-blocks give zeros) and the
product's native encoder is checked byte for byte against it.
"""
from __future__ import annotations

import math

import numpy as np

F = np.float32


def nearest_int(v: np.float32) -> int:
    """candle's nearest_int: f32::round (halves away from zero) as i32."""
    v = float(v)
    if math.isnan(v):
        return 0
    r = math.floor(abs(v) + 0.5) * (1 if v >= 0 else -1)
    return int(max(min(r, 2**31 - 1), -(2**31)))


def make_qkx1_quants(x: np.ndarray, nmax: int = 15, ntry: int = 5) -> tuple[np.float32, np.float32]:
    """(scale, -min) of one sub-block: GGML make_qkx1_quants."""
    x = [F(v) for v in x]
    n = len(x)
    mn, mx = min(x), max(x)
    if mx == mn:
        return F(0), F(0)
    if mn > 0:
        mn = F(0)
    iscale = F(nmax) / F(mx - mn)
    scale = F(1) / iscale
    L = [0] * n
    for _ in range(ntry):
        sumlx = F(0)
        suml2 = 0
        changed = False
        for i in range(n):
            li = max(0, min(nmax, nearest_int(F(iscale * F(x[i] - mn)))))
            if li != L[i]:
                L[i] = li
                changed = True
            sumlx = F(sumlx + F(F(x[i] - mn) * F(li)))
            suml2 += li * li
        scale = F(sumlx / F(suml2))
        s = F(0)
        for i in range(n):
            s = F(s + F(x[i] - F(scale * F(L[i]))))
        mn = F(s / F(n))
        if mn > 0:
            mn = F(0)
        iscale = F(F(1) / scale)
        if not changed:
            break
    return scale, F(-mn)


def quantize_block(x: np.ndarray) -> np.ndarray:
    """256 f32 values -> one 144-byte Q4_K block (BlockQ4K::from_float)."""
    x = np.asarray(x, np.float32).reshape(256)
    scales, mins = zip(*(make_qkx1_quants(x[32 * j:32 * j + 32]) for j in range(8)))
    max_scale = F(0)
    max_min = F(0)
    for j in range(8):
        max_scale = max(scales[j], max_scale)
        max_min = max(mins[j], max_min)
    inv_scale = F(F(63) / max_scale) if max_scale > 0 else F(0)
    inv_min = F(F(63) / max_min) if max_min > 0 else F(0)
    ls = [min(nearest_int(F(inv_scale * scales[j])), 63) for j in range(8)]
    lm = [min(nearest_int(F(inv_min * mins[j])), 63) for j in range(8)]
    sc = bytearray(12)
    for j in range(8):  # the packing get_scale_min_k4 reads back
        if j < 4:
            sc[j] = ls[j]
            sc[j + 4] = lm[j]
        else:
            sc[j + 4] = (ls[j] & 0xF) | ((lm[j] & 0xF) << 4)
            sc[j - 4] |= (ls[j] >> 4) << 6
            sc[j] |= (lm[j] >> 4) << 6
    d16 = np.float16(F(max_scale / F(63)))
    dmin16 = np.float16(F(max_min / F(63)))
    d, dmin = F(d16), F(dmin16)
    q = [0] * 256
    for j in range(8):
        dj = F(d * F(ls[j]))
        if dj == 0:
            continue
        dm = F(dmin * F(lm[j]))
        for i in range(32):
            q[32 * j + i] = max(0, min(15, nearest_int(F(F(x[32 * j + i] + dm) / dj))))
    out = bytearray(144)
    out[0:2] = d16.tobytes()
    out[2:4] = dmin16.tobytes()
    out[4:16] = sc
    for c in range(4):
        for i in range(32):
            out[16 + 32 * c + i] = q[64 * c + i] | (q[64 * c + 32 + i] << 4)
    return np.frombuffer(bytes(out), np.uint8)


def quantize(x: np.ndarray) -> np.ndarray:
    """[n * 256] f32 -> [n * 144] bytes, block by block."""
    x = np.asarray(x, np.float32).reshape(-1, 256)
    return np.concatenate([quantize_block(b) for b in x]) if len(x) else np.zeros(0, np.uint8)
