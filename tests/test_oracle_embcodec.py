"""Pins the CPU oracle of Witchcraft's embedding codecs (oracle/codec_oracle.c) to
independent formulations: float64 closed forms of the mu-law / 4-bit codes, an orthonormal
Haar matrix, a textbook exact-division rANS64 coder in Python integers, and exact rational
apportionment for scale_histogram.  The reference holds no tests or fixtures for these
functions (src/packops.rs's test module is commented out), so these are the pins.
"""
from __future__ import annotations

import struct
from fractions import Fraction

import numpy as np
import pytest

from oracle import oracle as orc


# ---------------------------------------------------------------- residual codec (mu-law q4)

def _table64() -> np.ndarray:
    v = (np.arange(16) - 7.5) * (2.0 / 15.0)
    return np.sign(v) * (np.power(256.0, np.abs(v)) - 1.0) / 255.0 / 4.0


def test_q4_table_closed_form_and_symmetry():
    t = orc.q4_dequant_table()
    # f32 pipeline bound: ln 256 rounded to f32 (2^-24 relative) is scaled by |v| ln 256 <= 5.6
    # inside exp, and p - 1 with p = 256^|v| >= 1.45 amplifies relative error by p / (p - 1) <= 3.3
    np.testing.assert_allclose(t.astype(np.float64), _table64(), rtol=2e-6, atol=0)
    for i in range(16):  # dequantize(4) is antisymmetric about 7.5 and inv_compand is odd
        assert t[15 - i] == -t[i]
    assert np.all(np.diff(t) > 0)


def test_compand_q4_closed_form():
    rng = np.random.default_rng(1)
    xs = np.concatenate([rng.uniform(-0.3, 0.3, 40000), rng.normal(0, 0.05, 40000)]).astype(np.float32)
    got = np.array([orc.compand_q4(x) for x in xs])
    x4 = 4.0 * xs.astype(np.float64)
    c = np.sign(x4) * np.log1p(255.0 * np.abs(x4)) / np.log(256.0)
    pre = 7.5 * c + 7.5
    want = np.clip(np.floor(pre + 0.5), 0, 15)  # pre >= 0 here: half away from zero = floor(+0.5)
    near = np.abs(pre - np.round(pre - 0.5) - 0.5) < 1e-5  # within 1e-5 of a .5 boundary
    assert np.all((got == want) | near)
    assert (got != want).sum() <= near.sum()


def test_compand_q4_specials():
    assert orc.compand_q4(0.0) == 8 and orc.compand_q4(-0.0) == 8  # round(7.5) = 8
    assert orc.compand_q4(float("nan")) == 0  # clamp(NaN) keeps the lower bound
    assert orc.compand_q4(float("inf")) == 15 and orc.compand_q4(float("-inf")) == 0
    assert orc.compand_q4(1.0) == 15 and orc.compand_q4(-1.0) == 0


def test_table_roundtrip_through_quantizer():
    t = orc.q4_dequant_table()
    assert [orc.compand_q4(v) for v in t] == list(range(16))


def test_residual_encode_decode():
    rng = np.random.default_rng(2)
    N, D, K = 300, 128, 7
    emb = rng.normal(0, 1, (N, D)).astype(np.float32)
    emb /= np.linalg.norm(emb, axis=1, keepdims=True)
    centers = (emb[rng.integers(0, N, K)] + rng.normal(0, 0.02, (K, D))).astype(np.float32)
    assign = rng.integers(0, K, N).astype(np.uint32)
    codes = orc.residual_encode(emb, centers, assign)
    assert codes.shape == (N, D // 2)
    r = emb - centers[assign]
    q = np.array([[orc.compand_q4(v) for v in row] for row in r[:20]])
    assert np.array_equal(codes[:20] >> 4, q[:, 0::2]) and np.array_equal(codes[:20] & 15, q[:, 1::2])
    dec = orc.residual_decode(codes, D)
    t = orc.q4_dequant_table()
    assert np.array_equal(dec[:20], t[q])
    # below 0.11 the largest decision interval is [0.0818, 0.1188] (codes 13 | 14), so a value
    # lands at most 0.037 from its reconstruction
    inner = np.abs(r) < 0.11
    assert np.max(np.abs(dec - r)[inner]) < 0.04


# --------------------------------------------------------------------------- Haar transform

def _haar_matrix(n: int) -> np.ndarray:
    """Orthonormal Haar analysis matrix in the reference's layout [a_L, d_L, ..., d_1] (n = 2^k),
    built as a product of per-level operators in float64."""
    H = np.eye(n)
    m = n
    while m > 1:
        L = np.eye(n)
        L[:m, :m] = 0
        for i in range(m // 2):
            L[i, 2 * i] = L[i, 2 * i + 1] = 2 ** -0.5
            L[m // 2 + i, 2 * i] = 2 ** -0.5
            L[m // 2 + i, 2 * i + 1] = -(2 ** -0.5)
        H = L @ H
        m //= 2
    return H


@pytest.mark.parametrize("n", [2, 8, 64, 128, 1024])
def test_haar_power_of_two_matches_orthonormal_basis(n):
    rng = np.random.default_rng(n)
    x = rng.normal(0, 1, n).astype(np.float32)
    H = _haar_matrix(n)
    assert np.allclose(H @ H.T, np.eye(n), atol=1e-12)
    y = orc.haar_forward(x)
    np.testing.assert_allclose(y, H @ x.astype(np.float64), atol=2e-6 * np.linalg.norm(x))


@pytest.mark.parametrize("n", list(range(1, 40)) + [127, 129, 255, 1000, 1023])
def test_haar_inverse_roundtrip_and_constant(n):
    rng = np.random.default_rng(1000 + n)
    x = rng.normal(0, 1, n).astype(np.float32)
    np.testing.assert_allclose(orc.haar_inverse(orc.haar_forward(x)), x, atol=2e-5)
    # a constant under the mirror extension has no detail; the DC term gains sqrt(2) per level
    levels, m = 0, n
    while m > 1:
        m = (m + 1) // 2
        levels += 1
    y = orc.haar_forward(np.full(n, 0.5, np.float32))
    assert np.all(y[1:] == 0)
    assert abs(y[0] - 0.5 * 2 ** (levels / 2)) <= 1e-5 * max(1.0, y[0])


# --------------------------------------------------------------------------- scale_histogram

def _apportion(counts: list[int], log2_scale: int) -> list[int]:
    """Largest remainders with exact rationals: 1 each plus floor quotas of the rest, the deficit
    to the largest remainders (earlier index first on ties), then any residue to the last
    maximum (Iterator::max_by_key)."""
    target = 1 << log2_scale
    m, total = len(counts), sum(counts)
    rest = target - m
    quotas = [Fraction(c * rest, total) for c in counts]
    out = [1 + (q.numerator // q.denominator) for q in quotas]
    fracs = [q - (q.numerator // q.denominator) for q in quotas]
    deficit = target - sum(out)
    for i in sorted(range(m), key=lambda i: (-fracs[i], i))[:deficit]:
        out[i] += 1
    if sum(out) != target:
        mx = max(out)
        last = max(i for i in range(m) if out[i] == mx)
        out[last] += target - sum(out)
    return out


@pytest.mark.parametrize("seed", range(12))
def test_scale_histogram_apportionment(seed):
    rng = np.random.default_rng(seed)
    m = int(rng.integers(1, 200))
    counts = rng.integers(1, 20000, m).astype(np.uint32)
    if seed % 3 == 0:
        counts[: m // 2] = 1  # many rare symbols
    f = orc.scale_histogram(counts, 12)
    assert int(f.astype(np.int64).sum()) == 4096 and f.min() >= 1
    assert f.tolist() == _apportion(counts.tolist(), 12)


def test_scale_histogram_rejects_what_the_reference_asserts():
    with pytest.raises(ValueError):
        orc.scale_histogram(np.ones(5000, np.uint32), 12)  # more symbols than slots


# ------------------------------------------------------------------------ rANS64 + packing

RANS_L = 1 << 31


def _rans_encode(symbols, start, freq, bits=12) -> bytes:
    """Textbook rANS64 with exact division (ryg_rans rans64.h without reciprocals): symbols
    pushed in order, 32-bit words emitted backwards, final 64-bit state in front."""
    x, words = RANS_L, []
    for s in symbols:
        f, c = freq[s], start[s]
        x_max = ((RANS_L >> bits) << 32) * f
        while x >= x_max:
            words.append(x & 0xFFFFFFFF)
            x >>= 32
        x = ((x // f) << bits) + (x % f) + c
    return struct.pack("<Q", x) + b"".join(struct.pack("<I", w) for w in reversed(words))


def _rans_decode(data: bytes, n: int, syms, start, freq, bits=12):
    cum2sym = np.zeros(1 << bits, np.int64)
    for s in syms:
        cum2sym[start[s]:start[s] + freq[s]] = s
    x = struct.unpack_from("<Q", data, 0)[0]
    pos, out = 8, [0] * n
    mask = (1 << bits) - 1
    for i in range(n - 1, -1, -1):
        s = int(cum2sym[x & mask])
        out[i] = s
        x = freq[s] * (x >> bits) + (x & mask) - start[s]
        if x < RANS_L:
            x = (x << 32) | struct.unpack_from("<I", data, pos)[0]
            pos += 4
    assert pos == len(data)
    return out


def _parse(buf: bytes, cols: int):
    rows = struct.unpack_from("<I", buf, 0)[0]
    pos, wins = 4, []
    for off in range(0, rows, 1024):
        wr = min(1024, rows - off)
        perm = list(buf[pos:pos + cols])
        pos += cols
        m = struct.unpack_from("<H", buf, pos)[0]
        pos += 2
        pairs = [struct.unpack_from("<HH", buf, pos + 4 * i) for i in range(m)]
        pos += 4 * m
        clen = struct.unpack_from("<H", buf, pos)[0]
        pos += 2
        wins.append((wr, perm, pairs, buf[pos:pos + clen]))
        pos += clen
    assert pos == len(buf)
    return rows, wins


def _smooth_embeddings(rows: int, cols: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    base = rng.normal(0, 1, cols)
    x = base + np.cumsum(rng.normal(0, 0.15, (rows, cols)), axis=0) + rng.normal(0, 0.3, (rows, cols))
    return (x / np.linalg.norm(x, axis=1, keepdims=True)).astype(np.float32)


@pytest.mark.parametrize("rows", [0, 1, 2, 7, 64, 333, 1024, 1025, 2500])
def test_packed_stream_is_textbook_rans(rows):
    cols = 128
    x = _smooth_embeddings(rows, cols, rows)
    buf = orc.embeddings_to_packed(x)
    nrows, wins = _parse(buf, cols)
    assert nrows == rows and len(wins) == (rows + 1023) // 1024
    for wr, perm, pairs, data in wins:
        assert sorted(perm) == list(range(cols))
        syms = [p[0] for p in pairs]
        assert syms == sorted(set(syms)) and sum(p[1] for p in pairs) == 4096
        start, freq, c = {}, {}, 0
        for s, f in pairs:
            start[s], freq[s] = c, f
            c += f
        symbols = _rans_decode(data, wr * cols, syms, start, freq)
        assert _rans_encode(symbols, start, freq) == data
    if rows:
        y = orc.embeddings_from_packed(buf, cols)
        assert y.shape == (rows, cols)
        np.testing.assert_allclose(np.linalg.norm(y, axis=1), 1.0, atol=1e-5)
        assert float((x * y).sum(1).min()) > 0.99


def test_packed_symbols_follow_the_quantizer():
    """Window symbols are round(29 x / max|x|<1) folded to 2|q| - 1 (+1 if negative) of the 2-D
    Haar coefficients of the column-sorted window (float64 restatement, boundary cases excepted)."""
    rows, cols = 40, 128
    x = _smooth_embeddings(rows, cols, 7)
    buf = orc.embeddings_to_packed(x)
    _, [(wr, perm_bytes, pairs, data)] = _parse(buf, cols)
    order = np.argsort(x.sum(0).astype(np.float64), kind="stable")
    assert [int(np.where(order == c)[0][0]) for c in range(cols)] == perm_bytes
    y = x[:, order].astype(np.float64)
    # separable 2-D Haar with mirror edges in float64: rows (n = 128 = 2^7), then columns (n = 40)
    y = y @ _haar_matrix(cols).T
    y = np.stack([orc.haar_forward(col.astype(np.float32)).astype(np.float64) for col in y.T], 1)
    a = np.abs(y)
    amax = max(1e-5, a[a < 1].max())
    v = 29 * y / amax
    q = np.sign(v) * np.floor(np.abs(v) + 0.5)
    s = np.where(q == 0, 0, 2 * np.abs(q) + (q < 0) - 1).astype(np.int64).reshape(-1)
    start, freq, c = {}, {}, 0
    for sy, f in pairs:
        start[sy], freq[sy] = c, f
        c += f
    got = np.array(_rans_decode(data, wr * cols, [p[0] for p in pairs], start, freq))
    boundary = np.abs(np.abs(v) - np.floor(np.abs(v)) - 0.5).reshape(-1) < 1e-3
    assert np.all((got == s) | boundary)


def test_packed_decoder_rejects_malformed():
    x = _smooth_embeddings(50, 128, 3)
    buf = orc.embeddings_to_packed(x)
    with pytest.raises(ValueError):
        orc.embeddings_from_packed(buf + b"\0", 128)  # leftover bytes
    with pytest.raises(ValueError):
        orc.embeddings_from_packed(buf[:-3], 128)  # truncated stream
