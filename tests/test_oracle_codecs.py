"""Pins the oracle's block codecs and scalar ops (CPU only).

Each check is independent of the oracle's own formula: exhaustive bit patterns against
numpy's IEEE conversion, exact closed forms evaluated in double precision, committed
golden vectors (tests/golden/), and mathematical identities.
"""
import math

import numpy as np
import pytest

from oracle import oracle as orc
from witchcraft_amd.quantize import quantize_q4k, quantize_q4k_minmax

GOLDEN = __import__("pathlib").Path(__file__).resolve().parent / "golden"


def exact_q4k(blocks: np.ndarray) -> np.ndarray:
    from tests.golden.make_codec_golden import closed_form
    return closed_form(blocks)


def test_f16_to_f32_all_bit_patterns():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([orc.lib().orc_f16_to_f32(int(b)) for b in bits[::7]], np.float32)
    r = ref[::7]
    same = (got.view(np.uint32) == r.view(np.uint32)) | (np.isnan(got) & np.isnan(r))
    assert same.all()


def test_q4k_golden_blocks_bit_exact():
    z = np.load(GOLDEN / "q4k_blocks.npz")
    got = orc.q4k_dequant(z["blocks"])
    assert np.array_equal(got.view(np.uint32), z["values"].view(np.uint32))


def _blocks_for_scale_sweep(j: int, d: float, dmin: float) -> np.ndarray:
    """4096 blocks: sub-block j takes every (sc, m) in [0,63]^2; nibbles cycle 0..15."""
    from tests.golden.make_codec_golden import make_blocks
    n = 4096
    blocks = make_blocks(n, seed=100 + j)
    sc = np.repeat(np.arange(64), 64).astype(np.int64)
    m = np.tile(np.arange(64), 64).astype(np.int64)
    s = blocks[:, 4:16].astype(np.int64)
    if j < 4:
        s[:, j] = (s[:, j] & 0xC0) | sc
        s[:, j + 4] = (s[:, j + 4] & 0xC0) | m
    else:
        s[:, j + 4] = (sc & 15) | ((m & 15) << 4)
        s[:, j - 4] = (s[:, j - 4] & 0x3F) | ((sc >> 4) << 6)
        s[:, j] = (s[:, j] & 0x3F) | ((m >> 4) << 6)
    blocks[:, 4:16] = s.astype(np.uint8)
    c, hi = j // 2, j % 2
    nib = np.arange(32) % 16
    qs = blocks[:, 16 + 32 * c: 16 + 32 * c + 32].astype(np.int64)
    qs = (qs & 0x0F) | (nib << 4) if hi else (qs & 0xF0) | nib
    blocks[:, 16 + 32 * c: 16 + 32 * c + 32] = qs.astype(np.uint8)
    blocks[:, 0:2] = np.array([d], np.float16).view(np.uint8)
    blocks[:, 2:4] = np.array([dmin], np.float16).view(np.uint8)
    return blocks


@pytest.mark.parametrize("j", range(8))
@pytest.mark.parametrize("d,dmin", [(0.0123, 0.0071), (6.1e-05, 5.96e-08), (65504.0, 1.0), (0.0, 0.5)])
def test_q4k_exhaustive_scale_min_sweep(j, d, dmin):
    blocks = _blocks_for_scale_sweep(j, d, dmin)
    got = orc.q4k_dequant(blocks)
    ref = exact_q4k(blocks)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_q4k_special_cases():
    # q = 0 or sc = 0 -> -dmin * m exactly
    blk = np.zeros(144, np.uint8)
    blk[0:2] = np.array([0.25], np.float16).view(np.uint8)
    blk[2:4] = np.array([0.125], np.float16).view(np.uint8)
    blk[4:8] = [0, 3, 63, 1]       # sc 0..3
    blk[8:12] = [5, 0, 7, 63]      # m 0..3
    blk[16:48] = 0xA0              # chunk 0: low nibble 0 (sub-block 0), high 10 (sub-block 1)
    v = orc.q4k_dequant(blk)
    assert np.all(v[0:32] == np.float32(-0.125 * 5))           # q = 0
    assert np.all(v[32:64] == np.float32(0.25 * 3 * 10 - 0))   # sc=3, q=10, m=0
    blk2 = blk.copy()
    blk2[4] = 0  # sc_0 = 0
    blk2[16:48] = 0x0F
    v2 = orc.q4k_dequant(blk2)
    assert np.all(v2[0:32] == np.float32(-0.125 * 5))


def test_quantizer_roundtrip_and_format():
    rng = np.random.default_rng(0)
    x = (rng.standard_normal((32, 768)) * 0.02).astype(np.float32)
    q = quantize_q4k_minmax(x)
    assert q.shape == (32, 3 * 144)
    y = orc.q4k_dequant(q).reshape(32, 768)
    rel = np.linalg.norm(y - x) / np.linalg.norm(x)
    assert rel < 0.1, rel
    # per sub-block: error bounded by the block's quantization step (plus min rounding)
    xb, yb = x.reshape(-1, 32), y.reshape(-1, 32)
    step = (np.maximum(xb.max(1), 0) - np.minimum(xb.min(1), 0)) / 15
    assert np.all(np.abs(xb - yb).max(1) <= 1.6 * step + 1e-6)
    # zero rows quantize to exact zeros
    z = orc.q4k_dequant(quantize_q4k_minmax(np.zeros((2, 256), np.float32)))
    assert np.all(z == 0)


def test_rel_buckets_match_threshold_table():
    z = np.load(GOLDEN / "rel_buckets.npz")
    got = np.array([orc.rel_bucket(max(-int(d), 0), max(int(d), 0)) for d in z["deltas"]])
    assert np.array_equal(got, z["buckets"])
    # thresholds of the log map: bucket 8+k starts at ceil(8 * 16^(k/8))
    for k, start in enumerate([8, 12, 16, 23, 32, 46, 64, 91]):
        assert orc.rel_bucket(start, 0) == 8 + k
        assert orc.rel_bucket(0, start) == 16 + 8 + k
        if start > 8:
            assert orc.rel_bucket(start - 1, 0) == 8 + k - 1


def test_gelu_forms():
    for x in np.linspace(-6, 6, 97):
        ref = 0.5 * x * (1 + math.tanh(math.sqrt(2 / math.pi) * (x + 0.044715 * x ** 3)))
        assert abs(orc.gelu_tanh(float(x)) - ref) <= 1e-6 * (1 + abs(ref))
        # Pade [3,3] tanh stays within 2e-3 of tanh on the clamp range
        assert abs(orc.fast_tanh(float(x)) - math.tanh(max(min(x, 4.97), -4.97))) < 2e-3
        g = float(x)
        pade_ref = 0.5 * g * (1 + orc.fast_tanh(0.7978845608 * g * (1 + 0.044715 * g * g)))
        assert abs(orc.gelu_pade(g) - pade_ref) <= 1e-6 * (1 + abs(pade_ref))


def test_q8k_and_vec_dot():
    rng = np.random.default_rng(3)
    x = rng.standard_normal(768).astype(np.float32)
    w = (rng.standard_normal(768) * 0.05).astype(np.float32)
    q8 = orc.q8k_quantize(x)
    assert q8.size == 3 * 292
    d8 = q8.reshape(3, 292)[:, :4].copy().view(np.float32)[:, 0]
    qs = q8.reshape(3, 292)[:, 4:260].view(np.int8).astype(np.float64)
    bsums = q8.reshape(3, 292)[:, 260:].copy().view(np.int16)
    assert np.array_equal(bsums, qs.reshape(3, 16, 16).sum(2).astype(np.int16))
    xq = (qs * d8[:, None]).reshape(-1)
    assert np.abs(xq - x).max() <= np.abs(x).max() / 127 * 0.51 + 1e-7  # half-step rounding
    q4 = quantize_q4k(w[None])[0]
    w4 = orc.q4k_dequant(q4).astype(np.float64)
    got = orc.q4k_q8k_vec_dot(768, q4, q8)
    ref = float(np.dot(w4, xq))
    assert abs(got - ref) <= 1e-5 * (abs(ref) + np.abs(w4).sum() * np.abs(xq).max() * 1e-3)


def test_bf16_truncation():
    for v in [1.0, -3.14159265, 1e-30, 65504.0, 0.1]:
        u = np.array([v], np.float32).view(np.uint32)[0] & 0xFFFF0000
        assert orc.bf16_trunc(v) == np.array([u], np.uint32).view(np.float32)[0]


def test_rmsnorm_and_softmax_identities():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((4, 256)).astype(np.float32) * 3
    w = np.ones(256, np.float32)
    y = orc.rmsnorm(x, w)
    assert np.allclose(np.sqrt((y.astype(np.float64) ** 2).mean(1)), 1.0, atol=1e-5)
    w2 = rng.standard_normal(256).astype(np.float32)
    assert np.allclose(orc.rmsnorm(x, w2), y * w2, rtol=1e-6, atol=1e-6)
    s = orc.softmax_rows(rng.standard_normal((3, 50)) * 10)
    assert np.allclose(s.sum(1), 1.0, atol=1e-6) and (s >= 0).all()


def test_linear_matches_float64():
    rng = np.random.default_rng(6)
    x = rng.standard_normal((37, 256)).astype(np.float32)
    w = rng.standard_normal((300, 256)).astype(np.float32)
    ref = x.astype(np.float64) @ w.astype(np.float64).T
    assert np.allclose(orc.linear(x, w, acc64=True), ref, rtol=1e-6, atol=1e-5)
    assert np.allclose(orc.linear(x, w, acc64=False), ref, rtol=1e-4, atol=1e-3)
