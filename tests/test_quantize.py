"""The Q4_K quantizer (`t5h_quantize_q4k`, the quantize tool's `QTensor::quantize(_, Q4K)`,
tools/quantize-tool/src/main.rs:12-24) against the scalar restatement in oracle/q4k_quant.py,
and both against what the algorithm fixes in closed form."""
import numpy as np
import pytest

from oracle import oracle as orc
from oracle import q4k_quant as ref
from witchcraft_amd.quantize import pack_q4k, quantize_q4k, quantize_q4k_minmax


def _blocks(seed: int) -> np.ndarray:
    """A mix of block kinds: weights, activations, one-signed, outliers, constants, zeros."""
    rng = np.random.default_rng(seed)
    b = [rng.standard_normal(256) * 0.02, rng.standard_normal(256), rng.uniform(0.5, 2.0, 256),
         -rng.uniform(0.0, 3.0, 256), rng.standard_normal(256) * 1e-3, np.zeros(256),
         rng.standard_normal(256) * 300.0]
    x = rng.standard_normal(256) * 0.05
    x[rng.integers(0, 256, 3)] = [4.0, -6.0, 9.5]          # outliers
    b.append(x)
    x = rng.standard_normal(256)
    x[32:64] = 0.75                                         # a constant sub-block
    x[128:160] = -1.25
    b.append(x)
    x = np.round(rng.standard_normal(256) * 4) / 4          # many exact ties
    b.append(x)
    return np.stack(b).astype(np.float32)


@pytest.mark.parametrize("seed", range(4))
def test_native_bytes_match_restatement(seed):
    x = _blocks(seed)
    assert np.array_equal(quantize_q4k(x), ref.quantize(x).reshape(x.shape[0], 144))


def test_native_bytes_match_restatement_random_weights():
    x = (np.random.default_rng(9).standard_normal((40, 256)) * 0.02).astype(np.float32)
    assert np.array_equal(quantize_q4k(x).reshape(-1), ref.quantize(x))


def _representable(seed: int, n: int):
    """Blocks whose values are exactly d * sc * q - dmin * m with the search's fixed point at
    the generating parameters: q covers 0 and 15 in every sub-block, sc >= 1, and the largest
    sc and m are 63 (so d and dmin are max / 63)."""
    rng = np.random.default_rng(seed)
    d = (2.0 ** rng.uniform(-12, -4, n)).astype(np.float16)
    dmin = (2.0 ** rng.uniform(-12, -4, n)).astype(np.float16)
    sc = rng.integers(1, 64, (n, 8))
    m = rng.integers(0, 64, (n, 8))
    sc[np.arange(n), rng.integers(0, 8, n)] = 63
    m[np.arange(n), rng.integers(0, 8, n)] = 63
    q = rng.integers(0, 16, (n, 8, 32))
    q[:, :, 0] = 0
    q[:, :, 1] = 15
    blocks = pack_q4k(d, dmin, sc, m, q)
    return blocks, orc.q4k_dequant(blocks).reshape(n, 256)


def test_representable_blocks_are_a_fixed_point():
    blocks, x = _representable(3, 64)
    qb = quantize_q4k(x)
    assert np.array_equal(orc.q4k_dequant(qb).reshape(x.shape), x)
    assert np.array_equal(qb, blocks)
    # the restatement reaches the same fixed point
    assert np.array_equal(ref.quantize(x[:8]), blocks[:8].reshape(-1))


def test_constant_and_zero_sub_blocks():
    """A sub-block with max == min gets scale 0 and min 0 (make_qkx1_quants' early return), so
    it dequantizes to zeros; the rest of the block is unaffected."""
    x = _blocks(1)[8:9]
    y = orc.q4k_dequant(quantize_q4k(x)).reshape(256)
    assert np.all(y[32:64] == 0) and np.all(y[128:160] == 0)
    assert np.abs(y[:32] - x[0, :32]).max() < 0.5
    assert np.all(orc.q4k_dequant(quantize_q4k(np.zeros((3, 256), np.float32))) == 0)


def test_search_beats_one_pass_encoder_on_weights():
    """RMS error on N(0, 0.02^2) rows no larger than the one-pass range/15 encoder's."""
    x = (np.random.default_rng(5).standard_normal((256, 768)) * 0.02).astype(np.float32)
    e_search = orc.q4k_dequant(quantize_q4k(x)).reshape(x.shape) - x
    e_minmax = orc.q4k_dequant(quantize_q4k_minmax(x)).reshape(x.shape) - x
    rms_s, rms_m = np.sqrt(np.mean(e_search ** 2)), np.sqrt(np.mean(e_minmax ** 2))
    assert rms_s <= rms_m, (rms_s, rms_m)
    assert rms_s < 0.08 * 0.02  # a few percent of the weights' spread


def test_threads_and_shapes():
    x = (np.random.default_rng(6).standard_normal((3000, 512)) * 0.02).astype(np.float32)
    a = quantize_q4k(x, threads=1)
    assert a.shape == (3000, 2 * 144)
    assert np.array_equal(a, quantize_q4k(x, threads=7))
    assert quantize_q4k(np.zeros((0, 256), np.float32)).shape == (0, 144)
    with pytest.raises(ValueError):
        quantize_q4k(np.zeros((2, 100), np.float32))
