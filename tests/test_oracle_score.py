"""CPU pins of the scoring oracle (oracle.matmul_t / oracle.matmul_argmax) and the host-side
argument checks of the scoring ABI.

The reference's scoring helpers have no tests of their own (src/fast_ops.rs:55-116,
src/lib.rs:187-208), so the oracle is pinned by what fixes the mathematics:
  * C = A . B^T against numpy's float64 matmul (a library routine, not the oracle's loop);
  * the fbgemm build's bf16 packing truncates (fbgemm-rs/src/bf16.rs:21-25), which values
    with known truncated and round-to-nearest images tell apart, sign included;
  * argmax against numpy's argmax of the float64 product (first occurrence on ties, as
    candle's argmax), and exact ties from duplicated rows of B.
"""
import numpy as np
import pytest

from oracle import oracle as orc


def _rng(seed):
    return np.random.default_rng(seed)


@pytest.mark.parametrize("M,N,D", [(1, 1, 1), (5, 7, 13), (32, 300, 128), (65, 64, 96), (3, 2, 0)])
def test_matmul_t_against_numpy_float64(M, N, D):
    r = _rng(M * 1000 + N + D)
    a = r.standard_normal((M, D)).astype(np.float32)
    b = r.standard_normal((N, D)).astype(np.float32)
    want = a.astype(np.float64) @ b.astype(np.float64).T
    got = orc.matmul_t(a, b)
    assert got.shape == (M, N)
    # the oracle sums in float64 and rounds once: at most half an f32 ulp off
    np.testing.assert_allclose(got, want, rtol=2 ** -23, atol=1e-30)
    got32 = orc.matmul_t(a, b, acc64=False)
    bound = D * 2 ** -23 * (np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64).T) + 1e-30
    assert np.all(np.abs(got32 - want) <= bound)


def test_matmul_t_transposed_operand_is_not_symmetric():
    # a plausible mistake -- reading B as [D, N] -- changes the result for non-square B
    r = _rng(3)
    a = r.standard_normal((4, 6)).astype(np.float32)
    b = r.standard_normal((5, 6)).astype(np.float32)
    c = orc.matmul_t(a, b)
    assert c.shape == (4, 5)
    assert abs(c[1, 3] - float(np.dot(a[1].astype(np.float64), b[3].astype(np.float64)))) < 1e-6


def test_bf16_packing_truncates_toward_zero():
    # values whose bf16 truncation differs from round-to-nearest-even
    x = np.array([1 + 2 ** -8 + 2 ** -9,       # RNE -> 1 + 2^-7, truncation -> 1.0
                  -(1 + 2 ** -8 + 2 ** -9),    # sign is kept: -1.0
                  1.9999999,                   # RNE -> 2.0, truncation -> 1.9921875
                  3.0,                         # exact in bf16
                  1 + 2 ** -7,                 # exact in bf16
                  -2.5e-39],                   # subnormal: keeps its top 7 mantissa bits
                 dtype=np.float32)
    want = np.array([1.0, -1.0, 1.9921875, 3.0, 1 + 2 ** -7,
                     (np.float32(-2.5e-39).view(np.uint32) & np.uint32(0xFFFF0000)).view(np.float32)],
                    dtype=np.float32)
    D = x.size
    eye = np.eye(D, dtype=np.float32)
    # C = I . B^T with B = x as one column per row: C[i, 0] = trunc(x[i])
    b = x.reshape(1, D)
    got = orc.matmul_t(eye, b, bf16_b=True)[:, 0]
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
    # A is not truncated: the same values on the A side pass through unchanged
    got_a = orc.matmul_t(x.reshape(1, D) * 1, eye, bf16_b=False)[0]
    np.testing.assert_array_equal(got_a.view(np.uint32), x.view(np.uint32))
    got_a16 = orc.matmul_t(x.reshape(1, D), eye, bf16_b=True)[0]  # I survives truncation
    np.testing.assert_array_equal(got_a16.view(np.uint32), x.view(np.uint32))


def test_bf16_mode_equals_product_with_masked_b():
    r = _rng(11)
    a = r.standard_normal((9, 48)).astype(np.float32)
    b = r.standard_normal((17, 48)).astype(np.float32)
    bt = (b.view(np.uint32) & np.uint32(0xFFFF0000)).view(np.float32)
    want = a.astype(np.float64) @ bt.astype(np.float64).T
    np.testing.assert_allclose(orc.matmul_t(a, b, bf16_b=True), want, rtol=2 ** -23, atol=1e-30)
    # and truncation changes the result (the flag is not ignored)
    assert not np.array_equal(orc.matmul_t(a, b, bf16_b=True), orc.matmul_t(a, b))


@pytest.mark.parametrize("M,N,D", [(1, 1, 8), (100, 37, 128), (70, 300, 16), (5, 1000, 7)])
def test_matmul_argmax_against_numpy(M, N, D):
    r = _rng(M + 7 * N + D)
    a = r.standard_normal((M, D)).astype(np.float32)
    b = r.standard_normal((N, D)).astype(np.float32)
    want = np.argmax(a.astype(np.float64) @ b.astype(np.float64).T, axis=1)
    got = orc.matmul_argmax(a, b)
    assert got.dtype == np.uint32 and got.shape == (M,)
    np.testing.assert_array_equal(got, want)
    bt = (b.view(np.uint32) & np.uint32(0xFFFF0000)).view(np.float32)
    want16 = np.argmax(a.astype(np.float64) @ bt.astype(np.float64).T, axis=1)
    np.testing.assert_array_equal(orc.matmul_argmax(a, b, bf16_b=True), want16)


def test_matmul_argmax_ties_go_to_first_index():
    r = _rng(5)
    a = r.standard_normal((20, 32)).astype(np.float32)
    base = r.standard_normal((6, 32)).astype(np.float32)
    # columns 2, 5 and 9 are the same centroid; whichever wins, the smallest index must
    b = np.concatenate([base, base[2:3], base[1:2], base[2:3], base[0:1]])  # rows 6..9
    b = np.concatenate([b[:5], base[2:3], b[5:]])  # row 5 = base[2] too
    got = orc.matmul_argmax(a, b)
    scores = a.astype(np.float64) @ b.astype(np.float64).T
    for i in range(a.shape[0]):
        best = np.flatnonzero(scores[i] == scores[i].max())
        assert got[i] == best[0]
    # all-equal scores (A = 0): index 0
    np.testing.assert_array_equal(orc.matmul_argmax(np.zeros((3, 32), np.float32), b), np.zeros(3, np.uint32))


def test_scoring_abi_rejects_bad_arguments_before_device_work():
    from witchcraft_amd import _lib, score

    a = np.ones((2, 16), np.float32)
    b = np.ones((3, 16), np.float32)
    out = np.empty(2, np.uint32)
    # argmax over zero columns is undefined
    rc = _lib.lib.t5h_matmul_argmax(0, a, 2, b, 0, 16, 0, out)
    assert rc == _lib.T5H_ERR_INVALID and b"N == 0" in _lib.lib.t5h_last_error()
    rc = _lib.lib.t5h_matmul_t(0, a, -1, b, 3, 16, 0, np.empty(6, np.float32))
    assert rc == _lib.T5H_ERR_INVALID
    # M == 0 and (for matmul_t) N == 0 are empty results, no device needed
    assert _lib.lib.t5h_matmul_t(0, a, 0, b, 3, 16, 0, np.empty(1, np.float32)) == _lib.T5H_OK
    assert _lib.lib.t5h_matmul_t(0, a, 2, b, 0, 16, 0, np.empty(1, np.float32)) == _lib.T5H_OK
    assert _lib.lib.t5h_matmul_argmax(0, a, 0, b, 3, 16, 0, out) == _lib.T5H_OK
    # the Python mirror checks dimensions like the reference's bail (src/fast_ops.rs:104-106)
    with pytest.raises(ValueError, match="dimension mismatch"):
        score.matmul_t(a, np.ones((3, 8), np.float32))
    with pytest.raises(ValueError, match="2-D"):
        score.matmul_argmax(np.ones(16, np.float32), b)
