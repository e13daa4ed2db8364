"""GPU parity of the residual codec (src/packops.rs) against the CPU oracle, through the C ABI.

Encoding and decoding are integer / table work: the GPU's code bytes and decoded floats must
equal the oracle's bit for bit, including NaN, infinities, signed zeros and values exactly at
(and one ulp beside) every decision threshold.  Scoring from codes (matmul_t over decoded
residuals, src/lib.rs:676-680,734-735) has exact f32 products on both sides, so the GPU may
differ from the float64 sum of the decoded values only by f32 summation rounding:
D * 2^-23 * sum_k |a_k r_k| per entry.
"""
import ctypes as C

import numpy as np
import pytest

from oracle import oracle as orc

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def codec():
    from witchcraft_amd import codec as c
    return c


def _unit_rows(n, d, rng):
    x = rng.standard_normal((n, d)).astype(np.float32)
    return x / np.linalg.norm(x, axis=1, keepdims=True)


@pytest.mark.parametrize("N,D,K", [(1, 8, 1), (37, 16, 5), (1000, 128, 64), (4099, 128, 300), (2, 64, 2)])
def test_residual_encode_bitexact(codec, N, D, K):
    rng = np.random.default_rng(N * 7 + D)
    emb = _unit_rows(N, D, rng)
    centers = (_unit_rows(K, D, rng) * 0.9).astype(np.float32)
    assign = rng.integers(0, K, N).astype(np.uint32)
    got = codec.residual_to_q4_bytes(emb, centers, assign)
    assert np.array_equal(got, orc.residual_encode(emb, centers, assign))


def test_residual_encode_edge_values(codec):
    t = codec.q4_compand_thresholds()
    specials = [0.0, -0.0, np.inf, -np.inf, np.nan, 1e-30, -1e-30, 3.4e38, -3.4e38, 1.0, -1.0, 0.25, -0.25]
    vals = list(specials)
    for x in t:
        x = np.float32(x)
        vals += [x, np.nextafter(x, np.float32(np.inf)), np.nextafter(x, np.float32(-np.inf))]
    vals = np.array(vals, np.float32)
    D = 8
    n = (vals.size + D - 1) // D
    r = np.zeros(n * D, np.float32)
    r[: vals.size] = vals
    emb = r.reshape(n, D)
    centers = np.zeros((1, D), np.float32)  # residual = emb exactly
    assign = np.zeros(n, np.uint32)
    got = codec.residual_to_q4_bytes(emb, centers, assign)
    want = orc.residual_encode(emb, centers, assign)
    assert np.array_equal(got, want)
    # and against the scalar quantizer, value by value
    codes = np.stack([got >> 4, got & 15], axis=-1).reshape(-1)
    assert [int(c) for c in codes[: vals.size]] == [orc.compand_q4(v) for v in vals]


def test_residual_encode_rejects_bad_assignment(codec):
    emb = np.zeros((4, 8), np.float32)
    with pytest.raises(RuntimeError):
        codec.residual_to_q4_bytes(emb, np.zeros((2, 8), np.float32), np.array([0, 1, 2, 0], np.uint32))


def test_residual_encode_device_flags_bad_assignment(codec):
    import torch
    from witchcraft_amd import _lib
    dev = torch.device("cuda", 0)
    emb = torch.zeros((3, 8), dtype=torch.float32, device=dev)
    cen = torch.zeros((2, 8), dtype=torch.float32, device=dev)
    asg = torch.tensor([0, 5, 1], dtype=torch.int32, device=dev)
    out = torch.full((3, 4), 0x77, dtype=torch.uint8, device=dev)
    bad = torch.zeros(1, dtype=torch.int32, device=dev)
    _lib.check(_lib.lib.t5h_residual_encode_device(emb.data_ptr(), 3, cen.data_ptr(), 2, asg.data_ptr(), 8,
                                                   out.data_ptr(), bad.data_ptr(), None))
    torch.cuda.synchronize()
    assert int(bad.item()) == 1
    o = out.cpu().numpy()
    assert np.all(o[1] == 0) and np.all(o[0] == 0x88) and np.all(o[2] == 0x88)  # zero residual -> code 8


@pytest.mark.parametrize("N,D", [(1, 2), (5, 6), (333, 128), (10000, 128)])
def test_residual_decode_bitexact(codec, N, D):
    rng = np.random.default_rng(N + D)
    codes = rng.integers(0, 256, (N, D // 2)).astype(np.uint8)
    got = codec.from_companded_q4_bytes(codes, D)
    want = orc.residual_decode(codes, D)
    assert got.view(np.uint32).tolist() == want.view(np.uint32).tolist()


SCORE_SHAPES = [
    (1, 1, 4),
    (5, 31, 12),        # D % 16 != 0
    (32, 1000, 128),    # tiled kernel
    (33, 300, 128),     # M > 32: tiled
    (100, 70, 64),
    (32, 65536, 128),   # streaming kernel: query tokens x residual codes
    (17, 4100, 128),    # 2 row blocks; last tile holds 4 rows
    (1, 4124, 128),     # last tile holds 28 rows
    (16, 4098, 128),    # N % 4 != 0: tiled
]


@pytest.mark.parametrize("M,N,D", SCORE_SHAPES)
def test_matmul_t_q4_within_f32_summation_bound(codec, M, N, D):
    rng = np.random.default_rng(M * 131 + N)
    a = _unit_rows(M, D, rng)
    codes = rng.integers(0, 256, (N, D // 2)).astype(np.uint8)
    got = codec.matmul_t_q4(a, codes)
    r = orc.residual_decode(codes, D).astype(np.float64)
    want = a.astype(np.float64) @ r.T
    bound = D * 2.0 ** -23 * (np.abs(a).astype(np.float64) @ np.abs(r).T) + 1e-30
    assert got.shape == (M, N)
    assert np.all(np.abs(got - want) <= bound)


def test_matmul_t_q4_matches_decode_then_matmul(codec):
    """Same scores as the reference's two steps, from_companded_q4_bytes then matmul_t."""
    from witchcraft_amd import score
    rng = np.random.default_rng(9)
    a = _unit_rows(32, 128, rng)
    codes = rng.integers(0, 256, (8192, 64)).astype(np.uint8)
    fused = codec.matmul_t_q4(a, codes)
    two_step = score.matmul_t(a, codec.from_companded_q4_bytes(codes, 128))
    r = orc.residual_decode(codes, 128).astype(np.float64)
    bound = 2 * 128 * 2.0 ** -23 * (np.abs(a).astype(np.float64) @ np.abs(r).T)
    assert np.all(np.abs(fused.astype(np.float64) - two_step) <= bound)


def test_matmul_t_q4_query_beyond_bf16_range(codec):
    """Finite query values of magnitude >= 0x7f7f8000 (about 3.396e38) round to a bf16 infinity,
    so the three-way bf16 split cannot carry them: their block takes the f32 kernel and gives
    the finite f32 scores.  A value just below the threshold stays on the split path."""
    from witchcraft_amd import score
    rng = np.random.default_rng(32)
    codes = rng.integers(0, 256, (4096, 64)).astype(np.uint8)  # the streaming shape: M <= 32
    r = orc.residual_decode(codes, 128).astype(np.float64)
    for big in (np.float32(3.4e38), -np.float32(3.39e38)):
        a = _unit_rows(20, 128, rng)
        a[2, 5] = big
        got = codec.matmul_t_q4(a, codes)
        two_step = score.matmul_t(a, codec.from_companded_q4_bytes(codes, 128))
        assert np.all(np.isfinite(two_step)) and np.all(np.isfinite(got)), big
        want = a.astype(np.float64) @ r.T
        bound = 3 * 128 * 2.0 ** -23 * (np.abs(a).astype(np.float64) @ np.abs(r).T)
        assert np.all(np.abs(got - want) <= bound), big


def test_matmul_t_q4_shape_errors(codec):
    with pytest.raises(ValueError):
        codec.matmul_t_q4(np.zeros((2, 128), np.float32), np.zeros((3, 32), np.uint8))


def test_matmul_t_q4_nonfinite_query(codec):
    """The streaming shape runs on bf16 MFMAs with both operands split in three parts, which
    cannot carry infinities (inf times parts of both signs would give NaN); a query block with a
    non-finite value takes the f32 kernel.  The NaN / inf pattern then equals the two-step f32
    result, and the finite rows of the same launch stay within the summation bound."""
    from witchcraft_amd import score
    rng = np.random.default_rng(31)
    a = _unit_rows(20, 128, rng)
    a[3, 7] = np.inf
    a[5, 100] = -np.inf
    a[9, 0] = np.nan
    codes = rng.integers(0, 256, (4096, 64)).astype(np.uint8)
    got = codec.matmul_t_q4(a, codes)
    two_step = score.matmul_t(a, codec.from_companded_q4_bytes(codes, 128))
    assert np.array_equal(np.isnan(got), np.isnan(two_step))
    inf = np.isinf(two_step)
    assert np.array_equal(np.isinf(got), inf)
    assert np.array_equal(np.sign(got[inf]), np.sign(two_step[inf]))
    fin = [i for i in range(20) if i not in (3, 5, 9)]
    r = orc.residual_decode(codes, 128).astype(np.float64)
    want = a[fin].astype(np.float64) @ r.T
    bound = 128 * 2.0 ** -23 * (np.abs(a[fin]).astype(np.float64) @ np.abs(r).T)
    assert np.all(np.abs(got[fin] - want) <= bound)
