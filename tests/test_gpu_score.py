"""GPU parity of the query-side scoring kernels against the CPU oracle, through the C ABI.

matmul_t (src/fast_ops.rs:98-116) is f32: products are exact f32 on both sides, so the GPU
may differ from the oracle's float64 sum only by f32 summation rounding, bounded per entry by
D * 2^-23 * sum_k |a_k b_k| -- the bound the tests use.  matmul_argmax (src/lib.rs:187-208)
must return the oracle's index wherever the best score leads the runner-up by more than
twice that bound; inside the bound, the GPU's pick must score within it of the maximum.
Exact ties (duplicated rows of B) must resolve to the first index, as candle's argmax does.
"""
import numpy as np
import pytest

from oracle import oracle as orc

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def score():
    from witchcraft_amd import score as s
    return s


def _data(M, N, D, seed, scale=1.0):
    r = np.random.default_rng(seed)
    return ((r.standard_normal((M, D)) * scale).astype(np.float32),
            r.standard_normal((N, D)).astype(np.float32))


def _trunc(b):
    return (b.view(np.uint32) & np.uint32(0xFFFF0000)).view(np.float32)


def _bound(a, b, bf16_b):
    bb = _trunc(b) if bf16_b else b
    D = a.shape[1]
    return D * 2.0 ** -23 * (np.abs(a).astype(np.float64) @ np.abs(bb).astype(np.float64).T) + 1e-30


SHAPES = [
    (1, 1, 128),       # single pair
    (32, 1000, 128),   # query tokens x residuals: 32-row tile, ragged last column tile
    (33, 257, 128),    # 48-row tile, N just past a workgroup
    (64, 64, 128),     # N <= 64: waves stacked along M
    (200, 40, 128),    # M > 64 with small N
    (65, 300, 128),    # two row tiles
    (3, 4096, 96),     # D % 16 != 0 (tail block), D % 4 == 0 (vector loads)
    (7, 5, 13),        # unaligned rows: scalar loads
    (1, 70, 1),
    # the persistent streaming kernel (M <= 32, D = 128, N >= 4096, N % 4 == 0)
    (32, 65536, 128),  # query tokens x residuals
    (17, 4100, 128),   # 2 row blocks; last 32-column tile holds 4 columns
    (16, 8192, 128),   # one row block
    (1, 4124, 128),    # single query row; last tile holds 28 columns
    (32, 4098, 128),   # N % 4 != 0: the tiled kernel instead
]


@pytest.mark.parametrize("bf16_b", [False, True])
@pytest.mark.parametrize("M,N,D", SHAPES)
def test_matmul_t_vs_oracle(score, M, N, D, bf16_b):
    print(f"matmul_t M={M} N={N} D={D} bf16_b={bf16_b}", flush=True)
    a, b = _data(M, N, D, seed=M * 31 + N + D)
    got = score.matmul_t(a, b, bf16_b=bf16_b)
    want = orc.matmul_t(a, b, bf16_b=bf16_b)
    assert got.shape == (M, N)
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    bound = _bound(a, b, bf16_b)
    assert np.all(err <= bound), f"max err/bound {(err / bound).max():.3f}"
    assert np.all(np.isfinite(got))


def test_matmul_t_d_zero_is_zero(score):
    a = np.zeros((5, 0), np.float32)
    b = np.zeros((9, 0), np.float32)
    np.testing.assert_array_equal(score.matmul_t(a, b), np.zeros((5, 9), np.float32))


def test_matmul_t_bf16_flag_changes_result(score):
    a, b = _data(16, 64, 128, seed=4)
    assert not np.array_equal(score.matmul_t(a, b, bf16_b=True), score.matmul_t(a, b))


def test_matmul_t_exact_small_integers(score):
    # integer-valued operands: every partial sum is exact, so the GPU must match bit for bit
    r = np.random.default_rng(8)
    a = r.integers(-8, 9, (40, 128)).astype(np.float32)
    b = r.integers(-8, 9, (333, 128)).astype(np.float32)
    want = (a.astype(np.int64) @ b.astype(np.int64).T).astype(np.float32)
    np.testing.assert_array_equal(score.matmul_t(a, b), want)
    np.testing.assert_array_equal(score.matmul_t(a, b, bf16_b=True), want)


def _check_argmax(a, b, got, bf16_b):
    want = orc.matmul_argmax(a, b, bf16_b=bf16_b)
    s = orc.matmul_t(a, b, bf16_b=bf16_b).astype(np.float64)
    bound = _bound(a, b, bf16_b)
    rows = np.arange(a.shape[0])
    top = s[rows, want]
    tol = 2 * bound[rows, want]
    s2 = s.copy()
    s2[rows, want] = -np.inf
    clear = top - s2.max(axis=1) > tol if s.shape[1] > 1 else np.ones(len(rows), bool)
    np.testing.assert_array_equal(got[clear], want[clear])
    assert np.all(s[rows, got] >= top - tol)
    return int(clear.sum())


@pytest.mark.parametrize("bf16_b", [False, True])
@pytest.mark.parametrize("M,N,D", [(1, 1, 128), (100, 37, 128), (64, 256, 128), (300, 1000, 128),
                                   (129, 4099, 128), (50, 300, 96), (17, 33, 13)])
def test_matmul_argmax_vs_oracle(score, M, N, D, bf16_b):
    print(f"argmax M={M} N={N} D={D} bf16_b={bf16_b}", flush=True)
    a, b = _data(M, N, D, seed=M + 5 * N + D)
    got = score.matmul_argmax(a, b, bf16_b=bf16_b)
    assert got.dtype == np.uint32 and got.shape == (M,)
    assert np.all(got < N)
    n_clear = _check_argmax(a, b, got, bf16_b)
    assert n_clear >= 0.9 * M


@pytest.mark.parametrize("bf16_b", [False, True])
def test_matmul_argmax_many_rows_vs_oracle(score, bf16_b):
    # M >= 256 x CUs routes to the register-A / LDS-B kernel; 300 columns = 4 full 64-column
    # chunks + 44, M = 512 x 128 + 37 leaves a partial last workgroup
    M, N, D = 65573, 300, 128
    print(f"argmax rows M={M} N={N} bf16_b={bf16_b}", flush=True)
    a, b = _data(M, N, D, seed=77)
    got = score.matmul_argmax(a, b, bf16_b=bf16_b)
    assert np.all(got < N)
    assert _check_argmax(a, b, got, bf16_b) >= 0.99 * M


def test_matmul_argmax_exact_ties_first_index(score):
    r = np.random.default_rng(12)
    base = r.standard_normal((40, 128)).astype(np.float32)
    # 1000 columns made of 40 distinct rows: every score appears 25 times; the copies sit in
    # different lanes, waves and 256-column chunks, and the first must win
    idx = r.integers(0, 40, 1000)
    b = base[idx]
    a = r.standard_normal((150, 128)).astype(np.float32)
    got = score.matmul_argmax(a, b)
    # the winner is the first column holding the best centroid; the best centroid is clear
    s = a.astype(np.float64) @ base.astype(np.float64).T
    best = np.argmax(s, axis=1)
    srt = np.sort(s, axis=1)
    clear = srt[:, -1] - srt[:, -2] > 1e-3
    first = np.array([np.flatnonzero(idx == c)[0] for c in best])
    np.testing.assert_array_equal(got[clear], first[clear])
    assert clear.sum() > 100
    # all scores equal: index 0
    np.testing.assert_array_equal(score.matmul_argmax(np.zeros((70, 128), np.float32), b), np.zeros(70, np.uint32))
    # the same through the many-rows kernel
    big = np.tile(a, (450, 1))
    got_big = score.matmul_argmax(big, b)
    np.testing.assert_array_equal(got_big[:150][clear], first[clear])
    np.testing.assert_array_equal(got_big.reshape(450, 150), np.tile(got_big[:150], (450, 1)))


def test_packed_right_device_path(score):
    import torch

    a, b = _data(32, 8192, 128, seed=9)  # the streaming kernel's shape
    pr = score.PackedRight(b)
    np.testing.assert_array_equal(pr.matmul(a), score.matmul_t(a, b))
    np.testing.assert_array_equal(pr.argmax(a), score.matmul_argmax(a, b))
    pr16 = score.PackedRight(b, bf16_b=True)
    np.testing.assert_array_equal(pr16.matmul(a), score.matmul_t(a, b, bf16_b=True))
    # reused against a second A of another height
    a2, _ = _data(5, 1, 128, seed=10)
    np.testing.assert_array_equal(pr.matmul(a2), score.matmul_t(a2, b))
    # device entry on a side stream
    s = torch.cuda.Stream()
    da = torch.from_numpy(a).cuda()
    db = torch.from_numpy(b).cuda()
    dc = torch.empty((32, 8192), device="cuda", dtype=torch.float32)
    torch.cuda.synchronize()
    score.matmul_t_device(da.data_ptr(), 32, db.data_ptr(), 8192, 128, dc.data_ptr(), stream=s.cuda_stream)
    s.synchronize()
    np.testing.assert_array_equal(dc.cpu().numpy(), score.matmul_t(a, b))


def test_kmeans_assignment_step(score):
    """One assignment step of kmeans (src/lib.rs:233-236) on clustered data: centers are
    sampled rows, so every row's own center scores highest among near-duplicates."""
    r = np.random.default_rng(21)
    k, per = 64, 40
    centers = r.standard_normal((k, 128)).astype(np.float32)
    centers /= np.linalg.norm(centers, axis=1, keepdims=True)
    labels = np.repeat(np.arange(k), per)
    data = centers[labels] + 0.01 * r.standard_normal((k * per, 128)).astype(np.float32)
    got = score.matmul_argmax(data, centers)
    np.testing.assert_array_equal(got, labels.astype(np.uint32))
    np.testing.assert_array_equal(got, orc.matmul_argmax(data, centers))
