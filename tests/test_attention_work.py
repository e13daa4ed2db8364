"""The attention work list (host planner, t5h_attention_work; no GPU): every query tile of every
(sequence, head) appears exactly once, the 8 per-XCD lists are padded to one length with empty
items, each (sequence, head) runs on one XCD in consecutive slots, and the list stays within
the capacity the workspace reserves for it."""
import numpy as np
import pytest

from witchcraft_amd.encoder import attention_work

QT, SMALL_L = 128, 128  # queries per workgroup; sequences up to SMALL_L tokens take 64


def item_queries(L):
    return 64 if L <= SMALL_L else QT


def _check(cu, heads, max_len=2048):
    items = attention_work(cu, heads)
    n = len(items)
    assert n % 8 == 0
    slots = n // 8
    B = len(cu) - 1
    # every (sequence, head, query tile) exactly once
    want = {(int(cu[b]), int(cu[b + 1] - cu[b]), q, h)
            for b in range(B) for h in range(heads) for q in range(0, int(cu[b + 1] - cu[b]), item_queries(int(cu[b + 1] - cu[b])))}
    real = [tuple(int(v) for v in it) for it in items if it[1] > 0]
    assert len(real) == len(set(real)) == len(want)
    assert set(real) == want
    # padding items are all zero
    assert all((it == 0).all() for it in items if it[1] == 0)
    # per XCD: real items first, then padding; a (sequence, head) stays on one XCD, in
    # consecutive slots, its query tiles in order
    where = {}
    for x in range(8):
        lst = items[x::8]
        lens = lst[:, 1]
        nz = np.nonzero(lens == 0)[0]
        if nz.size:
            assert (lens[nz[0]:] == 0).all()
        for slot, it in enumerate(lst):
            if it[1] == 0:
                continue
            key = (int(it[0]), int(it[3]))
            where.setdefault(key, []).append((x, slot, int(it[2])))
    for key, locs in where.items():
        assert len({x for x, _, _ in locs}) == 1, key
        slots_ = [s for _, s, _ in locs]
        assert slots_ == list(range(slots_[0], slots_[0] + len(slots_))), key
        assert [q for _, _, q in locs] == sorted(q for _, _, q in locs)
    # within the workspace's reservation: heads * (ceil(T / 64) + B) + 8 * (max(2, items(max_len)) + 1)
    T = int(cu[-1])
    assert n <= heads * ((T + 63) // 64 + B) + 8 * (max(2, (max_len + QT - 1) // QT) + 1)
    return items


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_ragged_batches(seed):
    r = np.random.default_rng(seed)
    for lens in (r.integers(32, 257, 32), r.integers(64, 513, 256), r.integers(1, 2049, 40),
                 np.full(40, 2048), r.integers(1, 65, 5)):
        cu = np.zeros(len(lens) + 1, np.int32)
        cu[1:] = np.cumsum(lens)
        _check(cu, 12)


def test_edge_batches():
    _check(np.array([0, 1], np.int32), 12)        # one token
    _check(np.array([0, 32], np.int32), 12)       # the query regime
    _check(np.array([0, 0, 5, 5, 70], np.int32), 3)  # empty sequences
    _check(np.array([0, 2048], np.int32), 1)
    _check(np.array([0, 64, 129, 193, 321], np.int32), 12)  # either side of the 64-query items
    _check(np.array([0, 65, 193], np.int32), 2)
    assert len(attention_work(np.array([0], np.int32), 12)) == 0  # no sequences


def test_xcd_load_is_balanced():
    # 2048-token windows: every XCD gets the same number of (sequence, head) groups
    cu = np.arange(0, 41 * 2048, 2048, dtype=np.int32)
    items = _check(cu, 12)
    per_xcd = [int((items[x::8][:, 1] > 0).sum()) for x in range(8)]
    assert max(per_xcd) - min(per_xcd) <= 32
