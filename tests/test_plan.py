"""The host segment planner of libhmx (hmx_plan_segments / _bounds): CPU only.

The C planner is checked against a plain-Python statement of the same policy
(segment counts handed to the sequence with the longest segments, one or two
waves of workgroups, whichever has the smaller makespan estimate) on random
batches, and against the table's invariants: every sequence has >= 1 segment,
its segments tile its chunks in order, and (n, seg_idx, first_seg, nseg) index
the rows consistently."""
import ctypes
import heapq
import random

import numpy as np
import pytest

from hmx import _lib

CHUNK = {_lib.PLAN_GDN: 32, _lib.PLAN_GKA: 64, _lib.PLAN_SSD: 64}
MIN_SEG, WARM, WG_PER_CU = 16, 3, 2


def _py_counts(chunks, budget):
    ns = [1] * len(chunks)
    heap = [(-c, n) for n, c in enumerate(chunks)]
    heapq.heapify(heap)
    total = len(chunks)
    while total < budget and heap:
        neg, n = heapq.heappop(heap)
        if -neg < 2 * MIN_SEG or chunks[n] / (ns[n] + 1) < MIN_SEG:
            continue
        ns[n] += 1
        total += 1
        heapq.heappush(heap, (-chunks[n] / ns[n], n))
    return ns


def _py_plan(op, bounds, H, cu_count, segment_chunks=None):
    chunk = CHUNK[op]
    chunks = [-(-(e - b) // chunk) for b, e in bounds]
    if segment_chunks:
        counts = [max(1, -(-nc // segment_chunks)) for nc in chunks]
    else:
        slots = max(1, WG_PER_CU * cu_count // H)
        best = None
        for waves in (1, 2):
            cnt = _py_counts(chunks, waves * slots)
            longest = max((-(-nc // ns) + (WARM if ns > 1 else 0) for nc, ns in zip(chunks, cnt)),
                          default=0)
            est = longest * min(waves, -(-sum(cnt) // slots))
            if best is None or est < best[0]:
                best = (est, cnt)
        counts = best[1]
    rows = []
    for n, ((b, e), nc, ns) in enumerate(zip(bounds, chunks, counts)):
        first = len(rows)
        rows += [[n, b, e, i * nc // ns, (i + 1) * nc // ns, i, first, ns] for i in range(ns)]
    return rows, sum(chunks)


def _check_invariants(op, rows, bounds):
    chunk = CHUNK[op]
    r = 0
    for n, (b, e) in enumerate(bounds):
        nc = -(-(e - b) // chunk)
        first, ns = rows[r][6], rows[r][7]
        assert first == r and ns >= 1
        assert [x[3] for x in rows[r:r + ns]][0] == 0 and rows[r + ns - 1][4] == nc
        for i in range(ns):
            row = rows[r + i]
            assert row[:3] == [n, b, e] and row[5] == i and row[6] == first and row[7] == ns
            if i:
                assert row[3] == rows[r + i - 1][4]
            assert row[3] <= row[4]
        r += ns
    assert r == len(rows)


@pytest.mark.parametrize("op", [_lib.PLAN_GDN, _lib.PLAN_GKA, _lib.PLAN_SSD])
def test_plan_matches_python_statement(op):
    rng = random.Random(7 + op)
    for trial in range(300):
        nseq = rng.choice([1, 1, 2, 3, 8, 17, 64, 300])
        lens = [rng.choice([0, 1, 31, 64, 65, rng.randint(1, 9000), rng.randint(1, 70000)])
                for _ in range(nseq)]
        bounds, t = [], 0
        for n in lens:
            bounds.append((t, t + n))
            t += n
        H = rng.choice([1, 8, 16, 32, 64])
        cu = rng.choice([80, 256, 304])
        seg = rng.choice([None, None, None, 1, 7, 128])
        table, nblk = _lib.plan_segments(op, bounds, t, H, cu, seg)
        exp, exp_blk = _py_plan(op, bounds, H, cu, seg)
        assert table.tolist() == exp, (trial, nseq, H, cu, seg)
        assert nblk == exp_blk
        _check_invariants(op, table.tolist(), bounds)


def test_plan_fills_the_gpu():
    # one long sequence: split into about two workgroups per CU over the heads
    table, _ = _lib.plan_segments(_lib.PLAN_GDN, [(0, 32768)], 32768, 32, 256)
    assert 8 <= len(table) <= 32
    # many short sequences keep one segment each
    b = [(i * 100, i * 100 + 100) for i in range(500)]
    table, _ = _lib.plan_segments(_lib.PLAN_GDN, b, 50000, 32, 256)
    assert len(table) == 500


def _plan_cu(op, cu, nseq, B, T, H=32, cu_count=256, max_rows=None, table=True):
    lib = _lib.load()
    cs = None if cu is None else np.asarray(cu, dtype=np.int64)
    nrows, nblk = ctypes.c_int32(0), ctypes.c_int32(0)
    rc = lib.hmx_plan_segments(op, None if cs is None else cs.ctypes.data_as(ctypes.c_void_p),
                               nseq, B, T, H, cu_count, 0, None, 0, ctypes.byref(nrows),
                               ctypes.byref(nblk))
    if rc or not table:
        return rc, nrows.value, None
    buf = np.zeros((max_rows if max_rows is not None else nrows.value, 8), dtype=np.int32)
    rc = lib.hmx_plan_segments(op, None if cs is None else cs.ctypes.data_as(ctypes.c_void_p),
                               nseq, B, T, H, cu_count, 0, buf.ctypes.data_as(ctypes.c_void_p),
                               buf.shape[0], ctypes.byref(nrows), ctypes.byref(nblk))
    return rc, nrows.value, buf


def test_plan_cu_seqlens_entry_matches_bounds_entry():
    cs = [0, 0, 100, 5000, 5001, 40000]
    rc, n, table = _plan_cu(_lib.PLAN_GKA, cs, 5, 1, 40000)
    assert rc == _lib.HMX_OK
    exp, _ = _lib.plan_segments(_lib.PLAN_GKA, list(zip(cs[:-1], cs[1:])), 40000, 32, 256)
    assert table.tolist() == exp.tolist()
    # no cu_seqlens: B rows of T tokens
    rc, n, table = _plan_cu(_lib.PLAN_GDN, None, 3, 3, 700)
    assert rc == _lib.HMX_OK
    exp, _ = _lib.plan_segments(_lib.PLAN_GDN, [(0, 700), (700, 1400), (1400, 2100)], 2100, 32, 256)
    assert table.tolist() == exp.tolist()


@pytest.mark.parametrize("cs", [[1, 5], [0, 5, 3], [0, 9]])
def test_plan_rejects_bad_offsets(cs):
    rc, _, _ = _plan_cu(_lib.PLAN_GDN, cs, len(cs) - 1, 1, 8)
    assert rc == _lib.HMX_EINVAL


@pytest.mark.parametrize("bounds", [[(5, 3)], [(0, 9)], [(-1, 2)]])
def test_plan_bounds_rejects_bad_ranges(bounds):
    with pytest.raises(ValueError):
        _lib.plan_segments(_lib.PLAN_GDN, bounds, 8, 32, 256)


def test_plan_rejects_short_table_and_bad_op():
    rc, n, _ = _plan_cu(_lib.PLAN_GDN, [0, 32768], 1, 1, 32768, table=False)
    assert rc == _lib.HMX_OK and n > 1
    rc, _, _ = _plan_cu(_lib.PLAN_GDN, [0, 32768], 1, 1, 32768, max_rows=n - 1)
    assert rc == _lib.HMX_EINVAL
    with pytest.raises(ValueError):
        _lib.plan_segments(7, [(0, 10)], 10, 32, 256)
