"""CPU: the GDN training op's host side — the block table, the state-gradient
chain's runs, and the C ABI's argument checks of hmx_gdn_train_fwd / _bwd, which
return before any launch (no GPU needed)."""
import ctypes

import numpy as np
import pytest

from hmx import _lib
from hmx.ops.gdn_train import block_table, chain_segments, check_chain_segments


BOUNDS = [(0, 200), (200, 200), (200, 201), (201, 2249), (2249, 2281)]


def test_block_table_covers_every_token_once():
    rows, cu = block_table(BOUNDS)
    assert cu.tolist() == [0, 7, 7, 8, 72, 73]
    covered = np.zeros(2281, dtype=int)
    for t0, nv, n, c in rows:
        bos, eos = BOUNDS[n]
        assert 1 <= nv <= 32 and t0 == bos + 32 * c and t0 + nv <= eos
        assert nv == 32 or t0 + nv == eos        # only a sequence's last block is short
        covered[t0:t0 + nv] += 1
    assert (covered == 1).all()
    assert [int(r[2]) for r in rows] == sorted(int(r[2]) for r in rows)


@pytest.mark.parametrize("seg", [None, 1, 3, 64, 1000])
def test_chain_runs_partition_each_sequence(seg):
    _, cu = block_table(BOUNDS)
    runs = chain_segments(cu, H=4, cu_count=256, seg_blocks=seg)
    for n in range(len(BOUNDS)):
        mine = [(a, b) for m, a, b in runs if m == n]
        assert mine, f"sequence {n} has no run (its dh0 would not be written)"
        if cu[n] == cu[n + 1]:
            assert mine == [(cu[n], cu[n])]      # one empty run for an empty sequence
            continue
        assert mine[0][0] == cu[n] and mine[-1][1] == cu[n + 1]
        for (a, b), (c, _) in zip(mine, mine[1:]):
            assert b == c                        # consecutive, no gap or overlap
        limit = seg if seg is not None else max(1, -(-int(cu[-1]) * 4 // 768))
        assert all(0 < b - a <= limit for a, b in mine)


def test_chain_runs_default_size():
    """By default about three workgroups per CU over all heads."""
    _, cu = block_table([(0, 32 * 1024)])
    runs = chain_segments(cu, H=32, cu_count=256)
    assert len(runs) == 24 and all(b - a <= 43 for _, a, b in runs)


def _bwd_args(**over):
    a = dict(q=None, q_ts=1024, k=None, v=None, kv_ts=1024, g=None, g_dt=0, beta=None, beta_dt=0,
             dout=None, do_ts=1024, dht=None, hc=None, tab=None, cu=None, nblk=1, N=1, cseg=None,
             ncseg=1, warm=16, thr=20.0, H=8, scale=0.088, l2=1, dq=None, dk=None, dv=None,
             dg=None, dbeta=None, dh0=None, ws=None, ws_bytes=0, stream=None)
    a.update(over)
    return list(a.values())


def test_train_bwd_rejects_bad_arguments():
    lib = _lib.load()
    assert lib.hmx_gdn_train_bwd(*_bwd_args()) == _lib.HMX_EINVAL       # null pointers
    assert b"null pointer" in lib.hmx_last_error()
    fake = ctypes.c_void_p(256)    # never dereferenced: the checks fail before any launch
    ptrs = {k: fake for k in ("q", "k", "v", "g", "beta", "dout", "hc", "tab", "cu", "cseg",
                              "dq", "dk", "dv", "dg", "dbeta")}
    assert lib.hmx_gdn_train_bwd(*_bwd_args(**ptrs, ncseg=0)) == _lib.HMX_EINVAL
    assert b"bad sizes" in lib.hmx_last_error()
    assert lib.hmx_gdn_train_bwd(*_bwd_args(**ptrs, g_dt=7)) == _lib.HMX_EUNSUPPORTED
    assert lib.hmx_gdn_train_bwd(*_bwd_args(**ptrs, q_ts=1001)) == _lib.HMX_EINVAL
    assert b"16-byte aligned" in lib.hmx_last_error()
    assert lib.hmx_gdn_train_bwd(*_bwd_args(**ptrs)) == _lib.HMX_EINVAL   # no workspace
    need = lib.hmx_gdn_train_bwd_workspace_bytes(1, 1, 1, 8)
    assert b"workspace of %d bytes" % need in lib.hmx_last_error()
    # one sequence walked as one run: no exact-run buffers
    assert need == 8 * (128 * 128 + 2 * 32 * 32) * 2 + 8 * 4 + 256


@pytest.mark.parametrize("nseq", [320, 2048])
def test_bwd_workspace_single_run_sequences_cost_no_exact_buffers(nseq):
    """Packed training batches of many short sequences (32768 tokens, H = 32, 256
    CUs): every sequence is one run, so the workspace is the per-block part plus one
    int per run and head; the R / Psi / exact-start buffers (3 x 64 KiB per run and
    head) are sized by the runs beyond each sequence's first only."""
    lib = _lib.load()
    T, H = 32768, 32
    L = T // nseq
    bounds = [(i * L, (i + 1) * L) for i in range(nseq)]
    rows, cu = block_table(bounds)
    runs = chain_segments(cu, H, 256)
    check_chain_segments(runs, cu)
    assert len(runs) == nseq
    nblk = rows.shape[0]
    base = nblk * H * (128 * 128 + 2 * 32 * 32) * 2 + len(runs) * H * 4 + 256
    assert lib.hmx_gdn_train_bwd_workspace_bytes(nblk, len(runs), nseq, H) == base
    # one long sequence cut into 24 runs: 23 runs carry the exact-run buffers
    rows1, cu1 = block_table([(0, T)])
    runs1 = chain_segments(cu1, H, 256)
    got = lib.hmx_gdn_train_bwd_workspace_bytes(rows1.shape[0], len(runs1), 1, H)
    assert got == (rows1.shape[0] * H * (128 * 128 + 2 * 32 * 32) * 2 + len(runs1) * H * 4
                   + (len(runs1) - 1) * H * 3 * 128 * 128 * 4 + 256)


@pytest.mark.parametrize("seg", [None, 1, 3])
def test_check_chain_segments_accepts_the_built_tables(seg):
    _, cu = block_table(BOUNDS)
    check_chain_segments(chain_segments(cu, H=4, cu_count=256, seg_blocks=seg), cu)


def test_check_chain_segments_rejects_other_orders():
    """The backward's compact exact-run indexing and its per-sequence binary search
    need the grouped, tiling order; the host check refuses anything else."""
    _, cu = block_table(BOUNDS)
    good = chain_segments(cu, H=4, cu_count=256, seg_blocks=3)
    bad = [good[::-1],                                   # sequences descending
           np.delete(good, 0, axis=0),                   # a sequence's first run missing
           good[[1, 0] + list(range(2, len(good)))],     # runs of a sequence swapped
           np.delete(good, [i for i, r in enumerate(good) if r[0] == 1], axis=0)]  # empty seq
    g2 = good.copy()
    g2[0, 2] -= 1                                        # a gap between two runs
    bad.append(g2)
    for b in bad:
        with pytest.raises(ValueError):
            check_chain_segments(b, cu)


def test_train_fwd_requires_block_states():
    lib = _lib.load()
    rc = lib.hmx_gdn_train_fwd(None, 1024, None, None, 1024, None, 0, None, 0, None, None, None,
                               None, 1, 1, 8, 0.088, 1, 16, 20.0, None, 0, None, None, None)
    assert rc == _lib.HMX_EINVAL
    assert b"block_states" in lib.hmx_last_error()
