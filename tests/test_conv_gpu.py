"""GPU parity: hmx.causal_conv1d_fn / causal_conv1d_update (the mixers' short
causal conv1d) against the CPU oracle.

Covers widths 2-4, bias and none, silu and none, varlen with empty and 1-token
sequences crossing the 64-token tiles, has_initial_state mixes, pad slots, a
state with speculative slack rows (state_len > width - 1), a strided x (the
transposed slice of a fused projection, as the layers pass it), fp32 rows, and T
decode steps against one prefill.  The pool is passed as the layers pass it: the
[slots, dim, state_len] transpose of the [slots, state_len, dim] cache.  States
hold raw inputs, so they must match bit for bit; outputs within the output
rounding.
"""
import pytest
import torch

import hmx
from oracle import conv as ref
from util import assert_out_close

pytestmark = pytest.mark.gpu


def _setup(lens, dim, W, slots, st_len, seed, dt=torch.bfloat16, bias=True):
    g = torch.Generator().manual_seed(seed)
    qs = torch.tensor([0] + list(torch.tensor(lens).cumsum(0)), dtype=torch.int32)
    total = int(qs[-1])
    x = torch.randn(total, dim, generator=g).to(dt)
    w = torch.randn(dim, W, generator=g) * 0.5
    b = torch.randn(dim, generator=g) * 0.1 if bias else None
    pool = torch.randn(slots, st_len, dim, generator=g).to(dt)
    return qs, x, w, b, pool, g


def _close(out, expect):
    """fp32 accumulation, one rounding to bf16: the error beyond half an ulp stays
    at fp32 level; the norm-wise error is bf16 rounding alone (about 1.7e-3)."""
    assert_out_close(out.cpu(), expect, max_abs_tol=1e-4, rel_tol=4e-3)


@pytest.mark.parametrize("W,bias,act", [(4, True, "silu"), (3, False, "silu"), (2, True, None)])
def test_prefill_varlen(dev, W, bias, act):
    lens = [130, 0, 1, 64, 7, 200]
    qs, x, w, b, pool, g = _setup(lens, 1024, W, 9, W - 1, W, bias=bias)
    idx = torch.tensor([3, 0, 8, 5, -1, 1], dtype=torch.int32)
    init = torch.tensor([True, True, False, True, True, False])
    out_r, pool_r = ref.causal_conv1d_varlen(x, w, b, pool, qs, idx, init, act)
    pool_d = pool.to(dev)
    d = lambda t: None if t is None else t.to(dev)
    out = hmx.causal_conv1d_fn(x.to(dev).t(), d(w), d(b), conv_states=pool_d.transpose(1, 2),
                               query_start_loc=d(qs), cache_indices=d(idx),
                               has_initial_state=d(init), activation=act)
    torch.cuda.synchronize()
    assert out.shape == (1024, x.shape[0])
    _close(out.t(), out_r)
    assert torch.equal(pool_d.cpu(), pool_r.to(pool.dtype))


def test_several_channel_groups(dev):
    """4608 channels: two full 2048-channel workgroups and a partial third, for the
    prefill (with states) and the decode update."""
    dim = 4608
    qs, x, w, b, pool, g = _setup([300, 45], dim, 4, 3, 3, 41)
    idx = torch.tensor([2, 0], dtype=torch.int32)
    init = torch.tensor([True, True])
    out_r, pool_r = ref.causal_conv1d_varlen(x, w, b, pool, qs, idx, init, "silu")
    pool_d = pool.to(dev)
    out = hmx.causal_conv1d_fn(x.to(dev).t(), w.to(dev), b.to(dev),
                               conv_states=pool_d.transpose(1, 2), query_start_loc=qs.to(dev),
                               cache_indices=idx.to(dev), has_initial_state=init.to(dev))
    torch.cuda.synchronize()
    _close(out.t(), out_r)
    assert torch.equal(pool_d.cpu(), pool_r.to(pool.dtype))
    xd = torch.randn(2, dim, generator=g).bfloat16()
    o_r, pool_r2 = ref.causal_conv1d_update(xd, pool_r, w, b, "silu", idx)
    o = hmx.causal_conv1d_update(xd.to(dev), pool_d.transpose(1, 2), w.to(dev), b.to(dev),
                                 "silu", conv_state_indices=idx.to(dev))
    torch.cuda.synchronize()
    _close(o, o_r)
    assert torch.equal(pool_d.cpu(), pool_r2.to(pool.dtype))


def test_tokens_past_last_sequence_are_zero(dev):
    """x longer than query_start_loc[-1] (a padded batch): the tail gives 0, and a
    batch of no sequences gives all zeros; validate_data rejects malformed bounds."""
    qs, x, w, b, pool, g = _setup([50, 70], 256, 4, 2, 3, 31)
    xp = torch.cat([x, torch.randn(90, 256, generator=g).bfloat16()])   # 90 padding tokens
    out_r, pool_r = ref.causal_conv1d_varlen(x, w, b, pool, qs, None, None, "silu")
    pool_d = pool.to(dev)
    out = hmx.causal_conv1d_fn(xp.to(dev).t(), w.to(dev), b.to(dev),
                               conv_states=pool_d.transpose(1, 2), query_start_loc=qs.to(dev))
    torch.cuda.synchronize()
    _close(out.t()[:120], out_r)
    assert torch.equal(out.t()[120:].cpu(), torch.zeros(90, 256, dtype=x.dtype))
    assert torch.equal(pool_d.cpu(), pool_r.to(pool.dtype))
    none = hmx.causal_conv1d_fn(xp[:40].to(dev).t(), w.to(dev), None,
                                query_start_loc=torch.zeros(1, dtype=torch.int32, device=dev))
    torch.cuda.synchronize()
    assert torch.equal(none.cpu(), torch.zeros(256, 40, dtype=x.dtype))
    with pytest.raises(ValueError):
        hmx.causal_conv1d_fn(xp[:40].to(dev).t(), w.to(dev), None, validate_data=True,
                             query_start_loc=torch.tensor([0, 30, 20], dtype=torch.int32,
                                                          device=dev))


def test_prefill_no_state_strided_and_fp32(dev):
    g = torch.Generator().manual_seed(11)
    proj = torch.randn(300, 3 * 512, generator=g).bfloat16().to(dev)
    x = proj[:, 512:1536]                 # a slice of a fused projection
    w = (torch.randn(1024, 4, generator=g) * 0.5).to(dev)
    out = hmx.causal_conv1d_fn(x.t(), w, None)
    torch.cuda.synchronize()
    o_r, _ = ref.conv_sequence(x.cpu(), None, w.cpu(), None, "silu")
    _close(out.t(), o_r)
    xf = torch.randn(90, 256, generator=g)
    wf = torch.randn(256, 3, generator=g)
    outf = hmx.causal_conv1d_fn(xf.to(dev).t(), wf.to(dev), None, activation=None)
    torch.cuda.synchronize()
    o_r, _ = ref.conv_sequence(xf, None, wf, None, None)
    assert_out_close(outf.t().cpu(), o_r, max_abs_tol=1e-5, rel_tol=1e-6)


@pytest.mark.parametrize("st_len", [3, 5])
def test_decode_steps_equal_prefill(dev, st_len):
    """T single-token updates == one prefill (outputs and final state), with a pad
    entry in the batch and state_len slack rows."""
    dim, W, T = 512, 4, 9
    qs, x, w, b, pool, g = _setup([T] * 3, dim, W, 4, st_len, 20 + st_len)
    xs = x.view(3, T, dim)
    idx = torch.tensor([2, 0, 3], dtype=torch.int32)
    pool_d = pool.to(dev)
    outs = []
    for t in range(T):
        bidx = idx.clone()
        if t == 4:
            bidx[1] = -1      # a padded entry in one step
        o = hmx.causal_conv1d_update(xs[:, t].contiguous().to(dev), pool_d.transpose(1, 2),
                                     w.to(dev), b.to(dev), "silu",
                                     conv_state_indices=bidx.to(dev))
        outs.append(o.cpu())
        if t == 4:
            assert torch.equal(o[1].cpu(), torch.zeros(dim, dtype=x.dtype))
    torch.cuda.synchronize()
    # sequences 0 and 2 never padded: equal the oracle's prefill from their slots
    for n in (0, 2):
        o_r, s_r = ref.conv_sequence(xs[n], pool[idx[n]], w, b, "silu")
        _close(torch.stack([outs[t][n] for t in range(T)]), o_r)
        assert torch.equal(pool_d[idx[n]].cpu(), s_r.to(pool.dtype))
    # the oracle's decode agrees step by step as well (pad skipped at step 4)
    pool_r = pool.clone().double()
    for t in range(T):
        bidx = idx.clone()
        if t == 4:
            bidx[1] = -1
        o_r, pool_r = ref.causal_conv1d_update(xs[:, t], pool_r, w, b, "silu", bidx)
        _close(outs[t], o_r)
    assert torch.equal(pool_d.cpu(), pool_r.to(pool.dtype))


def test_errors(dev):
    x = torch.zeros(8, 64, dtype=torch.bfloat16, device=dev)
    w = torch.zeros(64, 4, device=dev)
    pool = torch.zeros(2, 3, 64, dtype=torch.bfloat16, device=dev).transpose(1, 2)
    with pytest.raises(ValueError):   # the speculative form needs query_start_loc as well
        hmx.causal_conv1d_update(x, pool, w, num_accepted_tokens=torch.ones(8, device=dev))
    with pytest.raises(NotImplementedError):
        hmx.causal_conv1d_fn(x.t(), torch.zeros(64, 5, device=dev))    # width 5
    with pytest.raises(ValueError):
        hmx.causal_conv1d_fn(x.t(), torch.zeros(32, 4, device=dev))    # weight/dim mismatch
    with pytest.raises(ValueError):    # the cache rows themselves, not the [slots, dim, len] view
        hmx.causal_conv1d_update(x, pool.transpose(1, 2).contiguous(), w)
    with pytest.raises(ValueError):    # the block arguments come together, with a slot table
        hmx.causal_conv1d_update(x, pool, w, initial_state_idx=torch.zeros(8, device=dev))
    with pytest.raises(ValueError):
        hmx.causal_conv1d_fn(x.t(), w, conv_states=pool, num_computed_tokens=torch.zeros(
            1, dtype=torch.int32, device=dev))
    with pytest.raises(ValueError):    # prefix caching needs a [batch, blocks] table
        z = torch.zeros(8, dtype=torch.int32, device=dev)
        hmx.causal_conv1d_update(x, pool, w, conv_state_indices=z, initial_state_idx=z,
                                 block_idx_last_scheduled_token=z)


def test_prefill_more_tiles_than_one_launch(dev):
    """65535 * 64 + 200 tokens: the token tiles exceed one launch's grid (65535 in
    y), so the prefill runs as two launches; a sequence boundary falls inside the
    second.  8 channels keep it at 67 MB."""
    T = 65535 * 64 + 200
    lens = [T - 150, 150]
    qs, x, w, b, pool, g = _setup(lens, 8, 4, 3, 3, 11)
    idx = torch.tensor([2, 0], dtype=torch.int32)
    init = torch.tensor([True, False])
    out_r, pool_r = ref.causal_conv1d_varlen(x, w, b, pool, qs, idx, init, "silu")
    pool_d = pool.to(dev)
    d = lambda t: t.to(dev)
    out = hmx.causal_conv1d_fn(x.to(dev).t(), d(w), d(b), conv_states=pool_d.transpose(1, 2),
                               query_start_loc=d(qs), cache_indices=d(idx),
                               has_initial_state=d(init), activation="silu")
    torch.cuda.synchronize()
    _close(out.t(), out_r)
    assert torch.equal(pool_d.cpu(), pool_r.to(pool.dtype))


@pytest.mark.parametrize("W,L,act", [(4, 6, "silu"), (3, 5, None), (2, 4, "silu"), (4, 8, "silu")])
def test_update_spec_accepts_like_plain_conv(dev, W, L, act):
    """Speculative multi-token update (num_accepted_tokens, query_start_loc): every
    step carries 1 + L - W + 1 tokens per sequence (the draft slack the state holds).
    Step 1 from a random state with any accepted count a1: its window is state rows
    a1-1 .. a1+W-3, its outputs the plain causal conv over that window and the
    tokens, and its state the kept rows followed by the inputs.  Step 2 accepting a2
    of step 1's tokens then equals the plain conv over (window, the a2 accepted
    inputs, the new tokens) - the invariant that pins vLLM's un-vendored row
    arithmetic.  A padded sequence writes 0 and leaves the pool alone."""
    S1 = L - W + 2
    dim, slots = 64, 6
    g = torch.Generator().manual_seed(900 + 10 * W + L)
    idx = torch.tensor([4, 0, 2, -1], dtype=torch.int32)
    N = idx.numel()
    qs = torch.arange(0, N * S1 + 1, S1, dtype=torch.int32)
    pool = torch.randn(slots, L, dim, generator=g).bfloat16()
    w = torch.randn(dim, W, generator=g) * 0.5
    b = torch.randn(dim, generator=g) * 0.1
    a1 = torch.tensor([1, S1, min(2, S1), 1], dtype=torch.int32)
    a2 = torch.tensor([S1, 1, min(2, S1), 1], dtype=torch.int32)
    x1 = torch.randn(N * S1, dim, generator=g).bfloat16()
    x2 = torch.randn(N * S1, dim, generator=g).bfloat16()
    pool_d = pool.to(dev)
    view = pool_d.transpose(1, 2)
    o1 = hmx.causal_conv1d_update(x1.to(dev), view, w.to(dev), b.to(dev), act,
                                  conv_state_indices=idx.to(dev), num_accepted_tokens=a1.to(dev),
                                  query_start_loc=qs.to(dev), max_query_len=S1)
    st1 = pool_d.cpu()
    o2 = hmx.causal_conv1d_update(x2.to(dev), view, w.to(dev), b.to(dev), act,
                                  conv_state_indices=idx.to(dev), num_accepted_tokens=a2.to(dev),
                                  query_start_loc=qs.to(dev), max_query_len=S1)
    torch.cuda.synchronize()
    for n in range(N):
        r = slice(int(qs[n]), int(qs[n + 1]))
        if int(idx[n]) < 0:
            assert (o1[r] == 0).all() and (o2[r] == 0).all()
            continue
        slot, a = int(idx[n]), int(a1[n])
        win1 = pool[slot, a - 1:a + W - 2]
        o_r, _ = ref.conv_sequence(x1[r], win1, w, b, act)
        _close(o1[r], o_r)
        assert torch.equal(st1[slot], torch.cat([pool[slot, a:a + L - S1], x1[r]]))
        hist = torch.cat([win1, x1[r][:int(a2[n])]])           # accept a2 of step 1's tokens
        o_r2, _ = ref.conv_sequence(x2[r], hist[-(W - 1):], w, b, act)
        _close(o2[r], o_r2)
    untouched = [s for s in range(slots) if s not in set(int(i) for i in idx if i >= 0)]
    assert torch.equal(st1[untouched], pool[untouched])


@pytest.mark.parametrize("W,bs", [(4, 16), (3, 64), (2, 8)])
def test_prefill_prefix_cache_blocks(dev, W, bs):
    """Prefix caching (vLLM's block arguments, primed_mamba2_layer.py:770-793): a
    [batch, blocks] slot table, sequences continuing num_computed_tokens tokens (0,
    unaligned, aligned, a block boundary inside the first state_len tokens, one
    crossing 64-token tiles and several blocks), a padded last column and a pad
    in a middle column.  Outputs within the output rounding; every written block
    state and every untouched slot bit for bit."""
    dim, L = 1024, W - 1
    ncomp = [0, 2 * bs + 3, 3 * bs, bs - 1, 5, bs + 2]
    lens = [3 * bs + 7, 2 * bs + 11, 1, 2, 150, 2 * bs]
    slots = 128
    qs, x, w, b, pool, g = _setup(lens, dim, W, slots, L, 40 + W)
    nblk = max((n + t - 1) // bs + 1 for n, t in zip(ncomp, lens))
    assert len(lens) * nblk <= slots
    table = torch.randperm(slots, generator=g)[:len(lens) * nblk].view(len(lens), nblk)
    table = table.to(torch.int32)
    table[4, (ncomp[4] + lens[4] - 1) // bs] = -1    # sequence 4: padded entry
    table[5, ncomp[5] // bs] = -1                    # sequence 5: its first block (and read slot) pad
    init = torch.tensor([max(n - 1, 0) // bs for n in ncomp], dtype=torch.int32)
    first = torch.tensor([n // bs for n in ncomp], dtype=torch.int32)
    last = torch.tensor([(n + t - 1) // bs for n, t in zip(ncomp, lens)], dtype=torch.int32)
    has = torch.tensor([n > 0 for n in ncomp])
    nc = torch.tensor(ncomp, dtype=torch.int32)
    out_r, pool_r = ref.causal_conv1d_varlen_blocks(x, w, b, pool, qs, table, has, init, first,
                                                    last, nc, bs, "silu")
    pool_d = pool.to(dev)
    d = lambda t: t.to(dev)
    out = hmx.causal_conv1d_fn(x.to(dev).t(), d(w), d(b), conv_states=pool_d.transpose(1, 2),
                               query_start_loc=d(qs), cache_indices=d(table),
                               has_initial_state=d(has), activation="silu",
                               block_idx_first_scheduled_token=d(first),
                               block_idx_last_scheduled_token=d(last), initial_state_idx=d(init),
                               num_computed_tokens=d(nc), block_size_to_align=bs)
    torch.cuda.synchronize()
    _close(out.t(), out_r)
    assert torch.equal(pool_d.cpu(), pool_r.to(pool.dtype))


def test_update_prefix_cache_blocks(dev):
    """Decode with prefix caching (primed_mamba2_layer.py:964-973): the window from
    the column of the last computed token, the shifted state into the column of the
    scheduled one (the same column or the next block's), pad entries skipped."""
    W, dim = 4, 2048 + 512
    g = torch.Generator().manual_seed(77)
    pool = torch.randn(12, W - 1, dim, generator=g).bfloat16()
    x = torch.randn(4, dim, generator=g).bfloat16()
    w = torch.randn(dim, W, generator=g) * 0.5
    table = torch.tensor([[4, 7, 0], [1, 2, 3], [-1, 9, 10], [5, 6, 11]], dtype=torch.int32)
    init = torch.tensor([0, 2, 0, 1], dtype=torch.int32)
    last = torch.tensor([1, 2, 1, 2], dtype=torch.int32)
    out_r, pool_r = ref.causal_conv1d_update_blocks(x, pool, w, None, "silu", table, init, last)
    pool_d = pool.to(dev)
    out = hmx.causal_conv1d_update(x.to(dev), pool_d.transpose(1, 2), w.to(dev), None, "silu",
                                   conv_state_indices=table.to(dev),
                                   block_idx_last_scheduled_token=last.to(dev),
                                   initial_state_idx=init.to(dev))
    torch.cuda.synchronize()
    _close(out, out_r)
    assert torch.equal(pool_d.cpu(), pool_r.to(pool.dtype))
