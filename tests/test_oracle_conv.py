"""Pins the causal conv1d oracle (oracle/conv.py) against torch.nn.functional.conv1d
and its own state semantics (vLLM's causal_conv1d_fn / _update are un-vendored and
ship no vectors):
  - zero initial state: equals F.conv1d(groups=dim, padding=W-1) truncated to T,
    for W = 2, 3, 4 and with bias, with and without silu;
  - an initial state is the prefix: equals F.conv1d on [state; x] keeping the last
    T outputs;
  - a sequence split in two calls with the state carried equals one call;
  - T single-token updates equal one prefill over the T tokens (outputs and state);
  - pad slots are skipped; has_initial_state False ignores the stored state;
  - state_len > W - 1 (speculative slack): the window uses the last W - 1 rows;
  - prefix caching (block arguments): resuming from any written block state over
    the rest of the sequence, or decoding one more token from the last one, equals
    the uninterrupted run; the decode reads one column and writes another.
"""
import torch
import torch.nn.functional as F

from oracle import conv as ref

D64 = torch.float64


def _torch_conv(xfull, w, b, T):
    """Depthwise conv over [L, dim] rows via F.conv1d, last T outputs."""
    y = F.conv1d(xfull.t().unsqueeze(0), w.unsqueeze(1), b, groups=w.shape[0])
    return y[0].t()[-T:]


def test_zero_state_equals_conv1d():
    g = torch.Generator().manual_seed(0)
    for W in (2, 3, 4):
        x = torch.randn(37, 24, generator=g, dtype=D64)
        w = torch.randn(24, W, generator=g, dtype=D64)
        b = torch.randn(24, generator=g, dtype=D64)
        pad = torch.cat([torch.zeros(W - 1, 24, dtype=D64), x])
        for act, f in ((None, lambda y: y), ("silu", F.silu)):
            out, st = ref.conv_sequence(x, None, w, b, act)
            assert torch.allclose(out, f(_torch_conv(pad, w, b, 37)), rtol=1e-13, atol=1e-13)
            assert torch.equal(st, x[-(W - 1):])


def test_state_is_prefix():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(9, 16, generator=g, dtype=D64)
    w = torch.randn(16, 4, generator=g, dtype=D64)
    st = torch.randn(3, 16, generator=g, dtype=D64)
    out, ns = ref.conv_sequence(x, st, w, None, "silu")
    assert torch.allclose(out, F.silu(_torch_conv(torch.cat([st, x]), w, None, 9)), rtol=1e-13,
                          atol=1e-13)
    # a sequence shorter than the state keeps the older rows in front
    out2, ns2 = ref.conv_sequence(x[:2], st, w, None, "silu")
    assert torch.equal(ns2, torch.cat([st[2:], x[:2]]))


def test_split_and_decode_steps():
    g = torch.Generator().manual_seed(2)
    x = torch.randn(20, 8, generator=g, dtype=D64)
    w = torch.randn(8, 4, generator=g, dtype=D64)
    b = torch.randn(8, generator=g, dtype=D64)
    st0 = torch.randn(3, 8, generator=g, dtype=D64)
    full, stf = ref.conv_sequence(x, st0, w, b, "silu")
    o1, s1 = ref.conv_sequence(x[:7], st0, w, b, "silu")
    o2, s2 = ref.conv_sequence(x[7:], s1, w, b, "silu")
    assert torch.allclose(torch.cat([o1, o2]), full, rtol=1e-14, atol=1e-14) and torch.equal(s2, stf)
    pool = st0.unsqueeze(0).clone()
    outs = []
    for t in range(20):
        o, pool = ref.causal_conv1d_update(x[t:t + 1], pool, w, b, "silu", torch.tensor([0]))
        outs.append(o)
    assert torch.allclose(torch.cat(outs), full, rtol=1e-14, atol=1e-14)
    assert torch.equal(pool[0], stf)


def test_varlen_pad_and_initial_flags():
    g = torch.Generator().manual_seed(3)
    lens = [5, 0, 3, 7]
    qs = torch.tensor([0, 5, 5, 8, 15])
    x = torch.randn(15, 8, generator=g, dtype=D64)
    w = torch.randn(8, 3, generator=g, dtype=D64)
    pool = torch.randn(6, 2, 8, generator=g, dtype=D64)
    idx = torch.tensor([4, 1, -1, 0])
    init = torch.tensor([True, True, True, False])
    out, new = ref.causal_conv1d_varlen(x, w, None, pool, qs, idx, init, "silu")
    o0, s0 = ref.conv_sequence(x[0:5], pool[4], w, None, "silu")
    o3, s3 = ref.conv_sequence(x[8:15], None, w, None, "silu")
    assert torch.equal(out[0:5], o0) and torch.equal(new[4], s0)
    assert torch.equal(out[8:15], o3) and torch.equal(new[0], s3)
    assert torch.equal(out[5:8], torch.zeros(3, 8, dtype=D64))   # pad slot: untouched
    assert torch.equal(new[1], pool[1])                           # empty sequence: state kept
    # no flags: no initial states (vLLM's causal_conv1d_fn reads the cache only where a
    # has_initial_state tensor says so)
    out_n, new_n = ref.causal_conv1d_varlen(x, w, None, pool, qs, idx, None, "silu")
    out_f, new_f = ref.causal_conv1d_varlen(x, w, None, pool, qs, idx,
                                            torch.zeros(4, dtype=torch.bool), "silu")
    assert torch.equal(out_n, out_f) and torch.equal(new_n, new_f)


def test_state_slack_rows():
    """state_len = W - 1 + 2: the window reads the last W - 1 rows; the state shifts."""
    g = torch.Generator().manual_seed(4)
    w = torch.randn(8, 4, generator=g, dtype=D64)
    st = torch.randn(5, 8, generator=g, dtype=D64)
    x = torch.randn(1, 8, generator=g, dtype=D64)
    out, ns = ref.conv_sequence(x, st, w, None, None)
    assert torch.allclose(out, _torch_conv(torch.cat([st[2:], x]), w, None, 1), rtol=1e-14,
                          atol=1e-14)
    assert torch.equal(ns, torch.cat([st[1:], x]))


def _blocks_case(seed, ncomp, lens, bs, L, W, dim=8, slots=40):
    """Sequences continuing ncomp[b] computed tokens with lens[b] new ones, blocks
    of bs tokens: the [batch, blocks] table with distinct slots, block indices as
    vLLM's builder forms them (the block of the last computed token, of the first
    and of the last scheduled token)."""
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(dim, W, generator=g, dtype=D64)
    b = torch.randn(dim, generator=g, dtype=D64)
    pool = torch.randn(slots, L, dim, generator=g, dtype=D64)
    x = torch.randn(sum(lens), dim, generator=g, dtype=D64)
    nblk = max((n + t - 1) // bs + 1 for n, t in zip(ncomp, lens))
    perm = torch.randperm(slots, generator=g)
    table = perm[:len(lens) * nblk].view(len(lens), nblk).to(torch.int32)
    init = torch.tensor([max(n - 1, 0) // bs for n in ncomp])
    first = torch.tensor([n // bs for n in ncomp])
    last = torch.tensor([(n + t - 1) // bs for n, t in zip(ncomp, lens)])
    qs = torch.tensor([0] + list(torch.tensor(lens).cumsum(0)))
    has = torch.tensor([n > 0 for n in ncomp])
    return w, b, pool, x, table, init, first, last, qs, has


def test_prefix_cache_block_states_resume_the_run():
    """Prefix caching: the state written for a block is the state to resume from.
    Continuing from a block's slot over the rest of the sequence gives the same
    outputs as the uninterrupted run, and continuing from the last column's slot
    with one more token equals the run over one more token; blocks that end inside
    the initial state's window (a block boundary fewer than state_len tokens after
    num_computed_tokens) take their older rows from the initial state."""
    W, L, bs = 4, 3, 4
    ncomp, lens = [5, 0, 2, 7], [11, 9, 1, 2]
    w, b, pool, x, table, init, first, last, qs, has = _blocks_case(8, ncomp, lens, bs, L, W)
    out, st = ref.causal_conv1d_varlen_blocks(x, w, b, pool, qs, table, has, init, first, last,
                                              torch.tensor(ncomp), bs, "silu")
    g = torch.Generator().manual_seed(9)
    written = set()
    for s in range(len(lens)):
        xs = x[int(qs[s]):int(qs[s + 1])]
        s0 = pool[int(table[s, int(init[s])])] if ncomp[s] > 0 else None
        o_full, _ = ref.conv_sequence(xs, s0, w, b, "silu")
        assert torch.allclose(out[int(qs[s]):int(qs[s + 1])], o_full, rtol=1e-13, atol=1e-13)
        for k in range(int(first[s]), int(last[s])):
            end = (k + 1) * bs - ncomp[s]              # tokens of this step in block k and before
            assert 0 < end < lens[s]
            o_rest, _ = ref.conv_sequence(xs[end:], st[int(table[s, k])], w, b, "silu")
            assert torch.allclose(o_rest, o_full[end:], rtol=1e-13, atol=1e-13), (s, k)
            written.add(int(table[s, k]))
        nxt = torch.randn(1, xs.shape[1], generator=g, dtype=D64)
        o_next, _ = ref.conv_sequence(torch.cat([xs, nxt]), s0, w, b, "silu")
        o_dec, _ = ref.conv_sequence(nxt, st[int(table[s, int(last[s])])], w, b, "silu")
        assert torch.allclose(o_dec, o_next[-1:], rtol=1e-13, atol=1e-13)
        written.add(int(table[s, int(last[s])]))
    # sequence 3 (ncomp 7) crosses the boundary at 8 after one token, fewer than the
    # state's L = 3 rows: that block's state holds two rows of the initial state
    assert int(first[3]) == 1 < int(last[3]) and 0 < 2 * bs - ncomp[3] < L
    for slot in range(pool.shape[0]):
        if slot not in written:
            assert torch.equal(st[slot], pool[slot])


def test_prefix_cache_decode_reads_one_block_writes_another():
    """Decode with prefix caching: reads the column of the last computed token and
    writes the column of the scheduled one; one such step from a block boundary
    equals the plain decode on the read slot, and the read slot is unchanged."""
    g = torch.Generator().manual_seed(10)
    W, L, dim = 3, 2, 8
    w = torch.randn(dim, W, generator=g, dtype=D64)
    pool = torch.randn(10, L, dim, generator=g, dtype=D64)
    x = torch.randn(3, dim, generator=g, dtype=D64)
    table = torch.tensor([[4, 7], [1, 1], [-1, 9]], dtype=torch.int32)
    init = torch.tensor([0, 1, 0])
    last = torch.tensor([1, 1, 1])
    out, st = ref.causal_conv1d_update_blocks(x, pool, w, None, "silu", table, init, last)
    o_plain, st_plain = ref.causal_conv1d_update(x[:2], pool, w, None, "silu",
                                                 torch.tensor([4, 1]))
    assert torch.equal(out[:2], o_plain) and torch.equal(out[2], torch.zeros(dim, dtype=D64))
    assert torch.equal(st[7], st_plain[4]) and torch.equal(st[4], pool[4])
    assert torch.equal(st[1], st_plain[1]) and torch.equal(st[9], pool[9])
