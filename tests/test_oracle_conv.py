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
  - state_len > W - 1 (speculative slack): the window uses the last W - 1 rows.
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
