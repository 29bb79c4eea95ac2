"""GPU parity: hmx Mamba2 SSD chunk scan and selective_state_update vs the CPU oracle.

Scan: all four (headdim, d_state) tiles, GQA groups, initial/final states, D per
head and per (head, headdim), z gating, seq_idx restarts, cu_seqlens varlen
states, forced multi-segment decomposition (exact scalar-decay combine), the vLLM
varlen signature with non-contiguous (head-major) x/B views, empty and 1-token
sequences, and C4 (b=2, T=16384, H=64) checked on one group's heads over the full
length.  Decode: slot-indexed fp32 and bf16 pools, tied (per-head) and full A,
pad slots, separate destination slots, and T decode steps == the scan.
"""
import math

import pytest
import torch

import hmx
from oracle import ssd as ref
from util import assert_out_close, assert_state_close

pytestmark = pytest.mark.gpu


def _inputs(b, l, H, G, P, N, seed, z=False):
    g0 = torch.Generator().manual_seed(seed)
    x = torch.randn(b, l, H, P, generator=g0).bfloat16()
    B = torch.randn(b, l, G, N, generator=g0).bfloat16()
    C = torch.randn(b, l, G, N, generator=g0).bfloat16()
    dt = torch.randn(b, l, H, generator=g0) * 0.5 - 2.0
    u = torch.rand(H, generator=g0)
    bias = ref.softplus_inverse(torch.exp(u * (math.log(0.1) - math.log(1e-3)) + math.log(1e-3)))
    A = -torch.exp(torch.rand(H, generator=g0) * math.log(16))
    D = torch.randn(H, generator=g0) * 0.1 + 1.0
    zz = torch.randn(b, l, H, P, generator=g0).bfloat16() if z else None
    return x, dt, A, B, C, D, bias, zz, g0


def _d(dev, *ts):
    return [None if t is None else t.to(dev) for t in ts]


@pytest.mark.parametrize("P,N", [(64, 128), (128, 128), (64, 64), (128, 64)])
def test_scan_batch_initial_and_final_states(dev, P, N):
    b, l, H, G = 2, 300, 8, 2
    x, dt, A, B, C, D, bias, _, g0 = _inputs(b, l, H, G, P, N, 100 + P + N)
    h0 = torch.randn(b, H, P, N, generator=g0) * 0.1
    y_r, f_r = ref.mamba_chunk_scan_combined(x, dt, A, B, C, 256, D=D, dt_bias=bias,
                                             initial_states=h0, dt_softplus=True,
                                             return_final_states=True)
    y, f = hmx.mamba_chunk_scan_combined(*_d(dev, x, dt, A, B, C), 256, D=D.to(dev),
                                         dt_bias=bias.to(dev), initial_states=h0.to(dev),
                                         dt_softplus=True, return_final_states=True)
    torch.cuda.synchronize()
    assert y.dtype == torch.bfloat16 and y.shape == x.shape
    assert_out_close(y, y_r, what="y")
    assert_state_close(f, f_r, what="final_states")


@pytest.mark.parametrize("seg,P", [(None, 64), (2, 64), (2, 128)])
def test_scan_seq_idx_z_dhdim_varlen_states(dev, seg, P):
    l, H, G, N = 1000, 4, 1, 128
    x, dt, A, B, C, D, bias, z, g0 = _inputs(1, l, H, G, P, N, 7, z=True)
    Dh = torch.randn(H, P, generator=g0) * 0.1 + 1.0
    h0 = torch.randn(1, H, P, N, generator=g0) * 0.1
    lens = [390, 1, 609]
    cu = torch.tensor([0, 390, 391, 1000], dtype=torch.int32)
    seq_idx = torch.repeat_interleave(torch.arange(3, dtype=torch.int32), torch.tensor(lens))[None]
    y_r, f_r, v_r = ref.mamba_chunk_scan_combined(
        x, dt, A, B, C, 256, D=Dh, z=z, dt_bias=bias, initial_states=h0, seq_idx=seq_idx,
        cu_seqlens=cu, dt_softplus=True, return_final_states=True, return_varlen_states=True)
    y, f, v = hmx.mamba_chunk_scan_combined(
        *_d(dev, x, dt, A, B, C), 256, D=Dh.to(dev), z=z.to(dev), dt_bias=bias.to(dev),
        initial_states=h0.to(dev), seq_idx=seq_idx.to(dev), cu_seqlens=cu.to(dev),
        dt_softplus=True, return_final_states=True, return_varlen_states=True,
        _segment_chunks=seg)
    torch.cuda.synchronize()
    assert_out_close(y, y_r, what="y")
    assert_state_close(f, f_r, what="final_states")
    assert_state_close(v, v_r, what="varlen_states")


def test_scan_dt_limit_and_no_softplus(dev):
    l, H, G, P, N = 200, 4, 2, 64, 128
    x, dt, A, B, C, D, bias, _, _ = _inputs(1, l, H, G, P, N, 8)
    dtp = torch.rand(1, l, H) * 0.2     # already positive: dt_softplus=False
    y_r = ref.mamba_chunk_scan_combined(x, dtp, A, B, C, 64, D=D, dt_limit=(0.02, 0.15))
    y = hmx.mamba_chunk_scan_combined(*_d(dev, x, dtp, A, B, C), 64, D=D.to(dev),
                                      dt_limit=(0.02, 0.15))
    torch.cuda.synchronize()
    assert_out_close(y, y_r, what="y")


@pytest.mark.parametrize("seg", [None, 1])
def test_varlen_vllm_layout(dev, seg):
    """vLLM's call: x/B are head-major views rearranged to [T, H, P]; per-sequence
    initial states; ``out`` preallocated; ngroups == nheads (primed layout)."""
    H, P, N = 8, 64, 128
    lens = [130, 0, 1, 64, 500]
    T = sum(lens)
    cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0)), dtype=torch.int32)
    g0 = torch.Generator().manual_seed(9)
    xh = torch.randn(H, T, P, generator=g0).bfloat16()       # [group, seq, d] as in the layer
    Bh = torch.randn(H, T, N, generator=g0).bfloat16()
    C = torch.randn(T, H, N, generator=g0).bfloat16()
    dt = (torch.randn(T, H, generator=g0) * 0.5 - 2.0).bfloat16()
    bias = torch.randn(H, generator=g0) * 0.5 - 4.0
    A = -torch.exp(torch.rand(H, generator=g0) * math.log(16))
    D = torch.randn(H, generator=g0) * 0.1 + 1.0
    h0 = torch.randn(len(lens), H, P, N, generator=g0) * 0.1
    x, B = xh.transpose(0, 1), Bh.transpose(0, 1)              # non-contiguous [T, H, *]
    y_r, s_r = ref.mamba_chunk_scan_combined_varlen(x, dt, A, B, C, 256, cu, D=D, dt_bias=bias,
                                                    initial_states=h0, dt_softplus=True)
    xd, Bd = xh.to(dev).transpose(0, 1), Bh.to(dev).transpose(0, 1)
    out = torch.empty(T, H, P, dtype=torch.bfloat16, device=dev)
    s = hmx.mamba_chunk_scan_combined_varlen(
        xd, dt.to(dev), A.to(dev), Bd, C.to(dev), 256, cu_seqlens=cu.to(dev), out=out,
        D=D.to(dev), dt_bias=bias.to(dev), initial_states=h0.to(dev), dt_softplus=True,
        state_dtype=torch.float32, _segment_chunks=seg)
    torch.cuda.synchronize()
    assert_out_close(out, y_r, what="y")
    assert_state_close(s, s_r, what="varlen_states")
    assert torch.equal(s[1].cpu(), h0[1])          # empty sequence: state passes through


def test_scan_c4_full_size(dev):
    """C4 (b=2, T=16384, H=64, P=64, N=128, G=8): the whole call on the GPU, checked
    on heads 0-3 (group 0) of row 1 over the full length with the fp64 chunked form."""
    from hmx import workloads as wl
    d = wl.ssd_inputs(config_id=4)
    y, f = hmx.mamba_chunk_scan_combined(
        d["x"].to(dev), d["dt"].to(dev), d["A"].to(dev), d["B"].to(dev), d["C"].to(dev), 256,
        D=d["D"].to(dev), dt_bias=d["dt_bias"].to(dev), dt_softplus=True,
        return_final_states=True)
    torch.cuda.synchronize()
    assert torch.isfinite(y.float()).all() and torch.isfinite(f).all()
    r, hs = 1, slice(0, 4)
    dtp = ref.dt_transform(d["dt"][r, :, hs], d["dt_bias"][hs], True)
    y_r, s_r = ref.ssd_chunked(d["x"][r, :, hs], dtp, d["A"][hs], d["B"][r, :, 0:1],
                               d["C"][r, :, 0:1], 256, D=d["D"][hs])
    assert_out_close(y[r, :, hs], y_r, what="y")
    assert_state_close(f[r, hs], s_r, what="final_states")


@pytest.mark.parametrize("state_dtype,tied,use_z", [(torch.float32, True, True),
                                                    (torch.bfloat16, False, False),
                                                    (torch.float32, False, True)])
def test_state_update_pool(dev, state_dtype, tied, use_z):
    slots, bsz, H, G, P, N = 10, 6, 8, 2, 64, 128
    g0 = torch.Generator().manual_seed(11)
    pool = (torch.randn(slots, H, P, N, generator=g0) * 0.1).to(state_dtype)
    x = torch.randn(bsz, H, P, generator=g0).bfloat16()
    dth = torch.randn(bsz, H, generator=g0) * 0.5 - 2.0
    dt = dth[:, :, None].expand(bsz, H, P)
    if tied:
        A = (-torch.exp(torch.rand(H, generator=g0) * math.log(16)))[:, None, None].expand(H, P, N)
    else:
        A = -torch.rand(H, P, N, generator=g0) * 4
    B = torch.randn(bsz, G, N, generator=g0).bfloat16()
    C = torch.randn(bsz, G, N, generator=g0).bfloat16()
    D = (torch.randn(H, generator=g0) * 0.1 + 1.0)[:, None].expand(H, P)
    bias = (torch.randn(H, generator=g0) * 0.5 - 4.0)[:, None].expand(H, P)
    z = torch.randn(bsz, H, P, generator=g0).bfloat16() if use_z else None
    src = torch.tensor([3, 7, -1, 0, 9, 5], dtype=torch.int32)
    dst = torch.tensor([3, 1, -1, 0, 2, 5], dtype=torch.int32)
    o_r, new_r = ref.selective_state_update(pool, x, dt, A, B, C, D, z, bias, True, src, dst)
    pd = pool.to(dev)
    out = torch.zeros(bsz, H, P, dtype=torch.bfloat16, device=dev)
    ret = hmx.selective_state_update(pd, *_d(dev, x, dt, A, B, C, D, z, bias), dt_softplus=True,
                                     state_batch_indices=src.to(dev),
                                     dst_state_batch_indices=dst.to(dev), out=out)
    torch.cuda.synchronize()
    assert ret is out
    live = [0, 1, 3, 4, 5]
    assert_out_close(out[live], o_r[live], what="out")
    tol = 1e-2 if state_dtype == torch.bfloat16 else 1e-3
    assert_state_close(pd.float(), new_r, rel_tol=tol, what="state")
    for untouched in (4, 6, 8):
        assert torch.equal(pd[untouched].cpu(), pool[untouched])


def test_decode_steps_equal_scan(dev):
    T, H, G, P, N = 40, 4, 2, 64, 128
    x, dt, A, B, C, D, bias, z, g0 = _inputs(1, T, H, G, P, N, 12, z=True)
    h0 = torch.randn(1, H, P, N, generator=g0) * 0.1
    y_r, f_r = ref.mamba_chunk_scan_combined(x, dt, A, B, C, 256, D=D, z=z, dt_bias=bias,
                                             initial_states=h0, dt_softplus=True,
                                             return_final_states=True)
    pool = torch.zeros(3, H, P, N, device=dev)
    pool[1] = h0[0].to(dev)
    idx = torch.tensor([1], dtype=torch.int32, device=dev)
    Ae = A.to(dev)[:, None, None].expand(H, P, N)
    De, be = D.to(dev)[:, None].expand(H, P), bias.to(dev)[:, None].expand(H, P)
    ys = []
    for t in range(T):
        ys.append(hmx.selective_state_update(
            pool, x[0, t:t + 1].to(dev), dt[0, t:t + 1].to(dev)[:, :, None].expand(1, H, P), Ae,
            B[0, t:t + 1].to(dev), C[0, t:t + 1].to(dev), De, z[0, t:t + 1].to(dev), be, True,
            state_batch_indices=idx))
    torch.cuda.synchronize()
    assert_out_close(torch.cat(ys), y_r[0], what="y")
    assert_state_close(pool[1], f_r[0], what="state")


def test_errors(dev):
    x, dt, A, B, C, D, bias, _, _ = _inputs(1, 16, 2, 1, 64, 128, 13)
    with pytest.raises(NotImplementedError):
        hmx.mamba_chunk_scan_combined(*_d(dev, x.float(), dt, A, B, C), 256)
    with pytest.raises(NotImplementedError):
        hmx.mamba_chunk_scan_combined(*_d(dev, x[..., :32].contiguous(), dt, A, B, C), 256)
    with pytest.raises(RuntimeError):
        hmx.mamba_chunk_scan_combined(x, dt, A, B, C, 256)
    with pytest.raises(ValueError):                 # chunk states need the chunk metadata
        hmx.mamba_chunk_scan_combined_varlen(
            *_d(dev, x[0], dt[0], A, B[0], C[0]), 256,
            cu_seqlens=torch.tensor([0, 16], dtype=torch.int32, device=dev),
            return_intermediate_states=True)
    with pytest.raises(ValueError):                 # chunks that do not tile the sequence
        hmx.mamba_chunk_scan_combined_varlen(
            *_d(dev, x[0], dt[0], A, B[0], C[0]), 256,
            cu_seqlens=torch.tensor([0, 16], dtype=torch.int32, device=dev),
            cu_chunk_seqlens=torch.tensor([0, 10], dtype=torch.int32),
            seq_idx=torch.tensor([0], dtype=torch.int32), return_intermediate_states=True)
    with pytest.raises(ValueError):
        hmx.mamba_chunk_scan_combined(*_d(dev, x, dt, A, B, C), 256,
                                      initial_states=torch.zeros(2, 2, 64, 128, device=dev))


def _prefix_chunks(lens, computed, chunk=256):
    """vLLM's prefix-cache chunking (the metadata primed_mamba2_layer.py:862-921 reads):
    chunk ends fall where the sequence's absolute position (num_computed_tokens plus
    the offset) is a multiple of chunk, so a sequence's first chunk may be short."""
    cu, seq, last, pos = [0], [], [], 0
    for n, (L, nc) in enumerate(zip(lens, computed)):
        off = 0
        while off < L:
            step = min(chunk - (nc + off) % chunk, L - off)
            off += step
            cu.append(pos + off)
            seq.append(n)
        pos += L
        last.append(len(seq) - 1)
    return cu, seq, last


@pytest.mark.parametrize("pooled", [False, True])
def test_varlen_intermediate_chunk_states(dev, pooled):
    """return_intermediate_states (prefix caching): the state after every chunk of
    cu_chunk_seqlens, each chunk's from the fp64 recurrence chained chunk by chunk
    from the sequence's initial state; y as without it."""
    H, P, N = 4, 64, 128
    lens, computed = [300, 1, 640, 77], [100, 0, 256, 500]
    T = sum(lens)
    cs = [0] + list(torch.tensor(lens).cumsum(0).tolist())
    cu_c, seq, last = _prefix_chunks(lens, computed)
    g0 = torch.Generator().manual_seed(31)
    x = torch.randn(T, H, P, generator=g0).bfloat16()
    B = torch.randn(T, H, N, generator=g0).bfloat16()
    C = torch.randn(T, H, N, generator=g0).bfloat16()
    dt = torch.randn(T, H, generator=g0) * 0.5 - 2.0
    bias = torch.randn(H, generator=g0) * 0.5 - 4.0
    A = -torch.exp(torch.rand(H, generator=g0) * math.log(16))
    D = torch.randn(H, generator=g0) * 0.1 + 1.0
    h0 = torch.randn(len(lens), H, P, N, generator=g0) * 0.1
    dtp = ref.dt_transform(dt, bias, True)
    exp_states, y_r = [], torch.zeros(T, H, P, dtype=torch.float64)
    for n in range(len(lens)):
        S = h0[n]
        for c in range(len(seq)):
            if seq[c] != n:
                continue
            a, e = cu_c[c], cu_c[c + 1]
            y_r[a:e], S = ref.ssd_seq(x[a:e], dtp[a:e], A, B[a:e], C[a:e], D, None, S)
            exp_states.append(S)
    exp_states = torch.stack(exp_states)
    out = torch.empty(T, H, P, dtype=torch.bfloat16, device=dev)
    kw = dict(cu_seqlens=torch.tensor(cs, dtype=torch.int32, device=dev),
              cu_chunk_seqlens=torch.tensor(cu_c, dtype=torch.int32, device=dev),
              seq_idx=torch.tensor(seq, dtype=torch.int32, device=dev),
              last_chunk_indices=torch.tensor(last, dtype=torch.int32, device=dev), out=out,
              D=D.to(dev), dt_bias=bias.to(dev), dt_softplus=True,
              return_intermediate_states=True)
    if pooled:
        pool = torch.zeros(6, H, P, N, device=dev)
        slots = torch.tensor([4, 0, 5, 2], dtype=torch.int32, device=dev)
        pool[slots.long()] = h0.to(dev)
        st = hmx.mamba_chunk_scan_combined_varlen(
            *_d(dev, x, dt, A, B, C), 256, initial_states=pool, ssm_state_indices=slots, **kw)
        for n in range(len(lens)):         # the pool holds each sequence's end state
            assert_state_close(pool[int(slots[n])], exp_states[last[n]], what=f"pool slot {n}")
    else:
        st = hmx.mamba_chunk_scan_combined_varlen(*_d(dev, x, dt, A, B, C), 256,
                                                  initial_states=h0.to(dev), **kw)
    torch.cuda.synchronize()
    assert st.shape == (len(seq), H, P, N)
    assert_out_close(out, y_r, what="y")
    for c in range(len(seq)):
        assert_state_close(st[c], exp_states[c], what=f"chunk {c}")


@pytest.mark.parametrize("seg", [1, 2])
def test_scan_split_fast_and_slow_decay_heads(dev, seg):
    """Split sequences (forced 1- and 2-chunk segments) whose heads decay fast and
    very slowly (A down to -5e-4, so the segment combine carries nearly all of the
    state), with initial states, against the fp64 oracle: y of every head and the
    final states."""
    b, l, H, G, P, N = 2, 64 * 7 + 5, 4, 2, 64, 128
    x, dt, A, B, C, D, bias, _, g0 = _inputs(b, l, H, G, P, N, 77)
    A = torch.tensor([-8.0, -2e-3, -3.0, -5e-4])
    h0 = torch.randn(b, H, P, N, generator=g0) * 0.1
    y_r, f_r = ref.mamba_chunk_scan_combined(x, dt, A, B, C, 256, D=D, dt_bias=bias,
                                             initial_states=h0, dt_softplus=True,
                                             return_final_states=True)
    y, f = hmx.mamba_chunk_scan_combined(*_d(dev, x, dt, A, B, C), 256, D=D.to(dev),
                                         dt_bias=bias.to(dev), initial_states=h0.to(dev),
                                         dt_softplus=True, return_final_states=True,
                                         _segment_chunks=seg)
    torch.cuda.synchronize()
    assert_out_close(y, y_r, what="y")
    assert_state_close(f, f_r, what="final_states")
    for hh in range(H):
        assert_out_close(y[:, :, hh], y_r[:, :, hh], what=f"y head {hh}")


@pytest.mark.parametrize("case,seg", [("x", None), ("x", 2), ("B", None), ("C", 2),
                                      ("state", None), ("spike", 2)])
def test_scan_values_outside_fp16_range(dev, case, seg):
    """bf16 x, B or C (or an initial state) far outside fp16's range: the plain pass
    detects the overflow (inf reaches the end state or y) and the flagged walks run
    again with bf16 operands, so the result is the same computation at any
    magnitude.  The outputs and states divided by the scale a (a power of two:
    exact) meet the ordinary tolerances; seg 2 splits the sequences (the LOCAL pass
    and the combine see the large values too).  spike: one chunk of x at 2^20 between
    ordinary ones."""
    b, l, H, G, P, N = 2, 300, 4, 2, 64, 128
    x, dt, A, B, C, D, bias, _, g0 = _inputs(b, l, H, G, P, N, 61)
    h0 = torch.randn(b, H, P, N, generator=g0) * 0.1
    a = 2.0 ** 17
    if case == "x":
        x, h0 = (x.float() * a).bfloat16(), h0 * a
    elif case == "B":
        B = (B.float() * a).bfloat16()
    elif case == "C":
        C = (C.float() * a).bfloat16()
    elif case == "state":
        a = 2.0 ** 20
        h0 = h0 * a
    else:
        a = 2.0 ** 20
        x = x.float()
        x[:, 128:192] *= a
        x = x.bfloat16()
    big = max(x.float().abs().max(), B.float().abs().max(), C.float().abs().max(), h0.abs().max())
    assert big > 65504 * 4
    y_r, f_r = ref.mamba_chunk_scan_combined(x, dt, A, B, C, 256, D=D, dt_bias=bias,
                                             initial_states=h0, dt_softplus=True,
                                             return_final_states=True)
    y, f = hmx.mamba_chunk_scan_combined(*_d(dev, x, dt, A, B, C), 256, D=D.to(dev),
                                         dt_bias=bias.to(dev), initial_states=h0.to(dev),
                                         dt_softplus=True, return_final_states=True,
                                         _segment_chunks=seg)
    torch.cuda.synchronize()
    assert torch.isfinite(y.float()).all() and torch.isfinite(f).all()
    assert_out_close(y / a, y_r / a, what="y")      # a is a power of two: the division is exact
    assert_state_close(f / a, f_r / a, what="final_states")
