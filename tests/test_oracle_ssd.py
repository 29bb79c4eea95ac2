"""Pins the Mamba2 SSD oracle (oracle/ssd.py) with independent checks.

mamba_ssm and vLLM are un-vendored and ship no vectors for this path, so:
  - the per-token recurrence equals the SSD quadratic dual form
    y = (L o C B^T)(dt x) (an independent formula: one T x T matrix, no scan);
  - the scalar case P = N = 1 equals an explicit cumulative-product sum;
  - the chunked form equals the recurrence at chunk 256, 64, 16 and 7;
  - the initial state enters linearly with the scalar carry exp(sum dt'A)
    (mamba_mixer_cp_utils.py:44-65);
  - dt' = 0 leaves the state unchanged (y = S0 C + D x);
  - seq_idx / cu_seqlens equal separate runs per sequence;
  - T decode steps (selective_state_update) equal the scan, and one step equals
    its written-out update; pad slots are skipped;
  - dt transform: softplus threshold 20 and dt_limit clamp.
"""
import math

import torch
import torch.nn.functional as F

from oracle import ssd as ref

D64 = torch.float64


def _inputs(T, H, G, P, N, seed, b=None):
    g0 = torch.Generator().manual_seed(seed)
    sh = (T,) if b is None else (b, T)
    x = torch.randn(*sh, H, P, generator=g0, dtype=D64)
    dt = torch.randn(*sh, H, generator=g0, dtype=D64) * 0.5 - 2.0
    A = -torch.exp(torch.rand(H, generator=g0, dtype=D64) * math.log(16))
    B = torch.randn(*sh, G, N, generator=g0, dtype=D64)
    C = torch.randn(*sh, G, N, generator=g0, dtype=D64)
    D = torch.randn(H, generator=g0, dtype=D64) * 0.1 + 1.0
    dt_bias = ref.softplus_inverse(torch.exp(torch.rand(H, generator=g0, dtype=D64) *
                                             (math.log(0.1) - math.log(1e-3)) + math.log(1e-3)))
    return x, dt, A, B, C, D, dt_bias


def test_recurrence_equals_quadratic_dual_form():
    x, dt, A, B, C, D, bias = _inputs(40, 4, 2, 4, 8, 0)
    dtp = ref.dt_transform(dt, bias, True)
    y, _ = ref.ssd_seq(x, dtp, A, B, C)
    yq = ref.ssd_quadratic(x, dtp, A, B, C)
    assert torch.allclose(y, yq, rtol=1e-10, atol=1e-12)


def test_scalar_case_closed_form():
    T = 25
    g0 = torch.Generator().manual_seed(1)
    x = torch.randn(T, 1, 1, generator=g0, dtype=D64)
    dtp = torch.rand(T, 1, generator=g0, dtype=D64)
    A = torch.tensor([-0.7], dtype=D64)
    B = torch.randn(T, 1, 1, generator=g0, dtype=D64)
    C = torch.randn(T, 1, 1, generator=g0, dtype=D64)
    y, S = ref.ssd_seq(x, dtp, A, B, C)
    for t in range(T):
        h = sum(math.exp(-0.7 * float(dtp[j + 1:t + 1, 0].sum())) * float(dtp[j, 0] * x[j, 0, 0] * B[j, 0, 0])
                for j in range(t + 1))
        assert abs(float(y[t, 0, 0]) - h * float(C[t, 0, 0])) < 1e-12
    assert abs(float(S[0, 0, 0]) - h) < 1e-12


def test_chunked_equals_recurrence_any_chunk():
    x, dt, A, B, C, D, bias = _inputs(300, 4, 2, 8, 16, 2)
    dtp = ref.dt_transform(dt, bias, True)
    h0 = torch.randn(4, 8, 16, dtype=D64)
    z = torch.randn(300, 4, 8, dtype=D64)
    y, S = ref.ssd_seq(x, dtp, A, B, C, D, z, h0)
    for L in (256, 64, 16, 7):
        yc, Sc = ref.ssd_chunked(x, dtp, A, B, C, L, D, z, h0)
        assert torch.allclose(yc, y, rtol=1e-9, atol=1e-11), L
        assert torch.allclose(Sc, S, rtol=1e-9, atol=1e-11), L


def test_initial_state_carry_closed_form():
    """S_T(h0) = exp(sum dt'A) h0 + S_T(0) and y_t(h0) - y_t(0) = exp(cumsum_t) h0 C_t."""
    x, dt, A, B, C, D, bias = _inputs(50, 2, 1, 4, 6, 3)
    dtp = ref.dt_transform(dt, bias, True)
    h0 = torch.randn(2, 4, 6, dtype=D64)
    y1, S1 = ref.ssd_seq(x, dtp, A, B, C, D, None, h0)
    y0, S0 = ref.ssd_seq(x, dtp, A, B, C, D, None, None)
    cum = (dtp * A).cumsum(0)
    assert torch.allclose(S1, S0 + torch.exp(cum[-1])[:, None, None] * h0, rtol=1e-10)
    Ch = C.repeat_interleave(2, dim=1)
    carry = torch.exp(cum)[:, :, None] * torch.einsum("hpn,thn->thp", h0, Ch)
    assert torch.allclose(y1 - y0, carry, rtol=1e-9, atol=1e-12)


def test_zero_dt_keeps_state():
    x, dt, A, B, C, D, bias = _inputs(10, 2, 2, 4, 6, 4)
    h0 = torch.randn(2, 4, 6, dtype=D64)
    y, S = ref.ssd_seq(x, torch.zeros(10, 2, dtype=D64), A, B, C, D, None, h0)
    assert torch.equal(S, h0)
    assert torch.allclose(y, torch.einsum("hpn,thn->thp", h0, C) + x * D[None, :, None])


def test_seq_idx_and_cu_seqlens_equal_separate_runs():
    x, dt, A, B, C, D, bias = _inputs(60, 4, 2, 4, 8, 5, b=1)
    h0 = torch.randn(1, 4, 4, 8, dtype=D64)
    lens = [20, 5, 35]
    cu = torch.tensor([0, 20, 25, 60])
    seq_idx = torch.repeat_interleave(torch.arange(3), torch.tensor(lens))[None]
    y, fin, vs = ref.mamba_chunk_scan_combined(
        x, dt, A, B, C, 16, D=D, dt_bias=bias, initial_states=h0, seq_idx=seq_idx,
        cu_seqlens=cu, dt_softplus=True, return_final_states=True, return_varlen_states=True)
    dtp = ref.dt_transform(dt, bias, True)
    for i in range(3):
        s0, s1 = int(cu[i]), int(cu[i + 1])
        yy, S = ref.ssd_seq(x[0, s0:s1], dtp[0, s0:s1], A, B[0, s0:s1], C[0, s0:s1], D, None,
                            h0[0] if i == 0 else None)
        assert torch.allclose(y[0, s0:s1], yy)
        assert torch.allclose(vs[i], S)
    assert torch.allclose(fin[0], vs[2])
    yv, sv = ref.mamba_chunk_scan_combined_varlen(x[0], dt[0], A, B[0], C[0], 16, cu, D=D,
                                                  dt_bias=bias, initial_states=torch.cat(
                                                      [h0, torch.zeros(2, 4, 4, 8, dtype=D64)]),
                                                  dt_softplus=True)
    assert torch.allclose(yv, y[0]) and torch.allclose(sv, vs)


def test_decode_steps_equal_scan():
    T, H, G, P, N = 12, 4, 2, 4, 8
    x, dt, A, B, C, D, bias = _inputs(T, H, G, P, N, 6)
    h0 = torch.randn(H, P, N, dtype=D64)
    z = torch.randn(T, H, P, dtype=D64)
    y, S = ref.ssd_seq(x, ref.dt_transform(dt, bias, True), A, B, C, D, z, h0)
    pool = torch.zeros(3, H, P, N, dtype=D64)
    pool[2] = h0
    idx = torch.tensor([2])
    Ae = A[:, None, None].expand(H, P, N)
    for t in range(T):
        o, pool = ref.selective_state_update(
            pool, x[t:t + 1], dt[t:t + 1, :, None].expand(1, H, P), Ae, B[t:t + 1], C[t:t + 1],
            D[:, None].expand(H, P), z[t:t + 1], bias[:, None].expand(H, P), True, idx)
        assert torch.allclose(o[0], y[t])
    assert torch.allclose(pool[2], S) and torch.equal(pool[0], torch.zeros_like(pool[0]))


def test_decode_step_written_out_and_pad_slots():
    H, G, P, N = 2, 1, 3, 5
    g0 = torch.Generator().manual_seed(7)
    pool = torch.randn(4, H, P, N, generator=g0, dtype=D64)
    x = torch.randn(3, H, P, generator=g0, dtype=D64)
    dt = torch.randn(3, H, P, generator=g0, dtype=D64)
    A = -torch.rand(H, P, N, generator=g0, dtype=D64)
    B = torch.randn(3, G, N, generator=g0, dtype=D64)
    C = torch.randn(3, G, N, generator=g0, dtype=D64)
    src = torch.tensor([1, -1, 3])
    dst = torch.tensor([0, -1, 3])
    o, new = ref.selective_state_update(pool, x, dt, A, B, C, state_batch_indices=src,
                                        dst_state_batch_indices=dst)
    for i, s, d in ((0, 1, 0), (2, 3, 3)):
        Sx = pool[s] * torch.exp(A * dt[i][:, :, None]) + (dt[i] * x[i])[:, :, None] * B[i, 0]
        assert torch.allclose(new[d], Sx)
        assert torch.allclose(o[i], (Sx * C[i, 0]).sum(-1))
    assert torch.equal(o[1], torch.zeros_like(o[1]))
    assert torch.equal(new[1], pool[1]) and torch.equal(new[2], pool[2])


def test_dt_transform_threshold_and_limit():
    d = torch.tensor([-30.0, -1.0, 0.0, 19.9, 20.5, 40.0], dtype=D64)
    out = ref.dt_transform(d, None, True)
    assert torch.allclose(out[:4], F.softplus(d[:4]))
    assert torch.equal(out[4:], d[4:])
    lim = ref.dt_transform(d, torch.tensor(1.0, dtype=D64), True, (0.5, 10.0))
    assert lim.min() == 0.5 and lim.max() == 10.0
