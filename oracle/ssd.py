"""Mamba2 SSD CPU oracle — test infrastructure only (see package doc).

Reference call sites (paths relative to the reference repository root; the
kernels themselves live in un-vendored mamba_ssm 2.3.0 and vLLM 0.15.1):
  M2  = training/src/hmf/model/hybrid_zoo/layers/mamba/mamba2.py
  PML = vllm-inference/src/primed_vllm/primed_mamba2_layer.py
  CP  = training/src/hmf/model/hybrid_zoo/layers/mamba/mamba_mixer_cp_utils.py

Per head h with group g(h) = h // (H/G), state S in R^{P x N} (M2:555-580, :584-645):
    dt'  = clamp(softplus(dt + dt_bias), dt_limit)      softplus(x) = x for x > 20
    S_t  = e^{dt'_t A_h} S_{t-1} + dt'_t x_t B_t^T
    y_t  = S_t C_t + D_h x_t;   y_t *= z_t sigmoid(z_t) when z is given
Decode (selective_state_update, M2:776-800, PML:1000-1021) is one step of the
same recurrence on a slot of the state pool, with A, dt, dt_bias, D given per
(head, headdim[, dstate]) as the callers' expanded views.
Inter-chunk carry (CP:44-65): S_end += exp(sum dt'A) S_prev.
"""
from __future__ import annotations

import torch

DEFAULT = torch.float64


def dt_transform(dt, dt_bias=None, dt_softplus=False, dt_limit=(0.0, float("inf")), dtype=DEFAULT):
    """dt + dt_bias, softplus with threshold 20, clamp to dt_limit (M2:604-605)."""
    d = dt.to(dtype)
    if dt_bias is not None:
        d = d + dt_bias.to(dtype)
    if dt_softplus:
        d = torch.where(d <= 20.0, torch.log1p(torch.exp(d)), d)
    return d.clamp(min=dt_limit[0], max=dt_limit[1])


def _group_expand(t, H):
    return t.repeat_interleave(H // t.shape[-2], dim=-2)


def ssd_seq(x, dtp, A, B, C, D=None, z=None, h0=None, dtype=DEFAULT):
    """Per-token recurrence over ONE sequence.  x [T,H,P]; dtp [T,H] (transformed);
    A [H]; B, C [T,G,N]; D [H] or [H,P]; z [T,H,P]; h0 [H,P,N].
    Returns (y [T,H,P], S [H,P,N])."""
    T, H, P = x.shape
    N = B.shape[-1]
    x = x.to(dtype)
    Bh, Ch = _group_expand(B.to(dtype), H), _group_expand(C.to(dtype), H)
    S = torch.zeros(H, P, N, dtype=dtype) if h0 is None else h0.to(dtype).clone()
    y = torch.zeros(T, H, P, dtype=dtype)
    A = A.to(dtype)
    for t in range(T):
        S = S * torch.exp(dtp[t] * A)[:, None, None] + \
            (dtp[t][:, None] * x[t])[:, :, None] * Bh[t][:, None, :]
        y[t] = torch.einsum("hpn,hn->hp", S, Ch[t])
    if D is not None:
        Dv = D.to(dtype)
        y = y + x * (Dv[None, :, None] if Dv.dim() == 1 else Dv[None])
    if z is not None:
        zz = z.to(dtype)
        y = y * zz * torch.sigmoid(zz)
    return y, S


def ssd_quadratic(x, dtp, A, B, C, dtype=DEFAULT):
    """The SSD dual ('attention') form over one sequence from a zero state:
    y = (L o C B^T)(dt' x) with L_tj = exp(sum_{j<s<=t} dt'_s A) for j <= t
    (Dao & Gu 2024, 'Transformers are SSMs', the quadratic mode).  Materialises the
    full T x T matrix, so it is only for tiny T; an independent check of ssd_seq."""
    T, H, P = x.shape
    Bh, Ch = _group_expand(B.to(dtype), H), _group_expand(C.to(dtype), H)
    a = dtp.to(dtype) * A.to(dtype)                     # [T,H]
    cs = a.cumsum(0)
    Lm = torch.exp(cs[:, None, :] - cs[None, :, :])      # [t,j,H]
    Lm = Lm * torch.tril(torch.ones(T, T, dtype=dtype))[:, :, None]
    G = torch.einsum("thn,jhn->tjh", Ch, Bh)
    return torch.einsum("tjh,jh,jhp->thp", Lm * G, dtp.to(dtype), x.to(dtype))


def ssd_chunked(x, dtp, A, B, C, chunk, D=None, z=None, h0=None, dtype=DEFAULT):
    """The chunked form (intra-chunk quadratic + state carry) over one sequence;
    results equal ssd_seq for any chunk size.  Vectorised over heads; used as the
    CPU baseline and for chunk-size invariance."""
    T, H, P = x.shape
    N = B.shape[-1]
    x = x.to(dtype)
    Bh, Ch = _group_expand(B.to(dtype), H), _group_expand(C.to(dtype), H)
    S = torch.zeros(H, P, N, dtype=dtype) if h0 is None else h0.to(dtype).clone()
    y = torch.zeros(T, H, P, dtype=dtype)
    a_all = dtp.to(dtype) * A.to(dtype)
    for c0 in range(0, T, chunk):
        c1 = min(T, c0 + chunk)
        L = c1 - c0
        cs = a_all[c0:c1].cumsum(0)                                  # [L,H]
        mask = torch.tril(torch.ones(L, L, dtype=dtype))[:, :, None]
        decay = torch.exp((cs[:, None, :] - cs[None, :, :]) * mask) * mask
        G = torch.einsum("thn,jhn->tjh", Ch[c0:c1], Bh[c0:c1])
        dx = dtp[c0:c1].to(dtype)[:, :, None] * x[c0:c1]             # [L,H,P]
        y[c0:c1] = torch.einsum("tjh,jhp->thp", G * decay, dx) + \
            torch.exp(cs)[:, :, None] * torch.einsum("thn,hpn->thp", Ch[c0:c1], S)
        w = torch.exp(cs[-1][None, :] - cs)                          # [L,H]
        S = torch.exp(cs[-1])[:, None, None] * S + \
            torch.einsum("th,thp,thn->hpn", w, dx, Bh[c0:c1])
    if D is not None:
        Dv = D.to(dtype)
        y = y + x * (Dv[None, :, None] if Dv.dim() == 1 else Dv[None])
    if z is not None:
        zz = z.to(dtype)
        y = y * zz * torch.sigmoid(zz)
    return y, S


def _runs(seq_idx_row):
    """Maximal runs of equal seq_idx in one batch row -> [(start, end)]."""
    s = seq_idx_row.tolist()
    out, a = [], 0
    for i in range(1, len(s) + 1):
        if i == len(s) or s[i] != s[a]:
            out.append((a, i))
            a = i
    return out


def mamba_chunk_scan_combined(x, dt, A, B, C, chunk_size, D=None, z=None, dt_bias=None,
                              initial_states=None, seq_idx=None, cu_seqlens=None,
                              dt_softplus=False, dt_limit=(0.0, float("inf")),
                              return_final_states=False, return_varlen_states=False,
                              dtype=DEFAULT):
    """mamba_ssm 2.3.0 ``mamba_chunk_scan_combined`` semantics (call M2:555-580).

    x [b,l,H,P]; dt [b,l,H]; A [H]; B, C [b,l,G,N]; D [H] or [H,P]; z [b,l,H,P];
    initial_states [b,H,P,N] (seeds the first sequence of each row); seq_idx [b,l]
    (the state restarts from zero where it changes); cu_seqlens [n+1] (b == 1) picks
    the states returned as varlen_states (the state after each sequence's last
    token).  Returns y, then final_states [b,H,P,N] if asked, then varlen_states.
    The result does not depend on chunk_size (beyond rounding)."""
    b, l, H, P = x.shape
    N = B.shape[-1]
    dtp = dt_transform(dt, dt_bias, dt_softplus, dt_limit, dtype)
    y = torch.zeros(b, l, H, P, dtype=dtype)
    final = torch.zeros(b, H, P, N, dtype=dtype)
    ends = {}
    for r in range(b):
        if seq_idx is not None:
            runs = _runs(seq_idx[r])
        elif cu_seqlens is not None:
            cs = [int(v) for v in cu_seqlens.tolist()]
            runs = [(cs[i], cs[i + 1]) for i in range(len(cs) - 1) if cs[i + 1] > cs[i]]
        else:
            runs = [(0, l)]
        for i, (s0, s1) in enumerate(runs):
            h0 = initial_states[r] if (initial_states is not None and i == 0 and s0 == 0) else None
            yy, S = ssd_seq(x[r, s0:s1], dtp[r, s0:s1], A, B[r, s0:s1], C[r, s0:s1], D,
                            None if z is None else z[r, s0:s1], h0, dtype)
            y[r, s0:s1] = yy
            ends[(r, s1)] = S
        final[r] = ends[(r, l)] if l > 0 else (0 if initial_states is None else initial_states[r])
    out = [y]
    if return_final_states:
        out.append(final)
    if return_varlen_states:
        cs = [int(v) for v in cu_seqlens.tolist()]
        out.append(torch.stack([ends[(0, cs[i + 1])] for i in range(len(cs) - 1)]))
    return out[0] if len(out) == 1 else tuple(out)


def mamba_chunk_scan_combined_varlen(x, dt, A, B, C, chunk_size, cu_seqlens, D=None, z=None,
                                     dt_bias=None, initial_states=None, dt_softplus=False,
                                     dt_limit=(0.0, float("inf")), dtype=DEFAULT):
    """vLLM 0.15.1 ``mamba_chunk_scan_combined_varlen`` semantics (call PML:844-863):
    x [T,H,P]; dt [T,H]; B, C [T,G,N]; cu_seqlens [n+1]; initial_states [n,H,P,N] or
    None.  Returns (y [T,H,P], varlen_states [n,H,P,N]); every sequence starts from
    its own initial state (zero if none)."""
    T, H, P = x.shape
    N = B.shape[-1]
    dtp = dt_transform(dt, dt_bias, dt_softplus, dt_limit, dtype)
    cs = [int(v) for v in cu_seqlens.tolist()]
    y = torch.zeros(T, H, P, dtype=dtype)
    st = torch.zeros(len(cs) - 1, H, P, N, dtype=dtype)
    for i in range(len(cs) - 1):
        s0, s1 = cs[i], cs[i + 1]
        h0 = None if initial_states is None else initial_states[i]
        if s1 == s0:
            st[i] = 0 if h0 is None else h0.to(dtype)
            continue
        yy, S = ssd_seq(x[s0:s1], dtp[s0:s1], A, B[s0:s1], C[s0:s1], D,
                        None if z is None else z[s0:s1], h0, dtype)
        y[s0:s1] = yy
        st[i] = S
    return y, st


def selective_state_update(state, x, dt, A, B, C, D=None, z=None, dt_bias=None,
                           dt_softplus=False, state_batch_indices=None,
                           dst_state_batch_indices=None, pad_slot_id=-1, dtype=DEFAULT):
    """One decode step (mamba_ssm / vLLM ``selective_state_update``; calls M2:789-800,
    PML:1007-1021), out of place: returns (out [b,H,P], new state pool).

    state [slots,H,P,N]; x, dt [b,H,P]; A [H,P,N]; B, C [b,G,N]; D, dt_bias [H,P];
    z [b,H,P].  Entries whose source index equals pad_slot_id are skipped (out 0)."""
    bsz, H, P = x.shape
    new = state.to(dtype).clone()
    out = torch.zeros(bsz, H, P, dtype=dtype)
    Bh, Ch = _group_expand(B.to(dtype), H), _group_expand(C.to(dtype), H)
    for i in range(bsz):
        src = i if state_batch_indices is None else int(state_batch_indices[i])
        if src == pad_slot_id:
            continue
        dst = src if dst_state_batch_indices is None else int(dst_state_batch_indices[i])
        d = dt[i].to(dtype) + (0 if dt_bias is None else dt_bias.to(dtype))
        if dt_softplus:
            d = torch.where(d <= 20.0, torch.log1p(torch.exp(d)), d)
        dA = torch.exp(A.to(dtype) * d[:, :, None])                   # [H,P,N]
        S = state[src].to(dtype) * dA + (d * x[i].to(dtype))[:, :, None] * Bh[i][:, None, :]
        o = torch.einsum("hpn,hn->hp", S, Ch[i])
        if D is not None:
            o = o + x[i].to(dtype) * D.to(dtype)
        if z is not None:
            zz = z[i].to(dtype)
            o = o * zz * torch.sigmoid(zz)
        out[i] = o
        if dst != pad_slot_id:
            new[dst] = S
    return out, new


def softplus_inverse(y):
    """x with softplus(x) = y (used to draw dt_bias as M2:194-201 does)."""
    return y + torch.log(-torch.expm1(-y))


__all__ = ["dt_transform", "ssd_seq", "ssd_quadratic", "ssd_chunked", "mamba_chunk_scan_combined",
           "mamba_chunk_scan_combined_varlen", "selective_state_update", "softplus_inverse"]
