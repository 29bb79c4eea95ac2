"""Mamba2 SSD scan backward — CPU oracle (test infrastructure only, see package doc).

The chunked backward the kernels of csrc/ssd_backward.hip follow, restated in fp64
torch over one sequence: the gradients of the forward of oracle/ssd.py
(training/src/hmf/model/hybrid_zoo/layers/mamba/mamba2.py:555-580 calls the
scan under autograd; mamba_ssm's backward kernels are not vendored, so this is
the chain rule through that recurrence, arranged per chunk).

Per chunk of L tokens, a_t = dt'_t A_h, A_t = sum_{s<=t} a_s from the chunk start,
S0 / S1 the states entering / leaving the chunk, g = dy silu(z) (dy without z):
    M_ts = (C_t.B_s) e^{A_t-A_s},  Q_ts = g_t.x_s,  W_ts = dt'_s Q_ts e^{A_t-A_s}   (s<=t)
    dS0    = e^{A_L} dS1 + sum_t e^{A_t} g_t C_t^T                  (reverse chain)
    dx_s   = sum_t M_ts dt'_s g_t + e^{A_L-A_s} dt'_s dS1 B_s + D g_s
    dC_t   = sum_s W_ts B_s + e^{A_t} S0^T g_t
    dB_s   = sum_t W_ts C_t + e^{A_L-A_s} dt'_s dS1^T x_s
    ddt'_s = sum_t M_ts Q_ts + e^{A_L-A_s} x_s.(dS1 B_s) + A_h da_s
    dA_t   = sum_s W_ts C_t.B_s - sum_u W_ut C_u.B_t + g_t.(e^{A_t} S0 C_t)
             - dt'_t e^{A_L-A_t} x_t.(dS1 B_t) + [t = L-1] <dS1, S1>
    da_s   = sum_{t>=s} dA_t;   dA_h = sum_s dt'_s da_s;   dz = dy y' silu'(z)
with <dS1, S1> = e^{A_L} <dS1, S0> + sum_s dt'_s e^{A_L-A_s} x_s.(dS1 B_s).

``rnd`` (a callable or None) is applied where the kernels store a value in bf16
between launches (each chunk's local terms, S0, dS1), to measure what that storage
costs.  ``_drop_tail`` plants a mistake (the <dS1, S1> term left out) for the test
that shows the comparison against autograd catches it.
"""
from __future__ import annotations

import torch

from .ssd import _group_expand, dt_transform

DEFAULT = torch.float64


def chunk_grads(x, dt, A, B, C, D=None, z=None, dt_bias=None, h0=None, dy=None, d_final=None,
                dt_softplus=False, dt_limit=(0.0, float("inf")), chunk=64, rnd=None,
                _drop_tail=False, dtype=DEFAULT):
    """Gradients of one sequence's scan.  x [T,H,P]; dt [T,H]; A [H]; B [T,G,N];
    C [T,GC,N]; D [H] or [H,P]; z [T,H,P]; dt_bias [H]; h0 [H,P,N]; dy [T,H,P];
    d_final [H,P,N].  Returns a dict x, dt, A, B, C, D, z, dt_bias, h0 (None where
    the input is None), and A_abs = sum_t |dt'_t da_t| per head: dA is that sum of
    terms, which can cancel, so its rounding error scales with A_abs, not |dA|."""
    T, H, P = x.shape
    N = B.shape[-1]
    f = lambda t: None if t is None else t.to(dtype)
    x, dy, A, z, h0, d_final = f(x), f(dy), f(A), f(z), f(h0), f(d_final)
    r = (lambda t: t) if rnd is None else rnd
    Bh, Ch = _group_expand(B.to(dtype), H), _group_expand(C.to(dtype), H)
    # dt' and d dt'/d dt (torch.clamp passes the gradient on [min, max])
    d = dt.to(dtype) + (0 if dt_bias is None else dt_bias.to(dtype))
    sp, slope = d, torch.ones_like(d)
    if dt_softplus:
        sp = torch.where(d <= 20.0, torch.log1p(torch.exp(d)), d)
        slope = torch.where(d <= 20.0, torch.sigmoid(d), torch.ones_like(d))
    dtv = dt_transform(dt, dt_bias, dt_softplus, dt_limit, dtype)
    fac = slope * ((sp >= dt_limit[0]) & (sp <= dt_limit[1])).to(dtype)
    g = dy if z is None else dy * z * torch.sigmoid(z)
    Dm = None
    if D is not None:
        Dm = D.to(dtype)[:, None].expand(H, P) if D.dim() == 1 else D.to(dtype)
    a = dtv * A
    bounds = [(c0, min(T, c0 + chunk)) for c0 in range(0, T, chunk)]
    acs = [a[c0:c1].cumsum(0) for c0, c1 in bounds]                       # [L,H]
    # forward chain: every chunk's start state
    S = torch.zeros(H, P, N, dtype=dtype) if h0 is None else h0.clone()
    S0 = []
    for (c0, c1), cs in zip(bounds, acs):
        S0.append(r(S))
        w = dtv[c0:c1] * torch.exp(cs[-1][None] - cs)                    # [L,H]
        loc = r(torch.einsum("th,thp,thn->hpn", w, x[c0:c1], Bh[c0:c1]))
        S = torch.exp(cs[-1])[:, None, None] * S + loc
    # reverse chain: every chunk's end-state gradient, then the start state's
    G = torch.zeros(H, P, N, dtype=dtype) if d_final is None else d_final.clone()
    dS1 = [None] * len(bounds)
    for i in range(len(bounds) - 1, -1, -1):
        c0, c1 = bounds[i]
        cs = acs[i]
        dS1[i] = r(G)
        share = r(torch.einsum("th,thp,thn->hpn", torch.exp(cs), g[c0:c1], Ch[c0:c1]))
        G = torch.exp(cs[-1])[:, None, None] * G + share
    out = {k: None for k in ("x", "dt", "A", "B", "C", "D", "z", "dt_bias", "h0")}
    dx = torch.zeros_like(x)
    dBh, dCh = torch.zeros_like(Bh), torch.zeros_like(Ch)
    ddtv = torch.zeros(T, H, dtype=dtype)
    dA = torch.zeros(H, dtype=dtype)
    dA_abs = torch.zeros(H, dtype=dtype)
    dz = None if z is None else torch.zeros_like(z)
    for i, (c0, c1) in enumerate(bounds):
        L, cs = c1 - c0, acs[i]
        xs, gs, Bs, Cs, dts = x[c0:c1], g[c0:c1], Bh[c0:c1], Ch[c0:c1], dtv[c0:c1]
        mask = torch.tril(torch.ones(L, L, dtype=dtype))[:, :, None]
        dec = torch.exp((cs[:, None, :] - cs[None, :, :]) * mask) * mask   # [t,s,H]
        CB = torch.einsum("thn,shn->tsh", Cs, Bs)
        Q = torch.einsum("thp,shp->tsh", gs, xs)
        M = CB * dec
        Wm = dts[None, :, :] * Q * dec
        R = Wm * CB
        ea = torch.exp(cs)                                                   # [L,H]
        e = torch.exp(cs[-1][None] - cs)
        y_state = ea[:, :, None] * torch.einsum("thn,hpn->thp", Cs, S0[i])
        dHB = torch.einsum("hpn,shn->shp", dS1[i], Bs)
        dds = e * torch.einsum("shp,shp->sh", xs, dHB)
        if z is not None:
            ypre = torch.einsum("tsh,sh,shp->thp", M, dts, xs) + y_state
            if Dm is not None:
                ypre = ypre + xs * Dm[None]
            zz = z[c0:c1]
            sg = torch.sigmoid(zz)
            dz[c0:c1] = dy[c0:c1] * ypre * sg * (1 + zz * (1 - sg))
        dx[c0:c1] = (torch.einsum("tsh,sh,thp->shp", M, dts, gs)
                     + (e * dts)[:, :, None] * dHB)
        if Dm is not None:
            dx[c0:c1] += gs * Dm[None]
        dCh[c0:c1] = (torch.einsum("tsh,shn->thn", Wm, Bs)
                      + ea[:, :, None] * torch.einsum("thp,hpn->thn", gs, S0[i]))
        dBh[c0:c1] = (torch.einsum("tsh,thn->shn", Wm, Cs)
                      + (e * dts)[:, :, None] * torch.einsum("shp,hpn->shn", xs, dS1[i]))
        dacs = (R.sum(1) - R.sum(0) + torch.einsum("thp,thp->th", gs, y_state) - dts * dds)
        if not _drop_tail:
            dacs[-1] += (torch.exp(cs[-1]) * (dS1[i] * S0[i]).sum((1, 2))
                         + (dts * dds).sum(0))
        da = dacs.flip(0).cumsum(0).flip(0)
        ddtv[c0:c1] = (M * Q).sum(0) + dds + A[None] * da
        dA += (dts * da).sum(0)
        dA_abs += (dts * da).abs().sum(0)
    out["x"] = dx
    out["dt"] = ddtv * fac
    out["A"] = dA
    out["A_abs"] = dA_abs   # sum of |dt'_t da_t|: the scale dA's rounding error follows
    out["B"] = dBh.view(T, B.shape[1], H // B.shape[1], N).sum(2)
    out["C"] = dCh.view(T, C.shape[1], H // C.shape[1], N).sum(2)
    if Dm is not None:
        dD = torch.einsum("thp,thp->hp", g, x)
        out["D"] = dD.sum(1) if D.dim() == 1 else dD
    out["z"] = dz
    if dt_bias is not None:
        out["dt_bias"] = out["dt"].sum(0)
    if h0 is not None:
        out["h0"] = G
    return out
