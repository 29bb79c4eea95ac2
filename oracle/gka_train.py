"""The training-side Chebyshev solve of GKA, forward and backward — CPU oracle,
test infrastructure only (see package doc).

Reference (paths relative to the reference repository root):
  CI = training/src/hmf/model/hybrid_zoo/layers/gated_kalmanet/ops/chebyshev/chebyshev_iteration.py
  DK = .../ops/chebyshev/chunk_dk_backward.py, chunk_dk_backward_gating.py
  DH = .../ops/chebyshev/chunk_dh_kk_to_dk_backward.py, chunk_dh_kk_to_dk_gating_backward.py

``ChebyshevIteration`` (CI:560-688) solves (H_t + lam_t I) x_t = q_t per token with
H_t = sum_{s<=t} e^{G_t - G_s} k_s k_s^T (G the running sum of gk, h0 = None) and
lam_t = r |H_t|_F, by the Chebyshev recurrence of CI:308-460 (the same as the
serving kernels').  Its forward returns x and the final H; it saves fro_t = |H_t|_F.

Its backward (CI:606-688) treats x as the exact solution:
    dq_t = the same recurrence applied to dx_t, with lam_t from the saved fro_t
           (load_fro = 1, CI:621-632),
    dL/dH_t = G_t = -dq_t x_t^T - [bp_lambda] r (dq_t . x_t) H_t / fro_t,
and dk, dgk are the derivatives of sum_t <G_t, H_t(k, gk)> with G_t held fixed:
the chunked kernels of DK / DH spell these out (the reverse state chunk_bwd_dh
with q = dq, do = x; the in-chunk masked products; the lambda term's suffix sums
over h_kk; dgk as the chunk-local reverse cumsum of the per-position terms).
Here they come from autograd of that sum in float64 over the per-token H_t, which
is the same derivative without the chunking.

The chunk size (64 in the reference) only blocks the computation; it does not
change these values.
"""
from __future__ import annotations

import torch

DEFAULT = torch.float64


def _decays(gk, T, dtype):
    """G [B,T,H]: running sum of gk (zeros without a gate)."""
    return None if gk is None else torch.cumsum(gk.to(dtype), dim=1)


def h_states(k: torch.Tensor, gk: torch.Tensor | None, dtype=DEFAULT) -> torch.Tensor:
    """H_t [B,T,H,D,D] = e^{gk_t} H_{t-1} + k_t k_t^T from zero (CI:497-508,
    chunk_fwd_h with g = the chunk-local cumsum of gk, which composes to this)."""
    B, T, Hh, D = k.shape
    k = k.to(dtype)
    out = []
    Hs = torch.zeros(B, Hh, D, D, dtype=dtype)
    for t in range(T):
        if gk is not None:
            Hs = Hs * torch.exp(gk[:, t].to(dtype))[..., None, None]
        Hs = Hs + k[:, t, :, :, None] * k[:, t, :, None, :]
        out.append(Hs)
    return torch.stack(out, dim=1)


def chebyshev_fixed(Ht: torch.Tensor, rhs: torch.Tensor, fro: torch.Tensor, ridge_ratio: float,
                    num_iter: int) -> torch.Tensor:
    """The recurrence of CI:420-443 with |H_t|_F given (CI:397-406 load_fro):
    tau = 2/(2 lam + f), c = (f/(2 lam + f)/2)^2, x = tau q, x_prev = 0, w = 2;
    n times w <- 1/(1 - c w); x, x_prev <- w x - tau w (H x + lam x - q) - (w-1) x_prev, x.
    Ht [..., D, D], rhs [..., D], fro [...]."""
    lam = ridge_ratio * fro
    denom = 2.0 * lam + fro
    tau = 2.0 / denom
    c = (fro / denom * 0.5) ** 2
    x_prev = torch.zeros_like(rhs)
    x = tau[..., None] * rhs
    w = torch.full_like(fro, 2.0)
    for _ in range(num_iter):
        w = 1.0 / (1.0 - c * w)
        hx = (Ht @ x[..., None])[..., 0]
        grad = (tau * w)[..., None] * (hx + lam[..., None] * x - rhs) + (w - 1.0)[..., None] * x_prev
        x_prev = x
        x = w[..., None] * x - grad
    return x


def chebyshev_iteration_fwd(k, q, gk=None, num_iter=30, ridge_ratio=0.02, dtype=DEFAULT):
    """ChebyshevIteration.forward (CI:569-604) with h0 = None.
    k, q [B,T,H,D]; gk [B,T,H] or None.  Returns (x, fro [B,T,H], h_kk_final [B,H,D,D])."""
    Ht = h_states(k, gk, dtype)
    fro = torch.sqrt((Ht * Ht).sum((-1, -2)))
    x = chebyshev_fixed(Ht, q.to(dtype), fro, ridge_ratio, num_iter)
    return x, fro, Ht[:, -1]


def chebyshev_iteration_bwd(k, x, fro, gk, dx, num_iter=30, ridge_ratio=0.02, bp_lambda=True,
                            dtype=DEFAULT):
    """ChebyshevIteration.backward (CI:606-688) with h0 = None and no gradient of the
    final state.  Returns (dk, dq, dgk or None) in ``dtype``."""
    Ht = h_states(k, gk, dtype)
    fro = fro.to(dtype)
    x = x.to(dtype)
    dq = chebyshev_fixed(Ht, dx.to(dtype), fro, ridge_ratio, num_iter)
    G = -dq[..., :, None] * x[..., None, :]
    if bp_lambda:
        a = -ridge_ratio * (dq * x).sum(-1) / fro
        G = G + a[..., None, None] * Ht
    G = G.detach()
    kk = k.to(dtype).detach().requires_grad_(True)
    gg = None if gk is None else gk.to(dtype).detach().requires_grad_(True)
    sur = (G * h_states(kk, gg, dtype)).sum()
    grads = torch.autograd.grad(sur, [kk] + ([gg] if gg is not None else []))
    return grads[0], dq, (grads[1] if gg is not None else None)


# ---------------------------------------------------------------------------
# The whole training forward gka_chebyshev_gla (gka_chebyshev_solve.py:107-164):
# x = ChebyshevIteration(k, q, gk); u = q + alpha (x - q); o = chunk_simple_gla(u, k,
# v, scale, g) of fla (un-vendored; o_t = scale S_t^T u_t with S_t = e^{g_t} S_{t-1}
# + k_t v_t^T from zero).  Its backward is fla's GLA backward (the exact gradient,
# taken here by autograd of the recurrence), torch's autograd of the blend, and
# ChebyshevIteration.backward on dx = alpha du.
# ---------------------------------------------------------------------------
def gla(u, k, v, g, scale, dtype=DEFAULT):
    """o [B,T,H,V] and the final state [B,H,K,V] of the GLA recurrence (autograd-able)."""
    B, T, H, K = u.shape
    S = torch.zeros(B, H, K, v.shape[-1], dtype=dtype)
    out = []
    for t in range(T):
        S = S * torch.exp(g[:, t].to(dtype))[..., None, None] + k[:, t, :, :, None] * v[:, t, :, None, :]
        out.append(scale * (S * u[:, t, :, :, None]).sum(-2))
    return torch.stack(out, dim=1), S


def gka_chebyshev_gla_fwd(q, k, v, alpha, g, gk, scale, ridge_ratio, num_iter, dtype=DEFAULT):
    """(o, kk_final or None, kv_final, x or None, fro or None) in ``dtype``."""
    q, k, v = q.to(dtype), k.to(dtype), v.to(dtype)
    x = fro = hkk = None
    u = q
    if num_iter > 0:
        x, fro, hkk = chebyshev_iteration_fwd(k, q, gk, num_iter, ridge_ratio, dtype)
        u = q + alpha.to(dtype)[..., None] * (x - q)
    o, hkv = gla(u, k, v, g, scale, dtype)
    return o, hkk, hkv, x, fro


def gka_chebyshev_gla_bwd(q, k, v, alpha, g, gk, scale, ridge_ratio, num_iter, bp_lambda, do,
                          x=None, fro=None, dtype=DEFAULT):
    """Gradients (dq, dk, dv, dalpha or None, dg, dgk or None) of sum(o * do), with
    the solve's part as ChebyshevIteration.backward computes it, given the forward's
    saved x and |H_t|_F."""
    q, k, v, do = q.to(dtype), k.to(dtype), v.to(dtype), do.to(dtype)
    u = q if num_iter == 0 else q + alpha.to(dtype)[..., None] * (x.to(dtype) - q)
    uu = u.detach().requires_grad_(True)
    kk = k.detach().requires_grad_(True)
    vv = v.detach().requires_grad_(True)
    gg = g.to(dtype).detach().requires_grad_(True)
    o, _ = gla(uu, kk, vv, gg, scale, dtype)
    du, dk, dv, dg = torch.autograd.grad((o * do).sum(), [uu, kk, vv, gg])
    if num_iter == 0:
        return du, dk, dv, None, dg, None
    a = alpha.to(dtype)[..., None]
    xd = x.to(dtype)
    dalpha = (du * (xd - q)).sum(-1)
    dk_c, dq_c, dgk = chebyshev_iteration_bwd(k, xd, fro, gk, a * du, num_iter, ridge_ratio,
                                              bp_lambda, dtype)
    return (1 - a) * du + dq_c, dk + dk_c, dv, dalpha, dg, dgk
