"""The gated delta rule's backward (training) — CPU oracle, test infrastructure
only (see package doc).

Reference (paths relative to the reference repository root):
  GD = training/src/hmf/model/hybrid_zoo/layers/gated_deltanet/gdn.py
  M  = training/src/hmf/model/hybrid_zoo/models/qwen3_5_moe_hmf/modeling_qwen3_5_moe_hmf.py

The training layer calls fla's ``chunk_gated_delta_rule`` (GD:462-476) with q, k, v
expanded to H heads, g = -A_log.exp() softplus(a + dt_bias), beta = sigmoid(b),
and takes its gradient through fla's chunk backward (un-vendored; the layer's own
torch fallback, M:330-407, is the same recurrence differentiated by autograd).
The exact gradient of that recurrence is what both compute:

- ``recurrent_grads``: autograd, in float64, of oracle.gdn.recurrent_seq (the
  per-token recurrence of M:410-449) on one sequence - the oracle the GPU
  backward is compared with.  Pinned by finite differences (torch.autograd.gradcheck)
  in tests/test_oracle_gdn_train.py.
- ``chunk_grads``: the same gradient by the chunked formulas the HIP kernels
  implement (32-token blocks), pinned against ``recurrent_grads``.  Per block with
  S0 the state entering it, gamma the in-block cumsum of g, E = diag(e^gamma),
  F = diag(e^{gamma_L - gamma}), Gm_ij = e^{gamma_i - gamma_j}, unit-norm rows q^, k^:
      Mm = strict_lower(K^ K^T . Gm),  T = (I + diag(beta) Mm)^-1
      Ut = V - E K^ S0,  W = T diag(beta) Ut   (the forward's V_new)
      O  = scale (E Q^ S0 + lower(Q^ K^T . Gm) W),  S_L = e^{gamma_L} S0 + K^T F W
  and backward, with dS the gradient of S_L:
      dW = scale lower(Q^K^T . Gm)^T dO + F K^ dS;  Z = T^T dW;  dV = diag(beta) Z
      dN = -strict_lower(Z W^T);  Dm = diag(beta) dN . Gm;  Dp = scale lower(dO W^T) . Gm
      dQ^ = scale E dO S0^T + Dp K^
      dK^ = -E diag(beta) Z S0^T + F W dS^T + Dp^T Q^ + (Dm + Dm^T) K^
      dbeta = rowdot(Z, Ut) + rowsum(dN . Mm)
      dgamma = rowdot(Q^, scale E dO S0^T) + rowdot(K^, -E diag(beta) Z S0^T - F W dS^T)
               + (rowsum - colsum)(Dp . Q^K^T) + (rowsum - colsum)(Dm . K^K^T),
      dgamma_L += e^{gamma_L} <dS, S0> + sum_j k^_j . (F W dS^T)_j
      dS0 = e^{gamma_L} dS + scale Q^T E dO - K^T E diag(beta) Z
  dg is the in-block reverse cumsum of dgamma, and the L2 normalisation's backward
  maps dq^ to dq = (dq^ - q^ (q^ . dq^)) / sqrt(|q|^2 + 1e-6) (k likewise).
"""
from __future__ import annotations

import torch

from oracle import gdn as gd

DEFAULT = torch.float64


def recurrent_grads(q, k, v, g, beta, scale, S0=None, do=None, dST=None, use_qk_l2norm=True,
                    dtype=DEFAULT):
    """Gradients (dq, dk, dv, dg, dbeta, dS0 or None) of sum(o . do) + <S_T, dST> for ONE
    sequence of the per-token recurrence.  q, k, v [T,H,D]; g, beta [T,H]; S0, dST
    [H,D,D] or None."""
    ins = [t.to(dtype).detach().requires_grad_(True) for t in (q, k, v, g, beta)]
    s0 = None if S0 is None else S0.to(dtype).detach().requires_grad_(True)
    o, ST = gd.recurrent_seq(*ins, scale, s0, use_qk_l2norm, dtype)
    loss = (o * do.to(dtype)).sum()
    if dST is not None:
        loss = loss + (ST * dST.to(dtype)).sum()
    grads = torch.autograd.grad(loss, ins + ([s0] if s0 is not None else []), allow_unused=True)
    out = [torch.zeros_like(x) if gr is None else gr for x, gr in zip(ins, grads[:5])]
    return (*out, grads[5] if s0 is not None else None)


def _norm_rows(x, on):
    if not on:
        return x, torch.ones(x.shape[:-1] + (1,), dtype=x.dtype)
    r = torch.rsqrt((x * x).sum(-1, keepdim=True) + 1e-6)
    return x * r, r


def chunk_grads(q, k, v, g, beta, scale, S0=None, do=None, dST=None, use_qk_l2norm=True,
                chunk=32, dtype=DEFAULT):
    """The gradients of ``recurrent_grads`` by the blocked formulas of the module
    docstring (the HIP kernels' algorithm).  Same arguments and returns."""
    T, H, D = q.shape
    q, k, v, g, beta = (t.to(dtype) for t in (q, k, v, g, beta))
    do = do.to(dtype)
    qn, rq = _norm_rows(q, use_qk_l2norm)
    kn, rk = _norm_rows(k, use_qk_l2norm)
    S = torch.zeros(H, D, D, dtype=dtype) if S0 is None else S0.to(dtype).clone()
    blocks = [(c0, min(c0 + chunk, T)) for c0 in range(0, T, chunk)]
    # forward: the state entering each block
    states = []
    for a, b in blocks:
        states.append(S)
        gam = torch.cumsum(g[a:b], 0).T                              # [H, L]
        Gm = torch.exp(gam[:, :, None] - gam[:, None, :])
        Kh, Vh = kn[a:b].transpose(0, 1), v[a:b].transpose(0, 1)      # [H, L, D]
        L = b - a
        Mm = torch.tril(Kh @ Kh.transpose(1, 2) * Gm, -1)
        Tm = torch.linalg.inv(torch.eye(L, dtype=dtype) + beta[a:b].T[:, :, None] * Mm)
        Ut = Vh - torch.exp(gam)[:, :, None] * (Kh @ S)
        W = Tm @ (beta[a:b].T[:, :, None] * Ut)
        S = torch.exp(gam[:, -1])[:, None, None] * S + Kh.transpose(1, 2) @ (
            torch.exp(gam[:, -1:] - gam)[:, :, None] * W)
    dS = torch.zeros(H, D, D, dtype=dtype) if dST is None else dST.to(dtype).clone()
    dqn, dkn, dv = torch.zeros_like(q), torch.zeros_like(k), torch.zeros_like(v)
    dg, dbeta = torch.zeros_like(g), torch.zeros_like(beta)
    for (a, b), S0c in reversed(list(zip(blocks, states))):
        L = b - a
        gam = torch.cumsum(g[a:b], 0).T
        E = torch.exp(gam)[:, :, None]
        F = torch.exp(gam[:, -1:] - gam)[:, :, None]
        eL = torch.exp(gam[:, -1])[:, None, None]
        Gm = torch.exp(gam[:, :, None] - gam[:, None, :])
        Qh, Kh, Vh = (x[a:b].transpose(0, 1) for x in (qn, kn, v))
        dOh = do[a:b].transpose(0, 1)
        bt = beta[a:b].T[:, :, None]
        QK, KK = Qh @ Kh.transpose(1, 2), Kh @ Kh.transpose(1, 2)
        Mm = torch.tril(KK * Gm, -1)
        Pm = torch.tril(QK * Gm)
        Tm = torch.linalg.inv(torch.eye(L, dtype=dtype) + bt * Mm)
        Ut = Vh - E * (Kh @ S0c)
        W = Tm @ (bt * Ut)
        dW = scale * Pm.transpose(1, 2) @ dOh + F * (Kh @ dS)
        Z = Tm.transpose(1, 2) @ dW
        dN = -torch.tril(Z @ W.transpose(1, 2), -1)
        Dm = bt * dN * Gm
        Dp = scale * torch.tril(dOh @ W.transpose(1, 2)) * Gm
        Qt = scale * E * (dOh @ S0c.transpose(1, 2))
        Ut_ = -E * bt * (Z @ S0c.transpose(1, 2))
        St = F * (W @ dS.transpose(1, 2))
        dqh = Qt + Dp @ Kh
        dkh = Ut_ + St + Dp.transpose(1, 2) @ Qh + (Dm + Dm.transpose(1, 2)) @ Kh
        db = (Z * Ut).sum(-1) + (dN * Mm).sum(-1)
        c = (Kh * St).sum(-1)
        dgam = ((Qh * Qt).sum(-1) + (Kh * (Ut_ - St)).sum(-1)
                + (Dp * QK).sum(-1) - (Dp * QK).sum(-2) + (Dm * KK).sum(-1) - (Dm * KK).sum(-2))
        dgam[:, -1] += eL[:, 0, 0] * (dS * S0c).sum((-1, -2)) + c.sum(-1)
        dg[a:b] = torch.flip(torch.cumsum(torch.flip(dgam, [1]), 1), [1]).T
        dbeta[a:b] = db.T
        dqn[a:b], dkn[a:b], dv[a:b] = dqh.transpose(0, 1), dkh.transpose(0, 1), (bt * Z).transpose(0, 1)
        dS = eL * dS + scale * Qh.transpose(1, 2) @ (E * dOh) - Kh.transpose(1, 2) @ (E * bt * Z)
    if use_qk_l2norm:
        dq = rq * (dqn - qn * (qn * dqn).sum(-1, keepdim=True))
        dk = rk * (dkn - kn * (kn * dkn).sum(-1, keepdim=True))
    else:
        dq, dk = dqn, dkn
    return dq, dk, dv, dg, dbeta, (dS if S0 is not None else None)
