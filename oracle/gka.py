"""Gated KalmaNet (GKA) CPU oracle — test infrastructure only (see package doc).

Reference files (paths relative to the reference repository root):
  GF = vllm-inference/src/primed_vllm/gka/gka_forward.py
  CI = vllm-inference/src/primed_vllm/gka/ops/chebyshev_iteration_gqa.py   (decode)
  CP = vllm-inference/src/primed_vllm/gka/ops/chebyshev_prefill_gqa.py     (prefill solve)
  SG = vllm-inference/src/primed_vllm/gka/ops/chunk_simple_gla_gqa.py      (GLA states)
  CO = vllm-inference/src/primed_vllm/gka/ops/chunk_o_gqa.py               (GLA output)
  PL = vllm-inference/src/primed_vllm/primed_gka_layer.py                  (gating)

Per head, with eps = 1e-6, q and k L2-normalised WITHOUT eps (GF:114-159, CI:83-84):
    k~ = (beta + eps) k,  v~ = (beta + eps) v                  (CI:91-93, :141-142)
    H  <- e^{gk} H + k~ k~^T                                    (CI:95; CP:28-106 chunked)
    f  = |H|_F;  lam = r f;  tau = 2/(2 lam + f);  c = (f/(2 lam + f)/2)^2
    x = tau q; x_prev = 0; w = 2;  n times:                     (CI:115-134; CP:227-263)
        w <- 1/(1 - c w);  x, x_prev <- w x - tau w (H x + lam x - q) - (w-1) x_prev, x
    x <- q + alpha (x - q)                                      (CI:136; GF:225)
    S  <- e^{g} S + k~ v~^T;   o = scale S^T x                  (CI:154-157; SG:33-101; CO:25-114)
Decode uses gk for both decays (GF:305 asserts g is gk) and only the first token
of each sequence (CI:79).  Prefill runs the same recurrence for every token
(H_t includes token t; |H_t|_F is exact); with num_iter == 0 the query is only
normalised and no h_kk state is produced (GF:210-227).
"""
from __future__ import annotations

import torch

DEFAULT = torch.float64
EPS = 1e-6


def l2n(x: torch.Tensor) -> torch.Tensor:
    """x / |x| over the last dim, no eps (GF:136, CI:83-84)."""
    return x / torch.sqrt((x * x).sum(-1, keepdim=True))


def gka_gating(A_log, a, alpha_in, b, dt_bias, softplus_beta=1.0, threshold=20.0, dtype=DEFAULT):
    """g = -exp(A_log) softplus(a + dt_bias); alpha = sigmoid(alpha_in); beta = sigmoid(b)
    (PL:224-300).  Returns [1,T,H] tensors (g, alpha, beta)."""
    x = a.to(dtype) + dt_bias.to(dtype)
    bx = softplus_beta * x
    sp = torch.where(bx <= threshold, torch.log1p(torch.exp(bx)) / softplus_beta, x)
    g = -torch.exp(A_log.to(dtype)) * sp
    return (g.unsqueeze(0), torch.sigmoid(alpha_in.to(dtype)).unsqueeze(0),
            torch.sigmoid(b.to(dtype)).unsqueeze(0))


def chebyshev(H: torch.Tensor, q: torch.Tensor, ridge_ratio: float, num_iter: int):
    """The solver on one (H, q) pair (CI:115-134), batched over leading dims.

    H [..., D, D] symmetric; q [..., D].  Returns (x, fro).
    The matvec follows the reference's column-sum form sum_i x_i H[i, j].
    """
    fro = torch.sqrt((H * H).sum((-1, -2)))
    lam = ridge_ratio * fro
    denom = 2.0 * lam + fro
    tau = 2.0 / denom
    c = (fro / denom * 0.5) ** 2
    x_prev = torch.zeros_like(q)
    x = tau[..., None] * q
    w = torch.full_like(fro, 2.0)
    for _ in range(num_iter):
        w = 1.0 / (1.0 - c * w)
        hx = torch.einsum("...i,...ij->...j", x, H)
        grad = (tau * w)[..., None] * (hx + lam[..., None] * x - q) + (w - 1.0)[..., None] * x_prev
        x_prev = x
        x = w[..., None] * x - grad
    return x, fro


def _expand(x, H):
    return x.repeat_interleave(H // x.shape[-2], dim=-2)


def gka_seq(q, k, v, alpha, g, gk, beta, scale, ridge_ratio, num_iter, h_kk0=None, h_kv0=None,
            dtype=DEFAULT, normalize=True):
    """Per-token GKA over ONE sequence (prefill semantics).

    q [T,H,D]; k [T,HKV,D]; v [T,HKV,V]; alpha, g [T,H]; gk, beta [T,H] or None.
    ``normalize=False`` uses q and k as given (the training form, whose layer has
    normalised them).  Returns (o [T,H,V], h_kk [H,D,D] or None, h_kv [H,D,V]).
    """
    T, H, D = q.shape
    V = v.shape[-1]
    nz = l2n if normalize else (lambda x: x)
    q = nz(q.to(dtype))
    k = _expand(nz(k.to(dtype)), H)
    v = _expand(v.to(dtype), H)
    be = None if beta is None else beta.to(dtype) + EPS
    Hs = torch.zeros(H, D, D, dtype=dtype) if h_kk0 is None else h_kk0.to(dtype).clone()
    S = torch.zeros(H, D, V, dtype=dtype) if h_kv0 is None else h_kv0.to(dtype).clone()
    o = torch.zeros(T, H, V, dtype=dtype)
    for t in range(T):
        kt = k[t] if be is None else k[t] * be[t][:, None]
        vt = v[t] if be is None else v[t] * be[t][:, None]
        xq = q[t]
        if num_iter > 0:
            dk = 1.0 if gk is None else torch.exp(gk[t].to(dtype))[:, None, None]
            Hs = Hs * dk + kt[:, :, None] * kt[:, None, :]
            x, _ = chebyshev(Hs, q[t], ridge_ratio, num_iter)
            xq = q[t] + alpha[t].to(dtype)[:, None] * (x - q[t])
        S = S * torch.exp(g[t].to(dtype))[:, None, None] + kt[:, :, None] * vt[:, None, :]
        o[t] = scale * torch.einsum("hkv,hk->hv", S, xq)
    return o, (Hs if num_iter > 0 else None), S


def gka_seq_blocked(q, k, v, alpha, g, gk, beta, scale, ridge_ratio, num_iter, h_kk0=None,
                    h_kv0=None, dtype=DEFAULT, block=256):
    """``gka_seq`` (normalize=True) batched over blocks of up to ``block`` tokens: the
    states H_t and S_t of every token of a block are formed at once by unrolling the
    recurrences (a cumulative sum of e^{-G_j}-scaled outer products, then e^{G_t}),
    then every token's Chebyshev solve and output run as one batched call.  The same
    per-token states and solves in fp64, in another summation order; used where
    ``gka_seq``'s per-token Python loop is too slow (full-length C3 heads)."""
    T, H, D = q.shape
    V = v.shape[-1]
    q = l2n(q.to(dtype))
    k = _expand(l2n(k.to(dtype)), H)
    v = _expand(v.to(dtype), H)
    be = None if beta is None else beta.to(dtype) + EPS
    if be is not None:
        k = k * be[..., None]
        v = v * be[..., None]
    Hs = torch.zeros(H, D, D, dtype=dtype) if h_kk0 is None else h_kk0.to(dtype).clone()
    S = torch.zeros(H, D, V, dtype=dtype) if h_kv0 is None else h_kv0.to(dtype).clone()
    o = torch.zeros(T, H, V, dtype=dtype)
    gk_log = torch.zeros(T, H, dtype=dtype) if gk is None else gk.to(dtype)
    g_log = g.to(dtype)
    t0 = 0
    while t0 < T:
        # block [t0, t1): at most ``block`` tokens, and short enough that the
        # in-block log-decay sums stay above -500 (so e^{-G} stays finite)
        t1 = min(T, t0 + block)
        dec = torch.minimum(torch.cumsum(gk_log[t0:t1], 0).min(-1).values,
                            torch.cumsum(g_log[t0:t1], 0).min(-1).values)
        over = torch.nonzero(dec < -500.0)
        if len(over):
            t1 = t0 + max(1, int(over[0]))
        L = t1 - t0
        # the per-token recurrences H_t = e^{gk_t} H_{t-1} + k~ k~^T and
        # S_t = e^{g_t} S_{t-1} + k~ v~^T, unrolled over the block:
        #   X_t = e^{G_t} (X_{t0-1} + sum_{j<=t} e^{-G_j} x_j),  G = in-block cumsum
        kb, vb = k[t0:t1], v[t0:t1]
        Sst = None
        if num_iter > 0:
            G = torch.cumsum(gk_log[t0:t1], 0)
            Hst = torch.einsum("lhd,lhe->lhde", kb * torch.exp(-G)[..., None], kb)
            Hst = torch.cumsum(Hst, 0).add_(Hs).mul_(torch.exp(G)[..., None, None])
            Hs = Hst[L - 1].clone()
        G = torch.cumsum(g_log[t0:t1], 0)
        Sst = torch.einsum("lhd,lhe->lhde", kb * torch.exp(-G)[..., None], vb)
        Sst = torch.cumsum(Sst, 0).add_(S).mul_(torch.exp(G)[..., None, None])
        S = Sst[L - 1].clone()
        xq = q[t0:t1]
        if num_iter > 0:
            x, _ = chebyshev(Hst, xq, ridge_ratio, num_iter)
            xq = xq + alpha[t0:t1].to(dtype)[..., None] * (x - xq)
        o[t0:t1] = scale * torch.einsum("lhkv,lhk->lhv", Sst, xq)
        t0 = t1
    return o, (Hs if num_iter > 0 else None), S


def gka_chebyshev_gla_prefill(q, k, v, alpha, g, gk, beta, gla_scale, ridge_ratio=0.02,
                              num_iter=30, h_kk_initial=None, h_kv_initial=None,
                              output_final_state=True, cu_seqlens=None, dtype=DEFAULT):
    """GF:161-242 over B sequences or cu_seqlens.  Returns (o, h_kk_final, h_kv_final)."""
    B, T, H, D = q.shape
    V = v.shape[-1]
    if cu_seqlens is None:
        bounds = [(n * T, n * T + T) for n in range(B)]
    else:
        cs = [int(x) for x in cu_seqlens.tolist()]
        bounds = [(cs[n], cs[n + 1]) for n in range(len(cs) - 1)]
    N = len(bounds)
    flat = lambda x: None if x is None else x.reshape(B * T, *x.shape[2:])
    qf, kf, vf, af, gf, gkf, bf = map(flat, (q, k, v, alpha, g, gk, beta))
    o = torch.zeros(B * T, H, V, dtype=dtype)
    hkk = torch.zeros(N, H, D, D, dtype=dtype)
    hkv = torch.zeros(N, H, D, V, dtype=dtype)
    for n, (a, b) in enumerate(bounds):
        h0kk = None if h_kk_initial is None else h_kk_initial[n]
        h0kv = None if h_kv_initial is None else h_kv_initial[n]
        if b == a:
            hkk[n] = 0 if h0kk is None else h0kk.to(dtype)
            hkv[n] = 0 if h0kv is None else h0kv.to(dtype)
            continue
        sl = slice(a, b)
        on, hk, hv = gka_seq(qf[sl], kf[sl], vf[sl], af[sl], gf[sl],
                             None if gkf is None else gkf[sl], None if bf is None else bf[sl],
                             gla_scale, ridge_ratio, num_iter, h0kk, h0kv, dtype)
        o[sl] = on
        hkk[n] = hk if hk is not None else 0
        hkv[n] = hv
    o = o.view(B, T, H, V)
    if not output_final_state:
        return o, None, None
    return o, (hkk if num_iter > 0 else None), hkv


def gka_chebyshev_gla(q, k, v, alpha, g, gk, gla_scale, ridge_strength=0.02, num_iter=30,
                      dtype=DEFAULT):
    """Training-form GKA forward (layers/gated_kalmanet/ops/chebyshev/
    gka_chebyshev_solve.py:107-164): q, k, v [B,L,H,D] used as given (the layer
    normalised q, k with /(|x|+1e-6) and applied (beta+1e-6) to k and v,
    gka.py:477-490); H_t = e^{gk} H + k k^T from zero (ChebyshevIteration with
    h0=None, chebyshev_iteration.py:569-604); GLA with gate g from zero.
    Returns (o, kk_final or None, kv_final)."""
    B, T, H, D = q.shape
    V = v.shape[-1]
    o = torch.zeros(B, T, H, V, dtype=dtype)
    kk = torch.zeros(B, H, D, D, dtype=dtype)
    kv = torch.zeros(B, H, D, V, dtype=dtype)
    for b in range(B):
        gb = torch.zeros(T, H, dtype=dtype) if g is None else g[b]
        o[b], hk, kv[b] = gka_seq(q[b], k[b], v[b], alpha[b], gb, None if gk is None else gk[b],
                                  None, gla_scale, ridge_strength, num_iter, dtype=dtype,
                                  normalize=False)
        if hk is not None:
            kk[b] = hk
    return o, (kk if num_iter > 0 else None), kv


def torch_decoding_one_step(q, k, v, alpha, g, gk, gla_scale, ridge_strength, num_iter,
                            prev_h_kk=None, prev_h_kv=None, dtype=DEFAULT):
    """Training-form single-token step (gka_chebyshev_solve.py:324-397; the h_kk
    update and solve of its inference kernel :167-266): q, k, v [B,1,H,D].
    Returns (o [B,1,H,D], h_kk or None, h_kv)."""
    B, _, H, D = q.shape
    V = v.shape[-1]
    o = torch.zeros(B, 1, H, V, dtype=dtype)
    kk = torch.zeros(B, H, D, D, dtype=dtype)
    kv = torch.zeros(B, H, D, V, dtype=dtype)
    for b in range(B):
        gb = torch.zeros(1, H, dtype=dtype) if g is None else g[b]
        o[b], hk, kv[b] = gka_seq(q[b], k[b], v[b], alpha[b], gb, None if gk is None else gk[b],
                                  None, gla_scale, ridge_strength, num_iter,
                                  None if prev_h_kk is None else prev_h_kk[b],
                                  None if prev_h_kv is None else prev_h_kv[b], dtype=dtype,
                                  normalize=False)
        if hk is not None:
            kk[b] = hk
    return o, (kk if num_iter > 0 else None), kv


def gka_chebyshev_gla_decode(q, k, v, alpha, g, gk, beta, gla_scale, ridge_ratio=0.02,
                             num_iter=30, h_kk=None, h_kv=None, cu_seqlens=None,
                             ssm_state_indices=None, dtype=DEFAULT):
    """GF:248-326 / CI:22-238, out of place: returns (o, new h_kk, new h_kv) where the
    state pools are updated copies.  Only the first token of each sequence is used;
    num_iter == 0 runs one iteration (GF:293-303); decays use gk (GF:305)."""
    if num_iter == 0:
        num_iter = 1
    B, T, H, D = q.shape
    V = v.shape[-1]
    N = B if cu_seqlens is None else len(cu_seqlens) - 1
    hkk = (torch.zeros(N, H, D, D, dtype=dtype) if h_kk is None else h_kk.to(dtype).clone())
    hkv = (torch.zeros(N, H, D, V, dtype=dtype) if h_kv is None else h_kv.to(dtype).clone())
    o = torch.zeros(B, T, H, V, dtype=dtype)
    qf, kf, vf = q.reshape(B * T, H, D), k.reshape(B * T, -1, D), v.reshape(B * T, -1, V)
    af, gkf = alpha.reshape(B * T, H), gk.reshape(B * T, H) if gk is not None else None
    bf = beta.reshape(B * T, H) if beta is not None else None
    of = o.view(B * T, H, V)
    for n in range(N):
        if cu_seqlens is None:
            bos, ln = n * T, T
        else:
            bos, ln = int(cu_seqlens[n]), int(cu_seqlens[n + 1]) - int(cu_seqlens[n])
        if ln == 0:
            continue
        slot = n if ssm_state_indices is None else int(ssm_state_indices[n])
        qt = l2n(qf[bos].to(dtype))
        kt = _expand(l2n(kf[bos].to(dtype)), H)
        vt = _expand(vf[bos].to(dtype), H)
        if bf is not None:
            kt = kt * (bf[bos].to(dtype) + EPS)[:, None]
            vt = vt * (bf[bos].to(dtype) + EPS)[:, None]
        dk = torch.ones(H, dtype=dtype) if gkf is None else torch.exp(gkf[bos].to(dtype))
        Hn = hkk[slot] * dk[:, None, None] + kt[:, :, None] * kt[:, None, :]
        hkk[slot] = Hn
        x, _ = chebyshev(Hn, qt, ridge_ratio, num_iter)
        x = qt + af[bos].to(dtype)[:, None] * (x - qt)
        S = hkv[slot] * dk[:, None, None] + kt[:, :, None] * vt[:, None, :]
        hkv[slot] = S
        of[bos] = gla_scale * torch.einsum("hkv,hk->hv", S, x)
    return o, hkk, hkv
