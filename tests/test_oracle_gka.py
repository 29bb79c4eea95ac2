"""Pins the GKA oracle (oracle/gka.py) with independent checks.

The reference ships no torch implementation or vectors for GKA, so:
  - the solver is the Chebyshev semi-iteration: it converges to
    solve(H + lam I, q) and obeys the textbook error bound on [lam, lam + |H|_F];
  - |H_t|_F by the reference's closed form (chebyshev_prefill_gqa.py:227-235)
    equals the explicit Frobenius norm of the per-token H_t;
  - with alpha = 0 (or num_iter = 0) the op is beta^2 GLA, which equals the
    chunked matrix form of chunk_simple_gla / chunk_o (no solver involved);
  - a prefill over T tokens equals T decode steps through a state pool;
  - state passing is linear with scalar decay (gka_sp_utils.py:77-110);
  - gating matches torch's softplus / sigmoid.
"""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import gka as ref

D64 = torch.float64


def _inputs(T, H, HKV, D, seed, beta=True, gk=True):
    g0 = torch.Generator().manual_seed(seed)
    q = torch.randn(T, H, D, generator=g0, dtype=D64)
    k = torch.randn(T, HKV, D, generator=g0, dtype=D64)
    v = torch.randn(T, HKV, D, generator=g0, dtype=D64)
    alpha = torch.sigmoid(torch.randn(T, H, generator=g0, dtype=D64))
    g = F.logsigmoid(torch.randn(T, H, generator=g0, dtype=D64))
    gkk = F.logsigmoid(torch.randn(T, H, generator=g0, dtype=D64)) if gk else None
    be = torch.sigmoid(torch.randn(T, H, generator=g0, dtype=D64)) if beta else None
    return q, k, v, alpha, g, gkk, be


def test_chebyshev_converges_to_ridge_solution_within_bound():
    D = 12
    g0 = torch.Generator().manual_seed(0)
    Kx = torch.randn(30, D, generator=g0, dtype=D64)
    H = Kx.T @ Kx
    q = torch.randn(D, generator=g0, dtype=D64)
    r = 0.05
    fro = torch.linalg.matrix_norm(H)
    lam = r * fro
    xs = torch.linalg.solve(H + lam * torch.eye(D, dtype=D64), q)
    kappa = (lam + fro) / lam
    rho = (math.sqrt(kappa) - 1) / (math.sqrt(kappa) + 1)
    e0 = xs.norm()
    errs = []
    for n in (1, 4, 8, 16, 32, 64):
        x, f = ref.chebyshev(H, q, r, n)
        assert torch.allclose(f, fro)
        err = (x - xs).norm()
        bound = 2 * rho ** n / (1 + rho ** (2 * n))
        # the iterate starts from 0 in the Chebyshev recurrence's terms; allow the
        # spectral-norm slack sqrt(kappa) between error norms
        assert err <= bound * e0 * math.sqrt(kappa) + 1e-10, (n, err, bound)
        errs.append(err)
    assert errs[-1] < 1e-8 * e0
    assert all(b <= a * 1.000001 for a, b in zip(errs, errs[1:]))


def test_closed_form_frobenius_equals_explicit():
    T, H, D = 10, 1, 8
    q, k, v, alpha, g, gk, beta = _inputs(T, H, H, D, 1)
    kn = ref.l2n(k)[:, 0] * (beta[:, 0] + 1e-6)[:, None]
    Hc = torch.randn(D, D, generator=torch.Generator().manual_seed(2), dtype=D64)
    Hc = Hc @ Hc.T
    G = gk[:, 0].cumsum(0)
    M = torch.tril(torch.exp(G[:, None] - G[None, :]))
    KK = kn @ kn.T
    # closed form (chebyshev_prefill_gqa.py:227-235)
    fro_in = ((M @ (KK * KK)) * M).sum(1)
    cross = 2 * torch.exp(G) * (M * ((kn @ Hc) * kn).sum(1)[None, :]).sum(1)
    fro_cf = torch.sqrt(torch.exp(2 * G) * (Hc * Hc).sum() + cross + fro_in)
    # explicit H_t
    for t in range(T):
        Ht = torch.exp(G[t]) * Hc + sum(M[t, j] * torch.outer(kn[j], kn[j]) for j in range(t + 1))
        assert torch.allclose(fro_cf[t], torch.linalg.matrix_norm(Ht), rtol=1e-12)


@pytest.mark.parametrize("num_iter,zero_alpha", [(0, False), (8, True)])
def test_reduces_to_beta2_gla_chunked_form(num_iter, zero_alpha):
    T, H, HKV, D, C = 40, 2, 1, 8, 16
    q, k, v, alpha, g, gk, beta = _inputs(T, H, HKV, D, 3)
    if zero_alpha:
        alpha = torch.zeros_like(alpha)
    scale = 0.3
    S0 = torch.randn(H, D, D, generator=torch.Generator().manual_seed(4), dtype=D64)
    o, hkk, S = ref.gka_seq(q, k, v, alpha, g, gk, beta, scale, 0.02, num_iter, None, S0)
    # chunked simple-GLA form (chunk_simple_gla_gqa.py:33-101, chunk_o_gqa.py:25-114)
    qn, kn = ref.l2n(q), ref.l2n(k).repeat_interleave(H // HKV, 1)
    vb = v.repeat_interleave(H // HKV, 1) * ((beta + 1e-6) ** 2)[..., None]
    St = S0.clone()
    out = torch.zeros_like(o)
    for c0 in range(0, T, C):
        sl = slice(c0, min(T, c0 + C))
        G = g[sl].cumsum(0)                                     # [C, H]
        Dm = torch.tril(torch.exp(G[:, None, :] - G[None, :, :]).permute(2, 0, 1))
        A = torch.einsum("thd,jhd->htj", qn[sl], kn[sl]) * Dm
        out[sl] = scale * (torch.exp(G)[..., None] * torch.einsum("thd,hdv->thv", qn[sl], St)
                           + torch.einsum("htj,jhv->thv", A, vb[sl]))
        gl = G[-1]
        St = torch.exp(gl)[:, None, None] * St + torch.einsum(
            "thd,thv->hdv", kn[sl] * torch.exp(gl - G)[..., None], vb[sl])
    assert torch.allclose(out, o, atol=1e-10) and torch.allclose(St, S, atol=1e-10)
    if num_iter == 0:
        assert hkk is None


def test_prefill_equals_decode_steps():
    T, H, HKV, D = 7, 2, 1, 8
    q, k, v, alpha, g, gk, beta = _inputs(T, H, HKV, D, 5)
    g = gk  # decode uses gk for both decays
    o_p, hkk_p, hkv_p = ref.gka_chebyshev_gla_prefill(
        q[None], k[None], v[None], alpha[None], g[None], gk[None], beta[None], 0.5,
        ridge_ratio=0.03, num_iter=6)
    hkk = torch.zeros(3, H, D, D, dtype=D64)
    hkv = torch.zeros(3, H, D, D, dtype=D64)
    for t in range(T):
        sl = slice(t, t + 1)
        o_d, hkk, hkv = ref.gka_chebyshev_gla_decode(
            q[None, sl], k[None, sl], v[None, sl], alpha[None, sl], g[None, sl], gk[None, sl],
            beta[None, sl], 0.5, ridge_ratio=0.03, num_iter=6, h_kk=hkk, h_kv=hkv,
            cu_seqlens=torch.tensor([0, 1]), ssm_state_indices=torch.tensor([2]))
        assert torch.allclose(o_d[0, 0], o_p[0, t], atol=1e-10)
    assert torch.allclose(hkk[2], hkk_p[0], atol=1e-10)
    assert torch.allclose(hkv[2], hkv_p[0], atol=1e-10)


@pytest.mark.parametrize("block,num_iter,gates", [(1, 6, True), (5, 6, True), (64, 0, True),
                                                  (16, 4, False)])
def test_blocked_form_equals_per_token_form(block, num_iter, gates):
    """gka_seq_blocked (solves batched over token blocks) == gka_seq token by token,
    including a ragged last block and initial states."""
    T, H, HKV, D = 37, 2, 1, 8
    q, k, v, alpha, g, gk, beta = _inputs(T, H, HKV, D, 11, beta=gates, gk=gates)
    g0 = torch.Generator().manual_seed(12)
    kx = torch.randn(H, D, 3, generator=g0, dtype=D64)
    h0kk = kx @ kx.transpose(-1, -2)
    h0kv = torch.randn(H, D, D, generator=g0, dtype=D64) * 0.1
    a = ref.gka_seq(q, k, v, alpha, g, gk, beta, 0.3, 0.02, num_iter, h0kk, h0kv)
    b = ref.gka_seq_blocked(q, k, v, alpha, g, gk, beta, 0.3, 0.02, num_iter, h0kk, h0kv,
                            block=block)
    assert torch.allclose(a[0], b[0], rtol=1e-12, atol=1e-12)
    if num_iter:
        assert torch.allclose(a[1], b[1], rtol=1e-12, atol=1e-12)
    else:
        assert a[1] is None and b[1] is None
    assert torch.allclose(a[2], b[2], rtol=1e-12, atol=1e-12)


def test_state_passing_is_linear():
    T, H, D = 12, 2, 8
    q, k, v, alpha, g, gk, beta = _inputs(T, H, H, D, 6)
    h0kk = torch.randn(H, D, D, generator=torch.Generator().manual_seed(7), dtype=D64)
    h0kv = torch.randn(H, D, D, generator=torch.Generator().manual_seed(8), dtype=D64)
    _, hk, hv = ref.gka_seq(q, k, v, alpha, g, gk, beta, 1.0, 0.02, 3, h0kk, h0kv)
    _, hk0, hv0 = ref.gka_seq(q, k, v, alpha, g, gk, beta, 1.0, 0.02, 3, None, None)
    assert torch.allclose(hk, hk0 + torch.exp(gk.sum(0))[:, None, None] * h0kk, atol=1e-10)
    assert torch.allclose(hv, hv0 + torch.exp(g.sum(0))[:, None, None] * h0kv, atol=1e-10)


def test_gka_gating_matches_library():
    g0 = torch.Generator().manual_seed(9)
    a = torch.randn(20, 3, generator=g0, dtype=D64) * 12
    ai = torch.randn(20, 3, generator=g0, dtype=D64)
    b = torch.randn(20, 3, generator=g0, dtype=D64)
    A_log, dt = torch.randn(3, generator=g0, dtype=D64), torch.randn(3, generator=g0, dtype=D64)
    g, al, be = ref.gka_gating(A_log, a, ai, b, dt)
    assert torch.allclose(g[0], -A_log.exp() * F.softplus(a + dt))
    assert torch.allclose(al[0], torch.sigmoid(ai)) and torch.allclose(be[0], torch.sigmoid(b))


def test_training_form_equals_serving_form_on_layer_normalised_inputs():
    """gka_chebyshev_gla on inputs the layer prepared (unit q, k~ = (beta+eps) k^,
    v~ = (beta+eps) v) equals gka_chebyshev_gla_prefill on the raw inputs."""
    T, H, D = 24, 2, 8
    q, k, v, alpha, g, gk, be = _inputs(T, H, H, D, 30)
    o_s, hk_s, hv_s = ref.gka_chebyshev_gla_prefill(q[None], k[None], v[None], alpha[None], g[None],
                                                   gk[None], be[None], 0.3, ridge_ratio=0.05,
                                                   num_iter=6)
    s = (be + 1e-6)[..., None]
    qn, kn = ref.l2n(q), ref.l2n(k) * s
    o_t, hk_t, hv_t = ref.gka_chebyshev_gla(qn[None], kn[None], (v * s)[None], alpha[None], g[None],
                                           gk[None], 0.3, ridge_strength=0.05, num_iter=6)
    assert torch.allclose(o_t, o_s, rtol=1e-10, atol=1e-12)
    assert torch.allclose(hk_t, hk_s) and torch.allclose(hv_t, hv_s)


def test_training_decode_steps_equal_training_prefill():
    T, H, D = 9, 2, 8
    q, k, v, alpha, g, gk, _ = _inputs(T, H, H, D, 31)
    o_p, hk_p, hv_p = ref.gka_chebyshev_gla(q[None], k[None], v[None], alpha[None], g[None],
                                           gk[None], 0.2, ridge_strength=0.02, num_iter=5)
    hk = hv = None
    for t in range(T):
        o, hk, hv = ref.torch_decoding_one_step(q[None, t:t + 1], k[None, t:t + 1], v[None, t:t + 1],
                                                alpha[None, t:t + 1], g[None, t:t + 1],
                                                gk[None, t:t + 1], 0.2, 0.02, 5, hk, hv)
        assert torch.allclose(o[0, 0], o_p[0, t])
    assert torch.allclose(hk, hk_p) and torch.allclose(hv, hv_p)
