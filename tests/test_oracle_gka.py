"""Pins the GKA oracle (oracle/gka.py) with independent checks.

The reference ships no torch implementation or vectors for GKA, so:
  - the solver is the Chebyshev semi-iteration: it converges to
    solve(H + lam I, q) and obeys the textbook error bound on [lam, lam + |H|_F];
    at every finite num_iter its iterate equals the closed form x* - P(A) x*, with P
    the scaled Chebyshev residual polynomial of degree num_iter + 1 evaluated on the
    eigenvalues (both the serving solve and the training solve), and planted
    transcription mistakes (omega_0, rho^2/4, momentum sign, ...) fail that check;
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


# ---------------------------------------------------------------------------
# The solver at finite num_iter.  The C3 runs (ridge 0.01, n = 8 / 32) stop far from
# convergence, so the exact iterate is the contract.  The recurrence of
# chebyshev_iteration_gqa.py:115-134 is the Chebyshev semi-iteration (Golub & Varga
# 1961) on A = H + lam I over [a, b] = [lam, lam + |H|_F], started from y_0 = 0 with a
# Richardson step y_1 = tau q (omega_1 = 1; the loop's first omega, 1/(1 - c 2), is
# omega_2).  After n loop steps the iterate is y_{n+1}, whose error is the scaled
# Chebyshev residual polynomial of degree n+1 applied to the initial error -x*:
#     x* - y_{n+1} = P(A) x*,   P(mu) = T_{n+1}((b + a - 2 mu)/(b - a)) / T_{n+1}((b + a)/(b - a)).
# On an eigenbasis A = Q diag(mu + lam) Q^T this is a closed form in the eigenvalues,
# evaluated here with numpy's Chebyshev series (Clenshaw), independent of the
# three-term recurrence the oracle runs.
# ---------------------------------------------------------------------------
def _cheb_residual(Qm, mu, q, ridge_ratio, n):
    """x* - P(A) x* for H = Qm diag(mu) Qm^T, from the eigenvalues alone."""
    import numpy as np
    from numpy.polynomial import chebyshev as npc
    f = float(np.sqrt((mu.numpy() ** 2).sum()))
    lam = ridge_ratio * f
    a, b = lam, lam + f
    coef = np.zeros(n + 2)
    coef[n + 1] = 1.0
    s = mu.numpy() + lam
    P = npc.chebval((b + a - 2 * s) / (b - a), coef) / npc.chebval((b + a) / (b - a), coef)
    xs_eig = (Qm.T @ q).numpy() / s                       # x* in the eigenbasis
    return Qm @ torch.from_numpy(xs_eig * (1.0 - P))


def _spectra(seed, D=16):
    """(Q, mu) pairs: a random orthogonal basis with a spread PSD spectrum (one
    eigenvalue near 0, one near |H|_F), and the eigendecomposition of a real key
    Gram sum_j k~_j k~_j^T as the prefill forms it."""
    g0 = torch.Generator().manual_seed(seed)
    Qm, _ = torch.linalg.qr(torch.randn(D, D, generator=g0, dtype=D64))
    mu = torch.cat([torch.tensor([1e-4, 3.0], dtype=D64),
                    torch.rand(D - 2, generator=g0, dtype=D64) * 0.7])
    kk = ref.l2n(torch.randn(40, D, generator=g0, dtype=D64))
    kk = kk * (torch.sigmoid(torch.randn(40, 1, generator=g0, dtype=D64)) + 1e-6)
    mu2, Q2 = torch.linalg.eigh(kk.T @ kk)
    return [(Qm, mu), (Q2, mu2.clamp_min(0.0))]


@pytest.mark.parametrize("n", [0, 1, 2, 4, 8, 32])
@pytest.mark.parametrize("r", [0.01, 0.02])
def test_chebyshev_finite_n_equals_residual_polynomial(n, r):
    """ref.chebyshev after n loop steps == x* - P_{n+1}(A) x* to 1e-12, for both
    spectra, batched (leading dim) as the prefill calls it."""
    g0 = torch.Generator().manual_seed(100 + n)
    for Qm, mu in _spectra(7 + n):
        D = mu.numel()
        H = Qm @ torch.diag(mu) @ Qm.T
        H = 0.5 * (H + H.T)
        q = torch.randn(3, D, generator=g0, dtype=D64)
        x, fro = ref.chebyshev(H.expand(3, D, D), q, r, n)
        assert torch.allclose(fro, torch.linalg.matrix_norm(H).expand(3), rtol=1e-13)
        for i in range(3):
            want = _cheb_residual(Qm, mu, q[i], r, n)
            err = (x[i] - want).norm() / want.norm()
            assert err < 1e-12, (n, r, i, float(err))


@pytest.mark.parametrize("n", [0, 1, 4, 8, 32])
def test_training_chebyshev_fixed_equals_residual_polynomial(n):
    """oracle/gka_train.py:chebyshev_fixed (|H|_F given, CI:397-406) obeys the same
    closed form."""
    from oracle import gka_train as tr
    g0 = torch.Generator().manual_seed(200 + n)
    for Qm, mu in _spectra(17 + n):
        D = mu.numel()
        H = Qm @ torch.diag(mu) @ Qm.T
        H = 0.5 * (H + H.T)
        q = torch.randn(D, generator=g0, dtype=D64)
        x = tr.chebyshev_fixed(H[None], q[None], torch.linalg.matrix_norm(H)[None], 0.01, n)[0]
        want = _cheb_residual(Qm, mu, q, 0.01, n)
        assert (x - want).norm() / want.norm() < 1e-12


# Mistakes a transcription of CI:115-134 could plausibly make.  Each is planted in a
# copy of the oracle's own source (text substitution, then exec), which must still
# run but fail the closed form: the check above would catch it.
_MUTANTS = [
    ("torch.full_like(fro, 2.0)", "torch.full_like(fro, 1.0)"),      # omega_0 = 1
    ("(fro / denom * 0.5) ** 2", "(fro / denom) ** 2"),              # rho^2 without the 1/4
    ("(w - 1.0)[..., None] * x_prev", "(1.0 - w)[..., None] * x_prev"),  # sign of the momentum
    ("x = tau[..., None] * q", "x = q"),                             # no first Richardson step
    ("range(num_iter)", "range(num_iter - 1)"),                      # one step short
    ("hx + lam[..., None] * x - q", "hx - q"),                       # ridge dropped from A
]


@pytest.mark.parametrize("old,new", _MUTANTS)
def test_planted_chebyshev_mistakes_fail(old, new):
    import inspect
    import textwrap
    src = textwrap.dedent(inspect.getsource(ref.chebyshev))
    assert src.count(old) == 1, old
    ns = {"torch": torch}
    exec(compile(src.replace(old, new), "<mutant>", "exec"), ns)
    mutant = ns["chebyshev"]
    Qm, mu = _spectra(3)[0]
    H = Qm @ torch.diag(mu) @ Qm.T
    q = torch.randn(16, generator=torch.Generator().manual_seed(5), dtype=D64)
    want = _cheb_residual(Qm, mu, q, 0.01, 8)
    x, _ = mutant(H, q, 0.01, 8)
    assert (x - want).norm() / want.norm() > 1e-3, (old, new)
    x_ok, _ = ref.chebyshev(H, q, 0.01, 8)
    assert (x_ok - want).norm() / want.norm() < 1e-12
