"""CPU: the training-side Chebyshev oracle (oracle/gka_train.py) pinned by the
mathematics it stands for.

- Forward: with a ridge large enough for the recurrence to converge (r = 0.5 bounds
  the condition number of H_t + lam_t I by 3, so 40 steps reach float64 rounding),
  x_t equals the ridge solution torch.linalg.solve(H_t + r |H_t|_F I, q_t), and
  fro_t equals |H_t|_F of H_t summed from its definition.
- Backward at convergence: the reference's backward (chebyshev_iteration.py:606-688)
  treats x as the exact solution, so dk, dq, dgk must equal autograd of
  sum_t dx_t . solve(H_t(k, gk) + lam_t I, q_t) — with lam_t = r |H_t|_F
  differentiated (bp_lambda) or held fixed.
- dq at any iteration count: the recurrence is linear in its right-hand side with
  a symmetric polynomial of H_t, so dq is autograd of sum_t dx_t . x_t with respect
  to q through the unconverged recurrence itself.
- The whole training forward (solve, alpha blend, GLA readout): at convergence its
  backward equals autograd of the same chain with the exact ridge solve.
"""
import pytest
import torch

from oracle import gka_train as tr

D = 16


def _inputs(seed, B=1, T=24, H=2, gated=True):
    g0 = torch.Generator().manual_seed(seed)
    k = torch.randn(B, T, H, D, generator=g0, dtype=torch.float64)
    k = k / k.norm(dim=-1, keepdim=True)
    q = torch.randn(B, T, H, D, generator=g0, dtype=torch.float64)
    gk = (-0.3 * torch.rand(B, T, H, generator=g0, dtype=torch.float64)) if gated else None
    dx = torch.randn(B, T, H, D, generator=g0, dtype=torch.float64)
    return k, q, gk, dx


def _naive_h(k, gk):
    """H_t = sum_{s<=t} e^{sum_{s<u<=t} gk_u} k_s k_s^T, summed term by term."""
    B, T, H, _ = k.shape
    out = torch.zeros(B, T, H, D, D, dtype=torch.float64)
    for t in range(T):
        for s in range(t + 1):
            w = 1.0 if gk is None else torch.exp(gk[:, s + 1:t + 1].sum(1))[..., None, None]
            out[:, t] += w * k[:, s, :, :, None] * k[:, s, :, None, :]
    return out


def _ridge_solve(Ht, q, r, lam_grad=True):
    fro = torch.sqrt((Ht * Ht).sum((-1, -2)))
    if not lam_grad:
        fro = fro.detach()
    A = Ht + (r * fro)[..., None, None] * torch.eye(D, dtype=Ht.dtype)
    return torch.linalg.solve(A, q[..., None])[..., 0]


@pytest.mark.parametrize("gated", [False, True])
def test_forward_converged_equals_ridge_solution(gated):
    k, q, gk, _ = _inputs(1, gated=gated)
    x, fro, hT = tr.chebyshev_iteration_fwd(k, q, gk, num_iter=40, ridge_ratio=0.5)
    Hn = _naive_h(k, gk)
    assert torch.allclose(fro, torch.sqrt((Hn * Hn).sum((-1, -2))), rtol=1e-12, atol=0)
    assert torch.allclose(hT, Hn[:, -1], rtol=1e-12, atol=1e-14)
    xe = _ridge_solve(Hn, q, 0.5)
    assert (x - xe).norm() / xe.norm() < 1e-12


@pytest.mark.parametrize("gated", [False, True])
@pytest.mark.parametrize("bp_lambda", [True, False])
def test_backward_converged_equals_autograd_of_ridge_solution(gated, bp_lambda):
    k, q, gk, dx = _inputs(2, B=2, T=20, gated=gated)
    x, fro, _ = tr.chebyshev_iteration_fwd(k, q, gk, num_iter=40, ridge_ratio=0.5)
    dk, dq, dgk = tr.chebyshev_iteration_bwd(k, x, fro, gk, dx, num_iter=40, ridge_ratio=0.5,
                                             bp_lambda=bp_lambda)
    kk = k.clone().requires_grad_(True)
    qq = q.clone().requires_grad_(True)
    gg = None if gk is None else gk.clone().requires_grad_(True)
    xe = _ridge_solve(tr.h_states(kk, gg), qq, 0.5, lam_grad=bp_lambda)
    want = torch.autograd.grad((xe * dx).sum(), [kk, qq] + ([gg] if gg is not None else []))
    for got, exp, name in zip([dk, dq, dgk], want, ["dk", "dq", "dgk"]):
        err = ((got - exp).norm() / exp.norm()).item()
        assert err < 1e-10, f"{name}: {err:.2e}"
    if gk is None:
        assert dgk is None


def test_backward_lambda_term_matters():
    """bp_lambda changes dk (the check above would pass a dropped lambda term only if
    both paths agreed)."""
    k, q, gk, dx = _inputs(3)
    x, fro, _ = tr.chebyshev_iteration_fwd(k, q, gk, num_iter=40, ridge_ratio=0.5)
    a = tr.chebyshev_iteration_bwd(k, x, fro, gk, dx, 40, 0.5, bp_lambda=True)
    b = tr.chebyshev_iteration_bwd(k, x, fro, gk, dx, 40, 0.5, bp_lambda=False)
    assert (a[0] - b[0]).norm() > 1e-3 * a[0].norm()
    assert torch.equal(a[1], b[1])


@pytest.mark.parametrize("num_iter", [1, 8, 30])
def test_dq_is_the_recurrence_adjoint(num_iter):
    k, q, gk, dx = _inputs(4)
    x, fro, _ = tr.chebyshev_iteration_fwd(k, q, gk, num_iter=num_iter, ridge_ratio=0.02)
    _, dq, _ = tr.chebyshev_iteration_bwd(k, x, fro, gk, dx, num_iter=num_iter, ridge_ratio=0.02)
    qq = q.clone().requires_grad_(True)
    xq = tr.chebyshev_fixed(tr.h_states(k, gk), qq, fro, 0.02, num_iter)
    (want,) = torch.autograd.grad((xq * dx).sum(), [qq])
    assert ((dq - want).norm() / want.norm()).item() < 1e-12


def _ridge_gla(q, k, v, alpha, g, gk, r, lam_grad):
    """The training forward with the exact ridge solution in place of the recurrence."""
    x = _ridge_solve(tr.h_states(k, gk), q, r, lam_grad)
    u = q + alpha[..., None] * (x - q)
    return tr.gla(u, k, v, g, 0.3)[0]


@pytest.mark.parametrize("bp_lambda", [True, False])
def test_training_gka_backward_converged_equals_autograd(bp_lambda):
    """gka_chebyshev_gla_bwd at convergence equals autograd of the whole forward with
    the exact ridge solve (the GLA, the blend and the solve chained)."""
    k, q, gk, _ = _inputs(5, B=1, T=16)
    g0 = torch.Generator().manual_seed(6)
    v = torch.randn(1, 16, 2, D, generator=g0, dtype=torch.float64)
    alpha = torch.rand(1, 16, 2, generator=g0, dtype=torch.float64)
    g = -0.2 * torch.rand(1, 16, 2, generator=g0, dtype=torch.float64)
    do = torch.randn(1, 16, 2, D, generator=g0, dtype=torch.float64)
    o, _, _, x, fro = tr.gka_chebyshev_gla_fwd(q, k, v, alpha, g, gk, 0.3, 0.5, 40)
    got = tr.gka_chebyshev_gla_bwd(q, k, v, alpha, g, gk, 0.3, 0.5, 40, bp_lambda, do, x, fro)
    ins = [t.clone().requires_grad_(True) for t in (q, k, v, alpha, g, gk)]
    oe = _ridge_gla(*ins, 0.5, bp_lambda)
    assert (oe - o).norm() / oe.norm() < 1e-12
    want = torch.autograd.grad((oe * do).sum(), ins)
    for name, a, b in zip(["dq", "dk", "dv", "dalpha", "dg", "dgk"], got, want):
        err = ((a - b).norm() / b.norm()).item()
        assert err < 1e-10, f"{name}: {err:.2e}"
