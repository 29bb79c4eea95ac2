"""GPU: hmx.ChebyshevIteration (the training layer's solve with its backward,
chebyshev_iteration.py:560-688) through autograd against the float64 oracle
(oracle/gka_train.py, pinned in test_oracle_gka_train.py).

Inputs as the training layer prepares them (gka.py:477-490): unit-norm q, k
scaled by beta in (0, 1), gk a negative log-decay.  The forward is checked on x
(bf16, output tolerance), |H_t|_F and the final state (state tolerance).  The
backward is checked on the HIP path's own saved x and |H_t|_F fed to the oracle
(the reference's backward reads exactly these), so its tolerance measures the
backward kernels alone: norm-wise relative 1e-2 on dq, dk and dgk.  The backward
kernels round their operands once to fp16 (2^-11 relative); the reference's
kernels round theirs to bf16 (2^-8)."""
import pytest
import torch

import hmx
from hmx.ops.gka_train import GkaChebyshevGla, cheb_forward
from oracle import gka_train as tr
from util import STATE_REL, rel_err

pytestmark = pytest.mark.gpu

D = 128
GRAD_REL = 1e-2
OUT_ROW_REL = 1e-2


def _inputs(B, T, H, seed, gated, dev):
    g0 = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, H, D, generator=g0)
    q = q / q.norm(dim=-1, keepdim=True)
    k = torch.randn(B, T, H, D, generator=g0)
    beta = torch.rand(B, T, H, 1, generator=g0) * 0.9 + 0.1
    k = k / k.norm(dim=-1, keepdim=True) * beta
    gk = -0.1 * torch.rand(B, T, H, generator=g0) if gated else None
    dx = torch.randn(B, T, H, D, generator=g0)
    bf = lambda t: t.bfloat16().to(dev)
    return bf(q), bf(k), (None if gk is None else gk.to(dev)), bf(dx)


CASES = [  # B, T, H, gated, num_iter, bp_lambda, blocks per segment (None: the planner's)
    (2, 200, 2, True, 8, True, None),
    (1, 256, 2, False, 8, True, None),
    (2, 130, 2, True, 30, False, None),
    (1, 70, 3, True, 0, True, None),
    (2, 300, 2, True, 8, True, 1),      # segments of one block: the combine carries the states
    (1, 2048, 2, True, 8, True, None),  # one long sequence, which the planner cuts in two
]


@pytest.mark.parametrize("B,T,H,gated,num_iter,bp_lambda,seg", CASES)
def test_chebyshev_iteration_matches_oracle(dev, B, T, H, gated, num_iter, bp_lambda, seg):
    q, k, gk, dx = _inputs(B, T, H, 11, gated, dev)
    qq, kk = q.clone().requires_grad_(True), k.clone().requires_grad_(True)
    gg = None if gk is None else gk.clone().requires_grad_(True)
    x, h_final = hmx.ChebyshevIteration.apply(kk, qq, gg, num_iter, 0.02, bp_lambda, None, 64,
                                              seg)
    x_r, fro_r, h_r = tr.chebyshev_iteration_fwd(k.cpu(), q.cpu(), None if gk is None else gk.cpu(),
                                                 num_iter, 0.02)
    assert x.dtype == torch.bfloat16 and tuple(x.shape) == (B, T, H, D)
    (x.float() * dx.float()).sum().backward()
    # the oracle's backward on the saved x and |H_t|_F of this call
    ctx_fro = _saved_fro(kk, qq, gg, num_iter, seg)
    dk_r, dq_r, dgk_r = tr.chebyshev_iteration_bwd(k.cpu(), x.detach().cpu(), ctx_fro, None if gk is None
                                                   else gk.cpu(), dx.cpu(), num_iter, 0.02, bp_lambda)
    errs = {"x rows": _row_rel(x, x_r), "fro": rel_err(ctx_fro, fro_r),
            "h_kk_final": rel_err(h_final, h_r)}
    for got, exp, name in ((qq.grad, dq_r, "dq"), (kk.grad, dk_r, "dk"),
                           (None if gg is None else gg.grad, dgk_r, "dgk")):
        if exp is None:
            assert got is None
            continue
        assert torch.isfinite(got.float()).all(), name
        errs[name] = rel_err(got, exp)
    print("errors", {n: f"{e:.2e}" for n, e in errs.items()})
    # x grows like q / (r |H_t|_F): each token's row is compared norm-wise
    assert errs["x rows"] < OUT_ROW_REL
    assert errs["fro"] < 1e-4 and errs["h_kk_final"] < STATE_REL
    for name in ("dq", "dk", "dgk"):
        if name in errs:
            assert errs[name] < GRAD_REL, f"{name}: rel {errs[name]:.3e}"


def _row_rel(x, ref):
    """max over token rows of |x_t - ref_t| / |ref_t|"""
    d = (x.detach().double().cpu() - ref).norm(dim=-1)
    return (d / ref.norm(dim=-1)).max().item()


def _saved_fro(kk, qq, gg, num_iter, seg):
    """|H_t|_F as the forward saves it (the forward launches again; they are
    deterministic)."""
    with torch.no_grad():
        return cheb_forward(kk.detach(), qq.detach(), None if gg is None else gg.detach(),
                            num_iter, 0.02, seg)[1].cpu()


def test_chebyshev_iteration_deterministic(dev):
    q, k, gk, dx = _inputs(1, 150, 2, 5, True, dev)
    outs = []
    for _ in range(2):
        qq, kk, gg = (t.clone().requires_grad_(True) for t in (q, k, gk))
        x, hT = hmx.ChebyshevIteration.apply(kk, qq, gg, 8, 0.02, True)
        (x.float() * dx.float()).sum().backward()
        outs.append([x, hT, qq.grad, kk.grad, gg.grad])
    for a, b in zip(*outs):
        assert torch.equal(a, b)


def test_chebyshev_iteration_rejects(dev):
    q, k, gk, _ = _inputs(1, 10, 2, 1, True, dev)
    with pytest.raises(NotImplementedError):
        hmx.ChebyshevIteration.apply(k, q, gk, 8, 0.02, True, torch.zeros(1, 2, D, D, device=dev))
    with pytest.raises(NotImplementedError):
        hmx.ChebyshevIteration.apply(k.float(), q.float(), gk, 8, 0.02, True)
    with pytest.raises(ValueError):
        hmx.ChebyshevIteration.apply(k, q, gk[:, :5], 8, 0.02, True)


GLA_CASES = [  # B, T, H, gated gk, num_iter, bp_lambda, blocks per segment
    (2, 200, 2, True, 8, True, None),
    (1, 130, 2, False, 8, False, None),
    (1, 300, 2, True, 30, True, 1),
    (1, 100, 2, True, 0, True, None),
]


@pytest.mark.parametrize("B,T,H,gated,num_iter,bp_lambda,seg", GLA_CASES)
def test_gka_chebyshev_gla_backward_matches_oracle(dev, B, T, H, gated, num_iter, bp_lambda, seg):
    """The training GKA forward (gka_chebyshev_solve.py:107-164) with its backward:
    o and the final states against the oracle's forward, the six gradients against
    the oracle's backward on this call's saved x and |H_t|_F."""
    q, k, gk, _ = _inputs(B, T, H, 21, gated, dev)
    g0 = torch.Generator().manual_seed(22)
    v = torch.randn(B, T, H, D, generator=g0).bfloat16().to(dev)
    alpha = torch.rand(B, T, H, generator=g0).to(dev)
    g = (-0.1 * torch.rand(B, T, H, generator=g0)).to(dev)
    do = torch.randn(B, T, H, D, generator=g0).bfloat16().to(dev)
    ins = [None if t is None else t.clone().requires_grad_(True) for t in (q, k, v, alpha, g, gk)]
    o, hkk, hkv = GkaChebyshevGla.apply(*ins, 0.3, 0.02, num_iter, bp_lambda, seg)
    saved = o.grad_fn.saved_tensors
    x_s, fro_s = saved[6], saved[7]
    cpu = lambda t: None if t is None else t.detach().cpu()
    o_r, hkk_r, hkv_r, _, _ = tr.gka_chebyshev_gla_fwd(*(cpu(t) for t in (q, k, v, alpha, g, gk)),
                                                     0.3, 0.02, num_iter)
    (o.float() * do.float()).sum().backward()
    exp = tr.gka_chebyshev_gla_bwd(*(cpu(t) for t in (q, k, v, alpha, g, gk)), 0.3, 0.02,
                                   num_iter, bp_lambda, do.cpu(), cpu(x_s), cpu(fro_s))
    errs = {"o rows": _row_rel(o, o_r), "h_kv_final": rel_err(hkv, hkv_r)}
    if num_iter > 0:
        errs["h_kk_final"] = rel_err(hkk, hkk_r)
    for name, t, e in zip(["dq", "dk", "dv", "dalpha", "dg", "dgk"], ins, exp):
        if e is None:
            assert t is None or t.grad is None, name
            continue
        assert torch.isfinite(t.grad.float()).all(), name
        errs[name] = rel_err(t.grad, e)
    print("errors", {n: f"{e:.2e}" for n, e in errs.items()})
    assert errs["o rows"] < OUT_ROW_REL
    assert errs["h_kv_final"] < STATE_REL and errs.get("h_kk_final", 0.0) < STATE_REL
    for name in ("dq", "dk", "dv", "dalpha", "dg", "dgk"):
        if name in errs:
            assert errs[name] < GRAD_REL, f"{name}: rel {errs[name]:.3e}"


def test_gka_chebyshev_gla_routes_through_autograd(dev):
    """hmx.gka_chebyshev_gla takes the differentiable path when an input requires a
    gradient, with the same outputs as the forward-only path."""
    q, k, gk, _ = _inputs(1, 150, 2, 31, True, dev)
    v = torch.randn(1, 150, 2, D, device=dev).bfloat16()
    alpha = torch.rand(1, 150, 2, device=dev)
    g = -0.1 * torch.rand(1, 150, 2, device=dev)
    with torch.no_grad():
        o0, kk0, kv0 = hmx.gka_chebyshev_gla(q, k, v, alpha, g, gk, 0.3, 0.02, num_iter=8)
    qq = q.clone().requires_grad_(True)
    o1, kk1, kv1 = hmx.gka_chebyshev_gla(qq, k, v, alpha, g, gk, 0.3, 0.02, num_iter=8)
    assert o1.grad_fn is not None
    assert torch.equal(o0, o1) and torch.equal(kk0, kk1) and torch.equal(kv0, kv1)
    o1.float().sum().backward()
    assert qq.grad is not None and torch.isfinite(qq.grad.float()).all()


def test_gka_chebyshev_gla_final_state_gradient_refused(dev):
    """A loss that uses kv_final raises (its gradient would otherwise be dropped); a
    loss that also uses kk_final alone is accepted, as the reference's
    ChebyshevIteration.backward drops d_kk_final (chebyshev_iteration.py:606-688)."""
    q, k, gk, _ = _inputs(1, 100, 2, 32, True, dev)
    v = torch.randn(1, 100, 2, D, device=dev).bfloat16()
    alpha = torch.rand(1, 100, 2, device=dev)
    g = -0.1 * torch.rand(1, 100, 2, device=dev)
    qq = q.clone().requires_grad_(True)
    o, kk, kv = hmx.gka_chebyshev_gla(qq, k, v, alpha, g, gk, 0.3, 0.02, num_iter=4)
    with pytest.raises(NotImplementedError):
        (o.float().sum() + kv.sum()).backward()
    qq.grad = None
    o, kk, kv = hmx.gka_chebyshev_gla(qq, k, v, alpha, g, gk, 0.3, 0.02, num_iter=4)
    (o.float().sum() + kk.sum()).backward()
    g_kk = qq.grad.clone()
    qq.grad = None
    o, kk, kv = hmx.gka_chebyshev_gla(qq, k, v, alpha, g, gk, 0.3, 0.02, num_iter=4)
    o.float().sum().backward()
    assert torch.equal(qq.grad, g_kk)
