"""CPU: the GDN backward oracle (oracle/gdn_train.py) pinned by the mathematics.

- ``recurrent_grads`` is autograd of the float64 recurrence; torch.autograd.gradcheck
  checks that derivative against central finite differences on small inputs (every
  input: q, k, v, g, beta and the initial state, with and without the in-kernel
  L2 normalisation), so a wrong recurrence step would not pass unnoticed through
  autograd's own consistency.
- ``chunk_grads`` (the blocked formulas the HIP kernels implement) equals
  ``recurrent_grads`` on ragged multi-block sequences, with an initial state and a
  final-state gradient, at 1e-10 relative.
- Planted mistakes in the blocked formulas (a dropped decay term, a transposed T)
  make that comparison fail, so it pins each term.
"""
import pytest
import torch

from oracle import gdn as gd
from oracle import gdn_train as gt


def _inputs(seed, T, H, D, s0=True):
    g0 = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g0, dtype=torch.float64)
    q, k, v = r(T, H, D), r(T, H, D), r(T, H, D)
    g = torch.nn.functional.logsigmoid(r(T, H)) * 0.5
    beta = torch.sigmoid(r(T, H))
    S0 = r(H, D, D) * 0.3 if s0 else None
    do, dST = r(T, H, D), r(H, D, D)
    return q, k, v, g, beta, S0, do, dST


@pytest.mark.parametrize("l2", [True, False])
def test_recurrent_autograd_matches_finite_differences(l2):
    q, k, v, g, beta, S0, _, _ = _inputs(1, 5, 2, 4)
    if not l2:
        q, k = q / q.norm(dim=-1, keepdim=True) * 0.8, k / k.norm(dim=-1, keepdim=True) * 0.9

    def f(q, k, v, g, beta, S0):
        o, ST = gd.recurrent_seq(q, k, v, g, beta, 0.7, S0, l2)
        return o, ST
    ins = [t.clone().requires_grad_(True) for t in (q, k, v, g, beta, S0)]
    assert torch.autograd.gradcheck(f, ins, eps=1e-6, atol=1e-7, rtol=1e-6)


def _rel(a, b):
    return ((a - b).norm() / b.norm()).item()


@pytest.mark.parametrize("T,l2,s0,dst", [(70, True, True, True), (64, True, False, False),
                                         (33, False, True, False), (5, True, True, True)])
def test_chunk_formulas_equal_autograd(T, l2, s0, dst):
    q, k, v, g, beta, S0, do, dST = _inputs(2, T, 2, 8, s0)
    if not l2:
        k = k / k.norm(dim=-1, keepdim=True) * 0.9
    dST = dST if dst else None
    want = gt.recurrent_grads(q, k, v, g, beta, 0.5, S0, do, dST, l2)
    got = gt.chunk_grads(q, k, v, g, beta, 0.5, S0, do, dST, l2, chunk=32)
    names = ["dq", "dk", "dv", "dg", "dbeta", "dS0"]
    for name, a, b in zip(names, got, want):
        if b is None:
            assert a is None, name
            continue
        assert _rel(a, b) < 1e-10, f"{name}: {_rel(a, b):.2e}"


def test_chunk_formulas_small_blocks():
    """The blocked formulas at another block length (8) give the same gradient."""
    q, k, v, g, beta, S0, do, dST = _inputs(3, 40, 1, 8)
    a = gt.chunk_grads(q, k, v, g, beta, 0.5, S0, do, dST, True, chunk=8)
    b = gt.recurrent_grads(q, k, v, g, beta, 0.5, S0, do, dST, True)
    for x, y in zip(a, b):
        assert _rel(x, y) < 1e-10


def test_planted_mistakes_fail(monkeypatch):
    """A transposed T in the backward (Z = T dW instead of T^T dW) changes the
    gradients: the comparison above would catch it."""
    q, k, v, g, beta, S0, do, dST = _inputs(4, 40, 1, 8)
    want = gt.recurrent_grads(q, k, v, g, beta, 0.5, S0, do, dST, True)
    real_inv = torch.linalg.inv
    calls = {"n": 0}

    def inv_t(x):   # the forward's T is right; every backward T is transposed
        calls["n"] += 1
        y = real_inv(x)
        return y if calls["n"] <= 2 else y.transpose(-1, -2)
    monkeypatch.setattr(torch.linalg, "inv", inv_t)
    got = gt.chunk_grads(q, k, v, g, beta, 0.5, S0, do, dST, True, chunk=32)
    monkeypatch.undo()
    assert max(_rel(a, b) for a, b in zip(got, want)) > 1e-3
