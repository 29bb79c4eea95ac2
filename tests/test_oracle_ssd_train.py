"""CPU checks of oracle/ssd_train.py (the chunked SSD backward the kernels follow):
its gradients equal torch autograd through the fp64 forward of oracle/ssd.py (the
per-token recurrence, pinned by test_oracle_ssd.py) to 1e-9, at two chunk lengths,
with z, D per (head, headdim), dt_bias with softplus and an active dt_limit clamp,
B and C in different group counts, an initial state and the final state's gradient;
and a planted mistake (the end-decay term <dS1, S1> left out) fails that comparison."""
import math

import pytest
import torch

from oracle import ssd as ref
from oracle import ssd_train as oref


def _case(seed=3, T=150, H=4, P=8, N=16, GB=2, GC=1):
    g0 = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g0, dtype=torch.float64)
    x, B, C, z, dy = r(T, H, P), r(T, GB, N), r(T, GC, N), r(T, H, P), r(T, H, P)
    dt = r(T, H) * 0.5 - 2.0
    bias = ref.softplus_inverse(torch.exp(torch.rand(H, generator=g0, dtype=torch.float64)
                                          * (math.log(0.1) - math.log(1e-3)) + math.log(1e-3)))
    A = -torch.exp(torch.rand(H, generator=g0, dtype=torch.float64) * math.log(16))
    D = r(H, P) * 0.1 + 1.0
    h0, dfin = r(H, P, N) * 0.1, r(H, P, N)
    return dict(x=x, dt=dt, A=A, B=B, C=C, D=D, z=z, dt_bias=bias, h0=h0), dy, dfin


def _autograd(inp, dy, dfin, lim):
    leaves = {k: v.clone().requires_grad_(True) for k, v in inp.items()}
    l = leaves
    y, fin = ref.mamba_chunk_scan_combined(
        l["x"][None], l["dt"][None], l["A"], l["B"][None], l["C"][None], 64, D=l["D"], z=l["z"][None],
        dt_bias=l["dt_bias"], initial_states=l["h0"][None], dt_softplus=True, dt_limit=lim,
        return_final_states=True)
    ((y[0] * dy).sum() + (fin[0] * dfin).sum()).backward()
    return {k: v.grad for k, v in leaves.items()}


@pytest.mark.parametrize("chunk", [64, 16])
def test_chunk_grads_equal_autograd(chunk):
    inp, dy, dfin = _case()
    lim = (0.004, 0.2)
    want = _autograd(inp, dy, dfin, lim)
    got = oref.chunk_grads(inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"], D=inp["D"],
                           z=inp["z"], dt_bias=inp["dt_bias"], h0=inp["h0"], dy=dy, d_final=dfin,
                           dt_softplus=True, dt_limit=lim, chunk=chunk)
    for k, w in want.items():
        err = (got[k] - w).norm() / w.norm()
        assert err < 1e-9, f"d{k}: {err:.3e}"


def test_planted_missing_end_decay_term_is_caught():
    inp, dy, dfin = _case(seed=4)
    lim = (0.0, float("inf"))
    want = _autograd(inp, dy, dfin, lim)
    got = oref.chunk_grads(inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"], D=inp["D"],
                           z=inp["z"], dt_bias=inp["dt_bias"], h0=inp["h0"], dy=dy, d_final=dfin,
                           dt_softplus=True, dt_limit=lim, chunk=64, _drop_tail=True)
    assert (got["A"] - want["A"]).norm() / want["A"].norm() > 1e-3
    assert (got["dt"] - want["dt"]).norm() / want["dt"].norm() > 1e-4
