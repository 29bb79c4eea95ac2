"""GPU parity: the backward of hmx.mamba_chunk_scan_combined (the training scan,
training/src/hmf/model/hybrid_zoo/layers/mamba/mamba2.py:555-580, under autograd)
against autograd through the fp64 CPU oracle (oracle/ssd.py, whose forward is pinned
by test_oracle_ssd.py).

The loss is a fixed random weighting of y (and of the final states when returned),
so every gradient path is exercised: x, dt (through softplus and the dt_limit
clamp), A, B, C (groups shared by several heads: atomics), D per head and per
(head, headdim), z, dt_bias and initial_states; seq_idx restarts, ragged last
chunks, sequences shorter than one chunk.  Tolerance: the backward's products take
bf16 operands (as mamba_ssm's do) with fp32 accumulation; each gradient must match
to 2% of its norm with cosine above 1 - 1e-4 (measured: 0.1-0.9%, cosine above
1 - 2e-5), far below what a dropped or mis-signed term gives.
"""
import math

import pytest
import torch

import hmx
from oracle import ssd as ref

pytestmark = pytest.mark.gpu


def _inputs(b, l, H, G, P, N, seed, z, d_hdim):
    g0 = torch.Generator().manual_seed(seed)
    x = torch.randn(b, l, H, P, generator=g0).bfloat16()
    B = torch.randn(b, l, G, N, generator=g0).bfloat16()
    C = torch.randn(b, l, G, N, generator=g0).bfloat16()
    dt = torch.randn(b, l, H, generator=g0) * 0.5 - 2.0
    u = torch.rand(H, generator=g0)
    bias = ref.softplus_inverse(torch.exp(u * (math.log(0.1) - math.log(1e-3)) + math.log(1e-3)))
    A = -torch.exp(torch.rand(H, generator=g0) * math.log(16))
    D = (torch.randn(H, P, generator=g0) if d_hdim else torch.randn(H, generator=g0)) * 0.1 + 1.0
    zz = torch.randn(b, l, H, P, generator=g0).bfloat16() if z else None
    h0 = torch.randn(b, H, P, N, generator=g0) * 0.1
    wy = torch.randn(b, l, H, P, generator=g0)
    wf = torch.randn(b, H, P, N, generator=g0)
    return dict(x=x, dt=dt, A=A, B=B, C=C, D=D, dt_bias=bias, z=zz, initial_states=h0), wy, wf


def _grads(inp, wy, wf, kw, dev, dtype):
    """Gradients of sum(y * wy) (+ sum(final * wf)) through hmx (dev) or the oracle."""
    leaves = {k: (None if v is None else
                  v.to(dev if dev is not None else "cpu").to(dtype or v.dtype).requires_grad_(True))
              for k, v in inp.items()}
    args = dict(leaves)
    if dev is None:
        out = ref.mamba_chunk_scan_combined(args.pop("x"), args.pop("dt"), args.pop("A"),
                                            args.pop("B"), args.pop("C"), 256, **args, **kw)
    else:
        out = hmx.mamba_chunk_scan_combined(args.pop("x"), args.pop("dt"), args.pop("A"),
                                            args.pop("B"), args.pop("C"), 256, **args, **kw)
    y, fin = (out if isinstance(out, tuple) else (out, None))
    wy_ = wy.to(y.device, torch.float64 if dev is None else torch.float32)
    loss = (y.to(wy_.dtype) * wy_).sum()
    if fin is not None:
        loss = loss + (fin.to(wy_.dtype) * wf.to(fin.device, wy_.dtype)).sum()
    loss.backward()
    return {k: v.grad for k, v in leaves.items() if v is not None}


def _check(g, g_ref, name, tol=2e-2):
    a = g.detach().double().cpu().flatten()
    b = g_ref.detach().double().cpu().flatten()
    assert torch.isfinite(a).all(), f"{name}: non-finite gradient"
    nb = b.norm().item()
    err = (a - b).norm().item() / max(nb, 1e-30)
    cos = (a @ b).item() / max(a.norm().item() * nb, 1e-30)
    print(f"  {name}: rel err {err:.2e}, cosine {cos:.7f}")
    assert err <= tol and cos >= 1 - 1e-4, f"{name}: rel err {err:.3e}, cosine {cos:.6f}"


CASES = {
    # b, l, H, G, N, z, D per headdim, seq_idx runs, initial + final states, dt_limit
    "z_groups": (2, 160, 4, 1, 128, True, False, None, False, (0.0, float("inf"))),
    "seq_idx_states": (1, 300, 4, 4, 64, False, True, [100, 37, 163], True, (0.0, float("inf"))),
    "clamp_ragged": (2, 93, 4, 2, 128, True, True, None, True, (0.004, 0.05)),
    "long_runs": (1, 1100, 4, 2, 128, True, False, [700, 1, 399], True, (0.0, float("inf"))),
}


@pytest.mark.parametrize("case", list(CASES))
def test_scan_backward_matches_oracle_autograd(dev, case):
    b, l, H, G, N, z, d_hdim, runs, states, lim = CASES[case]
    inp, wy, wf = _inputs(b, l, H, G, 64, N, 700 + len(case), z, d_hdim)
    kw = dict(dt_softplus=True, dt_limit=lim)
    if not states:
        inp["initial_states"] = None
    else:
        kw["return_final_states"] = True
    if runs is not None:
        kw["seq_idx"] = torch.cat([torch.full((n,), i, dtype=torch.int32)
                                   for i, n in enumerate(runs)])[None].expand(b, l)
    kw_dev = dict(kw)
    if runs is not None:
        kw_dev["seq_idx"] = kw["seq_idx"].to(dev)
    print(f"[ssd bwd] case={case}", flush=True)
    g = _grads(inp, wy, wf, kw_dev, dev, None)
    torch.cuda.synchronize()
    g_ref = _grads(inp, wy, wf, kw, None, torch.float64)
    assert set(g) == set(g_ref)
    for k in g_ref:
        _check(g[k], g_ref[k], f"{case} d{k}")


def test_backward_needs_headdim_64(dev):
    inp, _, _ = _inputs(1, 64, 2, 1, 128, 64, 1, False, False)
    x = inp["x"].to(dev).requires_grad_(True)
    y = hmx.mamba_chunk_scan_combined(x, inp["dt"].to(dev), inp["A"].to(dev), inp["B"].to(dev),
                                      inp["C"].to(dev), 256, dt_softplus=True)
    with pytest.raises(NotImplementedError, match="headdim 64"):
        y.float().sum().backward()


def test_backward_training_layer_layout(dev):
    """The training layer's operands (mamba2.py:541-556): x and B repeated to the H
    heads, C with its own ngroups, D per head, no z."""
    inp, wy, wf = _inputs(1, 200, 4, 4, 64, 128, 900, False, False)
    g0 = torch.Generator().manual_seed(901)
    inp["C"] = torch.randn(1, 200, 2, 128, generator=g0).bfloat16()
    inp["initial_states"] = None
    kw = dict(dt_softplus=True)
    g = _grads(inp, wy, wf, kw, dev, None)
    torch.cuda.synchronize()
    g_ref = _grads(inp, wy, wf, kw, None, torch.float64)
    assert g["C"].shape == inp["C"].shape
    for k in g_ref:
        _check(g[k], g_ref[k], f"train_layout d{k}")
