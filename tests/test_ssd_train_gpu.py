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
1 - 2e-5), far below what a dropped or mis-signed term gives.  dA is a per-head sum
over every token of dt'_t da_t whose terms can cancel (23x in the B-groups-wider
case), so its error is measured against the norm of the per-head sums of |dt'_t
da_t| (from the fp64 chunked backward of oracle/ssd_train.py) and must stay under
1% of it (measured up to 0.4%).
"""
import math

import pytest
import torch

import hmx
from oracle import ssd as ref
from oracle import ssd_train as oref

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


def _dA_scale(inp, wy, wf, kw):
    """Per head, sum over every chunk of every sequence of |dt'_t da_t| (the fp64
    chunked backward): dA is the sum of these terms, which can cancel (23x in one
    case here), so dA's rounding error is measured against this scale."""
    b, l, H, _ = inp["x"].shape
    total = torch.zeros(H, dtype=torch.float64)
    seq_idx = kw.get("seq_idx")
    for row in range(b):
        runs = [(0, l)] if seq_idx is None else ref._runs(seq_idx[row])
        for i, (s0, s1) in enumerate(runs):
            h0 = inp["initial_states"]
            h0 = h0[row] if (h0 is not None and i == 0 and s0 == 0) else None
            fin = wf[row] if (kw.get("return_final_states") and s1 == l) else None
            sl = slice(s0, s1)
            o = oref.chunk_grads(inp["x"][row, sl], inp["dt"][row, sl], inp["A"], inp["B"][row, sl],
                                 inp["C"][row, sl], D=inp["D"],
                                 z=None if inp["z"] is None else inp["z"][row, sl],
                                 dt_bias=inp["dt_bias"], h0=h0, dy=wy[row, sl], d_final=fin,
                                 dt_softplus=kw.get("dt_softplus", False),
                                 dt_limit=kw.get("dt_limit", (0.0, float("inf"))))
            total += o["A_abs"]
    return total


def _check(g, g_ref, name, tol=2e-2, scale=None):
    a = g.detach().double().cpu().flatten()
    b = g_ref.detach().double().cpu().flatten()
    assert torch.isfinite(a).all(), f"{name}: non-finite gradient"
    if scale is not None:   # a sum of cancelling terms: error against the terms' scale
        err = (a - b).norm().item() / scale.norm().item()
        print(f"  {name}: error / ||sum|dt' da|||  {err:.2e}")
        assert err <= tol * 0.5, f"{name}: error {err:.3e} of the terms' scale"
        return
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
    sA = _dA_scale(inp, wy, wf, kw)
    for k in g_ref:
        _check(g[k], g_ref[k], f"{case} d{k}", scale=sA if k == "A" else None)


@pytest.mark.parametrize("N", [128, 64])
def test_backward_headdim_128(dev, N):
    """headdim 128 (the hybrid layers' headdim = d_state, mamba2.py:146): C shared by
    two heads, seq_idx restarts, initial and final states, D per head, no z."""
    inp, wy, wf = _inputs(1, 230, 4, 2, 128, N, 950 + N, False, False)
    kw = dict(dt_softplus=True, return_final_states=True,
              seq_idx=torch.cat([torch.zeros(150, dtype=torch.int32),
                                 torch.ones(80, dtype=torch.int32)])[None])
    kw_dev = dict(kw, seq_idx=kw["seq_idx"].to(dev))
    g = _grads(inp, wy, wf, kw_dev, dev, None)
    torch.cuda.synchronize()
    g_ref = _grads(inp, wy, wf, kw, None, torch.float64)
    sA = _dA_scale(inp, wy, wf, kw)
    for k in g_ref:
        _check(g[k], g_ref[k], f"hdim128 N={N} d{k}", scale=sA if k == "A" else None)


def test_backward_headdim_128_with_z_raises(dev):
    inp, _, _ = _inputs(1, 64, 2, 1, 128, 64, 1, True, False)
    x = inp["x"].to(dev).requires_grad_(True)
    y = hmx.mamba_chunk_scan_combined(x, inp["dt"].to(dev), inp["A"].to(dev), inp["B"].to(dev),
                                      inp["C"].to(dev), 256, z=inp["z"].to(dev), dt_softplus=True)
    with pytest.raises(NotImplementedError, match="z gate needs headdim 64"):
        y.float().sum().backward()


@pytest.mark.parametrize("gb,gc,bf16_params", [(4, 2, False), (1, 2, False), (4, 2, True)])
def test_backward_training_layer_layout(dev, gb, gc, bf16_params):
    """The training layer's operands (mamba2.py:541-556): x and B repeated to the H
    heads, C with its own ngroups, D per head, no z (gb = 4); B groups wider than C's
    (gb = 1: B's gradient accumulates across workgroups); and dt, D, dt_bias in the
    model's bf16 (their gradients come back in bf16)."""
    inp, wy, wf = _inputs(1, 200, 4, gb, 64, 128, 900 + gb, False, False)
    g0 = torch.Generator().manual_seed(901)
    inp["C"] = torch.randn(1, 200, gc, 128, generator=g0).bfloat16()
    if bf16_params:
        for k in ("dt", "D", "dt_bias"):
            inp[k] = inp[k].bfloat16()
    inp["initial_states"] = None
    kw = dict(dt_softplus=True)
    g = _grads(inp, wy, wf, kw, dev, None)
    torch.cuda.synchronize()
    g_ref = _grads(inp, wy, wf, kw, None, torch.float64)
    assert g["C"].shape == inp["C"].shape
    assert all(g[k].dtype == inp[k].dtype for k in g)
    sA = _dA_scale(inp, wy, wf, kw)
    for k in g_ref:
        _check(g[k], g_ref[k], f"train_layout d{k}", scale=sA if k == "A" else None)
