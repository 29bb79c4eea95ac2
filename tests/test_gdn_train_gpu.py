"""GPU: hmx.ChunkGatedDeltaRule (fla's chunk_gated_delta_rule with its backward, as
the training layer calls it, gated_deltanet/gdn.py:462-476) against the float64
oracle (oracle/gdn_train.py: autograd of the per-token recurrence, pinned by
finite differences and by the blocked formulas in test_oracle_gdn_train.py).

Inputs as the training layer forms them: q, k, v ~ N(0, 1) in bf16 with the
in-kernel L2 normalisation, g = -e^{A_log} softplus(x + dt_bias) in fp32, beta =
sigmoid(.) (times 2 with allow_neg_eigval).  The loss is sum(o . do) (+ <ht, dht>
when the final state is used).  Every gradient (q, k, v, g, beta and the initial
state) is compared norm-wise: relative error below 1e-2.  The kernels round each
MFMA operand once to fp16 (2^-11 relative) and write dq, dk, dv in bf16 (2^-8)."""
import pytest
import torch

import hmx
from hmx.ops.gdn_train import ChunkGatedDeltaRule
from oracle import gdn_train as gt
from util import rel_err

pytestmark = pytest.mark.gpu

D = 128
GRAD_REL = 1e-2


def _inputs(B, T, H, seed, dev, beta2=False, l2=True, weak=False):
    g0 = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, H, D, generator=g0)
    k = torch.randn(B, T, H, D, generator=g0)
    if not l2:   # unit-scale keys without the in-kernel normalisation
        q = q / q.norm(dim=-1, keepdim=True)
        k = k / k.norm(dim=-1, keepdim=True) * 0.9
    v = torch.randn(B, T, H, D, generator=g0)
    A_log = torch.rand(H, generator=g0) * 2.0 - 1.0
    g = -A_log.exp() * torch.nn.functional.softplus(torch.randn(B, T, H, generator=g0) - 2.0)
    if weak:     # too little decay for any warm-up: the state-gradient chain runs exact
        g = g * 1e-3
    beta = torch.sigmoid(torch.randn(B, T, H, generator=g0)) * (2.0 if beta2 else 1.0)
    do = torch.randn(B, T, H, D, generator=g0)
    bf = lambda t: t.bfloat16().to(dev)
    return bf(q), bf(k), bf(v), g.to(dev), beta.to(dev), bf(do)


# segment chunks: the recomputing forward's segments and the state-gradient chain's
# runs, in 32-token blocks (None: the planners'; at these sizes the chain's runs are
# one block each, every one after a warm-up)
CASES = [  # B, T, H, l2, h0, final-state grad, cu_seqlens, segment chunks, beta in (0, 2), beta bf16, weak decay
    (2, 200, 2, True, False, False, None, None, False, False, False),
    (1, 256, 2, True, True, True, None, None, False, False, False),
    (1, 180, 2, True, True, True, [0, 50, 51, 180], None, False, True, False),
    (1, 300, 2, True, True, False, None, 1, False, False, False),
    (2, 100, 3, False, False, True, None, None, False, False, False),
    (1, 160, 2, True, False, False, None, None, True, False, False),
    (1, 2048, 2, True, True, True, None, None, False, False, False),
    (1, 2048, 2, True, True, True, None, 5, False, False, False),
    (1, 700, 2, True, True, True, [0, 300, 300, 700], 3, False, False, True),
]


@pytest.mark.parametrize("B,T,H,l2,use_h0,use_dht,cu,seg,beta2,beta_bf,weak", CASES)
def test_chunk_gated_delta_rule_backward_matches_oracle(dev, B, T, H, l2, use_h0, use_dht, cu, seg,
                                                        beta2, beta_bf, weak):
    print("case", B, T, H, l2, use_h0, use_dht, cu, seg, beta2, beta_bf, weak, flush=True)
    q, k, v, g, beta, do = _inputs(B, T, H, 7, dev, beta2, l2, weak)
    if beta_bf:
        beta = beta.bfloat16()
    N = B if cu is None else len(cu) - 1
    g0 = torch.Generator().manual_seed(8)
    h0 = (torch.randn(N, H, D, D, generator=g0) * 0.1).to(dev) if use_h0 else None
    dht = torch.randn(N, H, D, D, generator=g0).to(dev) if use_dht else None
    cu_t = None if cu is None else torch.tensor(cu, dtype=torch.int32, device=dev)
    ins = [None if t is None else t.clone().requires_grad_(True) for t in (q, k, v, g, beta, h0)]
    o, ht = ChunkGatedDeltaRule.apply(*ins[:5], D ** -0.5, ins[5], use_dht, cu_t, l2, seg)
    loss = (o.float() * do.float()).sum()
    if use_dht:
        loss = loss + (ht * dht).sum()
    loss.backward()
    # the oracle, sequence by sequence
    bounds = [(b * T, b * T + T) for b in range(B)] if cu is None else list(zip(cu[:-1], cu[1:]))
    flat = lambda t: t.detach().reshape(B * T, *t.shape[2:]).cpu()
    qf, kf, vf, gf, bfl, dof = (flat(t) for t in (q, k, v, g, beta, do))
    exp = [torch.zeros(B * T, H, D, dtype=torch.float64) for _ in range(3)]
    exp += [torch.zeros(B * T, H, dtype=torch.float64) for _ in range(2)]
    exp_h0 = []
    for n, (a, b) in enumerate(bounds):
        r = gt.recurrent_grads(qf[a:b], kf[a:b], vf[a:b], gf[a:b], bfl[a:b], D ** -0.5,
                               None if h0 is None else h0[n].cpu(), dof[a:b],
                               None if dht is None else dht[n].cpu(), l2)
        for i in range(5):
            exp[i][a:b] = r[i]
        exp_h0.append(r[5])
    errs = {}
    for name, t, e in zip(["dq", "dk", "dv", "dg", "dbeta"], ins[:5], exp):
        got = t.grad.reshape(B * T, *t.shape[2:])
        assert got.dtype == t.dtype, name
        assert torch.isfinite(got.float()).all(), name
        errs[name] = rel_err(got, e)
    if use_h0:
        errs["dh0"] = rel_err(ins[5].grad, torch.stack(exp_h0))
    print("errors", {n: f"{e:.2e}" for n, e in errs.items()})
    for name, e in errs.items():
        assert e < GRAD_REL, f"{name}: rel {e:.3e}"


def test_backward_deterministic(dev):
    q, k, v, g, beta, do = _inputs(1, 150, 2, 5, dev)
    outs = []
    for _ in range(2):
        ins = [t.clone().requires_grad_(True) for t in (q, k, v, g, beta)]
        o, _ = ChunkGatedDeltaRule.apply(*ins, None, None, False, None, True, None)
        (o.float() * do.float()).sum().backward()
        outs.append([o] + [t.grad for t in ins])
    for a, b in zip(*outs):
        assert torch.equal(a, b)


def test_fla_entry_routes_through_autograd(dev):
    """hmx.chunk_gated_delta_rule takes the differentiable path when an input requires
    a gradient, with the forward-only path's outputs."""
    q, k, v, g, beta, do = _inputs(1, 130, 2, 9, dev)
    with torch.no_grad():
        o0, h0 = hmx.chunk_gated_delta_rule(q, k, v, g, beta, output_final_state=True,
                                            use_qk_l2norm_in_kernel=True)
    qq = q.clone().requires_grad_(True)
    o1, h1 = hmx.chunk_gated_delta_rule(qq, k, v, g, beta, output_final_state=True,
                                        use_qk_l2norm_in_kernel=True)
    assert o1.grad_fn is not None
    assert torch.equal(o0, o1) and torch.equal(h0, h1)
    (o1.float() * do.float()).sum().backward()
    assert qq.grad is not None and torch.isfinite(qq.grad.float()).all()


def test_backward_rejects(dev):
    q, k, v, g, beta, _ = _inputs(1, 10, 2, 1, dev)
    with pytest.raises(NotImplementedError):
        hmx.chunk_gated_delta_rule(q.float().requires_grad_(True), k.float(), v.float(), g, beta)
    with pytest.raises(ValueError):
        ChunkGatedDeltaRule.apply(q, k, v, g[:, :5], beta, None, None, False, None, True, None)


def test_backward_all_heads_subset_against_oracle(dev):
    """The training head count (H = 32) over two 1024-token sequences: every head runs
    on the GPU, three of them (first, middle, last) are checked against the oracle
    (heads are independent, so the others' indexing shows in these)."""
    B, T, H = 2, 1024, 32
    q, k, v, g, beta, do = _inputs(B, T, H, 12, dev)
    ins = [t.clone().requires_grad_(True) for t in (q, k, v, g, beta)]
    o, _ = ChunkGatedDeltaRule.apply(*ins, D ** -0.5, None, False, None, True, None)
    (o.float() * do.float()).sum().backward()
    for hh in (0, 13, 31):
        sl = lambda t: t.detach()[:, :, hh:hh + 1].cpu()
        for b in range(B):
            r = gt.recurrent_grads(*(sl(t)[b] for t in (q, k, v, g, beta)), D ** -0.5, None,
                                   sl(do)[b], None, True)
            errs = {name: rel_err(t.grad[b, :, hh:hh + 1], e)
                    for name, t, e in zip(["dq", "dk", "dv", "dg", "dbeta"], ins, r)}
            print("head", hh, "seq", b, {n: f"{e:.2e}" for n, e in errs.items()})
            for name, e in errs.items():
                assert e < GRAD_REL, f"head {hh} seq {b} {name}: rel {e:.3e}"


def test_backward_layer_gates_against_oracle(dev):
    """The gates a freshly initialised layer forms (hmx.workloads.gdn_layer_gates:
    A_log = log U(1, 16), Mamba2 dt_bias): several heads decay too slowly for any
    warm-up, so their state-gradient runs take the exact combine."""
    from hmx import workloads as wl
    T, H = 2048, 4
    q, k, v, _, _, do = _inputs(1, T, H, 13, dev)
    g, beta = wl.gdn_layer_gates(T, H, device=dev)
    ins = [t.clone().requires_grad_(True) for t in (q, k, v, g, beta)]
    o, _ = ChunkGatedDeltaRule.apply(*ins, D ** -0.5, None, False, None, True, None)
    (o.float() * do.float()).sum().backward()
    r = gt.recurrent_grads(*(t.detach()[0].cpu() for t in (q, k, v, g, beta)), D ** -0.5, None,
                           do[0].cpu(), None, True)
    errs = {name: rel_err(t.grad[0], e) for name, t, e in zip(["dq", "dk", "dv", "dg", "dbeta"],
                                                              ins, r)}
    print("errors", {n: f"{e:.2e}" for n, e in errs.items()})
    for name, e in errs.items():
        assert e < GRAD_REL, f"{name}: rel {e:.3e}"
