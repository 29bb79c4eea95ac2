"""Gates formed inside the mixer kernels from the layer's raw projections
(hmx.ProjGates, the hmx_gate_proj ABI) against the two-step path the layers take:
the gating op writes [tokens, H] gate tensors in the projections' dtype, the mixer
op reads them (fused_gdn_gating.py:79-125, primed_gdn_layer.py:798-802;
primed_gka_layer.py:224-358, :1138-1153).  Both paths share the gate arithmetic
and its rounding to the projection dtype, so outputs and states agree exactly;
the layer without a forgetting gate (torch's sigmoid in the two-step path) is
compared to the output tolerance.  The serving cores are checked to launch no
gating kernel."""
import pytest
import torch
import torch.nn.functional as F

import hmx
import hmx.serving as srv
from hmx import _lib
from util import assert_out_close, assert_state_close

pytestmark = pytest.mark.gpu

H, D = 8, 128


def _proj(T, seed, dev, width=3):
    """a, b, alpha_in as column slices of one [T, width*H] projection (strided), plus
    the layer parameters (A_log ~ log U(1,16), dt_bias from dt ~ logU(1e-3, 1e-1))."""
    g0 = torch.Generator().manual_seed(seed)
    proj = torch.randn(T, width * H, generator=g0).bfloat16().to(dev)
    a, b, ai = proj[:, :H], proj[:, H:2 * H], proj[:, 2 * H:3 * H]
    A_log = torch.log(torch.rand(H, generator=g0) * 15 + 1).to(dev)
    dt = torch.exp(torch.rand(H, generator=g0) * (torch.log(torch.tensor(0.1)) -
                                                    torch.log(torch.tensor(1e-3)))
                   + torch.log(torch.tensor(1e-3)))
    dt_bias = (dt + torch.log(-torch.expm1(-dt))).to(dev)
    return a, b, ai, A_log, dt_bias


def _qkv(T, seed, dev):
    g0 = torch.Generator().manual_seed(seed)
    return [torch.randn(1, T, H, D, generator=g0).bfloat16().to(dev) for _ in range(3)]


def _equal(xs, ys):
    for x, y in zip(xs, ys):
        if x is None:
            assert y is None
            continue
        assert torch.equal(x, y), (x.float() - y.float()).abs().max().item()


@pytest.mark.parametrize("neg", [False, True])
def test_gdn_prefill_gates_equal_two_step(dev, neg):
    T = 700
    cu = torch.tensor([0, 250, 251, 700], dtype=torch.int32, device=dev)
    q, k, v = _qkv(T, 1, dev)
    a, b, _, A_log, dt_bias = _proj(T, 2, dev)
    g, beta = hmx.fused_gdn_gating(A_log, a, b, dt_bias)
    if neg:
        beta = beta * 2.0
    h0 = torch.randn(3, H, D, D, device=dev) * 0.05
    ref = hmx.chunk_gated_delta_rule_gqa(q, k, v, g, beta, initial_state=h0,
                                         output_final_state=True, cu_seqlens=cu,
                                         use_qk_l2norm_in_kernel=True, _segment_chunks=4)
    gates = hmx.ProjGates(A_log, dt_bias, a, b, beta_scale=2.0 if neg else 1.0)
    got = hmx.chunk_gated_delta_rule_gqa(q, k, v, None, None, initial_state=h0,
                                         output_final_state=True, cu_seqlens=cu,
                                         use_qk_l2norm_in_kernel=True, gates=gates,
                                         _segment_chunks=4)
    _equal(got, ref)


def test_gdn_decode_gates_equal_two_step(dev):
    N, slots = 5, 9
    q, k, v = (x[:, :N] for x in _qkv(N, 3, dev))
    a, b, _, A_log, dt_bias = _proj(N, 4, dev)
    g, beta = hmx.fused_gdn_gating(A_log, a, b, dt_bias)
    pool = torch.randn(slots, H, D, D, device=dev) * 0.05
    idx = torch.tensor([3, 0, 8, 5, 1], dtype=torch.int32, device=dev)
    cu = torch.arange(N + 1, dtype=torch.int32, device=dev)
    p1, p2 = pool.clone(), pool.clone()
    o1, _ = hmx.fused_recurrent_gated_delta_rule_gqa(q, k, v, g, beta, initial_state=p1,
                                                     cu_seqlens=cu, ssm_state_indices=idx,
                                                     use_qk_l2norm_in_kernel=True)
    o2, _ = hmx.fused_recurrent_gated_delta_rule_gqa(q, k, v, None, None, initial_state=p2,
                                                     cu_seqlens=cu, ssm_state_indices=idx,
                                                     use_qk_l2norm_in_kernel=True,
                                                     gates=hmx.ProjGates(A_log, dt_bias, a, b))
    _equal([o2, p2], [o1, p1])


def _gka_two_step(A_log, dt_bias, a, b, ai, fg, kk, use_beta, num_iter, alpha_plus):
    if fg:
        g, alpha, beta = hmx.fused_gka_gating(A_log, a, ai, b if use_beta else None, dt_bias)
    else:
        g = None
        alpha = ai.sigmoid().unsqueeze(0)
        beta = b.sigmoid().unsqueeze(0) if use_beta else None
    if num_iter == 0:
        alpha = torch.zeros_like(alpha)
    elif alpha_plus:
        alpha = alpha + 0.5
    return alpha, g, (g if kk else None), beta


GKA_CASES = [  # forgetting gate, kk gate, beta gate, num_iter, alpha + 0.5
    (True, True, True, 8, True),
    (True, False, True, 4, False),
    (False, False, False, 8, True),
    (True, True, False, 0, True),
]


@pytest.mark.parametrize("fg,kk,use_beta,num_iter,alpha_plus", GKA_CASES)
def test_gka_prefill_gates_equal_two_step(dev, fg, kk, use_beta, num_iter, alpha_plus):
    T = 300
    cu = torch.tensor([0, 130, 300], dtype=torch.int32, device=dev)
    q, k, v = _qkv(T, 5, dev)
    a, b, ai, A_log, dt_bias = _proj(T, 6, dev)
    alpha, g, gk, beta = _gka_two_step(A_log, dt_bias, a, b, ai, fg, kk, use_beta, num_iter,
                                       alpha_plus)
    ref = hmx.gka_chebyshev_gla_prefill(q, k, v, alpha, g, gk, beta, D ** -0.5, ridge_ratio=0.02,
                                        num_iter=num_iter, cu_seqlens=cu, _segment_chunks=1)
    gates = hmx.ProjGates(A_log if fg else None, dt_bias, a, b if use_beta else None, ai,
                          alpha_add=0.5 if (num_iter != 0 and alpha_plus) else 0.0,
                          alpha_zero=num_iter == 0, gk_from_g=fg and kk)
    got = hmx.gka_chebyshev_gla_prefill(q, k, v, None, None, None, None, D ** -0.5,
                                        ridge_ratio=0.02, num_iter=num_iter, cu_seqlens=cu,
                                        gates=gates, _segment_chunks=1)
    if fg:
        _equal(got, ref)
    else:       # torch's sigmoid in the two-step path
        assert_out_close(got[0], ref[0].double())
        for x, y in zip(got[1:], ref[1:]):
            if x is not None:
                assert_state_close(x, y.double())


def test_gka_decode_gates_equal_two_step(dev):
    N, slots = 4, 6
    q, k, v = (x[:, :N] for x in _qkv(N, 7, dev))
    a, b, ai, A_log, dt_bias = _proj(N, 8, dev)
    alpha, g, gk, beta = _gka_two_step(A_log, dt_bias, a, b, ai, True, True, True, 8, True)
    x16 = torch.randn(slots, H, D, 16, device=dev) * 0.05
    hkk = x16 @ x16.transpose(-1, -2)
    hkv = torch.randn(slots, H, D, D, device=dev) * 0.02
    idx = torch.tensor([2, 5, 0, 3], dtype=torch.int32, device=dev)
    cu = torch.arange(N + 1, dtype=torch.int32, device=dev)
    s1, s2 = (hkk.clone(), hkv.clone()), (hkk.clone(), hkv.clone())
    o1 = hmx.gka_chebyshev_gla_decode(q, k, v, alpha, g, gk, beta, D ** -0.5, num_iter=8,
                                      h_kk=s1[0], h_kv=s1[1], cu_seqlens=cu,
                                      ssm_state_indices=idx)[0]
    gates = hmx.ProjGates(A_log, dt_bias, a, b, ai, alpha_add=0.5, gk_from_g=True)
    o2 = hmx.gka_chebyshev_gla_decode(q, k, v, None, None, None, None, D ** -0.5, num_iter=8,
                                      h_kk=s2[0], h_kv=s2[1], cu_seqlens=cu,
                                      ssm_state_indices=idx, gates=gates)[0]
    _equal([o2, *s2], [o1, *s1])


def test_gates_argument_errors(dev):
    T = 10
    q, k, v = _qkv(T, 9, dev)
    a, b, ai, A_log, dt_bias = _proj(T, 10, dev)
    with pytest.raises(ValueError):          # GDN needs b
        hmx.chunk_gated_delta_rule_gqa(q, k, v, None, None, gates=hmx.ProjGates(A_log, dt_bias, a))
    with pytest.raises(ValueError):          # wrong token count
        hmx.chunk_gated_delta_rule_gqa(q, k, v, None, None,
                                       gates=hmx.ProjGates(A_log, dt_bias, a[:5], b[:5]))


@pytest.mark.parametrize("kind", ["gdn", "gka"])
def test_serving_core_launches_no_gating(dev, kind, monkeypatch):
    """The serving cores form the gates inside the mixer kernels: no hmx_*_gating
    entry point is called."""
    import test_serving_gpu as ts
    called = []
    real = _lib.call

    def spy(name, *args):
        called.append(name)
        return real(name, *args)

    monkeypatch.setattr(_lib, "call", spy)
    r = ts._run(kind, "mixed", dev)
    assert not any("gating" in c for c in called), called
    assert any("fwd" in c for c in called)
    o_r, _, _ = ts._expected(kind, r["lay"], r["lens"], r["idx"], r["has"], r["nd"],
                             r["mixed_qkv"], r["gates"], r["conv_cache"], r["states"])
    assert_out_close(r["core"][:r["n"]], o_r)
