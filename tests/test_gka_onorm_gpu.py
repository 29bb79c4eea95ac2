"""GPU parity: the GKA prefill and decode ops with the layer's output gated RMSNorm
fused into the kernel (o_norm_weight / o_norm_gate, eps 1e-6) against the unfused
pair (the same op, then hmx.rms_norm_gated on its bf16 output: both norm the same
rounded o in fp32, so they agree to one unit in the last place), with the states
written identically.  Covers single- and multi-segment prefill, ragged tails, no
gate, and the slot-pool decode step.
"""
import pytest
import torch
import torch.nn.functional as F

import hmx
from util import half_ulp

pytestmark = pytest.mark.gpu


def _mk(n_tok, H, HKV, seed):
    g0 = torch.Generator().manual_seed(seed)
    q = torch.randn(1, n_tok, H, 128, generator=g0).bfloat16()
    k = torch.randn(1, n_tok, HKV, 128, generator=g0).bfloat16()
    v = torch.randn(1, n_tok, HKV, 128, generator=g0).bfloat16()
    alpha = torch.sigmoid(torch.randn(1, n_tok, H, generator=g0))
    g = F.logsigmoid(torch.randn(1, n_tok, H, generator=g0))
    beta = torch.sigmoid(torch.randn(1, n_tok, H, generator=g0))
    z = (torch.randn(1, n_tok, H, 128, generator=g0) * 1.5).bfloat16()
    w = torch.rand(128, generator=g0) + 0.5
    return q, k, v, alpha, g, beta, z, w, g0


def _close_ulp(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    assert ((a - b).abs() <= 2 * half_ulp(b, torch.bfloat16) + 1e-30).all()
    assert (a == b).double().mean().item() >= 0.98


@pytest.mark.parametrize("T,seg,gated", [(77, None, True), (32 * 20 + 5, 4, True), (100, None, False)])
def test_prefill_fused_norm(dev, T, seg, gated):
    q, k, v, alpha, g, beta, z, w, _ = _mk(T, 4, 2, T)
    d = [x.to(dev) for x in (q, k, v, alpha, g, g, beta)]
    zz = z.to(dev) if gated else None
    o, a1, b1 = hmx.gka_chebyshev_gla_prefill(*d, 0.09, ridge_ratio=0.02, num_iter=8,
                                              _segment_chunks=seg)
    on, a2, b2 = hmx.gka_chebyshev_gla_prefill(*d, 0.09, ridge_ratio=0.02, num_iter=8,
                                               _segment_chunks=seg, o_norm_weight=w.to(dev),
                                               o_norm_gate=zz)
    unf = hmx.rms_norm_gated(o, zz, w.to(dev), eps=1e-6)
    torch.cuda.synchronize()
    assert torch.equal(a1, a2) and torch.equal(b1, b2)
    _close_ulp(on, unf)


def test_decode_fused_norm(dev):
    N, H, HKV, slots = 6, 4, 2, 9
    q, k, v, alpha, g, beta, z, w, g0 = _mk(N, H, HKV, 3)
    x = torch.randn(slots, H, 128, 16, generator=g0) * 0.05
    hkk = x @ x.transpose(-1, -2)
    hkv = torch.randn(slots, H, 128, 128, generator=g0) * 0.02
    idx = torch.randperm(slots, generator=g0)[:N].to(torch.int32)
    cu = torch.arange(N + 1, dtype=torch.int32)
    gd = g.to(dev)   # the decode op needs the GLA gate to be the GKA gate (one tensor)
    d = [q.to(dev), k.to(dev), v.to(dev), alpha.to(dev), gd, gd, beta.to(dev)]
    kw = dict(ridge_ratio=0.02, num_iter=8, cu_seqlens=cu.to(dev), ssm_state_indices=idx.to(dev))
    k1, v1, k2, v2 = hkk.to(dev), hkv.to(dev), hkk.to(dev), hkv.to(dev)
    o, _, _ = hmx.gka_chebyshev_gla_decode(*d, 0.09, h_kk=k1, h_kv=v1, **kw)
    on, _, _ = hmx.gka_chebyshev_gla_decode(*d, 0.09, h_kk=k2, h_kv=v2, **kw,
                                            o_norm_weight=w.to(dev), o_norm_gate=z.to(dev))
    unf = hmx.rms_norm_gated(o, z.to(dev), w.to(dev), eps=1e-6)
    torch.cuda.synchronize()
    assert torch.equal(k1, k2) and torch.equal(v1, v2)
    _close_ulp(on, unf)
