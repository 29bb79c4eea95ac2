"""GPU: the GKA ops as the vLLM layer calls them (primed_gka_layer.py:1185-1300).

- q/k/v as column slices of one fused projection are read in place and give
  bit-identical results to contiguous copies (prefill and decode);
- the prefill with ``ssm_state_indices`` / ``has_initial_state`` reads and writes
  the h_kk / h_kv pools in place, bit-identical to the layer's gather -> zero ->
  op -> scatter sequence (primed_gka_layer.py:1245-1266) on fp32 and bf16 pools,
  single- and multi-segment (the combine launch then supplies every segment's
  start state), including num_iter == 0, where the layer rewrites h_kk from its
  zeroed gather (:1262-1265);
- a negative slot starts from zero and leaves the pools alone.

The dense paths these are compared with are checked against the oracle in
test_gka_gpu.py.
"""
import pytest
import torch
import torch.nn.functional as F

import hmx

pytestmark = pytest.mark.gpu

D = 128


def _fused(T, H, HKV, seed, dev):
    g0 = torch.Generator().manual_seed(seed)
    mixed = torch.randn(T, (H + 2 * HKV) * D, generator=g0).bfloat16().to(dev)
    q = mixed[:, :H * D].view(1, T, H, D)
    k = mixed[:, H * D:(H + HKV) * D].view(1, T, HKV, D)
    v = mixed[:, (H + HKV) * D:].view(1, T, HKV, D)
    gates = [torch.sigmoid(torch.randn(1, T, H, generator=g0)),        # alpha
             F.logsigmoid(torch.randn(1, T, H, generator=g0)),         # g (= gk)
             torch.sigmoid(torch.randn(1, T, H, generator=g0))]        # beta
    alpha, g, beta = (x.to(dev) for x in gates)
    return q, k, v, alpha, g, beta, g0


def _cu(lens, dev):
    return torch.tensor([0] + list(torch.tensor(lens).cumsum(0)), dtype=torch.int32, device=dev)


def _psd(slots, H, g0, dt, dev):
    x = torch.randn(slots, H, D, 16, generator=g0) * 0.05
    return (x @ x.transpose(-1, -2)).to(dt).to(dev)


@pytest.mark.parametrize("seg", [None, 2])
def test_prefill_strided_qkv_equals_contiguous(dev, seg):
    lens = [200, 0, 90, 130]
    H, HKV = 4, 2
    q, k, v, alpha, g, beta, g0 = _fused(sum(lens), H, HKV, 1, dev)
    cu = _cu(lens, dev)
    hkk = _psd(len(lens), H, g0, torch.float32, dev)
    hkv = (torch.randn(len(lens), H, D, D, generator=g0) * 0.02).to(dev)
    kw = dict(gla_scale=0.09, ridge_ratio=0.02, num_iter=8, h_kk_initial=hkk, h_kv_initial=hkv,
              output_final_state=True, cu_seqlens=cu, _segment_chunks=seg)
    r1 = hmx.gka_chebyshev_gla_prefill(q, k, v, alpha, g, g, beta, **kw)
    r2 = hmx.gka_chebyshev_gla_prefill(q.contiguous(), k.contiguous(), v.contiguous(), alpha, g,
                                       g, beta, **kw)
    torch.cuda.synchronize()
    for a, b in zip(r1, r2):
        assert torch.equal(a, b)


@pytest.mark.parametrize("kk_dt,kv_dt", [(torch.float32, torch.float32),
                                         (torch.float32, torch.bfloat16)])
@pytest.mark.parametrize("seg,num_iter", [(None, 8), (2, 8), (2, 0)])
def test_prefill_pools_in_place_equal_gather_scatter(dev, kk_dt, kv_dt, seg, num_iter):
    lens = [100, 0, 64, 170, 1, 90]
    H, HKV = 4, 2
    q, k, v, alpha, g, beta, g0 = _fused(sum(lens), H, HKV, 2, dev)
    cu = _cu(lens, dev)
    pkk = _psd(9, H, g0, kk_dt, dev)
    pkv = (torch.randn(9, H, D, D, generator=g0) * 0.02).to(kv_dt).to(dev)
    idx = torch.tensor([5, 2, 0, 8, 3, 1], dtype=torch.int32, device=dev)
    has = torch.tensor([True, True, False, True, False, True], device=dev)
    il = idx.long()
    # the layer's sequence (primed_gka_layer.py:1245-1266)
    hkk0, hkv0 = pkk[il].contiguous(), pkv[il].contiguous()
    hkk0[~has] = 0
    hkv0[~has] = 0
    o_ref, kk_f, kv_f = hmx.gka_chebyshev_gla_prefill(
        q, k, v, alpha, g, g, beta, 0.09, ridge_ratio=0.02, num_iter=num_iter,
        h_kk_initial=hkk0, h_kv_initial=hkv0, output_final_state=True, cu_seqlens=cu,
        _segment_chunks=seg)
    pkk_ref, pkv_ref = pkk.clone(), pkv.clone()
    pkk_ref[il] = hkk0 if num_iter == 0 else kk_f.to(kk_dt)
    pkv_ref[il] = kv_f.to(kv_dt)
    # in place
    pkk2, pkv2 = pkk.clone(), pkv.clone()
    out = torch.empty_like(o_ref)
    o, a, b = hmx.gka_chebyshev_gla_prefill(
        q, k, v, alpha, g, g, beta, 0.09, ridge_ratio=0.02, num_iter=num_iter,
        h_kk_initial=pkk2, h_kv_initial=pkv2, output_final_state=True, cu_seqlens=cu,
        ssm_state_indices=idx, has_initial_state=has, out=out, _segment_chunks=seg)
    torch.cuda.synchronize()
    assert o is out and b is pkv2 and (a is None if num_iter == 0 else a is pkk2)
    assert torch.equal(o, o_ref)
    assert torch.equal(pkv2, pkv_ref)
    assert torch.equal(pkk2, pkk_ref)


def test_prefill_pool_negative_slot(dev):
    lens = [70, 120]
    H = 2
    q, k, v, alpha, g, beta, g0 = _fused(sum(lens), H, H, 3, dev)
    cu = _cu(lens, dev)
    pkk = _psd(3, H, g0, torch.float32, dev)
    pkv = (torch.randn(3, H, D, D, generator=g0) * 0.02).to(dev)
    idx = torch.tensor([-1, 2], dtype=torch.int32, device=dev)
    pkk2, pkv2 = pkk.clone(), pkv.clone()
    o, _, _ = hmx.gka_chebyshev_gla_prefill(
        q, k, v, alpha, g, g, beta, 0.09, num_iter=8, h_kk_initial=pkk2, h_kv_initial=pkv2,
        cu_seqlens=cu, ssm_state_indices=idx, _segment_chunks=2)
    z = torch.zeros_like(pkk[0])
    o_ref, kk_f, kv_f = hmx.gka_chebyshev_gla_prefill(
        q, k, v, alpha, g, g, beta, 0.09, num_iter=8, h_kk_initial=torch.stack([z, pkk[2]]),
        h_kv_initial=torch.stack([z, pkv[2]]), cu_seqlens=cu, _segment_chunks=2)
    torch.cuda.synchronize()
    assert torch.equal(o, o_ref)
    assert torch.equal(pkk2[:2], pkk[:2]) and torch.equal(pkv2[:2], pkv[:2])
    assert torch.equal(pkk2[2], kk_f[1]) and torch.equal(pkv2[2], kv_f[1])


def test_decode_strided_qkv_equals_contiguous(dev):
    N, H, HKV = 6, 4, 2
    q, k, v, alpha, g, beta, g0 = _fused(N, H, HKV, 4, dev)
    pkk = _psd(8, H, g0, torch.float32, dev)
    pkv = (torch.randn(8, H, D, D, generator=g0) * 0.02).to(dev)
    idx = torch.tensor([3, 7, 0, 5, 2, 1], dtype=torch.int32, device=dev)
    cu = torch.arange(N + 1, dtype=torch.int32, device=dev)
    s1 = (pkk.clone(), pkv.clone())
    s2 = (pkk.clone(), pkv.clone())
    o1, _, _ = hmx.gka_chebyshev_gla_decode(q, k, v, alpha, g, g, beta, 0.09, num_iter=8,
                                            h_kk=s1[0], h_kv=s1[1], cu_seqlens=cu,
                                            ssm_state_indices=idx)
    o2, _, _ = hmx.gka_chebyshev_gla_decode(q.contiguous(), k.contiguous(), v.contiguous(), alpha,
                                            g, g, beta, 0.09, num_iter=8, h_kk=s2[0], h_kv=s2[1],
                                            cu_seqlens=cu, ssm_state_indices=idx)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(s1[0], s2[0]) and torch.equal(s1[1], s2[1])
