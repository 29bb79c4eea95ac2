"""GPU: the GDN ops as the vLLM layer calls them (primed_gdn_layer.py:790-936).

- q/k/v as column slices of one fused [tokens, (H + 2 HKV) x 128] projection are
  read in place and give bit-identical results to contiguous copies (prefill and
  decode);
- the prefill with ``ssm_state_indices`` / ``has_initial_state`` reads and writes
  the state pool in place, bit-identical to the layer's own gather -> zero ->
  op -> scatter sequence (primed_gdn_layer.py:868-879) on fp32 and bf16 pools,
  with sequences split into segments (the staged end states) and the exact
  segment scan (which reads the pool in an earlier launch);
- a negative slot starts from zero and leaves the pool alone;
- ``out=`` receives o.

The dense paths these are compared with are checked against the oracle in
test_gdn_prefill_gpu.py / test_gdn_decode_gpu.py.
"""
import pytest
import torch
import torch.nn.functional as F

import hmx

pytestmark = pytest.mark.gpu

D = 128


def _fused(T, H, HKV, seed, dev, weak_head=False):
    g0 = torch.Generator().manual_seed(seed)
    mixed = torch.randn(T, (H + 2 * HKV) * D, generator=g0).bfloat16().to(dev)
    q = mixed[:, :H * D].view(1, T, H, D)
    k = mixed[:, H * D:(H + HKV) * D].view(1, T, HKV, D)
    v = mixed[:, (H + HKV) * D:].view(1, T, HKV, D)
    g = F.logsigmoid(torch.randn(1, T, H, generator=g0))
    if weak_head:   # head 0 decays weakly: the exact segment scan runs for it
        g[..., 0] = F.logsigmoid(torch.randn(1, T, generator=g0) * 0.1 + 8.0)
    beta = torch.sigmoid(torch.randn(1, T, H, generator=g0))
    return q, k, v, g.to(dev), beta.to(dev), g0


def _cu(lens, dev):
    return torch.tensor([0] + list(torch.tensor(lens).cumsum(0)), dtype=torch.int32, device=dev)


@pytest.mark.parametrize("H,HKV,seg", [(4, 4, None), (4, 2, 2)])
def test_prefill_strided_qkv_equals_contiguous(dev, H, HKV, seg):
    lens = [300, 0, 77, 450]
    q, k, v, g, beta, g0 = _fused(sum(lens), H, HKV, 1, dev)
    assert q.stride(1) == (H + 2 * HKV) * D
    cu = _cu(lens, dev)
    h0 = (torch.randn(len(lens), H, D, D, generator=g0) * 0.05).to(dev)
    kw = dict(initial_state=h0, output_final_state=True, cu_seqlens=cu,
              use_qk_l2norm_in_kernel=True, _segment_chunks=seg)
    o1, s1 = hmx.chunk_gated_delta_rule_gqa(q, k, v, g, beta, **kw)
    o2, s2 = hmx.chunk_gated_delta_rule_gqa(q.contiguous(), k.contiguous(), v.contiguous(), g,
                                            beta, **kw)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(s1, s2)


@pytest.mark.parametrize("pool_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("seg,weak", [(None, False), (3, False), (3, True)])
def test_prefill_pool_in_place_equals_gather_scatter(dev, pool_dtype, seg, weak):
    lens = [130, 0, 64, 400, 1, 200]
    H, HKV = 4, 2
    q, k, v, g, beta, g0 = _fused(sum(lens), H, HKV, 2, dev, weak_head=weak)
    cu = _cu(lens, dev)
    pool = (torch.randn(9, H, D, D, generator=g0) * 0.05).to(pool_dtype).to(dev)
    idx = torch.tensor([5, 2, 0, 8, 3, 1], dtype=torch.int32, device=dev)
    has = torch.tensor([True, True, False, True, False, True], device=dev)
    # the layer's sequence: gather, zero, op, scatter
    init = pool[idx.long()].contiguous()
    init[~has] = 0
    o_ref, s_ref = hmx.chunk_gated_delta_rule_gqa(q, k, v, g, beta, initial_state=init,
                                                  output_final_state=True, cu_seqlens=cu,
                                                  use_qk_l2norm_in_kernel=True,
                                                  _segment_chunks=seg)
    pool_ref = pool.clone()
    pool_ref[idx.long()] = s_ref.to(pool_dtype)
    # in place
    pool2 = pool.clone()
    out = torch.empty(1, sum(lens), H, D, dtype=torch.bfloat16, device=dev)
    o, st = hmx.chunk_gated_delta_rule_gqa(q, k, v, g, beta, initial_state=pool2,
                                           output_final_state=True, cu_seqlens=cu,
                                           use_qk_l2norm_in_kernel=True, ssm_state_indices=idx,
                                           has_initial_state=has, out=out, _segment_chunks=seg)
    torch.cuda.synchronize()
    assert st is pool2 and o is out
    assert torch.equal(o, o_ref)
    assert torch.equal(pool2, pool_ref)


def test_prefill_pool_negative_slot_and_no_final(dev):
    lens = [90, 150]
    H = 2
    q, k, v, g, beta, g0 = _fused(sum(lens), H, H, 3, dev)
    cu = _cu(lens, dev)
    pool = (torch.randn(3, H, D, D, generator=g0) * 0.05).to(dev)
    idx = torch.tensor([-1, 2], dtype=torch.int32, device=dev)
    pool2 = pool.clone()
    o, _ = hmx.chunk_gated_delta_rule_gqa(q, k, v, g, beta, initial_state=pool2,
                                          output_final_state=True, cu_seqlens=cu,
                                          use_qk_l2norm_in_kernel=True, ssm_state_indices=idx,
                                          _segment_chunks=2)
    init = torch.stack([torch.zeros_like(pool[0]), pool[2]])
    o_ref, s_ref = hmx.chunk_gated_delta_rule_gqa(q, k, v, g, beta, initial_state=init,
                                                  output_final_state=True, cu_seqlens=cu,
                                                  use_qk_l2norm_in_kernel=True,
                                                  _segment_chunks=2)
    torch.cuda.synchronize()
    assert torch.equal(o, o_ref)
    assert torch.equal(pool2[:2], pool[:2]) and torch.equal(pool2[2], s_ref[1])
    # output_final_state=False: the pool is read, never written
    pool3 = pool.clone()
    o3, s3 = hmx.chunk_gated_delta_rule_gqa(q, k, v, g, beta, initial_state=pool3,
                                            output_final_state=False, cu_seqlens=cu,
                                            use_qk_l2norm_in_kernel=True, ssm_state_indices=idx)
    torch.cuda.synchronize()
    assert s3 is None and torch.equal(pool3, pool) and torch.equal(o3, o_ref)


def test_decode_strided_qkv_equals_contiguous(dev):
    N, H, HKV = 6, 4, 2
    q, k, v, g, beta, g0 = _fused(N, H, HKV, 4, dev)
    pool = (torch.randn(8, H, D, D, generator=g0) * 0.05).to(dev)
    idx = torch.tensor([3, 7, 0, 5, -1, 1], dtype=torch.int32, device=dev)
    cu = torch.arange(N + 1, dtype=torch.int32, device=dev)
    p1, p2 = pool.clone(), pool.clone()
    o1, _ = hmx.fused_recurrent_gated_delta_rule_gqa(q, k, v, g, beta, initial_state=p1,
                                                     cu_seqlens=cu, ssm_state_indices=idx,
                                                     use_qk_l2norm_in_kernel=True)
    o2, _ = hmx.fused_recurrent_gated_delta_rule_gqa(q.contiguous(), k.contiguous(),
                                                     v.contiguous(), g, beta, initial_state=p2,
                                                     cu_seqlens=cu, ssm_state_indices=idx,
                                                     use_qk_l2norm_in_kernel=True)
    torch.cuda.synchronize()
    live = (idx >= 0).nonzero().flatten()      # a padded entry's output is never written
    assert torch.equal(o1[:, live], o2[:, live]) and torch.equal(p1, p2)


def test_pool_argument_errors(dev):
    q, k, v, g, beta, _ = _fused(10, 2, 2, 5, dev)
    pool = torch.zeros(2, 2, D, D, device=dev)
    with pytest.raises(ValueError, match="state pool"):
        hmx.chunk_gated_delta_rule_gqa(q, k, v, g, beta, initial_state=pool[:, :1],
                                       ssm_state_indices=torch.zeros(1, dtype=torch.int32,
                                                                     device=dev))
    with pytest.raises(ValueError, match="slots"):
        hmx.chunk_gated_delta_rule_gqa(q, k, v, g, beta, initial_state=pool,
                                       ssm_state_indices=torch.zeros(2, dtype=torch.int32,
                                                                     device=dev))
    with pytest.raises(ValueError, match="out must be"):
        hmx.chunk_gated_delta_rule_gqa(q, k, v, g, beta,
                                       out=torch.empty(1, 10, 2, D, device=dev))


def test_prefill_pool_in_place_c1_varlen(dev):
    """C1's varlen case (8 sequences, 36-42K tokens, H = 32) with the pool read and
    written in place: the planner splits the long sequences into segments (staged
    end states) exactly as at full scale; bit-identical to gather -> op -> scatter."""
    from hmx import workloads as wl
    lens = wl.varlen_lengths()
    cu = wl.cu_from_lengths(lens).to(dev)
    T = int(lens.sum())
    d = wl.gdn_inputs(T=T, H=32, HKV=32, D=D, config_id=1, device=dev, gen_device=dev)
    args = [d[n] for n in ("q", "k", "v", "g", "beta")]
    g0 = torch.Generator(device=dev).manual_seed(9)
    pool = torch.randn(12, 32, D, D, generator=g0, device=dev) * 0.02
    idx = torch.tensor([7, 2, 11, 0, 5, 9, 1, 4], dtype=torch.int32, device=dev)
    has = torch.tensor([True, False, True, True, False, True, True, True], device=dev)
    init = pool[idx.long()].contiguous()
    init[~has] = 0
    o_ref, s_ref = hmx.chunk_gated_delta_rule_gqa(*args, initial_state=init, output_final_state=True,
                                                  cu_seqlens=cu, use_qk_l2norm_in_kernel=True)
    pool_ref = pool.clone()
    pool_ref[idx.long()] = s_ref
    pool2 = pool.clone()
    o, _ = hmx.chunk_gated_delta_rule_gqa(*args, initial_state=pool2, output_final_state=True,
                                          cu_seqlens=cu, use_qk_l2norm_in_kernel=True,
                                          ssm_state_indices=idx, has_initial_state=has)
    torch.cuda.synchronize()
    assert torch.equal(o, o_ref) and torch.equal(pool2, pool_ref)
