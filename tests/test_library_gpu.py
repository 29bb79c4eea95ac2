"""GPU: the torch.ops.hmx registrations run the same kernels as the direct calls
(bit-identical outputs), their declared mutations match what the kernels write,
and torch.library.opcheck accepts the schemas and fake implementations."""
import pytest
import torch
import torch.nn.functional as F

import hmx
import hmx.library as hl

pytestmark = pytest.mark.gpu


def _gdn(dev, T=100, H=4, HKV=2, seed=0):
    g0 = torch.Generator().manual_seed(seed)
    q = torch.randn(1, T, H, 128, generator=g0).bfloat16().to(dev)
    k = torch.randn(1, T, HKV, 128, generator=g0).bfloat16().to(dev)
    v = torch.randn(1, T, HKV, 128, generator=g0).bfloat16().to(dev)
    g = F.logsigmoid(torch.randn(1, T, H, generator=g0)).to(dev)
    beta = torch.sigmoid(torch.randn(1, T, H, generator=g0)).to(dev)
    return q, k, v, g, beta


def test_chunk_gdn_registered_equals_direct(dev):
    q, k, v, g, beta = _gdn(dev)
    cu = torch.tensor([0, 40, 100], dtype=torch.int32, device=dev)
    o1, s1 = hmx.chunk_gated_delta_rule_gqa(q, k, v, g, beta, output_final_state=True,
                                            cu_seqlens=cu, use_qk_l2norm_in_kernel=True)
    o2, s2 = hl.chunk_gated_delta_rule_gqa(q, k, v, g, beta, output_final_state=True,
                                           cu_seqlens=cu, use_qk_l2norm_in_kernel=True)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(s1, s2)
    o3, s3 = hl.chunk_gated_delta_rule_gqa(q, k, v, g, beta, use_qk_l2norm_in_kernel=True,
                                           cu_seqlens=cu)
    assert s3 is None and torch.equal(o3, o1)


def test_recurrent_gdn_registered_mutates_pool(dev):
    q, k, v, g, beta = _gdn(dev, T=3, seed=1)
    pool = torch.randn(5, 4, 128, 128, device=dev) * 0.02
    pool2 = pool.clone()
    idx = torch.tensor([4, 0, 2], dtype=torch.int32, device=dev)
    cu = torch.arange(4, dtype=torch.int32, device=dev)
    o1, _ = hmx.fused_recurrent_gated_delta_rule_gqa(q, k, v, g, beta, initial_state=pool,
                                                     cu_seqlens=cu, ssm_state_indices=idx,
                                                     use_qk_l2norm_in_kernel=True)
    o2, st = hl.fused_recurrent_gated_delta_rule_gqa(q, k, v, g, beta, initial_state=pool2,
                                                     cu_seqlens=cu, ssm_state_indices=idx,
                                                     use_qk_l2norm_in_kernel=True)
    torch.cuda.synchronize()
    assert st is pool2 and torch.equal(o1, o2) and torch.equal(pool, pool2)


def test_selective_state_update_registered(dev):
    g0 = torch.Generator().manual_seed(2)
    H, P, N = 4, 64, 128
    state = (torch.randn(3, H, P, N, generator=g0) * 0.1).to(dev)
    state2 = state.clone()
    x = torch.randn(2, H, P, generator=g0).bfloat16().to(dev)
    dt = (torch.randn(2, H, generator=g0) - 2).to(dev)[:, :, None].expand(2, H, P)
    A = (-torch.rand(H, generator=g0) * 4).to(dev)[:, None, None].expand(H, P, N)
    B = torch.randn(2, 1, N, generator=g0).bfloat16().to(dev)
    idx = torch.tensor([2, 0], dtype=torch.int32, device=dev)
    o1 = hmx.selective_state_update(state, x, dt, A, B, B, dt_softplus=True, state_batch_indices=idx)
    o2 = hl.selective_state_update(state2, x, dt, A, B, B, dt_softplus=True, state_batch_indices=idx)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(state, state2)


def test_opcheck_functional_ops(dev):
    q, k, v, g, beta = _gdn(dev, T=40, seed=3)
    torch.library.opcheck(torch.ops.hmx.chunk_gated_delta_rule_gqa.default,
                          (q, k, v, g, beta, 0.088, None, True, None, True),
                          test_utils=("test_schema", "test_faketensor",
                                      "test_autograd_registration"))
    x = torch.randn(1, 70, 4, 64, device=dev).bfloat16()
    dt = torch.randn(1, 70, 4, device=dev) - 2
    Bm = torch.randn(1, 70, 1, 128, device=dev).bfloat16()
    A = -torch.rand(4, device=dev)
    torch.library.opcheck(torch.ops.hmx.mamba_chunk_scan_combined.default,
                          (x, dt, A, Bm, Bm, 256, None, None, None, None, None, True, 0.0,
                           float("inf")),
                          test_utils=("test_schema", "test_faketensor",
                                      "test_autograd_registration"))


def test_conv_and_norm_registered_equal_direct(dev):
    g0 = torch.Generator().manual_seed(4)
    x = torch.randn(150, 256, generator=g0).bfloat16().to(dev)
    w = torch.randn(256, 4, generator=g0).to(dev)
    b = torch.randn(256, generator=g0).to(dev)
    pool = torch.randn(4, 3, 256, generator=g0).bfloat16().to(dev).transpose(1, 2)
    pool2 = pool.clone(memory_format=torch.preserve_format)
    qs = torch.tensor([0, 60, 150], dtype=torch.int32, device=dev)
    idx = torch.tensor([3, 1], dtype=torch.int32, device=dev)
    o1 = hmx.causal_conv1d_fn(x.t(), w, b, conv_states=pool, query_start_loc=qs, cache_indices=idx)
    o2 = hl.causal_conv1d_fn(x.t(), w, b, conv_states=pool2, query_start_loc=qs, cache_indices=idx)
    torch.cuda.synchronize()
    assert o2.shape == (256, 150) and torch.equal(o1, o2) and torch.equal(pool, pool2)
    u1 = hmx.causal_conv1d_update(x[:2], pool, w, b, "silu", conv_state_indices=idx)
    u2 = hl.causal_conv1d_update(x[:2], pool2, w, b, True, conv_state_indices=idx)
    torch.cuda.synchronize()
    assert torch.equal(u1, u2) and torch.equal(pool, pool2)
    z = torch.randn(2, 9, 4, 128, generator=g0).bfloat16().to(dev)
    wn = torch.rand(128, generator=g0).to(dev)
    assert torch.equal(hmx.rms_norm_gated(z, z.flip(0), wn, 1e-6),
                       hl.rms_norm_gated(z, z.flip(0), wn, 1e-6))
    torch.library.opcheck(torch.ops.hmx.rms_norm_gated.default, (z, z.flip(0), wn, 1e-6, True),
                          test_utils=("test_schema", "test_faketensor",
                                      "test_autograd_registration"))
    torch.library.opcheck(torch.ops.hmx.causal_conv1d_update.default,
                          (x[:2], pool.clone(memory_format=torch.preserve_format), w, b, "silu",
                           idx, -1),
                          test_utils=("test_schema", "test_faketensor"))
