"""GPU: the Mamba2 varlen scan with the layer's state pool read and written in place
(``ssm_state_indices`` / ``has_initial_state``), bit-identical to the layer's
own sequence (primed_mamba2_layer.py:812-824 gather with has_initial_states,
the op, :941 scatter) on fp32 and bf16 pools, single- and multi-segment (the
combine launch then supplies every segment's start state); a negative slot
starts from zero and leaves the pool alone.  The dense path compared with is
checked against the oracle in test_ssd_gpu.py.
"""
import math

import pytest
import torch

import hmx

pytestmark = pytest.mark.gpu


def _inputs(lens, H, P, N, seed, dev):
    g0 = torch.Generator().manual_seed(seed)
    T = sum(lens)
    x = torch.randn(T, H, P, generator=g0).bfloat16().to(dev)
    B = torch.randn(T, H, N, generator=g0).bfloat16().to(dev)
    C = torch.randn(T, H, N, generator=g0).bfloat16().to(dev)
    dt = (torch.randn(T, H, generator=g0) * 0.5 - 2.0).to(dev)
    bias = (torch.randn(H, generator=g0) * 0.5 - 4.0).to(dev)
    A = (-torch.exp(torch.rand(H, generator=g0) * math.log(16))).to(dev)
    D = (torch.randn(H, generator=g0) * 0.1 + 1.0).to(dev)
    cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0)), dtype=torch.int32, device=dev)
    return x, dt, A, B, C, D, bias, cu, g0


@pytest.mark.parametrize("pool_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("seg", [None, 1])
def test_varlen_pool_in_place_equals_gather_scatter(dev, pool_dtype, seg):
    H, P, N = 8, 64, 128
    lens = [130, 0, 1, 64, 300, 70]
    x, dt, A, B, C, D, bias, cu, g0 = _inputs(lens, H, P, N, 1, dev)
    pool = (torch.randn(9, H, P, N, generator=g0) * 0.1).to(pool_dtype).to(dev)
    idx = torch.tensor([5, 2, 0, 8, 3, 1], dtype=torch.int32, device=dev)
    has = torch.tensor([True, True, False, True, False, True], device=dev)
    il = idx.long()
    init = torch.where(has[:, None, None, None], pool[il], 0)        # :818-823
    y_ref = torch.empty_like(x)
    s_ref = hmx.mamba_chunk_scan_combined_varlen(x, dt, A, B, C, 256, cu_seqlens=cu, out=y_ref,
                                                 D=D, dt_bias=bias, initial_states=init,
                                                 dt_softplus=True, _segment_chunks=seg)
    pool_ref = pool.clone()
    pool_ref[il] = s_ref.to(pool_dtype)                               # :941
    pool2 = pool.clone()
    y = torch.empty_like(x)
    st = hmx.mamba_chunk_scan_combined_varlen(x, dt, A, B, C, 256, cu_seqlens=cu, out=y, D=D,
                                              dt_bias=bias, initial_states=pool2,
                                              dt_softplus=True, ssm_state_indices=idx,
                                              has_initial_state=has, _segment_chunks=seg)
    torch.cuda.synchronize()
    assert st is pool2
    assert torch.equal(y, y_ref)
    assert torch.equal(pool2, pool_ref)


def test_varlen_pool_negative_slot(dev):
    H, P, N = 4, 64, 64
    lens = [200, 90]
    x, dt, A, B, C, D, bias, cu, g0 = _inputs(lens, H, P, N, 2, dev)
    pool = (torch.randn(3, H, P, N, generator=g0) * 0.1).to(dev)
    idx = torch.tensor([-1, 2], dtype=torch.int32, device=dev)
    pool2 = pool.clone()
    y = torch.empty_like(x)
    hmx.mamba_chunk_scan_combined_varlen(x, dt, A, B, C, 256, cu_seqlens=cu, out=y, D=D,
                                         dt_bias=bias, initial_states=pool2, dt_softplus=True,
                                         ssm_state_indices=idx, _segment_chunks=1)
    init = torch.stack([torch.zeros_like(pool[0]), pool[2]])
    y_ref = torch.empty_like(x)
    s_ref = hmx.mamba_chunk_scan_combined_varlen(x, dt, A, B, C, 256, cu_seqlens=cu, out=y_ref,
                                                 D=D, dt_bias=bias, initial_states=init,
                                                 dt_softplus=True, _segment_chunks=1)
    torch.cuda.synchronize()
    assert torch.equal(y, y_ref)
    assert torch.equal(pool2[:2], pool[:2]) and torch.equal(pool2[2], s_ref[1])
