"""GPU: hmx.gdn_conv_decode (the GDN layer's decode conv fused into the recurrent
step, hmx_gdn_conv_recurrent_fwd) equals hmx.causal_conv1d_update followed by
hmx.fused_recurrent_gated_delta_rule_gqa on q, k, v views of its output, as the
layer runs them (primed_gdn_layer.py:775-785, :805-823): outputs, the recurrent
state pool and the conv state pool bit for bit.  HKV == H (every channel's conv
state shifts in the kernel) and HKV < H (the group-shared k / v channels shift in a
second launch), fp32 and bf16 state pools, a padded entry (slot -1), and the gated
output norm."""
import pytest
import torch

import hmx

pytestmark = pytest.mark.gpu

K = V = 128


def _case(H, HKV, N, sdt, seed, dev, W=4, slots=12):
    g0 = torch.Generator().manual_seed(seed)
    dim = H * K + 2 * HKV * K
    x = torch.randn(N, dim, generator=g0).bfloat16().to(dev)
    w = (torch.randn(dim, W, generator=g0) * 0.4).bfloat16().to(dev)
    conv = torch.randn(slots, W - 1, dim, generator=g0).bfloat16().to(dev)
    pool = (torch.randn(slots, H, K, V, generator=g0) * 0.05).to(sdt).to(dev)
    idx = torch.randperm(slots, generator=g0)[:N].to(torch.int32)
    idx[N // 2] = -1
    A_log = (torch.rand(H, generator=g0) * 2 - 1).to(dev)
    dt_bias = (torch.randn(H, generator=g0) * 0.5).to(dev)
    a = torch.randn(N, H, generator=g0).bfloat16().to(dev)
    b = torch.randn(N, H, generator=g0).bfloat16().to(dev)
    z = torch.randn(1, N, H, V, generator=g0).bfloat16().to(dev)
    wn = (torch.rand(V, generator=g0) + 0.5).bfloat16().to(dev)
    return x, w, conv, pool, idx.to(dev), hmx.ProjGates(A_log, dt_bias, a, b), z, wn


@pytest.mark.parametrize("H,HKV,sdt,norm", [(8, 8, torch.float32, False),
                                            (8, 4, torch.float32, False),
                                            (8, 8, torch.bfloat16, True),
                                            (16, 2, torch.float32, True)])
def test_conv_decode_equals_conv_then_recurrent(dev, H, HKV, sdt, norm):
    N = 6
    x, w, conv, pool, idx, gates, z, wn = _case(H, HKV, N, sdt, 100 + H + HKV, dev)
    kw = dict(o_norm_weight=wn, o_norm_gate=z, o_norm_eps=1e-6) if norm else {}
    # reference order: the conv op, then the recurrent op on views of its output
    conv_r, pool_r = conv.clone(), pool.clone()
    xc = hmx.causal_conv1d_update(x, conv_r.transpose(1, 2), w, None, "silu",
                                  conv_state_indices=idx)
    q = xc[:, :H * K].view(1, N, H, K)
    k = xc[:, H * K:(H + HKV) * K].view(1, N, HKV, K)
    v = xc[:, (H + HKV) * K:].view(1, N, HKV, V)
    o_r = torch.zeros(1, N, H, V, dtype=torch.bfloat16, device=dev)
    hmx.fused_recurrent_gated_delta_rule_gqa(
        q, k, v, None, None, initial_state=pool_r, inplace_final_state=True,
        cu_seqlens=torch.arange(N + 1, dtype=torch.int32, device=dev), ssm_state_indices=idx,
        use_qk_l2norm_in_kernel=True, out=o_r, gates=gates, **kw)
    # fused
    conv_f, pool_f = conv.clone(), pool.clone()
    o_f = torch.zeros(1, N, H, V, dtype=torch.bfloat16, device=dev)
    hmx.gdn_conv_decode(x, w, None, conv_f.transpose(1, 2), "silu", pool_f, idx, H, HKV,
                        gates=gates, out=o_f, **kw)
    torch.cuda.synchronize()
    assert torch.equal(o_f, o_r)
    assert torch.equal(pool_f, pool_r)
    assert torch.equal(conv_f, conv_r)
    assert torch.equal(o_f[:, N // 2], torch.zeros_like(o_f[:, N // 2]))   # padded entry
