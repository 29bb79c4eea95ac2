"""GPU parity: hmx GDN fused recurrent decode vs the CPU oracle (fp64).

Covers the reference kernel's modes (fused_recurrent_gqa.py:25-277): slot-indexed
in-place pool update, GQA, varlen multi-token (speculative) sequences with
num_accepted_tokens and 2-D indices, zero-length sequences, non-in-place final
state, head-wise beta, f16/f32 inputs, bf16 state, K/V in {64,128,256}, and the
C2 shape (256 seqs x 32 heads, random slot permutation) over several steps.
"""
import pytest
import torch

import hmx
from hmx import workloads as wl
from oracle import gdn as ref
from util import assert_out_close, assert_state_close

pytestmark = pytest.mark.gpu


def _mk(n_tok, H, HKV, K, V, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.nn.functional.normalize(torch.randn(1, n_tok, H, K, generator=g), dim=-1).to(dtype)
    k = torch.nn.functional.normalize(torch.randn(1, n_tok, HKV, K, generator=g), dim=-1).to(dtype)
    v = torch.randn(1, n_tok, HKV, V, generator=g).to(dtype)
    gg = torch.nn.functional.logsigmoid(torch.randn(1, n_tok, H, generator=g))
    beta = torch.sigmoid(torch.randn(1, n_tok, H, generator=g))
    return q, k, v, gg, beta, g


@pytest.mark.parametrize("K,V,H,HKV", [(128, 128, 4, 4), (128, 128, 8, 2), (64, 64, 4, 1),
                                       (256, 128, 2, 2), (128, 256, 2, 1), (128, 32, 2, 2),
                                       (128, 160, 2, 2)])
def test_decode_pool_inplace(dev, K, V, H, HKV):
    N, slots = 7, 12
    q, k, v, g, beta, gen = _mk(N, H, HKV, K, V, torch.bfloat16, 1 + K + V + H)
    pool = torch.randn(slots, H, K, V, generator=gen) * 0.02
    idx = torch.randperm(slots, generator=gen)[:N].to(torch.int32)
    cu = torch.arange(N + 1, dtype=torch.int32)
    o_ref, pool_ref = ref.fused_recurrent_gated_delta_rule_gqa(
        q, k, v, g, beta, initial_state=pool, inplace_final_state=True, cu_seqlens=cu,
        ssm_state_indices=idx, use_qk_l2norm_in_kernel=True)
    pool_d = pool.to(dev)
    o, fs = hmx.fused_recurrent_gated_delta_rule_gqa(
        q.to(dev), k.to(dev), v.to(dev), g.to(dev), beta.to(dev), initial_state=pool_d,
        inplace_final_state=True, cu_seqlens=cu.to(dev), ssm_state_indices=idx.to(dev),
        use_qk_l2norm_in_kernel=True)
    torch.cuda.synchronize()
    assert fs.data_ptr() == pool_d.data_ptr()
    assert o.shape == (1, N, H, V) and o.dtype == torch.bfloat16
    assert_out_close(o, o_ref)
    assert_state_close(pool_d, pool_ref)
    # untouched slots stay bit-identical
    untouched = sorted(set(range(slots)) - set(idx.tolist()))
    assert torch.equal(pool_d.cpu()[untouched], pool[untouched])


def test_decode_spec_varlen(dev):
    """Multi-token sequences, zero-length entries, 2-D indices + num_accepted_tokens."""
    H, HKV, K, V = 4, 2, 128, 128
    lens = [3, 0, 5, 1, 4]
    cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0)), dtype=torch.int32)
    n_tok = int(cu[-1])
    q, k, v, g, beta, gen = _mk(n_tok, H, HKV, K, V, torch.bfloat16, 7)
    slots, S = 20, 3
    pool = torch.randn(slots, H, K, V, generator=gen) * 0.02
    idx = torch.randperm(slots, generator=gen)[:len(lens) * S].view(len(lens), S).to(torch.int32)
    nacc = torch.tensor([2, 1, 3, 1, 2], dtype=torch.int32)
    o_ref, pool_ref = ref.fused_recurrent_gated_delta_rule_gqa(
        q, k, v, g, beta, initial_state=pool, inplace_final_state=True, cu_seqlens=cu,
        ssm_state_indices=idx, num_accepted_tokens=nacc, use_qk_l2norm_in_kernel=True)
    pool_d = pool.to(dev)
    o, _ = hmx.fused_recurrent_gated_delta_rule_gqa(
        q.to(dev), k.to(dev), v.to(dev), g.to(dev), beta.to(dev), initial_state=pool_d,
        inplace_final_state=True, cu_seqlens=cu.to(dev), ssm_state_indices=idx.to(dev),
        num_accepted_tokens=nacc.to(dev), use_qk_l2norm_in_kernel=True)
    torch.cuda.synchronize()
    assert_out_close(o, o_ref)
    assert_state_close(pool_d, pool_ref)


@pytest.mark.parametrize("dtype,T", [(torch.float16, 1), (torch.float32, 1), (torch.float32, 3)])
def test_decode_not_inplace_headwise_beta(dev, dtype, T):
    H, HKV, K, V, B = 4, 4, 128, 64, 3
    g0 = torch.Generator().manual_seed(3)
    q = torch.randn(B, T, H, K, generator=g0).to(dtype)
    k = torch.randn(B, T, HKV, K, generator=g0).to(dtype)
    v = torch.randn(B, T, HKV, V, generator=g0).to(dtype)
    g = torch.nn.functional.logsigmoid(torch.randn(B, T, H, generator=g0))
    beta = torch.sigmoid(torch.randn(B, T, H, V, generator=g0))
    h0 = torch.randn(B * T, H, K, V, generator=g0) * 0.05
    o_ref, f_ref = ref.fused_recurrent_gated_delta_rule_gqa(
        q, k, v, g, beta, initial_state=h0, inplace_final_state=False,
        use_qk_l2norm_in_kernel=True)
    o, f = hmx.fused_recurrent_gated_delta_rule_gqa(
        q.to(dev), k.to(dev), v.to(dev), g.to(dev), beta.to(dev), initial_state=h0.to(dev),
        inplace_final_state=False, use_qk_l2norm_in_kernel=True)
    torch.cuda.synchronize()
    assert f.shape == (B, T, H, K, V)
    assert_out_close(o, o_ref)
    rows = [n * T for n in range(B)]    # sequence n's final state sits at row bos = n*T
    assert_state_close(f.view(B * T, H, K, V)[rows], f_ref.view(B * T, H, K, V)[rows])


def test_decode_not_inplace_varlen_rows(dev):
    """Without inplace_final_state, sequence n's state goes to flat row cu_seqlens[n]
    (fused_recurrent_gqa.py:137-139), also after a leading empty sequence."""
    H, K, V = 2, 128, 128
    q, k, v, g, beta, gen = _mk(5, H, H, K, V, torch.bfloat16, 12)
    cu = torch.tensor([0, 0, 2, 5], dtype=torch.int32)
    h0 = torch.randn(5, H, K, V, generator=gen) * 0.05
    o_ref, f_ref = ref.fused_recurrent_gated_delta_rule_gqa(
        q, k, v, g, beta, initial_state=h0, inplace_final_state=False, cu_seqlens=cu,
        use_qk_l2norm_in_kernel=True)
    o, f = hmx.fused_recurrent_gated_delta_rule_gqa(
        q.to(dev), k.to(dev), v.to(dev), g.to(dev), beta.to(dev), initial_state=h0.to(dev),
        inplace_final_state=False, cu_seqlens=cu.to(dev), use_qk_l2norm_in_kernel=True)
    torch.cuda.synchronize()
    assert_out_close(o, o_ref)
    assert_state_close(f.view(5, H, K, V)[[0, 2]], f_ref.view(5, H, K, V)[[0, 2]])


def test_decode_bf16_state_and_no_l2norm(dev):
    H, K, V, N = 2, 64, 64, 4
    q, k, v, g, beta, gen = _mk(N, H, H, K, V, torch.bfloat16, 11)
    pool = (torch.randn(N, H, K, V, generator=gen) * 0.02).to(torch.bfloat16)
    idx = torch.arange(N, dtype=torch.int32)
    cu = torch.arange(N + 1, dtype=torch.int32)
    o_ref, pool_ref = ref.fused_recurrent_gated_delta_rule_gqa(
        q, k, v, g, beta, initial_state=pool, inplace_final_state=True, cu_seqlens=cu,
        ssm_state_indices=idx, use_qk_l2norm_in_kernel=False)
    pool_d = pool.to(dev)
    o, _ = hmx.fused_recurrent_gated_delta_rule_gqa(
        q.to(dev), k.to(dev), v.to(dev), g.to(dev), beta.to(dev), initial_state=pool_d,
        inplace_final_state=True, cu_seqlens=cu.to(dev), ssm_state_indices=idx.to(dev),
        use_qk_l2norm_in_kernel=False)
    torch.cuda.synchronize()
    assert_out_close(o, o_ref)
    assert_state_close(pool_d, pool_ref, rel_tol=1e-2)  # bf16 storage of the state


def test_decode_c2_shape_steps(dev):
    """C2 shape: 256 seqs x 32 heads, random slot permutation, 3 consecutive steps."""
    steps = 3
    d = wl.decode_inputs(n_seqs=256, H=32, HKV=32, D=128, steps=steps)
    pool_ref = d["pool"].double()
    pool_d = d["pool"].to(dev)
    cu_d, idx_d = d["cu_seqlens"].to(dev), d["idx"].to(dev)
    for s in range(steps):
        args = [d[n][s] for n in ("q", "k", "v", "g", "beta")]
        o_ref, pool_ref = ref.fused_recurrent_gated_delta_rule_gqa(
            *args, initial_state=pool_ref, inplace_final_state=True, cu_seqlens=d["cu_seqlens"],
            ssm_state_indices=d["idx"], use_qk_l2norm_in_kernel=True)
        o, _ = hmx.fused_recurrent_gated_delta_rule_gqa(
            *[a.to(dev) for a in args], initial_state=pool_d, inplace_final_state=True,
            cu_seqlens=cu_d, ssm_state_indices=idx_d, use_qk_l2norm_in_kernel=True)
        torch.cuda.synchronize()
        assert_out_close(o, o_ref, what=f"o step {s}")
    assert_state_close(pool_d, pool_ref)


def test_decode_c2_all_512_steps_slice(dev):
    """C2 over its whole run: 512 consecutive in-place steps of the full 256-sequence
    x 32-head batch (randperm slots), with sequences 0-15 (all 32 heads, their 16
    random slots) checked at every step against the fp64 recurrence: every step's
    output and, at the end, their 16 slots; the other 240 slots against the GPU's own
    run are covered by the 3-step full-batch test above."""
    steps, ns = 512, 16
    d = wl.decode_inputs(n_seqs=256, H=32, HKV=32, D=128, steps=steps, device=dev,
                         gen_device=dev)
    pool_d = d["pool"]
    slots = d["idx"][:ns].long()
    pool_ref = pool_d[slots].double().cpu()          # the slice's slots, compact
    idx_ref = torch.arange(ns, dtype=torch.int32)
    cu_ref = torch.arange(ns + 1, dtype=torch.int32)
    for s in range(steps):
        args = [d[n][s] for n in ("q", "k", "v", "g", "beta")]
        o, _ = hmx.fused_recurrent_gated_delta_rule_gqa(
            *args, initial_state=pool_d, inplace_final_state=True, cu_seqlens=d["cu_seqlens"],
            ssm_state_indices=d["idx"], use_qk_l2norm_in_kernel=True)
        sl = [a[:, :ns].cpu() for a in args]
        o_ref, pool_ref = ref.fused_recurrent_gated_delta_rule_gqa(
            *sl, initial_state=pool_ref, inplace_final_state=True, cu_seqlens=cu_ref,
            ssm_state_indices=idx_ref, use_qk_l2norm_in_kernel=True)
        assert_out_close(o[:, :ns], o_ref, what=f"o step {s}")
    torch.cuda.synchronize()
    assert_state_close(pool_d[slots], pool_ref, what="the slice's slots after 512 steps")


def test_fla_style_fused_recurrent(dev):
    B, T, H, K, V = 2, 5, 2, 128, 128
    q, k, v, g, beta, gen = _mk(B * T, H, H, K, V, torch.bfloat16, 5)
    q, k, v = (x.view(B, T, H, -1) for x in (q, k, v))
    g, beta = g.view(B, T, H), beta.view(B, T, H)
    h0 = torch.randn(B, H, K, V, generator=gen) * 0.02
    o_ref, f_ref = ref.chunk_gated_delta_rule_gqa(q, k, v, g, beta, initial_state=h0,
                                                 output_final_state=True,
                                                 use_qk_l2norm_in_kernel=True, form="recurrent")
    o, f = hmx.fused_recurrent_gated_delta_rule(q.to(dev), k.to(dev), v.to(dev), g.to(dev),
                                                beta.to(dev), initial_state=h0.to(dev),
                                                output_final_state=True,
                                                use_qk_l2norm_in_kernel=True)
    torch.cuda.synchronize()
    assert_out_close(o, o_ref)
    assert_state_close(f, f_ref)


def test_gdn_gating(dev):
    g0 = torch.Generator().manual_seed(9)
    T, H = 37, 12
    ab = torch.randn(T, 3 * H, generator=g0).to(torch.bfloat16) * 8  # strided split, spans threshold
    a, b = ab[:, :H], ab[:, 2 * H:]
    A_log = torch.randn(H, generator=g0)
    dt_bias = torch.randn(H, generator=g0)
    g_ref, b_ref = ref.gdn_gating(A_log, a, b, dt_bias)
    ab_d = ab.to(dev)
    g, bo = hmx.fused_gdn_gating(A_log.to(dev), ab_d[:, :H], ab_d[:, 2 * H:], dt_bias.to(dev))
    torch.cuda.synchronize()
    assert g.shape == (1, T, H) and g.dtype == torch.bfloat16
    # outputs are rounded to bf16: compare at bf16 resolution
    assert torch.allclose(g.float().cpu(), g_ref.float(), rtol=8e-3, atol=1e-6)
    assert torch.allclose(bo.float().cpu(), b_ref.float(), rtol=8e-3, atol=1e-6)
    g32, b32 = hmx.fused_gdn_gating(A_log.to(dev), ab_d[:, :H].float(), ab_d[:, 2 * H:].float(),
                                    dt_bias.to(dev))
    assert torch.allclose(g32.cpu().double(), g_ref, rtol=1e-5, atol=1e-6)
    assert torch.allclose(b32.cpu().double(), b_ref, rtol=1e-5, atol=1e-6)
