"""GPU parity: hmx GKA gating, decode step and chunked prefill vs the CPU oracle.

Decode covers slot-indexed pools, GQA, beta/gk present or absent, bf16 h_kv,
num_iter 1/8/30, zero-length entries and the num_iter=0 -> 1 rule.  Prefill
covers num_iter 0/8/32, initial states, multi-segment (exact scalar-decay
combine), varlen with empty sequences, no beta/gk, C3 (T=32768, H=32) at num_iter
8 and 32 on two whole heads against the fp64 recurrence (across the planner's
segment edges, and the final states), and prefill == T decode steps.
"""
import pytest
import torch
import torch.nn.functional as F

import hmx
from oracle import gka as ref
from util import assert_out_close, assert_state_close

pytestmark = pytest.mark.gpu


def _mk(n_tok, H, HKV, seed, B=1, bf16=True):
    g0 = torch.Generator().manual_seed(seed)
    dt = torch.bfloat16 if bf16 else torch.float32
    q = torch.randn(B, n_tok, H, 128, generator=g0).to(dt)
    k = torch.randn(B, n_tok, HKV, 128, generator=g0).to(dt)
    v = torch.randn(B, n_tok, HKV, 128, generator=g0).to(dt)
    alpha = torch.sigmoid(torch.randn(B, n_tok, H, generator=g0))
    g = F.logsigmoid(torch.randn(B, n_tok, H, generator=g0))
    gk = F.logsigmoid(torch.randn(B, n_tok, H, generator=g0))
    beta = torch.sigmoid(torch.randn(B, n_tok, H, generator=g0))
    return q, k, v, alpha, g, gk, beta, g0


def _psd_pool(slots, H, g0, scale=0.05):
    x = torch.randn(slots, H, 128, 16, generator=g0) * scale
    return x @ x.transpose(-1, -2)


@pytest.mark.parametrize("num_iter,use_beta,use_gk,kv_bf16", [
    (8, True, True, False), (30, True, True, False), (1, False, False, False), (8, True, True, True)])
def test_gka_decode(dev, num_iter, use_beta, use_gk, kv_bf16):
    N, H, HKV, slots = 6, 4, 2, 9
    q, k, v, alpha, g, gk, beta, g0 = _mk(N, H, HKV, 10 + num_iter)
    gk = gk if use_gk else None
    beta = beta if use_beta else None
    hkk = _psd_pool(slots, H, g0)
    hkv = torch.randn(slots, H, 128, 128, generator=g0) * 0.02
    if kv_bf16:
        hkv = hkv.bfloat16()
    idx = torch.randperm(slots, generator=g0)[:N].to(torch.int32)
    cu = torch.arange(N + 1, dtype=torch.int32)
    o_r, hkk_r, hkv_r = ref.gka_chebyshev_gla_decode(
        q, k, v, alpha, gk, gk, beta, 0.09, ridge_ratio=0.02, num_iter=num_iter,
        h_kk=hkk, h_kv=hkv, cu_seqlens=cu, ssm_state_indices=idx)
    d = lambda x: None if x is None else x.to(dev)
    hkk_d, hkv_d = hkk.to(dev), hkv.to(dev)
    gk_d = d(gk)
    o, a, b = hmx.gka_chebyshev_gla_decode(d(q), d(k), d(v), d(alpha), gk_d, gk_d, d(beta), 0.09,
                                           ridge_ratio=0.02, num_iter=num_iter, h_kk=hkk_d,
                                           h_kv=hkv_d, cu_seqlens=d(cu), ssm_state_indices=d(idx))
    torch.cuda.synchronize()
    assert a.data_ptr() == hkk_d.data_ptr() and b.data_ptr() == hkv_d.data_ptr()
    assert_out_close(o, o_r)
    assert_state_close(hkk_d, hkk_r, what="h_kk")
    assert_state_close(hkv_d, hkv_r, rel_tol=1e-2 if kv_bf16 else 1e-3, what="h_kv")


def test_gka_decode_zero_length_and_num_iter_zero(dev):
    H = 2
    q, k, v, alpha, g, gk, beta, g0 = _mk(3, H, H, 20)
    cu = torch.tensor([0, 2, 2, 3], dtype=torch.int32)  # seq 1 empty; seq 0 uses token 0 only
    hkk = _psd_pool(3, H, g0)
    hkv = torch.randn(3, H, 128, 128, generator=g0) * 0.02
    o_r, hkk_r, hkv_r = ref.gka_chebyshev_gla_decode(
        q, k, v, alpha, gk, gk, beta, 0.1, num_iter=0, h_kk=hkk, h_kv=hkv, cu_seqlens=cu)
    hkk_d, hkv_d = hkk.to(dev), hkv.to(dev)
    gk_d = gk.to(dev)
    o, _, _ = hmx.gka_chebyshev_gla_decode(q.to(dev), k.to(dev), v.to(dev), alpha.to(dev), gk_d,
                                           gk_d, beta.to(dev), 0.1, num_iter=0, h_kk=hkk_d,
                                           h_kv=hkv_d, cu_seqlens=cu.to(dev))
    torch.cuda.synchronize()
    assert_out_close(o[0, [0, 2]], o_r[0, [0, 2]])
    assert torch.equal(hkk_d[1].cpu(), hkk[1])  # empty sequence untouched
    assert_state_close(hkk_d, hkk_r)
    assert_state_close(hkv_d, hkv_r)


def test_gka_gating(dev):
    g0 = torch.Generator().manual_seed(21)
    T, H = 33, 6
    a = (torch.randn(T, 2 * H, generator=g0) * 10).bfloat16()[:, :H]
    ai = torch.randn(T, H, generator=g0).bfloat16()
    b = torch.randn(T, H, generator=g0).bfloat16()
    A_log, dtb = torch.randn(H, generator=g0), torch.randn(H, generator=g0)
    g_r, a_r, b_r = ref.gka_gating(A_log, a, ai, b, dtb)
    g, al, be = hmx.fused_gka_gating(A_log.to(dev), a.to(dev), ai.to(dev), b.to(dev), dtb.to(dev))
    g2, al2, be2 = hmx.fused_gka_gating(A_log.to(dev), a.to(dev), ai.to(dev), None, dtb.to(dev))
    torch.cuda.synchronize()
    assert be2 is None and g.dtype == torch.bfloat16
    for x, y in ((g, g_r), (al, a_r), (be, b_r), (g2, g_r), (al2, a_r)):
        assert torch.allclose(x.float().cpu(), y.float(), rtol=8e-3, atol=1e-6)


def _prefill_check(dev, q, k, v, alpha, g, gk, beta, num_iter, h0kk=None, h0kv=None, cu=None,
                   seg=None, ridge=0.01):
    o_r, hkk_r, hkv_r = ref.gka_chebyshev_gla_prefill(
        q, k, v, alpha, g, gk, beta, 128 ** -0.5, ridge_ratio=ridge, num_iter=num_iter,
        h_kk_initial=h0kk, h_kv_initial=h0kv, cu_seqlens=cu)
    d = lambda x: None if x is None else x.to(dev)
    o, hkk, hkv = hmx.gka_chebyshev_gla_prefill(
        d(q), d(k), d(v), d(alpha), d(g), d(gk), d(beta), 128 ** -0.5, ridge_ratio=ridge,
        num_iter=num_iter, h_kk_initial=d(h0kk), h_kv_initial=d(h0kv), cu_seqlens=d(cu),
        _segment_chunks=seg)
    torch.cuda.synchronize()
    assert o.shape == o_r.shape
    assert_out_close(o, o_r)
    assert_state_close(hkv, hkv_r, what="h_kv")
    if num_iter > 0:
        assert_state_close(hkk, hkk_r, what="h_kk")
    else:
        assert hkk is None
    return o, hkk, hkv


@pytest.mark.parametrize("T,num_iter", [(40, 8), (100, 0), (70, 32), (1, 8)])
def test_gka_prefill_single_segment(dev, T, num_iter):
    q, k, v, alpha, g, gk, beta, g0 = _mk(T, 4, 2, 30 + T)
    h0kk = _psd_pool(1, 4, g0)
    h0kv = torch.randn(1, 4, 128, 128, generator=g0) * 0.02
    _prefill_check(dev, q, k, v, alpha, g, gk, beta, num_iter, h0kk, h0kv)


def test_gka_prefill_multi_segment_and_no_gates(dev):
    q, k, v, alpha, g, gk, beta, g0 = _mk(32 * 7 + 9, 2, 2, 40)
    g = F.logsigmoid(torch.randn(1, 32 * 7 + 9, 2, generator=g0) * 0.1 + 5)  # long memory
    # ~150 tokens of memory sum into h_kv: scale v so |o| stays O(1), where a bf16
    # output can meet the absolute bound (unscaled, |o| reaches 64 and rounding the
    # exact answer to bf16 alone moves it by 0.12).
    v = (v.float() * 0.05).to(v.dtype)
    h0kk = _psd_pool(1, 2, g0)
    h0kv = torch.randn(1, 2, 128, 128, generator=g0) * 0.02
    _prefill_check(dev, q, k, v, alpha, g, gk, beta, 8, h0kk, h0kv, seg=2)
    _prefill_check(dev, q, k, v, alpha, g, None, None, 8, h0kk, h0kv, seg=3)


def test_gka_prefill_varlen(dev):
    lens = [50, 0, 33, 100, 1]
    cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0)), dtype=torch.int32)
    q, k, v, alpha, g, gk, beta, g0 = _mk(int(cu[-1]), 2, 1, 41)
    h0kk = _psd_pool(len(lens), 2, g0)
    h0kv = torch.randn(len(lens), 2, 128, 128, generator=g0) * 0.02
    for seg in (None, 1):
        _, hkk, hkv = _prefill_check(dev, q, k, v, alpha, g, gk, beta, 8, h0kk, h0kv, cu=cu, seg=seg)
        assert torch.equal(hkv[1].cpu(), h0kv[1])


_C3_CACHE = {}


def _c3_inputs():
    if "d" not in _C3_CACHE:
        from hmx import workloads as wl
        _C3_CACHE["d"] = wl.gka_inputs(T=32768, H=32, HKV=32, D=128, config_id=3)
    return _C3_CACHE["d"]


@pytest.mark.parametrize("num_iter", [8, 32])
def test_gka_prefill_c3_full_size(dev, num_iter):
    """C3 (T=32768, H=32, bf16, ridge 0.01) at num_iter 8 and 32: two heads over the
    whole sequence vs the fp64 per-token recurrence (its block-batched form), with
    the output window around the first segment boundary the planner cuts, the whole
    output of both heads and their final h_kk / h_kv."""
    from hmx import _lib
    from hmx.ops import gdn as gops
    from hmx.ops.gka import GKA_BLOCK
    d = _c3_inputs()
    T, H = 32768, 32
    args = [d[n] for n in ("q", "k", "v", "alpha", "g", "gk", "beta")]
    o, hkk, hkv = hmx.gka_chebyshev_gla_prefill(*[a.to(dev) for a in args], 128 ** -0.5,
                                                ridge_ratio=0.01, num_iter=num_iter)
    torch.cuda.synchronize()
    rows, _ = gops._segment_table(_lib.PLAN_GKA, [(0, T)], T, H, dev)
    assert len(rows) > 1, "C3 is expected to run as several segments per head"
    edge = rows[1][3] * GKA_BLOCK           # first token of the second segment
    hs = [0, 17]
    sub = [a[0][:, hs] for a in args]
    o_r, hkk_r, hkv_r = ref.gka_seq_blocked(*sub, 128 ** -0.5, 0.01, num_iter)
    o_h = o[0][:, hs]
    win = slice(edge - 256, edge + 256)
    assert_out_close(o_h[win], o_r[win], what=f"o around the segment edge at {edge}")
    assert_out_close(o_h, o_r, what="o, whole sequence")
    assert_state_close(hkk[0, hs], hkk_r, what="h_kk final")
    assert_state_close(hkv[0, hs], hkv_r, what="h_kv final")
    assert torch.isfinite(o.float()).all()


def test_gka_prefill_equals_decode_steps(dev):
    """A prefill over T tokens equals T single-token decode steps through a pool slot
    (decode decays both states by gk, so g = gk here): outputs token by token and
    the final h_kk / h_kv."""
    T, H, HKV = 150, 2, 1
    q, k, v, alpha, _, gk, beta, g0 = _mk(T, H, HKV, 42)
    h0kk = _psd_pool(1, H, g0)
    h0kv = torch.randn(1, H, 128, 128, generator=g0) * 0.02
    d = lambda x: x.to(dev)
    o_p, hkk_p, hkv_p = hmx.gka_chebyshev_gla_prefill(
        d(q), d(k), d(v), d(alpha), d(gk), d(gk), d(beta), 0.09, ridge_ratio=0.02, num_iter=8,
        h_kk_initial=d(h0kk), h_kv_initial=d(h0kv), _segment_chunks=2)
    pool_kk = torch.zeros(3, H, 128, 128, device=dev)
    pool_kv = torch.zeros(3, H, 128, 128, device=dev)
    pool_kk[1], pool_kv[1] = d(h0kk[0]), d(h0kv[0])
    idx = torch.tensor([1], dtype=torch.int32, device=dev)
    cu = torch.tensor([0, 1], dtype=torch.int32, device=dev)
    o_d = torch.empty_like(o_p)
    for t in range(T):
        sl = slice(t, t + 1)
        gt = d(gk[:, sl])
        o_t, _, _ = hmx.gka_chebyshev_gla_decode(
            d(q[:, sl]), d(k[:, sl]), d(v[:, sl]), d(alpha[:, sl]), gt, gt, d(beta[:, sl]), 0.09,
            ridge_ratio=0.02, num_iter=8, h_kk=pool_kk, h_kv=pool_kv, cu_seqlens=cu,
            ssm_state_indices=idx)
        o_d[:, sl] = o_t
    torch.cuda.synchronize()
    assert_out_close(o_p, o_d.float(), what="prefill vs decode o")
    assert_state_close(hkk_p[0], pool_kk[1], what="prefill vs decode h_kk")
    assert_state_close(hkv_p[0], pool_kv[1], what="prefill vs decode h_kv")


def _layer_prepared(B, T, H, seed):
    """Inputs as the training layer hands them over (gka.py:477-490): q, k divided by
    (|x| + 1e-6), (beta + 1e-6) applied to k and v, all cast back to bf16."""
    g0 = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, H, 128, generator=g0)
    k = torch.randn(B, T, H, 128, generator=g0)
    v = torch.randn(B, T, H, 128, generator=g0)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=g0))
    q = (q / (q.norm(dim=-1, keepdim=True) + 1e-6)).bfloat16()
    k = (k / (k.norm(dim=-1, keepdim=True) + 1e-6) * (beta[..., None] + 1e-6)).bfloat16()
    v = (v * (beta[..., None] + 1e-6)).bfloat16()
    alpha = torch.sigmoid(torch.randn(B, T, H, generator=g0))
    g = F.logsigmoid(torch.randn(B, T, H, generator=g0))
    gk = F.logsigmoid(torch.randn(B, T, H, generator=g0) + 1.0)
    return q, k, v, alpha, g, gk


@pytest.mark.parametrize("num_iter", [8, 0])
def test_gka_training_form(dev, num_iter):
    q, k, v, alpha, g, gk = _layer_prepared(2, 70, 2, 50 + num_iter)
    o_r, hk_r, hv_r = ref.gka_chebyshev_gla(q, k, v, alpha, g, gk, 128 ** -0.5,
                                           ridge_strength=0.02, num_iter=num_iter)
    d = [x.to(dev) for x in (q, k, v, alpha, g, gk)]
    o, hk, hv = hmx.gka_chebyshev_gla(*d, 128 ** -0.5, ridge_strength=0.02, num_iter=num_iter)
    torch.cuda.synchronize()
    assert_out_close(o, o_r)
    assert_state_close(hv, hv_r, what="kv_final")
    if num_iter:
        assert_state_close(hk, hk_r, what="kk_final")
    else:
        assert hk is None


def test_gka_training_decode_steps(dev):
    q, k, v, alpha, g, gk = _layer_prepared(3, 6, 2, 60)
    g0 = torch.Generator().manual_seed(61)
    hk0 = _psd_pool(3, 2, g0)
    hv0 = torch.randn(3, 2, 128, 128, generator=g0) * 0.02
    hk_r, hv_r, hk, hv = hk0, hv0, hk0.to(dev), hv0.to(dev)
    for t in range(q.shape[1]):
        sl = slice(t, t + 1)
        o_r, hk_r, hv_r = ref.torch_decoding_one_step(q[:, sl], k[:, sl], v[:, sl], alpha[:, sl],
                                                      g[:, sl], gk[:, sl], 0.1, 0.02, 8, hk_r, hv_r)
        o, hk, hv = hmx.torch_decoding_one_step(*(x[:, sl].to(dev) for x in (q, k, v, alpha, g, gk)),
                                                0.1, 0.02, "chebyshev", 8, hk, hv)
        torch.cuda.synchronize()
        assert o.shape == (3, 1, 2, 128)
        assert_out_close(o, o_r)
    assert_state_close(hk, hk_r, what="h_kk")
    assert_state_close(hv, hv_r, what="h_kv")
    # unbatched [1, H, D] inputs and no h_kk (num_iter = 0)
    o, hk1, hv1 = hmx.torch_decoding_one_step(*(x[0, 0:1].to(dev) for x in (q, k, v, alpha, g, gk)),
                                              0.1, 0.02, "chebyshev", 0, None, None)
    torch.cuda.synchronize()
    assert hk1 is None and o.shape == (1, 1, 2, 128)
