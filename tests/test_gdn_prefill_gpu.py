"""GPU parity: hmx GDN chunked prefill vs the CPU oracle (fp64) and vs the GPU
recurrent kernel at the full C1 size.

Covers: single segment with h0, ragged tails, GQA, multi-segment warm-up start
states, the exact segment scan (weak decay, and use_qk_l2norm_in_kernel=False),
heads mixing both, varlen with empty and 1-token sequences, B > 1 without
cu_seqlens, bf16 g/beta, and C1 (T=32768, H=32, HKV 32 and 8) with the benchmark's
gates and with a freshly initialised layer's gates, plus the 8-sequence varlen C1
case.
"""
import pytest
import torch
import torch.nn.functional as F

import hmx
from hmx import workloads as wl
from oracle import gdn as ref
from util import assert_out_close, assert_state_close

pytestmark = pytest.mark.gpu


def _mk(B, T, H, HKV, seed, gscale=1.0, gshift=0.0, normalize=True):
    g0 = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, H, 128, generator=g0)
    k = torch.randn(B, T, HKV, 128, generator=g0)
    if normalize:
        q, k = F.normalize(q, dim=-1), F.normalize(k, dim=-1)
    v = torch.randn(B, T, HKV, 128, generator=g0)
    g = F.logsigmoid(torch.randn(B, T, H, generator=g0) * gscale + gshift)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=g0))
    return q.bfloat16(), k.bfloat16(), v.bfloat16(), g, beta, g0


def _run(dev, q, k, v, g, beta, h0=None, cu=None, l2=True, seg=None):
    args = [x.to(dev) for x in (q, k, v, g, beta)]
    o, s = hmx.chunk_gated_delta_rule_gqa(
        *args, initial_state=None if h0 is None else h0.to(dev), output_final_state=True,
        cu_seqlens=None if cu is None else cu.to(dev), use_qk_l2norm_in_kernel=l2,
        _segment_chunks=seg)
    torch.cuda.synchronize()
    return o, s


def _check(dev, q, k, v, g, beta, h0=None, cu=None, l2=True, seg=None):
    o_ref, s_ref = ref.chunk_gated_delta_rule_gqa(q, k, v, g, beta, initial_state=h0,
                                                 output_final_state=True, cu_seqlens=cu,
                                                 use_qk_l2norm_in_kernel=l2)
    o, s = _run(dev, q, k, v, g, beta, h0, cu, l2, seg)
    assert o.shape == o_ref.shape and o.dtype == torch.bfloat16
    assert_out_close(o, o_ref)
    assert_state_close(s, s_ref)
    return o, s


@pytest.mark.parametrize("T,H,HKV", [(64, 2, 2), (200, 4, 2), (37, 2, 1), (1, 2, 2)])
def test_prefill_single_segment(dev, T, H, HKV):
    q, k, v, g, beta, g0 = _mk(1, T, H, HKV, T + H)
    h0 = torch.randn(1, H, 128, 128, generator=g0) * 0.05
    _check(dev, q, k, v, g, beta, h0=h0)


def test_prefill_no_initial_state(dev):
    q, k, v, g, beta, _ = _mk(1, 150, 2, 2, 3)
    _check(dev, q, k, v, g, beta)


def test_prefill_multi_segment_warmup(dev):
    """Typical decay: every later segment starts from a warm-up (zero state)."""
    q, k, v, g, beta, g0 = _mk(1, 64 * 20 + 17, 4, 2, 4)
    h0 = torch.randn(1, 4, 128, 128, generator=g0) * 0.05
    _check(dev, q, k, v, g, beta, h0=h0, seg=3)


def test_prefill_multi_segment_exact_scan(dev):
    """Weak decay (g ~ -1e-3): the warm-up bound is not met -> exact segment scan."""
    q, k, v, g, beta, g0 = _mk(1, 64 * 9 + 5, 2, 2, 5, gscale=0.1, gshift=7.0)
    assert g.mean() > -2e-3
    h0 = torch.randn(1, 2, 128, 128, generator=g0) * 0.05
    _check(dev, q, k, v, g, beta, h0=h0, seg=2)


def test_prefill_mixed_heads(dev):
    """Head 0 decays strongly (warm-up), head 1 weakly (exact scan) in one call."""
    q, k, v, g, beta, g0 = _mk(1, 64 * 12, 2, 2, 6)
    g[..., 1] = F.logsigmoid(torch.randn(1, 64 * 12, generator=g0) * 0.1 + 8.0)
    _check(dev, q, k, v, g, beta, seg=4)


def test_prefill_without_l2norm_uses_exact_scan(dev):
    q, k, v, g, beta, _ = _mk(1, 64 * 8, 2, 2, 7)
    _check(dev, q, k, v, g, beta, l2=False, seg=2)


def test_prefill_varlen(dev):
    lens = [130, 0, 64, 500, 1, 77]
    cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0)), dtype=torch.int32)
    q, k, v, g, beta, g0 = _mk(1, int(cu[-1]), 4, 1, 8)
    h0 = torch.randn(len(lens), 4, 128, 128, generator=g0) * 0.05
    for seg in (None, 2):
        o, s = _check(dev, q, k, v, g, beta, h0=h0, cu=cu, seg=seg)
        assert torch.equal(s[1].cpu(), h0[1])  # empty sequence returns its initial state


def test_prefill_batched_no_cu(dev):
    q, k, v, g, beta, g0 = _mk(3, 100, 2, 2, 9)
    h0 = torch.randn(3, 2, 128, 128, generator=g0) * 0.05
    _check(dev, q, k, v, g, beta, h0=h0, seg=1)


def test_prefill_bf16_gates(dev):
    q, k, v, g, beta, _ = _mk(1, 96, 2, 2, 10)
    g, beta = g.bfloat16(), beta.bfloat16()
    o_ref, s_ref = ref.chunk_gated_delta_rule_gqa(q, k, v, g, beta, output_final_state=True,
                                                 use_qk_l2norm_in_kernel=True)
    o, s = _run(dev, q, k, v, g, beta)
    assert_out_close(o, o_ref)
    assert_state_close(s, s_ref)


def test_prefill_errors(dev):
    q, k, v, g, beta, _ = _mk(2, 8, 2, 2, 11)
    d = lambda *xs: [x.to(dev) for x in xs]
    with pytest.raises(AssertionError):
        hmx.chunk_gated_delta_rule_gqa(*d(q.float(), k.float(), v.float(), g, beta))
    with pytest.raises(ValueError, match="Batch size"):
        hmx.chunk_gated_delta_rule_gqa(*d(q, k, v, g, beta),
                                       cu_seqlens=torch.tensor([0, 8], device=dev))
    with pytest.raises(ValueError, match="Initial states count"):
        hmx.chunk_gated_delta_rule_gqa(*d(q[:1], k[:1], v[:1], g[:1], beta[:1]),
                                       initial_state=torch.zeros(2, 2, 128, 128, device=dev),
                                       cu_seqlens=torch.tensor([0, 8], device=dev))


@pytest.mark.parametrize("HKV", [32, 8])
def test_prefill_c1_full_size(dev, HKV):
    """C1: T=32768, H=32.  All heads vs the GPU recurrent kernel (chunked == recurrent);
    heads 0-3 vs the fp64 oracle."""
    T, H = 32768, 32
    d = wl.gdn_inputs(T=T, H=H, HKV=HKV, D=128, config_id=1)
    q, k, v, g, beta = (d[n] for n in ("q", "k", "v", "g", "beta"))
    o, s = _run(dev, q, k, v, g, beta)
    # recurrent kernel over the same sequence through a 1-slot pool
    pool = torch.zeros(1, H, 128, 128, device=dev)
    o_r, _ = hmx.fused_recurrent_gated_delta_rule_gqa(
        *[x.to(dev) for x in (q, k, v, g, beta)], initial_state=pool, inplace_final_state=True,
        cu_seqlens=torch.tensor([0, T], dtype=torch.int32, device=dev),
        ssm_state_indices=torch.zeros(1, dtype=torch.int32, device=dev),
        use_qk_l2norm_in_kernel=True)
    torch.cuda.synchronize()
    assert_out_close(o, o_r.float(), what="chunked vs recurrent o")
    assert_state_close(s, pool, what="chunked vs recurrent state")
    # fp64 oracle on the first 4 query heads (they read kv heads 0..4/(H/HKV))
    hs = 4
    nkv = max(1, hs // (H // HKV))
    o_ref, s_ref = ref.chunk_gated_delta_rule_gqa(
        q[:, :, :hs], k[:, :, :nkv], v[:, :, :nkv], g[:, :, :hs], beta[:, :, :hs],
        output_final_state=True, use_qk_l2norm_in_kernel=True)
    assert_out_close(o[:, :, :hs], o_ref)
    assert_state_close(s[:, :hs], s_ref)


def test_prefill_c1_layer_gates(dev):
    """C1 with the gates of a freshly initialised GDN layer (weak decay on several
    heads, so later segments of those heads take the exact segment scan).  All heads
    vs the GPU recurrent kernel; the fp64 oracle on two heads that run the exact scan
    and two that do not."""
    from hmx import _lib
    T, H = 32768, 32
    d = wl.gdn_inputs(T=T, H=H, HKV=H, D=128, config_id=1)
    q, k, v = d["q"], d["k"], d["v"]
    g, beta = wl.gdn_layer_gates(T, H)
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    table, _ = _lib.plan_segments(_lib.PLAN_GDN, [(0, T)], T, H, cus)
    pairs, exact = wl.gdn_exact_pairs(g, beta, table)
    print(f"{len(table)} segments, {pairs} exact (segment, head) pairs, "
          f"{int(exact.sum())} heads", flush=True)
    assert pairs > 0 and 0 < int(exact.sum()) < H
    o, s = _run(dev, q, k, v, g, beta)
    pool = torch.zeros(1, H, 128, 128, device=dev)
    o_r, _ = hmx.fused_recurrent_gated_delta_rule_gqa(
        *[x.to(dev) for x in (q, k, v, g, beta)], initial_state=pool, inplace_final_state=True,
        cu_seqlens=torch.tensor([0, T], dtype=torch.int32, device=dev),
        ssm_state_indices=torch.zeros(1, dtype=torch.int32, device=dev),
        use_qk_l2norm_in_kernel=True)
    torch.cuda.synchronize()
    assert_out_close(o, o_r.float(), what="chunked vs recurrent o")
    assert_state_close(s, pool, what="chunked vs recurrent state")
    idx = torch.cat([exact.nonzero()[:2, 0], (~exact).nonzero()[:2, 0]])
    o_ref, s_ref = ref.chunk_gated_delta_rule_gqa(
        *(x[:, :, idx] for x in (q, k, v, g, beta)), output_final_state=True,
        use_qk_l2norm_in_kernel=True)
    assert_out_close(o[:, :, idx.to(dev)], o_ref)
    assert_state_close(s[:, idx.to(dev)], s_ref)


def test_prefill_c1_varlen(dev):
    lens = wl.varlen_lengths()
    cu = wl.cu_from_lengths(lens)
    T = int(cu[-1])
    d = wl.gdn_inputs(T=T, H=8, HKV=8, D=128, config_id=1)
    _check(dev, *(d[n] for n in ("q", "k", "v", "g", "beta")), cu=cu)


def test_prefill_c1_varlen_h32(dev):
    """C1-varlen at its real head count (8 sequences of randint(1024, 8193) tokens,
    H = 32, zero initial states): the planner's H = 32 segment table.  All heads vs
    the GPU recurrent kernel per sequence (a pool slot each); heads 0-3 vs the fp64
    oracle, outputs and every sequence's final state."""
    from hmx import _lib
    from hmx.ops import gdn as gops
    lens = wl.varlen_lengths()
    cu = wl.cu_from_lengths(lens)
    T, H, N = int(cu[-1]), 32, len(lens)
    d = wl.gdn_inputs(T=T, H=H, HKV=H, D=128, config_id=1)
    q, k, v, g, beta = (d[n] for n in ("q", "k", "v", "g", "beta"))
    bounds = [(int(cu[i]), int(cu[i + 1])) for i in range(N)]
    rows, _ = gops._segment_table(_lib.PLAN_GDN, bounds, T, H, torch.device(dev))
    assert len(rows) > N, "the H = 32 plan is expected to split the sequences"
    h0 = torch.zeros(N, H, 128, 128)
    o, s = _run(dev, q, k, v, g, beta, h0=h0, cu=cu)
    pool = torch.zeros(N, H, 128, 128, device=dev)
    o_r, _ = hmx.fused_recurrent_gated_delta_rule_gqa(
        *[x.to(dev) for x in (q, k, v, g, beta)], initial_state=pool, inplace_final_state=True,
        cu_seqlens=cu.to(dev), ssm_state_indices=torch.arange(N, dtype=torch.int32, device=dev),
        use_qk_l2norm_in_kernel=True)
    torch.cuda.synchronize()
    assert_out_close(o, o_r.float(), what="varlen H=32 chunked vs recurrent o")
    assert_state_close(s, pool, what="varlen H=32 chunked vs recurrent states")
    hs = 4
    o_ref, s_ref = ref.chunk_gated_delta_rule_gqa(
        q[:, :, :hs], k[:, :, :hs], v[:, :, :hs], g[:, :, :hs], beta[:, :, :hs],
        initial_state=h0[:, :hs], output_final_state=True, cu_seqlens=cu,
        use_qk_l2norm_in_kernel=True)
    assert_out_close(o[:, :, :hs], o_ref, what="varlen H=32 o, heads 0-3 vs oracle")
    assert_state_close(s[:, :hs], s_ref, what="varlen H=32 final states, heads 0-3 vs oracle")


def test_c0_exact_shape(dev):
    """C0 at its exact shape (B=1, T=2048, H=16, d=128, fp32 inputs, zero initial
    state, in-kernel L2 norm): the fp32 inputs through the fp32 recurrent kernel and
    their bf16 casts through the chunked kernel, each against the oracle's chunked
    fp32 form on the same inputs (and the recurrent fp64 form for the first)."""
    d = wl.gdn_inputs(T=2048, H=16, HKV=16, D=128, dtype=torch.float32, config_id=0)
    q, k, v, g, beta = (d[n] for n in ("q", "k", "v", "g", "beta"))
    o32, s32 = hmx.chunk_gated_delta_rule(
        *[x.to(dev) for x in (q, k, v, g, beta)], output_final_state=True,
        use_qk_l2norm_in_kernel=True)
    torch.cuda.synchronize()
    o_ref, s_ref = ref.chunk_gated_delta_rule_gqa(q, k, v, g, beta, output_final_state=True,
                                                 use_qk_l2norm_in_kernel=True,
                                                 dtype=torch.float32)
    assert o32.dtype == torch.float32 and s32.shape == (1, 16, 128, 128)
    assert_out_close(o32, o_ref, what="C0 fp32 o (recurrent kernel)")
    assert_state_close(s32, s_ref, what="C0 fp32 state (recurrent kernel)")
    o_rr, s_rr = ref.fused_recurrent_gated_delta_rule_gqa(
        q, k, v, g, beta, initial_state=torch.zeros(1, 16, 128, 128),
        inplace_final_state=True, ssm_state_indices=torch.zeros(1, dtype=torch.int32),
        use_qk_l2norm_in_kernel=True)
    assert_state_close(s32, s_rr[0:1], rel_tol=1e-5, what="C0 fp32 state vs fp64 recurrence")
    qb, kb, vb = (x.bfloat16() for x in (q, k, v))
    ob, sb = _run(dev, qb, kb, vb, g, beta)
    o_ref_b, s_ref_b = ref.chunk_gated_delta_rule_gqa(qb, kb, vb, g, beta, output_final_state=True,
                                                     use_qk_l2norm_in_kernel=True,
                                                     dtype=torch.float32)
    assert_out_close(ob, o_ref_b, what="C0 bf16 o (chunked kernel)")
    assert_state_close(sb, s_ref_b, what="C0 bf16 state (chunked kernel)")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_fla_chunk_gated_delta_rule(dev, dtype):
    """The training layer's call (gdn.py:462-476): fla keyword arguments, k/v with H
    heads, B > 1 with initial_state and output_final_state, then the same tokens
    packed with cu_seqlens (B = 1)."""
    B, T, H = 3, 150, 2
    q, k, v, g, beta, g0 = _mk(B, T, H, H, 13, normalize=False)
    if dtype == torch.float32:
        q, k, v = (x.float() for x in (q, k, v))
    h0 = torch.randn(B, H, 128, 128, generator=g0) * 0.05
    d = lambda x: x.to(dev)
    o, s = hmx.chunk_gated_delta_rule(q=d(q), k=d(k), v=d(v), g=d(g), beta=d(beta),
                                      initial_state=d(h0), output_final_state=True,
                                      cu_seqlens=None, use_qk_l2norm_in_kernel=True)
    torch.cuda.synchronize()
    o_ref, s_ref = ref.chunk_gated_delta_rule_gqa(q, k, v, g, beta, initial_state=h0,
                                                 output_final_state=True,
                                                 use_qk_l2norm_in_kernel=True)
    assert o.dtype == dtype and s.dtype == torch.float32
    assert_out_close(o, o_ref)
    assert_state_close(s, s_ref)
    cu = torch.arange(0, (B + 1) * T, T, dtype=torch.int32)
    flat = lambda x: x.reshape(1, B * T, *x.shape[2:])
    o2, s2 = hmx.chunk_gated_delta_rule(q=d(flat(q)), k=d(flat(k)), v=d(flat(v)), g=d(flat(g)),
                                        beta=d(flat(beta)), initial_state=d(h0),
                                        output_final_state=True, cu_seqlens=d(cu),
                                        use_qk_l2norm_in_kernel=True)
    o3, s3 = hmx.chunk_gated_delta_rule(q=d(flat(q)), k=d(flat(k)), v=d(flat(v)), g=d(flat(g)),
                                        beta=d(flat(beta)), cu_seqlens=d(cu),
                                        use_qk_l2norm_in_kernel=True)
    torch.cuda.synchronize()
    assert_out_close(o2, o_ref.reshape(1, B * T, H, 128))
    assert_state_close(s2, s_ref)
    assert s3 is None and o3.shape == (1, B * T, H, 128)


@pytest.mark.parametrize("seg", [None, 2])
def test_prefill_rows_outside_fp16_range(dev, seg):
    """With the in-kernel L2 norm, k and q rows are normalised in fp32 before their
    fp16 rounding, so bf16 rows far outside fp16's range (|x| ~ 1e5) or tiny
    (~1e-6) stage safely.  Such rows and a zero key row, in the first chunk, a
    later chunk and a multi-segment split, against the fp64 oracle."""
    q, k, v, g, beta, g0 = _mk(1, 64 * 5 + 9, 4, 2, 31, normalize=False)
    q, k = q.float(), k.float()
    k[0, 3] *= 3e4          # first chunk: |k| elements past fp16's range
    k[0, 70, 1] *= 1e5
    q[0, 40] *= 4e4
    q[0, 200, 2] *= 1e-6    # a tiny query row
    k[0, 150, 0] *= 1e-6    # a tiny key row
    k[0, 260, 1] = 0.0      # a zero key row (stays on the fast path)
    q, k = q.bfloat16(), k.bfloat16()
    assert k.float().abs().max() > 65504 and q.float().abs().max() > 65504
    h0 = torch.randn(1, 4, 128, 128, generator=g0) * 0.05
    _check(dev, q, k, v, g, beta, h0=h0, seg=seg)


@pytest.mark.parametrize("case", ["uniform", "uniform_seg", "weak_decay_exact", "spike"])
def test_prefill_values_outside_fp16_range(dev, case):
    """bf16 values (and an initial state) far outside fp16's range: the walk scales
    its fp16 operands per wave by a power of two from a running bound on the state's
    column norms, so the result is the same computation at any magnitude.

    uniform*: v and h0 multiplied by 2^17 (|v| up to ~6e5) - the outputs and state
    divided by 2^17 (exact in bf16 / fp32) meet the ordinary tolerances; single
    walk, split into warm-up segments, and weak decay through the exact segment
    scan (where the state grows over the whole sequence).  spike: one chunk's values
    at 2^20 (~1e6) between ordinary chunks, so the scale drops and recovers within
    one walk; compared at the spike's magnitude."""
    gs = dict(gscale=0.1, gshift=7.0) if case == "weak_decay_exact" else {}
    q, k, v, g, beta, g0 = _mk(1, 64 * 5 + 9, 4, 2, 41, **gs)
    h0 = torch.randn(1, 4, 128, 128, generator=g0) * 0.05
    if case == "spike":
        a = 2.0 ** 20
        v = v.float()
        v[0, 96:128] *= a
        v = v.bfloat16()
    else:
        a = 2.0 ** 17
        v = (v.float() * a).bfloat16()
        h0 = h0 * a
    assert v.float().abs().max() > 65504 * 4
    seg = {"uniform": None, "spike": None}.get(case, 2)
    o_ref, s_ref = ref.chunk_gated_delta_rule_gqa(q, k, v, g, beta, initial_state=h0,
                                                 output_final_state=True,
                                                 use_qk_l2norm_in_kernel=True)
    o, s = _run(dev, q, k, v, g, beta, h0=h0, seg=seg)
    assert torch.isfinite(o.float()).all() and torch.isfinite(s).all()
    assert_out_close(o / a, o_ref / a)     # a is a power of two: the division is exact
    assert_state_close(s / a, s_ref / a)
