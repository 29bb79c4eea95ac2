"""Benchmark of the linear-recurrent mixer hot path on one MI355X.

Headline (``value``): GDN chunked prefill at BASELINE config C1 — B=1, T=32768,
H=32, d=128 (the kernel walks 32-token chunks), bf16 q/k/v, fp32 g/beta, zero initial state, fp32 final
state — in tokens/s; one "step" is one call of chunk_gated_delta_rule_gqa over
the whole sequence with inputs resident in HBM.  Also reported: GDN decode at
C2 (256 sequences x 1 token, H=32, fp32 state pool of 512 MiB through a random
slot permutation, 512 consecutive steps) in steps/s, each with its roofline,
and the CPU oracle timed on a bounded sample of the same workloads.

GKA prefill at C3 (the C1 shape, Chebyshev solve at 8 and 32 iterations) is
reported under ``gka`` against the bf16 MFMA roofline; the Mamba2 SSD chunk scan
at C4 under ``ssd`` and its single-token state update under ``ssd_decode``, both
against HBM.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--only LEGS]
  --only takes comma-separated legs (c1, prefill_gqa, prefill_varlen,
  prefill_layer_gates, onorm, conv, gdn_core, gdn_decode_core, mamba2_core, gka_core,
  gdn_decode, gka_decode, ssd_c4, ssd_primed, ssd_decode, gka8, gka32, gka_train,
  gdn_train, ssd_train) or groups (prefill, core, decode, ssd, gka, train); one leg
  alone is what the committed rocprofv3 counter runs profile.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
for _p in (REPO, REPO / "hybrid-model-factory_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

HBM_PEAK_GBS = 8000.0       # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0   # MI355X dense bf16 MFMA


def _steady_state(fn, seconds=0.3, min_calls=3):
    """Untimed: run the leg's own step back to back for about ``seconds`` so the
    chip settles into the clock and power state of that op before the timed
    steps.  Without it the first calls run at the idle state's clocks (after
    input generation the C1 prefill's first 20 calls took 474 us against 381 us
    later); a warm-up on another workload (dense GEMMs) leaves the power state of
    that workload instead, which measured 25% slower for the prefill than its own
    steady state."""
    import torch
    t0 = time.perf_counter()
    n = 0
    while n < min_calls or time.perf_counter() - t0 < seconds:
        fn()
        n += 1
        if n % 8 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()


def _timed(fn, steps, warmup, stream=None):
    import torch
    _steady_state(fn)
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(steps):
        fn()
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps  # ms per step


def bench_prefill(dev, steps, warmup, HKV=32):
    import torch
    import hmx
    from hmx import workloads as wl
    T, H, D = 32768, 32, 128
    d = wl.gdn_inputs(T=T, H=H, HKV=HKV, D=D, config_id=1, device=dev, gen_device=dev)
    args = [d[n] for n in ("q", "k", "v", "g", "beta")]

    def step():
        hmx.chunk_gated_delta_rule_gqa(*args, output_final_state=True,
                                       use_qk_l2norm_in_kernel=True)

    ms = _timed(step, steps, warmup)
    by = wl.gdn_prefill_bytes(T, H, HKV)
    fl = wl.gdn_prefill_flops(T, H)
    fl32 = wl.gdn_prefill_flops(T, H, C=32)     # the same count at the kernel's 32-token chunk
    gbs = by / (ms * 1e-3) / 1e9
    tfs = fl / (ms * 1e-3) / 1e12
    return dict(ms=ms, tokens_per_s=T / (ms * 1e-3), bytes=by, flops=fl, GBps=gbs, TFLOPs=tfs,
                flops_c32=fl32, TFLOPs_c32=fl32 / (ms * 1e-3) / 1e12)


def bench_prefill_layer_gates(dev, steps, warmup):
    """C1 with the gates a GDN layer forms at initialisation (A_log ~ log U(1,16),
    dt_bias from dt ~ logU(1e-3, 1e-1), fused_gdn_gating of N(0,1) projections):
    weak decay on some heads sends their later segments through the exact segment
    scan.  Reports how many (segment, head) pairs take it."""
    import hmx
    from hmx import _lib, workloads as wl
    T, H, D = 32768, 32, 128
    d = wl.gdn_inputs(T=T, H=H, HKV=H, D=D, config_id=1, device=dev, gen_device=dev)
    g, beta = wl.gdn_layer_gates(T, H, device=dev, gen_device=dev)
    args = [d["q"], d["k"], d["v"], g, beta]

    def step():
        hmx.chunk_gated_delta_rule_gqa(*args, output_final_state=True,
                                       use_qk_l2norm_in_kernel=True)

    ms = _timed(step, steps, warmup)
    import torch
    table, _ = _lib.plan_segments(_lib.PLAN_GDN, [(0, T)], T, H,
                                  torch.cuda.get_device_properties(dev).multi_processor_count)
    pairs, heads = wl.gdn_exact_pairs(g, beta, table)
    by = wl.gdn_prefill_bytes(T, H, H)
    return dict(ms=ms, tokens_per_s=T / (ms * 1e-3), bytes=by, GBps=by / (ms * 1e-3) / 1e9,
                segments=len(table), exact_pairs=pairs, exact_heads=int(heads.sum()))


def bench_prefill_varlen(dev, steps, warmup):
    """C1 varlen: 8 sequences with randint(1024, 8193) tokens (the config generator's
    first draw), zero fp32 initial states, final states out."""
    import torch
    import hmx
    from hmx import workloads as wl
    H, D = 32, 128
    lens = wl.varlen_lengths()
    cu = wl.cu_from_lengths(lens).to(dev)
    T = int(lens.sum())
    d = wl.gdn_inputs(T=T, H=H, HKV=H, D=D, config_id=1, device=dev, gen_device=dev)
    args = [d[n] for n in ("q", "k", "v", "g", "beta")]
    h0 = torch.zeros(len(lens), H, D, D, device=dev)

    def step():
        hmx.chunk_gated_delta_rule_gqa(*args, initial_state=h0, output_final_state=True,
                                       cu_seqlens=cu, use_qk_l2norm_in_kernel=True)

    ms = _timed(step, steps, warmup)
    by = wl.gdn_prefill_bytes(T, H, H, n_seqs=len(lens))
    return dict(ms=ms, tokens=T, lengths=[int(x) for x in lens], tokens_per_s=T / (ms * 1e-3),
                bytes=by, GBps=by / (ms * 1e-3) / 1e9)


def bench_onorm(dev, steps, warmup):
    """The layer's output norm o_norm(o, z) at C1: the standalone gated RMSNorm kernel,
    prefill + norm as two ops, and the prefill with the norm fused into its epilogue."""
    import torch
    import hmx
    from hmx import workloads as wl
    T, H, D = 32768, 32, 128
    d = wl.gdn_inputs(T=T, H=H, HKV=H, D=D, config_id=1, device=dev, gen_device=dev)
    args = [d[n] for n in ("q", "k", "v", "g", "beta")]
    g = torch.Generator(device=dev).manual_seed(wl.SEED_BASE + 6)
    z = torch.randn(1, T, H, D, generator=g, device=dev).bfloat16()
    w = torch.rand(D, generator=g, device=dev) + 0.5
    o, _ = hmx.chunk_gated_delta_rule_gqa(*args, use_qk_l2norm_in_kernel=True)
    ms_norm = _timed(lambda: hmx.rms_norm_gated(o, z, w), steps, warmup)

    def unfused():
        oo, _ = hmx.chunk_gated_delta_rule_gqa(*args, output_final_state=True,
                                               use_qk_l2norm_in_kernel=True)
        hmx.rms_norm_gated(oo, z, w)

    def fused():
        hmx.chunk_gated_delta_rule_gqa(*args, output_final_state=True, use_qk_l2norm_in_kernel=True,
                                       o_norm_weight=w, o_norm_gate=z)

    ms_unf = _timed(unfused, steps, warmup)
    ms_fus = _timed(fused, steps, warmup)
    norm_bytes = 3 * T * H * D * 2   # o, z read; out written (bf16)
    return dict(ms_norm=ms_norm, ms_unfused=ms_unf, ms_fused=ms_fus, norm_bytes=norm_bytes,
                norm_GBps=norm_bytes / (ms_norm * 1e-3) / 1e9)


def bench_conv(dev, steps, warmup):
    """The GDN layer's input conv at the C1 shape: causal_conv1d_fn over q|k|v
    (dim 3*32*128 = 12288, width 4, silu) for 8 sequences x 4096 tokens with a
    state pool, and causal_conv1d_update for 256 sequences x 1 token."""
    import torch
    import hmx
    from hmx import workloads as wl
    T, dim, W, nseq, st_len = 32768, 3 * 32 * 128, 4, 8, 3
    g = torch.Generator(device=dev).manual_seed(wl.SEED_BASE + 7)
    x = torch.randn(T, dim, generator=g, device=dev).bfloat16()
    w = torch.randn(dim, W, generator=g, device=dev) * 0.5
    b = torch.randn(dim, generator=g, device=dev) * 0.1
    pool = torch.randn(nseq, st_len, dim, generator=g, device=dev).bfloat16()
    qs = torch.arange(0, T + 1, T // nseq, dtype=torch.int32, device=dev)
    init = torch.ones(nseq, dtype=torch.bool, device=dev)
    pool = pool.transpose(1, 2)        # the layers pass the [slots, dim, state_len] view
    ms_fwd = _timed(lambda: hmx.causal_conv1d_fn(x.t(), w, b, conv_states=pool, query_start_loc=qs,
                                                 has_initial_state=init), steps, warmup)
    fwd_bytes = 2 * T * dim * 2 + 2 * nseq * st_len * dim * 2   # x read, out written; states
    N = 256
    xd = torch.randn(N, dim, generator=g, device=dev).bfloat16()
    dpool = torch.randn(N, st_len, dim, generator=g, device=dev).bfloat16().transpose(1, 2)
    idx = torch.randperm(N, device=dev, generator=g).to(torch.int32)
    ms_dec = _timed(lambda: hmx.causal_conv1d_update(xd, dpool, w, b, "silu",
                                                     conv_state_indices=idx), 200, 10)
    dec_bytes = N * dim * 2 * (2 + 2 * st_len)                  # x, out; state read + written
    return dict(ms_fwd=ms_fwd, fwd_bytes=fwd_bytes, fwd_GBps=fwd_bytes / (ms_fwd * 1e-3) / 1e9,
                ms_dec=ms_dec, dec_bytes=dec_bytes, dec_GBps=dec_bytes / (ms_dec * 1e-3) / 1e9)


def bench_mamba2_core(dev, steps, warmup):
    """The primed Mamba2 layer's conv_ssm_forward on a prefill batch (8 sequences x
    4096 tokens; 32 heads, head_dim = d_state = 128, d_xb = 1024, conv width 4 with
    bias, fp32 state pool of 8 slots, B/C RMSNorm): the reference layer's call
    sequence over hmx ops (primed_mamba2_layer.py:663-669 norms, :775-790 conv,
    :800-835 rearrange + repeat_kv copies, :812-824 gather, :844-863 scan, :941
    scatter) against hmx.serving.mamba2_conv_ssm_forward."""
    from types import SimpleNamespace
    import torch
    import hmx
    import hmx.serving as srv
    T, H, P, nseq, W = 32768, 32, 128, 8, 4
    N, XB = P, 1024
    I, HX = H * P, XB // P
    CD = I + 2 * XB
    dproj = 2 * I + 2 * XB + H
    g = torch.Generator(device=dev).manual_seed(7)
    rnd = lambda *s, sc=1.0: torch.randn(*s, generator=g, device=dev) * sc

    class Norm:
        """Stand-in for the layer's fused vLLM RMSNorm modules: one pass."""
        def __init__(self):
            self.weight = (torch.rand(P, generator=g, device=dev) + 0.5).bfloat16()

        def __call__(self, x):
            return hmx.rms_norm_gated(x, None, self.weight, 1e-6)

    lay = SimpleNamespace(
        tp_size=1, tped_intermediate_size=I, tped_conv_size=CD, dt_pad=0, num_heads=H,
        xb_size=XB, ssm_state_size=N, head_dim=P, n_groups=H, chunk_size=256,
        conv_weights=rnd(CD, W, sc=0.4).bfloat16(), conv1d=SimpleNamespace(bias=rnd(CD, sc=0.1).bfloat16()),
        activation="silu", A=-torch.exp(torch.rand(H, generator=g, device=dev) * 2), D=rnd(H),
        dt_bias=rnd(H, sc=0.5), B_norm=Norm(), C_norm=Norm(), use_pos_embed=False,
        cache_config=SimpleNamespace(mamba_cache_mode="none"))
    proj = rnd(T, dproj).bfloat16()
    proj[:, I + CD:] = proj[:, I + CD:] * 0.5 - 1.5
    conv_cache = rnd(nseq, W - 1, CD).bfloat16()
    pool = rnd(nseq, H, P, N, sc=0.05)
    idx = torch.randperm(nseq, generator=g, device=dev).to(torch.int32)
    has = torch.ones(nseq, dtype=torch.bool, device=dev)
    qsl = torch.arange(0, T + 1, T // nseq, dtype=torch.int32, device=dev)
    md = SimpleNamespace(num_prefills=nseq, num_decode_tokens=0, num_prefill_tokens=T,
                         state_indices_tensor=idx, has_initial_states_p=has,
                         prep_initial_states=True, query_start_loc_p=qsl)
    output = torch.empty(T, I, dtype=torch.bfloat16, device=dev)
    cs = conv_cache.transpose(1, 2)

    def reference_sequence():
        hbc = proj[:, I:I + CD]
        hs, B, C = torch.split(hbc, [XB, XB, I], dim=-1)
        B = lay.B_norm(B.reshape(-1, P)).view(B.shape)
        C = lay.C_norm(C.reshape(-1, P)).view(C.shape)
        hbc = torch.cat([hs, B, C], dim=-1)
        x = hmx.causal_conv1d_fn(hbc.t(), lay.conv_weights, lay.conv1d.bias, conv_states=cs,
                                 has_initial_state=has, cache_indices=idx,
                                 query_start_loc=qsl).t()
        hs, B, C = torch.split(x, [XB, XB, I], dim=-1)
        rep = lambda t: (t.reshape(T, HX, P).permute(1, 0, 2)[:, None]
                         .expand(HX, H // HX, T, P).reshape(H, T, P))        # repeat_kv
        hs, B = rep(hs).permute(1, 0, 2), rep(B).permute(1, 0, 2)
        init = torch.where(has[:, None, None, None], pool[idx.long()], 0)
        st = hmx.mamba_chunk_scan_combined_varlen(
            hs, proj[:, I + CD:], lay.A, B, C.reshape(T, H, N), 256, cu_seqlens=qsl,
            out=output.view(T, H, P), D=lay.D, dt_bias=lay.dt_bias, initial_states=init,
            dt_softplus=True)
        pool[idx.long()] = st

    def hmx_core():
        srv.mamba2_conv_ssm_forward(lay, proj, output, md, cs, pool)

    ms_ref = _timed(reference_sequence, steps, warmup)
    ms_core = _timed(hmx_core, steps, warmup)
    return dict(ms_ref=ms_ref, ms_core=ms_core, tokens=T)


def bench_gka_core(dev, steps, warmup):
    """The GKA layer's core on the same prefill batch (8 sequences x 4096 tokens,
    H = HKV = 32, d = 128, num_iter 8): the reference call sequence over hmx ops
    (primed_gka_layer.py:1060-1300 then o_norm: conv to a new tensor, contiguous
    q/k/v, gating, gather and zeroing of both pools, prefill, scatter of both,
    copy into core_attn_out, separate norm) against hmx.serving.gka_forward_core
    with the norm fused."""
    from types import SimpleNamespace
    import torch
    import hmx
    import hmx.serving as srv
    from hmx import workloads as wl
    T, H, D, nseq = 32768, 32, 128, 8
    cd = 3 * H * D
    g = torch.Generator(device=dev).manual_seed(wl.SEED_BASE + 9)
    lay = SimpleNamespace(
        conv1d=SimpleNamespace(weight=(torch.randn(cd, 1, 4, generator=g, device=dev) * 0.4)
                               .bfloat16()),
        activation="silu", A=torch.rand(H, generator=g, device=dev),
        dt_bias=torch.randn(H, generator=g, device=dev), key_dim=H * D, kv_k_dim=H * D,
        kv_v_dim=H * D, num_heads=H, num_kv_heads=H, head_k_dim=D, head_v_dim=D, tp_size=1,
        proj_k=None, use_forgetting_gate=True, use_forgetting_gate_kk=True, use_beta_gate=True,
        num_iter=8, ridge_strength=0.02, gla_scale=D ** -0.5, _alpha_idx=None)
    mixed = torch.randn(T, cd, generator=g, device=dev).bfloat16()
    a, alpha_in, b = (torch.randn(T, H, generator=g, device=dev).bfloat16() for _ in range(3))
    z = torch.randn(T, H, D, generator=g, device=dev).bfloat16()
    wn = torch.rand(D, generator=g, device=dev) + 0.5
    conv_cache = torch.randn(nseq, 3, cd, generator=g, device=dev).bfloat16()
    x16 = torch.randn(nseq, H, D, 16, generator=g, device=dev) * 0.05
    hkk = x16 @ x16.transpose(-1, -2)
    hkv = torch.randn(nseq, H, D, D, generator=g, device=dev) * 0.02
    qs = torch.arange(0, T + 1, T // nseq, dtype=torch.int32, device=dev)
    idx = torch.randperm(nseq, generator=g, device=dev).to(torch.int32)
    has = torch.ones(nseq, dtype=torch.bool, device=dev)
    md = SimpleNamespace(spec_sequence_masks=None, num_actual_tokens=T, num_decodes=0,
                         num_decode_tokens=0, num_prefills=nseq, non_spec_query_start_loc=qs,
                         non_spec_state_indices_tensor=idx, has_initial_state=has,
                         non_spec_query_start_loc_d=None, non_spec_query_start_loc_p=None)
    core = torch.zeros(T, H, D, dtype=torch.bfloat16, device=dev)
    cs = conv_cache.transpose(1, 2)
    w2 = lay.conv1d.weight.view(cd, 4)

    def reference_sequence():
        x = hmx.causal_conv1d_fn(mixed.t(), w2, None, conv_states=cs, query_start_loc=qs,
                                 cache_indices=idx, has_initial_state=has).t()
        q = x[:, :H * D].reshape(1, T, H, D).contiguous()
        k = x[:, H * D:2 * H * D].reshape(1, T, H, D).contiguous()
        v = x[:, 2 * H * D:].reshape(1, T, H, D).contiguous()
        gg, alpha, beta = hmx.fused_gka_gating(lay.A, a, alpha_in, b, lay.dt_bias)
        alpha = alpha + 0.5
        il = idx.long()
        kk0, kv0 = hkk[il].contiguous(), hkv[il].contiguous()
        kk0[~has] = 0
        kv0[~has] = 0
        o, kkf, kvf = hmx.gka_chebyshev_gla_prefill(
            q, k, v, alpha, gg, gg, beta, lay.gla_scale, ridge_ratio=lay.ridge_strength,
            num_iter=lay.num_iter, h_kk_initial=kk0, h_kv_initial=kv0,
            output_final_state=True, cu_seqlens=qs)
        hkk[il] = kkf
        hkv[il] = kvf
        core[:T] = o.squeeze(0)
        return hmx.rms_norm_gated(core, z, wn, 1e-6)

    def hmx_core():
        srv.gka_forward_core(lay, mixed, a, alpha_in, b, core, md, cs, hkk, hkv,
                             o_norm=(wn, z, 1e-6))

    ms_ref = _timed(reference_sequence, steps, warmup)
    ms_core = _timed(hmx_core, steps, warmup)
    return dict(ms_ref=ms_ref, ms_core=ms_core, tokens=T)


def bench_core(dev, steps, warmup):
    """The GDN layer's core at the C1 shape (8 sequences x 4096 tokens, H = HKV = 32,
    d = 128, conv width 4, state pools of 8 slots): the reference layer's call
    sequence over hmx ops (primed_gdn_layer.py:747-936 then o_norm, :621-626: conv
    to a new tensor, contiguous q/k/v, gating, state gather and zeroing, prefill,
    scatter, copy into core_attn_out, separate norm) against
    hmx.serving.gdn_forward_core with the norm fused."""
    from types import SimpleNamespace
    import torch
    import hmx
    import hmx.serving as srv
    from hmx import workloads as wl
    T, H, D, nseq = 32768, 32, 128, 8
    cd = 3 * H * D
    g = torch.Generator(device=dev).manual_seed(wl.SEED_BASE + 8)
    lay = SimpleNamespace(
        conv1d=SimpleNamespace(weight=(torch.randn(cd, 1, 4, generator=g, device=dev) * 0.4)
                               .bfloat16()),
        activation="silu", A=torch.rand(H, generator=g, device=dev),
        dt_bias=torch.randn(H, generator=g, device=dev), key_dim=H * D, kv_k_dim=H * D,
        kv_v_dim=H * D, num_heads=H, num_kv_heads=H, head_k_dim=D, head_v_dim=D, tp_size=1,
        proj_k=None, allow_neg_eigval=False)
    mixed = torch.randn(T, cd, generator=g, device=dev).bfloat16()
    a = torch.randn(T, H, generator=g, device=dev).bfloat16()
    b = torch.randn(T, H, generator=g, device=dev).bfloat16()
    z = torch.randn(T, H, D, generator=g, device=dev).bfloat16()
    wn = torch.rand(D, generator=g, device=dev) + 0.5
    conv_cache = torch.randn(nseq, 3, cd, generator=g, device=dev).bfloat16()
    ssm = torch.randn(nseq, H, D, D, generator=g, device=dev) * 0.02
    qs = torch.arange(0, T + 1, T // nseq, dtype=torch.int32, device=dev)
    idx = torch.randperm(nseq, generator=g, device=dev).to(torch.int32)
    has = torch.ones(nseq, dtype=torch.bool, device=dev)
    md = SimpleNamespace(spec_sequence_masks=None, num_actual_tokens=T, num_decodes=0,
                         num_decode_tokens=0, num_prefills=nseq, non_spec_query_start_loc=qs,
                         non_spec_state_indices_tensor=idx, has_initial_state=has,
                         non_spec_query_start_loc_d=None, non_spec_query_start_loc_p=None)
    core = torch.zeros(T, H, D, dtype=torch.bfloat16, device=dev)
    cs = conv_cache.transpose(1, 2)
    w2 = lay.conv1d.weight.view(cd, 4)

    def reference_sequence():
        x = hmx.causal_conv1d_fn(mixed.t(), w2, None, conv_states=cs, query_start_loc=qs,
                                 cache_indices=idx, has_initial_state=has).t()
        q = x[:, :H * D].reshape(1, T, H, D).contiguous()
        k = x[:, H * D:2 * H * D].reshape(1, T, H, D).contiguous()
        v = x[:, 2 * H * D:].reshape(1, T, H, D).contiguous()
        gg, beta = hmx.fused_gdn_gating(lay.A, a, b, lay.dt_bias)
        init = ssm[idx.long()].contiguous()
        init[~has] = 0
        o, st = hmx.chunk_gated_delta_rule_gqa(q, k, v, gg, beta, initial_state=init,
                                               output_final_state=True, cu_seqlens=qs,
                                               use_qk_l2norm_in_kernel=True)
        ssm[idx.long()] = st
        core[:T] = o.squeeze(0)
        return hmx.rms_norm_gated(core, z, wn, 1e-6)

    def hmx_core():
        srv.gdn_forward_core(lay, mixed, b, a, core, md, cs, ssm, o_norm=(wn, z, 1e-6))

    ms_ref = _timed(reference_sequence, steps, warmup)
    ms_core = _timed(hmx_core, steps, warmup)
    return dict(ms_ref=ms_ref, ms_core=ms_core, tokens=T)


def bench_core_decode(dev, steps=64, warmup=8):
    """The GDN layer's core on a decode batch at the C2 shape (256 sequences x 1 token,
    H = HKV = 32, d = 128, conv width 4, fp32 state pool, randperm slots), with the
    output norm: the reference layer's call sequence over hmx ops (conv update into a
    new tensor, contiguous q/k/v, gating, recurrent step in place, copy into
    core_attn_out, separate norm; primed_gdn_layer.py:775-823, :925-936, :621-626)
    against hmx.serving.gdn_forward_core (the conv update, then the recurrent step on
    views of its output with the gating and the norm in its loads and epilogue)."""
    from types import SimpleNamespace
    import torch
    import hmx
    import hmx.serving as srv
    from hmx import workloads as wl
    N, H, D = 256, 32, 128
    cd = 3 * H * D
    g = torch.Generator(device=dev).manual_seed(wl.SEED_BASE + 14)
    lay = SimpleNamespace(
        conv1d=SimpleNamespace(weight=(torch.randn(cd, 1, 4, generator=g, device=dev) * 0.4)
                               .bfloat16()),
        activation="silu", A=torch.rand(H, generator=g, device=dev),
        dt_bias=torch.randn(H, generator=g, device=dev), key_dim=H * D, kv_k_dim=H * D,
        kv_v_dim=H * D, num_heads=H, num_kv_heads=H, head_k_dim=D, head_v_dim=D, tp_size=1,
        proj_k=None, allow_neg_eigval=False)
    nstep = 8                              # distinct inputs, cycled
    mixed = torch.randn(nstep, N, cd, generator=g, device=dev).bfloat16()
    a = torch.randn(nstep, N, H, generator=g, device=dev).bfloat16()
    b = torch.randn(nstep, N, H, generator=g, device=dev).bfloat16()
    z = torch.randn(nstep, N, H, D, generator=g, device=dev).bfloat16()
    wn = torch.rand(D, generator=g, device=dev) + 0.5
    conv_cache = torch.randn(N, 3, cd, generator=g, device=dev).bfloat16()
    ssm = torch.randn(N, H, D, D, generator=g, device=dev) * 0.02
    idx = torch.randperm(N, generator=g, device=dev).to(torch.int32)
    cu = torch.arange(N + 1, dtype=torch.int32, device=dev)
    md = SimpleNamespace(spec_sequence_masks=None, num_actual_tokens=N, num_decodes=N,
                         num_decode_tokens=N, num_prefills=0, non_spec_query_start_loc=cu,
                         non_spec_state_indices_tensor=idx, has_initial_state=None,
                         non_spec_query_start_loc_d=None, non_spec_query_start_loc_p=None)
    core = torch.zeros(N, H, D, dtype=torch.bfloat16, device=dev)
    cs = conv_cache.transpose(1, 2)
    w2 = lay.conv1d.weight.view(cd, 4)
    it = {"s": 0}

    def nxt():
        s = it["s"] % nstep
        it["s"] += 1
        return s

    def reference_sequence():
        s = nxt()
        x = hmx.causal_conv1d_update(mixed[s], cs, w2, None, "silu", conv_state_indices=idx)
        q = x[:, :H * D].reshape(1, N, H, D).contiguous()
        k = x[:, H * D:2 * H * D].reshape(1, N, H, D).contiguous()
        v = x[:, 2 * H * D:].reshape(1, N, H, D).contiguous()
        gg, beta = hmx.fused_gdn_gating(lay.A, a[s], b[s], lay.dt_bias)
        o, _ = hmx.fused_recurrent_gated_delta_rule_gqa(
            q, k, v, gg, beta, initial_state=ssm, inplace_final_state=True, cu_seqlens=cu,
            ssm_state_indices=idx, use_qk_l2norm_in_kernel=True)
        core[:N] = o.squeeze(0)
        return hmx.rms_norm_gated(core, z[s], wn, 1e-6)

    def hmx_core():
        s = nxt()
        srv.gdn_forward_core(lay, mixed[s], b[s], a[s], core, md, cs, ssm,
                             o_norm=(wn, z[s], 1e-6))

    ms_ref = _timed(reference_sequence, steps, warmup)
    ms_core = _timed(hmx_core, steps, warmup)
    return dict(ms_ref=ms_ref, ms_core=ms_core, tokens=N)


def bench_decode(dev, steps_total=512, warmup=8):
    import torch
    import hmx
    from hmx import workloads as wl
    N, H, D = 256, 32, 128
    d = wl.decode_inputs(n_seqs=N, H=H, HKV=H, D=D, steps=steps_total, device=dev, gen_device=dev)
    pool, idx, cu = d["pool"], d["idx"], d["cu_seqlens"]
    it = {"s": 0}

    def step():
        s = it["s"] % steps_total
        it["s"] += 1
        hmx.fused_recurrent_gated_delta_rule_gqa(
            d["q"][s], d["k"][s], d["v"][s], d["g"][s], d["beta"][s], initial_state=pool,
            inplace_final_state=True, cu_seqlens=cu, ssm_state_indices=idx,
            use_qk_l2norm_in_kernel=True)

    ms = _timed(step, steps_total, warmup)
    by = wl.gdn_decode_bytes(N, H, H)
    gbs = by / (ms * 1e-3) / 1e9
    return dict(ms=ms, steps_per_s=1e3 / ms, tokens_per_s=N * 1e3 / ms, bytes=by, GBps=gbs)


def bench_gka_decode(dev, num_iter=8, steps_total=128, warmup=4):
    """K7: gka_chebyshev_gla_decode over 256 sequences x 1 token, H = 32, d = 128, in
    place on fp32 h_kk / h_kv pools (randperm slots), the C2 batch shape."""
    import torch
    import torch.nn.functional as F
    import hmx
    from hmx import workloads as wl
    N, H, D = 256, 32, 128
    g = torch.Generator(device=dev).manual_seed(wl.SEED_BASE + 6)
    q = torch.randn(steps_total, 1, N, H, D, generator=g, device=dev).bfloat16()
    k = torch.randn(steps_total, 1, N, H, D, generator=g, device=dev).bfloat16()
    v = torch.randn(steps_total, 1, N, H, D, generator=g, device=dev).bfloat16()
    alpha = torch.sigmoid(torch.randn(steps_total, 1, N, H, generator=g, device=dev))
    gk = F.logsigmoid(torch.randn(steps_total, 1, N, H, generator=g, device=dev))
    beta = torch.sigmoid(torch.randn(steps_total, 1, N, H, generator=g, device=dev))
    x = torch.randn(N, H, D, 16, generator=g, device=dev) * 0.05
    hkk = x @ x.transpose(-1, -2)
    hkv = torch.randn(N, H, D, D, generator=g, device=dev) * 0.02
    idx = torch.randperm(N, generator=g, device=dev).to(torch.int32)
    cu = torch.arange(N + 1, dtype=torch.int32, device=dev)
    out = torch.empty(1, N, H, D, dtype=torch.bfloat16, device=dev)
    it = {"s": 0}

    def step():
        s = it["s"] % steps_total
        it["s"] += 1
        gs = gk[s]                                   # the op requires g is gk
        hmx.gka_chebyshev_gla_decode(q[s], k[s], v[s], alpha[s], gs, gs, beta[s],
                                     D ** -0.5, num_iter=num_iter, h_kk=hkk, h_kv=hkv,
                                     cu_seqlens=cu, ssm_state_indices=idx, out=out)

    ms = _timed(step, steps_total, warmup)
    by = wl.gka_decode_bytes(N, H, H, D)
    return dict(ms=ms, steps_per_s=1e3 / ms, bytes=by, GBps=by / (ms * 1e-3) / 1e9)


def bench_gka(dev, steps, warmup, num_iter):
    """C3: gka_chebyshev_gla_prefill at the C1 shape, ridge 0.01, zero initial states."""
    import hmx
    from hmx import workloads as wl
    T, H, D = 32768, 32, 128
    d = wl.gka_inputs(T=T, H=H, HKV=H, D=D, config_id=3, device=dev, gen_device=dev)
    args = [d[n] for n in ("q", "k", "v", "alpha", "g", "gk", "beta")]

    def step():
        hmx.gka_chebyshev_gla_prefill(*args, D ** -0.5, ridge_ratio=0.01, num_iter=num_iter,
                                      output_final_state=True)

    ms = _timed(step, steps, warmup)
    fl = wl.gka_prefill_flops(T, H, num_iter)
    by = wl.gka_prefill_bytes(T, H, H)
    tfs = fl / (ms * 1e-3) / 1e12
    return dict(ms=ms, tokens_per_s=T / (ms * 1e-3), flops=fl, bytes=by, TFLOPs=tfs,
                GBps=by / (ms * 1e-3) / 1e9)


def bench_gka_train(dev, steps, warmup, num_iter=8, B=8, T=4096, H=32):
    """F4: the training layer's Chebyshev solve (hmx.ChebyshevIteration) forward and
    forward + backward through autograd, B=8 x T=4096 tokens (the C3 token count),
    H=32, d=128, ridge 0.02, bp_lambda; inputs as the layer prepares them (unit q,
    k = beta k^ with beta in (0.1, 1), gk = logsigmoid(N(2, 1)) / 8).  Also the
    whole training GKA op (hmx.gka_chebyshev_gla: solve, blend, GLA) forward +
    backward on the same shape."""
    import torch
    import torch.nn.functional as F
    import hmx
    from hmx import workloads as wl
    D = 128
    g = torch.Generator(device=dev).manual_seed(wl.SEED_BASE + 12)
    q = F.normalize(torch.randn(B, T, H, D, generator=g, device=dev), dim=-1).bfloat16()
    beta = torch.rand(B, T, H, 1, generator=g, device=dev) * 0.9 + 0.1
    k = (F.normalize(torch.randn(B, T, H, D, generator=g, device=dev), dim=-1) * beta).bfloat16()
    gk = F.logsigmoid(torch.randn(B, T, H, generator=g, device=dev) + 2.0) / 8
    dx = torch.randn(B, T, H, D, generator=g, device=dev).bfloat16()
    kk, qq, gg = (t.clone().requires_grad_(True) for t in (k, q, gk))

    def fwd():
        with torch.no_grad():
            hmx.ChebyshevIteration.apply(k, q, gk, num_iter, 0.02, True)

    def fwd_bwd():
        x, _ = hmx.ChebyshevIteration.apply(kk, qq, gg, num_iter, 0.02, True)
        torch.autograd.backward(x, dx)

    ms_f = _timed(fwd, steps, warmup)
    ms_fb = _timed(fwd_bwd, steps, warmup)
    ff, fb = wl.gka_train_flops(B * T, H, num_iter)
    # the whole training GKA forward (solve, blend, GLA) with its backward
    v = torch.randn(B, T, H, D, generator=g, device=dev).bfloat16()
    alpha = torch.rand(B, T, H, generator=g, device=dev)
    gg_ = F.logsigmoid(torch.randn(B, T, H, generator=g, device=dev) + 2.0) / 8
    do = torch.randn(B, T, H, D, generator=g, device=dev).bfloat16()
    ins = [t.clone().requires_grad_(True) for t in (q, k, v, alpha, gg_, gk)]

    def layer_fwd_bwd():
        o, _, _ = hmx.gka_chebyshev_gla(*ins, D ** -0.5, 0.02, num_iter=num_iter)
        torch.autograd.backward(o, do)

    ms_l = _timed(layer_fwd_bwd, steps, warmup)
    return dict(ms_fwd=ms_f, ms_fwd_bwd=ms_fb, flops_fwd=ff, flops_bwd=fb,
                tokens_per_s=B * T / (ms_fb * 1e-3),
                TFLOPs_fwd=ff / (ms_f * 1e-3) / 1e12,
                TFLOPs_fwd_bwd=(ff + fb) / (ms_fb * 1e-3) / 1e12,
                ms_gka_chebyshev_gla_fwd_bwd=ms_l)


def bench_gdn_train(dev, steps, warmup, B=8, T=4096, H=32):
    """F4: the training GDN op (hmx.chunk_gated_delta_rule with the in-kernel L2
    normalisation, through hmx.ChunkGatedDeltaRule under autograd) forward and
    forward + backward, B=8 x T=4096 tokens, H=32, d=128; inputs as the training
    layer forms them (q, k, v ~ N(0, 1) bf16, g = -e^{A_log} softplus(x + dt_bias)
    fp32, beta = sigmoid(x) bf16, do ~ N(0, 1)).  Also forward + backward at the C1
    shape (B=1, T=32768), with these gates and with a fresh layer's gates (many heads
    decay too slowly for a warm-up: their state-gradient runs take the exact combine)."""
    import torch
    import torch.nn.functional as F
    import hmx
    from hmx import workloads as wl
    D = 128
    g = torch.Generator(device=dev).manual_seed(wl.SEED_BASE + 13)

    def inputs(B, T):
        r = lambda *s: torch.randn(*s, generator=g, device=dev)
        q, k, v, do = (r(B, T, H, D).bfloat16() for _ in range(4))
        A_log = torch.rand(H, generator=g, device=dev) * 2.0 - 1.0
        gate = -A_log.exp() * F.softplus(r(B, T, H) - 2.0)
        beta = torch.sigmoid(r(B, T, H)).bfloat16()
        return q, k, v, gate, beta, do

    def run(B, T, with_bwd, layer_gates=False):
        q, k, v, gate, beta, do = inputs(B, T)
        if layer_gates:    # a fresh layer's gates: many heads decay slowly (exact runs)
            gate, beta = wl.gdn_layer_gates(T, H, device=dev)
            beta = beta.bfloat16()
        ins = [t.clone().requires_grad_(True) for t in (q, k, v, gate, beta)]

        def fwd():
            with torch.no_grad():
                hmx.chunk_gated_delta_rule(q, k, v, gate, beta, use_qk_l2norm_in_kernel=True)

        def fwd_bwd():   # the gradients returned, not accumulated into .grad
            o, _ = hmx.chunk_gated_delta_rule(*ins, use_qk_l2norm_in_kernel=True)
            torch.autograd.grad(o, ins, do)
        return _timed(fwd_bwd if with_bwd else fwd, steps, warmup)

    ms_f = run(B, T, False)
    ms_fb = run(B, T, True)
    ms_c1 = run(1, 32768, True)
    ms_c1_layer = run(1, 32768, True, layer_gates=True)
    ff, fb = wl.gdn_train_flops(B * T, H)
    return dict(ms_fwd=ms_f, ms_fwd_bwd=ms_fb, ms_c1_fwd_bwd=ms_c1,
                ms_c1_layer_gates_fwd_bwd=ms_c1_layer, flops_fwd=ff, flops_bwd=fb,
                tokens_per_s=B * T / (ms_fb * 1e-3),
                TFLOPs_fwd_bwd=(ff + fb) / (ms_fb * 1e-3) / 1e12)


def bench_ssd_train(dev, steps, warmup):
    """F4 Mamba2: the training scan (hmx.mamba_chunk_scan_combined through
    hmx.MambaChunkScanCombined under autograd, mamba2.py:555-580) at the C4 shape
    (b=2, T=16384, H=64, P=64, N=128, G=8, D, dt_bias, softplus), forward alone and
    forward + backward with dy ~ N(0, 1).  The backward recomputes the forward (one
    segment per 64-token chunk, for the chunk start states), then runs the local,
    reverse-scan and chunk-gradient launches."""
    import torch
    import hmx
    from hmx import workloads as wl
    d = wl.ssd_inputs(config_id=4, device=dev, gen_device=dev)
    b, T, H, P = d["x"].shape
    G, N = d["B"].shape[2], d["B"].shape[3]
    g = torch.Generator(device=dev).manual_seed(wl.SEED_BASE + 15)
    dy = torch.randn(b, T, H, P, generator=g, device=dev).bfloat16()
    leaves = [d[k].clone().requires_grad_(True) for k in ("x", "dt", "A", "B", "C", "D",
                                                          "dt_bias")]

    def fwd():
        with torch.no_grad():
            hmx.mamba_chunk_scan_combined(d["x"], d["dt"], d["A"], d["B"], d["C"], 256,
                                          D=d["D"], dt_bias=d["dt_bias"], dt_softplus=True)

    def fwd_bwd():   # the gradients returned, not accumulated into .grad
        x, dt, A, B, C, D, bias = leaves
        y = hmx.mamba_chunk_scan_combined(x, dt, A, B, C, 256, D=D, dt_bias=bias,
                                          dt_softplus=True)
        torch.autograd.grad(y, leaves, dy)

    ms_f = _timed(fwd, steps, warmup)
    ms_fb = _timed(fwd_bwd, steps, warmup)
    L = 64   # the backward's chunk: per (chunk, head) 3 L^2 N + 3 L^2 P + 5 L P N MACs
    flops_bwd = 2.0 * (b * T // L) * H * (3 * L * L * N + 3 * L * L * P + 5 * L * P * N)
    del leaves, d, dy

    # the hybrid layer's training shape (mamba2.py:541-580 with headdim = d_state =
    # 128 as mamba2.py:146 sets it): 8 x 4096 tokens, 32 heads, x and B repeated to
    # the heads, C in 32 groups, D per head, no z (the layer's RMSNorm path)
    b2, T2, H2, P2 = 8, 4096, 32, 128
    r = lambda *sh: torch.randn(*sh, generator=g, device=dev)
    x2, B2, C2, dy2 = (r(b2, T2, H2, P2).bfloat16() for _ in range(4))
    dt2 = r(b2, T2, H2) * 0.5 - 2.0
    A2 = -torch.rand(H2, generator=g, device=dev) * 15.0 - 1.0
    D2, bias2 = torch.ones(H2, device=dev), torch.full((H2,), -4.0, device=dev)
    leaves2 = [t.clone().requires_grad_(True) for t in (x2, dt2, A2, B2, C2, D2, bias2)]

    def fwd_bwd_hybrid():
        x, dt, A, B, C, D, bias = leaves2
        y = hmx.mamba_chunk_scan_combined(x, dt, A, B, C, 256, D=D, dt_bias=bias,
                                          dt_softplus=True)
        torch.autograd.grad(y, leaves2, dy2)

    def fwd_hybrid():
        with torch.no_grad():
            hmx.mamba_chunk_scan_combined(x2, dt2, A2, B2, C2, 256, D=D2, dt_bias=bias2,
                                          dt_softplus=True)

    ms_f2 = _timed(fwd_hybrid, steps, warmup)
    ms_fb2 = _timed(fwd_bwd_hybrid, steps, warmup)
    return dict(ms_fwd=ms_f, ms_fwd_bwd=ms_fb, tokens=b * T, flops_bwd=flops_bwd,
                tokens_per_s=b * T / (ms_fb * 1e-3), ms_fwd_hybrid=ms_f2,
                ms_fwd_bwd_hybrid=ms_fb2)


def bench_ssd(dev, steps, warmup, b=2, T=16384, H=64, P=64, N=128, G=8):
    """C4: mamba_chunk_scan_combined, b=2, T=16384, H=64, P=64, N=128, G=8, fp32 final
    state (other shapes through the keywords: the primed layout is P = N = 128, G = H)."""
    import hmx
    from hmx import workloads as wl
    d = wl.ssd_inputs(b=b, T=T, H=H, P=P, N=N, G=G, config_id=4, device=dev, gen_device=dev)

    def step():
        hmx.mamba_chunk_scan_combined(d["x"], d["dt"], d["A"], d["B"], d["C"], 256, D=d["D"],
                                      dt_bias=d["dt_bias"], dt_softplus=True,
                                      return_final_states=True)

    ms = _timed(step, steps, warmup)
    by = wl.ssd_bytes(b * T, H, G, P, N, n_seqs=b)
    fl = wl.ssd_flops(b * T, H, G, P, N)
    return dict(ms=ms, tokens_per_s=b * T / (ms * 1e-3), bytes=by, flops=fl,
                GBps=by / (ms * 1e-3) / 1e9, TFLOPs=fl / (ms * 1e-3) / 1e12)


def bench_ssd_decode(dev, steps=64, warmup=4):
    """selective_state_update over a 256-slot fp32 pool (H=64, P=64, N=128, G=8; vLLM's
    expanded A/dt/D views), randperm slots -- the C2 batch shape on the C4 layer."""
    import torch
    import hmx
    from hmx import workloads as wl
    bsz, H, P, N, G = 256, 64, 64, 128, 8
    g = torch.Generator(device=dev).manual_seed(wl.SEED_BASE + 5)
    pool = torch.randn(bsz, H, P, N, generator=g, device=dev) * 0.02
    idx = torch.randperm(bsz, generator=g, device=dev).to(torch.int32)
    x = torch.randn(steps, bsz, H, P, generator=g, device=dev).bfloat16()
    dt = torch.randn(steps, bsz, H, generator=g, device=dev) * 0.5 - 2.0
    B = torch.randn(steps, bsz, G, N, generator=g, device=dev).bfloat16()
    C = torch.randn(steps, bsz, G, N, generator=g, device=dev).bfloat16()
    A = -torch.exp(torch.rand(H, generator=g, device=dev) * 2.77)
    Ae = A[:, None, None].expand(H, P, N)
    De = torch.ones(H, device=dev)[:, None].expand(H, P)
    be = torch.full((H,), -4.0, device=dev)[:, None].expand(H, P)
    out = torch.empty(bsz, H, P, dtype=torch.bfloat16, device=dev)
    it = {"s": 0}

    def step():
        s = it["s"] % steps
        it["s"] += 1
        hmx.selective_state_update(pool, x[s], dt[s][:, :, None].expand(bsz, H, P), Ae, B[s], C[s],
                                   De, None, be, True, state_batch_indices=idx, out=out)

    ms = _timed(step, steps, warmup)
    by = wl.ssd_decode_bytes(bsz, H, G, P, N)
    return dict(ms=ms, steps_per_s=1e3 / ms, bytes=by, GBps=by / (ms * 1e-3) / 1e9)


def cpu_model():
    """The host CPU as lscpu reports it: model name, vendor, family / model /
    stepping (the model name alone can be a bare "AMD EPYC" under virtualisation)."""
    fields = {}
    try:
        import subprocess
        txt = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in txt.splitlines():
            k, _, v = line.partition(":")
            fields[k.strip()] = v.strip()
    except (OSError, ValueError, subprocess.SubprocessError):
        pass
    if not fields.get("Model name"):
        try:
            for line in open("/proc/cpuinfo"):
                k, _, v = line.partition(":")
                k = {"model name": "Model name", "vendor_id": "Vendor ID",
                     "cpu family": "CPU family", "model": "Model", "stepping": "Stepping"}.get(k.strip())
                if k and k not in fields:
                    fields[k] = v.strip()
        except OSError:
            pass
    name = fields.get("Model name")
    if name is None:
        return None
    ident = ", ".join(f"{k.lower()} {fields[k]}" for k in ("CPU family", "Model", "Stepping")
                      if fields.get(k))
    vend = fields.get("Vendor ID")
    return f"{name} ({vend}{', ' if vend and ident else ''}{ident})" if (vend or ident) else name


def _median_time(fn, reps=3):
    """1 untimed warm-up call, then the median of ``reps`` timed calls (seconds)."""
    fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return sorted(ts)[len(ts) // 2]


def cpu_baseline(sample_tokens=32768):
    """The oracle's chunked fp32 restatement on the host, on the whole C1 workload
    (T=32768, H=32; a few seconds on the box's host cores)."""
    import torch
    from hmx import workloads as wl
    from oracle import gdn as ref
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    d = wl.gdn_inputs(T=sample_tokens, H=32, HKV=32, D=128, config_id=1)
    args = [d[n] for n in ("q", "k", "v", "g", "beta")]
    dt = _median_time(lambda: ref.chunk_gated_delta_rule_gqa(
        *args, output_final_state=True, use_qk_l2norm_in_kernel=True, dtype=torch.float32))
    return dict(value=sample_tokens / dt, unit="tokens/s", cores=torch.get_num_threads(),
                cpu=cpu_model(), kind="port", sample=f"C1 {sample_tokens} tokens x 32 heads (the whole workload), "
                f"oracle chunked form (chunk 64) in fp32 torch on CPU, median of 3 after a warm-up: "
                f"{dt:.2f} s")


def cpu_baselines_more(c3_n32_budget_s=300.0):
    """The oracle beside C1 on every other config, same host, fp32 torch on all cores:
    C0 whole (T=2048, H=16, chunked form) and C4 whole (chunked form), each the
    median of 3 after a warm-up; C2 all 512 decode steps (256 sequences x 32 heads,
    the 512 MiB pool) and C3 whole at num_iter 8 (per-token form, ~20 s), once each;
    C3 at num_iter 32 whole if its first 4096 tokens project the whole run under
    ``c3_n32_budget_s``, else those 4096 tokens, labelled."""
    import torch
    from hmx import workloads as wl
    from oracle import gdn as gref, gka as kref, ssd as sref
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    f32 = torch.float32
    out = {}
    model = cpu_model()

    def row(value, unit, sample):
        return dict(value=value, unit=unit, cores=cores, cpu=model, kind="port", sample=sample)
    d0 = wl.gdn_inputs(T=2048, H=16, HKV=16, D=128, dtype=f32, config_id=0)
    a0 = [d0[n] for n in ("q", "k", "v", "g", "beta")]
    dt = _median_time(lambda: gref.chunk_gated_delta_rule_gqa(
        *a0, output_final_state=True, use_qk_l2norm_in_kernel=True, dtype=f32))
    out["c0"] = row(2048 / dt, "tokens/s", f"C0 whole (2048 tokens x 16 heads, fp32 inputs), oracle "
                    f"chunked form (chunk 64) in fp32 torch on CPU, median of 3: {dt:.3f} s")
    steps = 512
    d = wl.decode_inputs(n_seqs=256, H=32, HKV=32, D=128, steps=steps)
    pool = d["pool"].clone()
    t0 = time.perf_counter()
    for s in range(steps):
        _, pool = gref.fused_recurrent_gated_delta_rule_gqa(
            d["q"][s], d["k"][s], d["v"][s], d["g"][s], d["beta"][s], initial_state=pool,
            inplace_final_state=True, cu_seqlens=d["cu_seqlens"], ssm_state_indices=d["idx"],
            use_qk_l2norm_in_kernel=True, dtype=f32)
    dt = time.perf_counter() - t0
    del d, pool
    out["decode"] = row(steps / dt, "steps/s", f"C2 all {steps} steps (256 seqs x 32 heads, the "
                        f"state carried step to step), oracle recurrence in fp32 torch on CPU, "
                        f"{dt:.2f} s")
    T = 32768
    g = wl.gka_inputs(T=T, H=32, HKV=32, D=128)
    ga = [g[n] for n in ("q", "k", "v", "alpha", "g", "gk", "beta")]

    def gka(n, t):
        return kref.gka_chebyshev_gla_prefill(*[a[:, :t] for a in ga], 128 ** -0.5,
                                              ridge_ratio=0.01, num_iter=n, dtype=f32)
    t0 = time.perf_counter()
    gka(8, T)
    dt = time.perf_counter() - t0
    out["gka_num_iter_8"] = row(T / dt, "tokens/s", f"C3 whole workload ({T} tokens x 32 heads), "
                                f"num_iter 8, oracle per-token form in fp32 torch on CPU, {dt:.2f} s")
    t_part = 4096
    t0 = time.perf_counter()
    gka(32, t_part)
    dt = time.perf_counter() - t0
    if dt * T / t_part < c3_n32_budget_s:
        t0 = time.perf_counter()
        gka(32, T)
        dt = time.perf_counter() - t0
        out["gka_num_iter_32"] = row(T / dt, "tokens/s", f"C3 whole workload ({T} tokens x 32 "
                                     f"heads), num_iter 32, oracle per-token form in fp32 torch "
                                     f"on CPU, {dt:.2f} s")
    else:
        out["gka_num_iter_32"] = row(t_part / dt, "tokens/s", f"C3 FIRST {t_part} TOKENS ONLY x 32 "
                                     f"heads (the whole run projects past {c3_n32_budget_s:.0f} "
                                     f"s), num_iter 32, oracle per-token form in fp32 torch on "
                                     f"CPU, {dt:.2f} s")
    del g, ga
    x = wl.ssd_inputs()
    dt = _median_time(lambda: sref.mamba_chunk_scan_combined(
        x["x"], x["dt"], x["A"], x["B"], x["C"], 256, D=x["D"], dt_bias=x["dt_bias"],
        dt_softplus=True, return_final_states=True, dtype=f32))
    out["ssd"] = row(2 * 16384 / dt, "tokens/s", f"C4 whole workload (2 x 16384 tokens x 64 "
                     f"heads), oracle chunked form in fp32 torch on CPU, median of 3: {dt:.2f} s")
    return out


def copy_calibration(dev, nbytes=1 << 30, reps=5):
    """A plain device copy of known size: what FETCH_SIZE / WRITE_SIZE read for it
    calibrates the counters (bytes moved per dispatch = nbytes each way)."""
    import torch
    src = torch.empty(nbytes // 4, dtype=torch.float32, device=dev).uniform_()
    dst = torch.empty_like(src)
    ms = _timed(lambda: dst.copy_(src), reps, 1)
    return dict(bytes_each_way=nbytes, ms=ms, GBps=2 * nbytes / (ms * 1e-3) / 1e9)


def measured_traffic(key):
    """HBM bytes per launch from the committed rocprofv3 PMC summary (profiles/), if any."""
    f = REPO / "profiles" / "traffic.json"
    try:
        return json.loads(f.read_text())[key]["hbm_bytes"]
    except (OSError, KeyError, ValueError):
        return None


# bench legs in run order (the long compute-bound GKA legs last), and the groups
# --only accepts beside single legs
LEGS = ["c1", "prefill_gqa", "prefill_varlen", "prefill_layer_gates", "onorm", "conv", "gdn_core",
        "gdn_decode_core", "mamba2_core", "gka_core", "gdn_decode", "gka_decode", "ssd_c4", "ssd_primed",
        "ssd_decode", "gka8", "gka32", "gka_train", "gdn_train", "ssd_train"]
GROUPS = {"prefill": ["c1", "prefill_gqa", "prefill_varlen", "prefill_layer_gates"],
          "core": ["gdn_core", "gdn_decode_core", "mamba2_core", "gka_core"], "decode": ["gdn_decode", "gka_decode"],
          "ssd": ["ssd_c4", "ssd_primed", "ssd_decode"], "gka": ["gka8", "gka32"],
          "train": ["gka_train", "gdn_train", "ssd_train"]}


def measured_mfma_busy(key):
    """Counter-based MFMA busy fraction of the leg's dominant kernel
    (SQ_VALU_MFMA_BUSY_CYCLES over the SIMDs' cycles) from the committed summary."""
    f = REPO / "profiles" / "traffic.json"
    try:
        return json.loads(f.read_text())[key]["mfma_busy"]["frac"]
    except (OSError, KeyError, ValueError):
        return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", default=None,
                    help="comma-separated legs (" + ", ".join(LEGS) + ") or groups (" +
                         ", ".join(GROUPS) + "); default: all")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a 1 GiB device copy (HBM counter calibration)")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the mixer ops shard by head/sequence with no "
              "communication inside the op, so multi-GPU runs are not part of this build.",
              file=sys.stderr)
        sys.exit(2)
    sel = []
    for name in (a.only.split(",") if a.only else LEGS):
        name = name.strip()
        if name in GROUPS:
            sel += GROUPS[name]
        elif name in LEGS:
            sel.append(name)
        else:
            ap.error(f"unknown leg {name!r}")
    import torch
    dev = torch.device("cuda:0")
    if a.copy_calibration:
        print(json.dumps({"copy_calibration": copy_calibration(dev)}), flush=True)
        return
    out = {}
    S, W = a.steps, a.warmup
    run = {
        "c1": lambda: out.__setitem__("prefill", bench_prefill(dev, S, W)),
        "prefill_gqa": lambda: out.__setitem__("prefill_gqa", bench_prefill(dev, S, W, HKV=8)),
        "prefill_varlen": lambda: out.__setitem__("prefill_varlen", bench_prefill_varlen(dev, S, W)),
        "prefill_layer_gates": lambda: out.__setitem__("prefill_layer_gates",
                                                       bench_prefill_layer_gates(dev, S, W)),
        "onorm": lambda: out.__setitem__("onorm", bench_onorm(dev, S, W)),
        "conv": lambda: out.__setitem__("conv", bench_conv(dev, S, W)),
        "gdn_core": lambda: out.__setitem__("core", bench_core(dev, max(2, S // 2), W)),
        "gdn_decode_core": lambda: out.__setitem__("decode_core", bench_core_decode(dev)),
        "mamba2_core": lambda: out.__setitem__("mamba2_core", bench_mamba2_core(dev, max(2, S // 2), W)),
        "gka_core": lambda: out.__setitem__("gka_core", bench_gka_core(dev, max(2, S // 4), 1)),
        "gdn_decode": lambda: out.__setitem__("decode", bench_decode(dev)),
        "gka_decode": lambda: out.__setitem__("gka_decode", bench_gka_decode(dev)),
        "ssd_c4": lambda: out.__setitem__("ssd", bench_ssd(dev, S, W)),
        "ssd_primed": lambda: out.__setitem__(
            "ssd_primed", bench_ssd(dev, max(2, S // 2), W, P=128, N=128, G=64)),
        "ssd_decode": lambda: out.__setitem__("ssd_decode", bench_ssd_decode(dev)),
        "gka8": lambda: out.setdefault("gka", {}).__setitem__(8, bench_gka(dev, max(2, S // 4), 1, 8)),
        "gka32": lambda: out.setdefault("gka", {}).__setitem__(32, bench_gka(dev, max(2, S // 4), 1, 32)),
        "gka_train": lambda: out.__setitem__("gka_train", bench_gka_train(dev, max(2, S // 4), 1)),
        "gdn_train": lambda: out.__setitem__("gdn_train", bench_gdn_train(dev, max(2, S // 4), 1)),
        "ssd_train": lambda: out.__setitem__("ssd_train", bench_ssd_train(dev, max(2, S // 4), 1)),
    }
    for name in LEGS:           # run order: the long compute-bound GKA legs last
        if name in sel:
            run[name]()
    line = {
        "metric": "mixer prefill tokens/sec + decode steps/sec at 8B shape; % of roofline (1 GPU)",
        "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic",
    }
    if "prefill" in out:
        pf = out["prefill"]
        line.update({
            "value": round(pf["tokens_per_s"], 1), "unit": "tokens/s",
            "ms_per_step": round(pf["ms"], 4),
            "config": {"workload": "C1 GDN chunked prefill (chunk_gated_delta_rule_gqa)",
                       "B": 1, "T": 32768, "H": 32, "HKV": 32, "d": 128, "chunk": 32,
                       "qkv_dtype": "bf16", "state_dtype": "fp32"},
            "roofline": {"bound": "hbm", "achieved": round(pf["GBps"], 1),
                         "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(pf["GBps"] / HBM_PEAK_GBS, 4),
                         "traffic": measured_traffic("gdn_prefill_c1"),
                         "kernel": "all launches of one prefill op call",
                         "algorithmic_bytes": pf["bytes"],
                         "mfma_TFLOPs": round(pf["TFLOPs"], 1),
                         "mfma_frac": round(pf["TFLOPs"] / BF16_PEAK_TFLOPS, 4),
                         "mfma_flops_basis": "2 T H (5 C d + 3 d^2) at C = 64: 188.98 GFLOP",
                         "mfma_frac_chunk32": round(pf["TFLOPs_c32"] / BF16_PEAK_TFLOPS, 4),
                         "mfma_flops_chunk32": pf["flops_c32"],
                         "mfma_busy_counter": measured_mfma_busy("gdn_prefill_c1")},
        })
    if "prefill_gqa" in out:
        r = out["prefill_gqa"]
        line["prefill_gqa"] = {
            "value": round(r["tokens_per_s"], 1), "unit": "tokens/s", "ms_per_step": round(r["ms"], 4),
            "config": {"workload": "C1 with HKV=8 (Qwen3-8B GQA layout)", "T": 32768, "H": 32,
                       "HKV": 8, "d": 128},
            "roofline": {"bound": "hbm", "achieved": round(r["GBps"], 1), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(r["GBps"] / HBM_PEAK_GBS, 4),
                         "algorithmic_bytes": r["bytes"],
                         "traffic": measured_traffic("gdn_prefill_gqa"),
                         "mfma_TFLOPs": round(r["TFLOPs"], 1)},
        }
    if "prefill_varlen" in out:
        r = out["prefill_varlen"]
        line["prefill_varlen"] = {
            "value": round(r["tokens_per_s"], 1), "unit": "tokens/s", "ms_per_step": round(r["ms"], 4),
            "config": {"workload": "C1 varlen: 8 sequences, randint(1024, 8193) tokens",
                       "lengths": r["lengths"], "tokens": r["tokens"], "H": 32, "d": 128,
                       "initial_state": "zeros fp32 [8,32,128,128]"},
            "roofline": {"bound": "hbm", "achieved": round(r["GBps"], 1), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(r["GBps"] / HBM_PEAK_GBS, 4),
                         "algorithmic_bytes": r["bytes"],
                         "traffic": measured_traffic("gdn_prefill_varlen")},
        }
    if "prefill_layer_gates" in out:
        r = out["prefill_layer_gates"]
        line["prefill_layer_gates"] = {
            "value": round(r["tokens_per_s"], 1), "unit": "tokens/s", "ms_per_step": round(r["ms"], 4),
            "vs_c1_bench_gates": (round(r["ms"] / out["prefill"]["ms"], 3)
                                  if "prefill" in out else None),
            "config": {"workload": "C1 with layer-initialisation gates (A_log ~ log U(1,16), "
                                   "dt ~ logU(1e-3, 1e-1), a, b ~ N(0,1))",
                       "T": 32768, "H": 32, "HKV": 32, "d": 128, "segments": r["segments"],
                       "exact_scan_pairs": r["exact_pairs"],
                       "exact_scan_pairs_of": (r["segments"] - 1) * 32,
                       "heads_running_exact_scan": r["exact_heads"]},
            "roofline": {"bound": "hbm", "achieved": round(r["GBps"], 1), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(r["GBps"] / HBM_PEAK_GBS, 4),
                         "algorithmic_bytes": r["bytes"],
                         "traffic": measured_traffic("gdn_prefill_layer_gates")},
        }
    if "decode" in out:
        dc = out["decode"]
        line["decode"] = {
            "value": round(dc["steps_per_s"], 1), "unit": "steps/s",
            "ms_per_step": round(dc["ms"], 4), "tokens_per_s": round(dc["tokens_per_s"], 1),
            "config": {"workload": "C2 GDN fused recurrent decode", "seqs": 256, "H": 32,
                       "d": 128, "steps": 512, "pool": "fp32 [256,32,128,128] randperm slots"},
            "roofline": {"bound": "hbm", "achieved": round(dc["GBps"], 1), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(dc["GBps"] / HBM_PEAK_GBS, 4),
                         "traffic": measured_traffic("gdn_decode_c2"),
                         "algorithmic_bytes": dc["bytes"]},
        }
        if "value" not in line:
            line.update({"value": line["decode"]["value"], "unit": "steps/s",
                         "ms_per_step": line["decode"]["ms_per_step"],
                         "config": line["decode"]["config"],
                         "roofline": line["decode"]["roofline"]})
    if "onorm" in out:
        r = out["onorm"]
        line["o_norm"] = {
            "config": {"workload": "C1 GDN prefill output norm o_norm(o, z) (gated RMSNorm, "
                                   "norm before gate)", "T": 32768, "H": 32, "d": 128},
            "prefill_then_norm_ms": round(r["ms_unfused"], 4),
            "prefill_fused_norm_ms": round(r["ms_fused"], 4),
            "norm_kernel_ms": round(r["ms_norm"], 4),
            "norm_roofline": {"bound": "hbm", "achieved": round(r["norm_GBps"], 1),
                              "peak": HBM_PEAK_GBS, "unit": "GB/s",
                              "frac": round(r["norm_GBps"] / HBM_PEAK_GBS, 4),
                              "algorithmic_bytes": r["norm_bytes"],
                              "traffic": measured_traffic("gated_norm")},
        }
    if "conv" in out:
        r = out["conv"]
        line["conv1d"] = {
            "config": {"workload": "GDN input conv (causal_conv1d_fn / causal_conv1d_update), "
                                   "q|k|v dim 12288, width 4, silu, bf16",
                       "prefill": "8 seqs x 4096 tokens, state cache [8,3,12288] "
                                  "(passed as its [8,12288,3] view)",
                       "decode": "256 seqs x 1 token, cache [256,3,12288] randperm slots"},
            "prefill_ms": round(r["ms_fwd"], 4),
            "prefill_roofline": {"bound": "hbm", "achieved": round(r["fwd_GBps"], 1),
                                 "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                 "frac": round(r["fwd_GBps"] / HBM_PEAK_GBS, 4),
                                 "algorithmic_bytes": r["fwd_bytes"],
                                 "traffic": measured_traffic("conv1d_prefill")},
            "decode_ms": round(r["ms_dec"], 4),
            "decode_roofline": {"bound": "hbm", "achieved": round(r["dec_GBps"], 1),
                                "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                "frac": round(r["dec_GBps"] / HBM_PEAK_GBS, 4),
                                "algorithmic_bytes": r["dec_bytes"],
                                "traffic": measured_traffic("conv1d_decode")},
        }
    if "core" in out:
        r = out["core"]
        line["gdn_layer_core"] = {
            "config": {"workload": "GDN layer core + output norm at C1 (8 seqs x 4096 tokens, "
                                   "H=HKV=32, d=128, conv width 4, pooled states)"},
            "reference_call_sequence_ms": round(r["ms_ref"], 4),
            "hmx_serving_core_ms": round(r["ms_core"], 4),
            "tokens_per_s": round(r["tokens"] / (r["ms_core"] * 1e-3), 1),
        }
    if "decode_core" in out:
        r = out["decode_core"]
        line["gdn_decode_core"] = {
            "config": {"workload": "GDN layer core + output norm on a decode batch (256 seqs x "
                                   "1 token, H=HKV=32, d=128, conv width 4, fp32 pool)"},
            "reference_call_sequence_ms": round(r["ms_ref"], 4),
            "hmx_serving_core_ms": round(r["ms_core"], 4),
            "tokens_per_s": round(r["tokens"] / (r["ms_core"] * 1e-3), 1),
        }
    if "gka_core" in out:
        r = out["gka_core"]
        line["gka_layer_core"] = {
            "config": {"workload": "GKA layer core + output norm, prefill of 8 seqs x 4096 "
                                   "tokens (H=HKV=32, d=128, num_iter 8, pooled states)"},
            "reference_call_sequence_ms": round(r["ms_ref"], 4),
            "hmx_serving_core_ms": round(r["ms_core"], 4),
            "tokens_per_s": round(r["tokens"] / (r["ms_core"] * 1e-3), 1),
        }
    if "mamba2_core" in out:
        r = out["mamba2_core"]
        line["mamba2_layer_core"] = {
            "config": {"workload": "Mamba2 conv_ssm_forward, prefill of 8 seqs x 4096 tokens "
                                   "(H=32, head_dim=d_state=128, d_xb=1024, conv width 4, "
                                   "B/C norm, fp32 pool)"},
            "reference_call_sequence_ms": round(r["ms_ref"], 4),
            "hmx_serving_core_ms": round(r["ms_core"], 4),
            "tokens_per_s": round(r["tokens"] / (r["ms_core"] * 1e-3), 1),
        }
    if "gka" in out:
        line["gka"] = {}
        for n, r in out["gka"].items():
            line["gka"][f"num_iter_{n}"] = {
                "value": round(r["tokens_per_s"], 1), "unit": "tokens/s",
                "ms_per_step": round(r["ms"], 4),
                "config": {"workload": "C3 GKA prefill (gka_chebyshev_gla_prefill)", "B": 1,
                           "T": 32768, "H": 32, "d": 128, "num_iter": n, "ridge_ratio": 0.01},
                "roofline": {"bound": "mfma", "achieved": round(r["TFLOPs"], 1),
                             "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                             "frac": round(r["TFLOPs"] / BF16_PEAK_TFLOPS, 4),
                             "traffic": measured_traffic(f"gka_prefill_c3_n{n}"),
                             "mfma_busy_counter": measured_mfma_busy(f"gka_prefill_c3_n{n}"),
                             "algorithmic_flops": r["flops"],
                             "hbm_GBps": round(r["GBps"], 1)},
            }
    if "gdn_train" in out:
        r = out["gdn_train"]
        line["gdn_train"] = {
            "value": round(r["tokens_per_s"], 1), "unit": "tokens/s (forward + backward)",
            "ms_fwd": round(r["ms_fwd"], 4), "ms_fwd_bwd": round(r["ms_fwd_bwd"], 4),
            "ms_fwd_bwd_at_c1_shape": round(r["ms_c1_fwd_bwd"], 4),
            "ms_fwd_bwd_at_c1_shape_layer_gates": round(r["ms_c1_layer_gates_fwd_bwd"], 4),
            "config": {"workload": "F4 GDN training op (chunk_gated_delta_rule fwd + bwd)",
                       "B": 8, "T": 4096, "H": 32, "d": 128, "use_qk_l2norm_in_kernel": True},
            "roofline": {"bound": "mfma", "achieved": round(r["TFLOPs_fwd_bwd"], 1),
                         "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(r["TFLOPs_fwd_bwd"] / BF16_PEAK_TFLOPS, 4),
                         "algorithmic_flops_fwd": r["flops_fwd"],
                         "algorithmic_flops_bwd": r["flops_bwd"]},
        }
    if "ssd_train" in out:
        r = out["ssd_train"]
        line["ssd_train"] = {
            "value": round(r["tokens_per_s"], 1), "unit": "tokens/s (forward + backward)",
            "ms_fwd": round(r["ms_fwd"], 4), "ms_fwd_bwd": round(r["ms_fwd_bwd"], 4),
            "config": {"workload": "F4 Mamba2 training scan (mamba_chunk_scan_combined fwd + bwd)",
                       "B": 2, "T": 16384, "H": 64, "P": 64, "N": 128, "G": 8},
            "backward_TFLOPs": round(r["flops_bwd"] / ((r["ms_fwd_bwd"] - r["ms_fwd"]) * 1e-3)
                                     / 1e12, 1),
            "algorithmic_flops_bwd": r["flops_bwd"],
            "hybrid_layer_shape": {
                "config": {"B": 8, "T": 4096, "H": 32, "P": 128, "N": 128, "G": 32,
                           "note": "x and B repeated to the heads, headdim = d_state"},
                "ms_fwd": round(r["ms_fwd_hybrid"], 4),
                "ms_fwd_bwd": round(r["ms_fwd_bwd_hybrid"], 4),
                "tokens_per_s": round(8 * 4096 / (r["ms_fwd_bwd_hybrid"] * 1e-3), 1)},
        }
    if "gka_train" in out:
        r = out["gka_train"]
        line["gka_train"] = {
            "value": round(r["tokens_per_s"], 1), "unit": "tokens/s (forward + backward)",
            "ms_fwd": round(r["ms_fwd"], 4), "ms_fwd_bwd": round(r["ms_fwd_bwd"], 4),
            "gka_chebyshev_gla_ms_fwd_bwd": round(r["ms_gka_chebyshev_gla_fwd_bwd"], 4),
            "config": {"workload": "F4 GKA training solve (ChebyshevIteration fwd + bwd)",
                       "B": 8, "T": 4096, "H": 32, "d": 128, "num_iter": 8, "ridge_ratio": 0.02,
                       "bp_lambda": True},
            "roofline": {"bound": "mfma", "achieved": round(r["TFLOPs_fwd_bwd"], 1),
                         "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(r["TFLOPs_fwd_bwd"] / BF16_PEAK_TFLOPS, 4),
                         "forward_TFLOPs": round(r["TFLOPs_fwd"], 1),
                         "algorithmic_flops_fwd": r["flops_fwd"],
                         "algorithmic_flops_bwd": r["flops_bwd"]},
        }
    if "ssd" in out:
        r = out["ssd"]
        line["ssd"] = {
            "value": round(r["tokens_per_s"], 1), "unit": "tokens/s", "ms_per_step": round(r["ms"], 4),
            "config": {"workload": "C4 Mamba2 SSD chunk scan (mamba_chunk_scan_combined)", "B": 2,
                       "T": 16384, "H": 64, "P": 64, "N": 128, "G": 8, "chunk": 256},
            "roofline": {"bound": "hbm", "achieved": round(r["GBps"], 1), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(r["GBps"] / HBM_PEAK_GBS, 4),
                         "traffic": measured_traffic("ssd_c4"), "algorithmic_bytes": r["bytes"],
                         "mfma_TFLOPs": round(r["TFLOPs"], 1),
                         "mfma_frac": round(r["TFLOPs"] / BF16_PEAK_TFLOPS, 4),
                         "mfma_busy_counter": measured_mfma_busy("ssd_c4")},
        }
    if "ssd_primed" in out:
        r = out["ssd_primed"]
        line["ssd_primed"] = {
            "value": round(r["tokens_per_s"], 1), "unit": "tokens/s", "ms_per_step": round(r["ms"], 4),
            "config": {"workload": "Mamba2 SSD scan, primed layout (secondary shape)", "B": 2,
                       "T": 16384, "H": 64, "P": 128, "N": 128, "G": 64},
            "roofline": {"bound": "hbm", "achieved": round(r["GBps"], 1), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(r["GBps"] / HBM_PEAK_GBS, 4),
                         "algorithmic_bytes": r["bytes"], "traffic": measured_traffic("ssd_primed")},
        }
    if "ssd_decode" in out:
        r = out["ssd_decode"]
        line["ssd_decode"] = {
            "value": round(r["steps_per_s"], 1), "unit": "steps/s", "ms_per_step": round(r["ms"], 4),
            "config": {"workload": "Mamba2 selective_state_update, 256 seqs x 1 token",
                       "H": 64, "P": 64, "N": 128, "G": 8, "pool": "fp32 [256,64,64,128]"},
            "roofline": {"bound": "hbm", "achieved": round(r["GBps"], 1), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(r["GBps"] / HBM_PEAK_GBS, 4),
                         "traffic": measured_traffic("ssd_decode"),
                         "algorithmic_bytes": r["bytes"]},
        }
    if "gka_decode" in out:
        r = out["gka_decode"]
        line["gka_decode"] = {
            "value": round(r["steps_per_s"], 1), "unit": "steps/s", "ms_per_step": round(r["ms"], 4),
            "config": {"workload": "GKA decode (gka_chebyshev_gla_decode), 256 seqs x 1 token",
                       "H": 32, "d": 128, "num_iter": 8, "pools": "fp32 h_kk, h_kv [256,32,128,128]"},
            "roofline": {"bound": "hbm", "achieved": round(r["GBps"], 1), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(r["GBps"] / HBM_PEAK_GBS, 4),
                         "traffic": measured_traffic("gka_decode"), "algorithmic_bytes": r["bytes"]},
        }
    if not a.no_cpu:
        line["cpu_baseline"] = cpu_baseline()
        if a.only is None:
            line["cpu_baselines_more"] = cpu_baselines_more()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
