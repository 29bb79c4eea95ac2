"""The chunked gated delta rule with its backward (training), over libhmx.

Entry point: ``ChunkGatedDeltaRule.apply(q, k, v, g, beta, scale, initial_state,
output_final_state, cu_seqlens, use_qk_l2norm_in_kernel, segment_chunks) ->
(o, final_state)``, the autograd function behind ``hmx.chunk_gated_delta_rule``
when a gradient is needed.  It stands for fla's ``chunk_gated_delta_rule`` as the
training layer calls it (training/src/hmf/model/hybrid_zoo/layers/gated_deltanet/
gdn.py:462-476: q, k, v [B,T,H,D] with k, v expanded to H heads, g [B,T,H] fp32,
beta [B,T,H], cu_seqlens with B == 1) and returns the gradients of q, k, v, g,
beta and initial_state, including the final state's gradient when it is used.

The forward is the serving prefill (hmx_gdn_chunk_fwd).  The backward
recomputes the state entering every 32-token block (hmx_gdn_train_fwd: the
same walk writing those states, fp16) instead of keeping them from the forward,
as fla's backward recomputes them, then runs hmx_gdn_train_bwd: the blocks' T and
masked Q K^T, the reverse chain of the state gradient (each sequence's blocks cut
into runs walked in parallel, a run that ends early starting after a warm-up
over the following blocks where the gates decay, as the forward's segments do),
and the per-block gradients.  bf16 q/k/v with head dim 128 only.
"""
from __future__ import annotations

import numpy as np
import torch

from .. import _lib
from .gdn import (CHUNK, DECAY_THRESHOLD, MAX_WARM_CHUNKS, _cu_count, _device_table,
                  _segment_table, chunk_gated_delta_rule_gqa, seq_bounds)


def block_table(bounds: list[tuple[int, int]]):
    """int32 rows (first token, tokens, sequence, block in sequence) of every
    CHUNK-token block, and cu_blocks [N+1]."""
    rows, cu = [], [0]
    for n, (bos, eos) in enumerate(bounds):
        for c, t0 in enumerate(range(bos, eos, CHUNK)):
            rows.append((t0, min(CHUNK, eos - t0), n, c))
        cu.append(len(rows))
    return np.asarray(rows, dtype=np.int32).reshape(-1, 4), np.asarray(cu, dtype=np.int32)


def chain_segments(cu_blocks: np.ndarray, H: int, cu_count: int, seg_blocks: int | None = None):
    """int32 rows (sequence, first block, end block): every sequence's blocks cut into
    runs of at most ``seg_blocks`` blocks (by default as long as gives about three
    workgroups per CU over all heads, as many as fit one), one (empty) row for a
    sequence without blocks."""
    total = int(cu_blocks[-1])
    if seg_blocks is None:
        seg_blocks = max(1, -(-total * H // (3 * cu_count)))
    rows = []
    for n in range(len(cu_blocks) - 1):
        a, e = int(cu_blocks[n]), int(cu_blocks[n + 1])
        if a == e:
            rows.append((n, a, e))
        for b in range(a, e, seg_blocks):
            rows.append((n, b, min(b + seg_blocks, e)))
    return np.asarray(rows, dtype=np.int32).reshape(-1, 3)


def check_chain_segments(cseg: np.ndarray, cu_blocks: np.ndarray) -> None:
    """Raise ValueError unless the chain-run rows are in the order hmx_gdn_train_bwd
    requires: grouped by ascending sequence 0..N-1, every sequence with at least one
    row, and each sequence's rows tiling its blocks [cu[n], cu[n+1]) in ascending
    order (an empty sequence has the one row (n, cu[n], cu[n]))."""
    cseg = np.asarray(cseg).reshape(-1, 3)
    N = len(cu_blocks) - 1
    n, a, e = cseg[:, 0].astype(np.int64), cseg[:, 1].astype(np.int64), cseg[:, 2].astype(np.int64)
    if len(n) < N or (len(n) and (n[0] != 0 or n[-1] != N - 1)) or np.any(np.diff(n) < 0) \
            or np.any(np.diff(n) > 1):
        raise ValueError("chain_segments: rows must be grouped by ascending sequence, "
                         "every sequence with at least one row")
    first = np.r_[True, n[1:] != n[:-1]]
    last = np.r_[n[1:] != n[:-1], True]
    cu = np.asarray(cu_blocks, dtype=np.int64)
    ok = (np.all(a[first] == cu[n[first]]) and np.all(e[last] == cu[n[last] + 1])
          and np.all(a[~first] == e[np.flatnonzero(~first) - 1]) and np.all(e >= a)
          and np.all((e > a) | (first & last)))
    if not ok:
        raise ValueError("chain_segments: each sequence's rows must tile its blocks in "
                         "ascending order")


def _check(q, k, v, g, beta):
    if q.dim() != 4 or k.shape != q.shape or v.shape != q.shape:
        raise ValueError(f"q, k, v must be [B, T, H, D] alike (k, v expanded to H heads), got "
                         f"{tuple(q.shape)}, {tuple(k.shape)}, {tuple(v.shape)}")
    if not (q.dtype == k.dtype == v.dtype == torch.bfloat16):
        raise NotImplementedError(f"hmx chunk_gated_delta_rule backward: q, k, v must be "
                                  f"bfloat16, got {q.dtype}")
    if q.shape[-1] != 128:
        raise NotImplementedError(f"hmx chunk_gated_delta_rule backward: head dim must be 128, "
                                  f"got {q.shape[-1]}")
    if tuple(g.shape) != tuple(q.shape[:3]) or tuple(beta.shape) != tuple(q.shape[:3]):
        raise ValueError(f"g {tuple(g.shape)} and beta {tuple(beta.shape)} must be "
                         f"[B, T, H] = {tuple(q.shape[:3])}")
    _lib.require_gpu(q, k, v, g, beta)


def _rows(x):
    """x [B,T,H,D] with unit element and head strides: (x, token stride)."""
    if x.stride(-1) != 1 or x.stride(-2) != x.shape[-1] or x.stride(0) != x.shape[1] * x.stride(1):
        x = x.contiguous()
    return x, x.stride(1)


def block_states(q, k, v, g, beta, scale, h0, bounds, l2norm, segment_chunks=None):
    """The state entering every block, fp16 [nblk, H, D, D], and the block table
    (host rows, device table, device cu_blocks, host cu_blocks)."""
    B, T, H, D = q.shape
    N = len(bounds)
    rows_np, cu_np = block_table(bounds)
    nblk = rows_np.shape[0]
    hc = torch.empty(max(nblk, 1), H, D, D, dtype=torch.float16, device=q.device)
    cu_dev = _device_table(cu_np, q.device)
    seg_rows, _ = _segment_table(_lib.PLAN_GDN, bounds, B * T, H, q.device, segment_chunks)
    if nblk == 0:
        return hc, rows_np, _device_table(np.zeros((1, 4), np.int32), q.device), cu_dev, cu_np
    seg = _device_table(seg_rows, q.device)
    lib = _lib.load()
    ws_bytes = int(lib.hmx_gdn_chunk_workspace_bytes(len(seg_rows), N, H, 0))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=q.device)
    o = torch.empty(B, T, H, D, dtype=q.dtype, device=q.device)
    (q, q_ts), (k, kv_ts), (v, v_ts) = _rows(q), _rows(k), _rows(v)
    if v_ts != kv_ts:
        raise ValueError("k and v must share a token stride")
    _lib.call("hmx_gdn_train_fwd",
              _lib.ptr(q), q_ts, _lib.ptr(k), _lib.ptr(v), kv_ts,
              _lib.ptr(g), _lib.dtype_code(g), _lib.ptr(beta), _lib.dtype_code(beta),
              _lib.ptr(o), _lib.ptr(h0), None, _lib.ptr(seg), len(seg_rows), N, H, float(scale),
              int(bool(l2norm)), MAX_WARM_CHUNKS, DECAY_THRESHOLD, _lib.ptr(ws), ws.numel(),
              _lib.ptr(hc), _lib.ptr(cu_dev), _lib.stream_of(q))
    return hc, rows_np, _device_table(rows_np, q.device), cu_dev, cu_np


def chunk_backward(q, k, v, g, beta, scale, h0, do, dht, bounds, l2norm, segment_chunks=None,
                   want_dh0=False):
    """(dq, dk, dv bf16, dg, dbeta, dh0 or None fp32) of the chunked gated delta rule.
    ``segment_chunks`` (tests) bounds both the recomputing forward's segments and the
    state-gradient chain's runs, in 32-token blocks."""
    B, T, H, D = q.shape
    N = len(bounds)
    g, beta = g.contiguous(), beta.contiguous()
    hc, rows_np, tab, cu_dev, cu_np = block_states(q, k, v, g, beta, scale, h0, bounds, l2norm,
                                                   segment_chunks)
    nblk = rows_np.shape[0]
    cseg_np = chain_segments(cu_np, H, _cu_count(q.device), segment_chunks)
    check_chain_segments(cseg_np, cu_np)
    cseg = _device_table(cseg_np, q.device)
    covered = sum(e - b for b, e in bounds) == B * T
    alloc = torch.empty if covered else torch.zeros
    dq, dk, dv = (alloc(B, T, H, D, dtype=torch.bfloat16, device=q.device) for _ in range(3))
    dg = alloc(B, T, H, dtype=torch.float32, device=q.device)
    dbeta = alloc(B, T, H, dtype=torch.float32, device=q.device)
    dh0 = torch.empty(N, H, D, D, dtype=torch.float32, device=q.device) if want_dh0 else None
    if dht is not None:
        dht = dht.to(torch.float32).contiguous()
    lib = _lib.load()
    ws = torch.empty(max(int(lib.hmx_gdn_train_bwd_workspace_bytes(nblk, cseg_np.shape[0], N, H)),
                         16),
                     dtype=torch.uint8, device=q.device)
    (q, q_ts), (k, kv_ts), (v, _), (do, do_ts) = _rows(q), _rows(k), _rows(v), _rows(do)
    _lib.call("hmx_gdn_train_bwd",
              _lib.ptr(q), q_ts, _lib.ptr(k), _lib.ptr(v), kv_ts,
              _lib.ptr(g), _lib.dtype_code(g), _lib.ptr(beta), _lib.dtype_code(beta),
              _lib.ptr(do), do_ts, _lib.ptr(dht), _lib.ptr(hc), _lib.ptr(tab), _lib.ptr(cu_dev),
              nblk, N, _lib.ptr(cseg), cseg_np.shape[0], MAX_WARM_CHUNKS, DECAY_THRESHOLD, H,
              float(scale), int(bool(l2norm)),
              _lib.ptr(dq), _lib.ptr(dk), _lib.ptr(dv), _lib.ptr(dg), _lib.ptr(dbeta),
              _lib.ptr(dh0), _lib.ptr(ws), ws.numel(), _lib.stream_of(q))
    return dq, dk, dv, dg, dbeta, dh0


class ChunkGatedDeltaRule(torch.autograd.Function):
    """fla's chunk_gated_delta_rule with its backward (see module doc)."""

    @staticmethod
    def forward(ctx, q, k, v, g, beta, scale=None, initial_state=None, output_final_state=False,
                cu_seqlens=None, use_qk_l2norm_in_kernel=False, segment_chunks=None):
        _check(q, k, v, g, beta)
        if scale is None:
            scale = q.shape[-1] ** -0.5
        B, T, H, D = q.shape
        if cu_seqlens is not None and B != 1:
            raise ValueError(f"Batch size expected to be 1 with cu_seqlens, got {B}")
        bounds = seq_bounds(cu_seqlens, B, T)
        h0 = None
        if initial_state is not None:
            if tuple(initial_state.shape) != (len(bounds), H, D, D):
                raise ValueError(f"initial_state must be [{len(bounds)},{H},{D},{D}], got "
                                 f"{tuple(initial_state.shape)}")
            h0 = initial_state.to(torch.float32).contiguous()
        o, ht = chunk_gated_delta_rule_gqa(q, k, v, g, beta, scale, h0, output_final_state,
                                           cu_seqlens, use_qk_l2norm_in_kernel,
                                           _segment_chunks=segment_chunks)
        ctx.save_for_backward(q, k, v, g, beta, h0)
        ctx.scale, ctx.bounds, ctx.l2 = scale, bounds, use_qk_l2norm_in_kernel
        ctx.seg, ctx.has_h0 = segment_chunks, initial_state is not None
        ctx.dt = (g.dtype, beta.dtype, None if initial_state is None else initial_state.dtype)
        ctx.set_materialize_grads(False)
        return o, ht

    @staticmethod
    def backward(ctx, do, dht):
        q, k, v, g, beta, h0 = ctx.saved_tensors
        if do is None:
            do = torch.zeros_like(q)
        want_dh0 = ctx.has_h0 and ctx.needs_input_grad[6]
        dq, dk, dv, dg, dbeta, dh0 = chunk_backward(
            q, k, v, g, beta, ctx.scale, h0, do.to(torch.bfloat16), dht, ctx.bounds, ctx.l2,
            ctx.seg, want_dh0)
        gdt, bdt, sdt = ctx.dt
        return (dq, dk, dv, dg.to(gdt), dbeta.to(bdt), None,
                dh0.to(sdt) if dh0 is not None else None, None, None, None, None)
