"""Gated delta rule (GDN) ops — the reference's Python signatures over libhmx.

Entry points (reference paths relative to the reference repository root):

- ``fused_gdn_gating``  — vllm-inference/src/primed_vllm/gdn/ops/fused_gdn_gating.py:79-125
- ``fused_recurrent_gated_delta_rule_gqa`` — .../gdn/ops/fused_recurrent_gqa.py:227-277
- ``chunk_gated_delta_rule_gqa`` — .../gdn/ops/chunk_gqa.py:15-83
- fla-style training names ``chunk_gated_delta_rule`` / ``fused_recurrent_gated_delta_rule``
  (called at training/src/hmf/model/hybrid_zoo/layers/gated_deltanet/gdn.py:462-489):
  the GQA entries with HKV == H.

Every op validates on the host with the reference's exception types, allocates
its outputs through torch's caching allocator, and launches on torch's current
stream.  There is no CPU fallback.
"""
from __future__ import annotations

import collections

import numpy as np
import torch

from .. import _lib
from .gates import ProjGates


def _i32(t: torch.Tensor | None) -> torch.Tensor | None:
    if t is None:
        return None
    if t.dtype != torch.int32:
        t = t.to(torch.int32)
    return t.contiguous()


def _token_rows(t: torch.Tensor, mult: int) -> tuple[torch.Tensor, int]:
    """(t, token stride) for a [B, T, heads, dim] tensor whose B*T tokens sit at one
    stride with each token's heads contiguous -- the column slices of a fused
    projection, as the layers pass q/k/v -- so the kernels read it in place; a
    contiguous copy otherwise.  The stride must be a multiple of ``mult`` elements
    and the base 16-byte aligned."""
    B, T, Hh, Dd = t.shape
    if B * T <= 1:
        ts = Hh * Dd          # one token: the stride is never used
    else:
        ts = t.stride(1) if T > 1 else t.stride(0)
    ok = (t.stride(-1) == 1 and (t.stride(2) == Dd or Hh == 1) and ts % mult == 0
          and ts >= Hh * Dd and (B == 1 or t.stride(0) == T * ts) and t.data_ptr() % 16 == 0)
    if not ok:
        t = t.contiguous()
        ts = Hh * Dd
    return t, ts


def fused_gdn_gating(A_log: torch.Tensor, a: torch.Tensor, b: torch.Tensor,
                     dt_bias: torch.Tensor, beta: float = 1.0,
                     threshold: float = 20.0) -> tuple[torch.Tensor, torch.Tensor]:
    """g = -exp(A_log) * softplus(a + dt_bias), beta = sigmoid(b).

    a, b: [num_tokens, num_heads], any strides.  Returns (g, beta), each
    [1, num_tokens, num_heads] in ``a.dtype`` (fused_gdn_gating.py:79-125).
    """
    _lib.require_gpu(A_log, a, b, dt_bias)
    num_tokens, num_heads = a.shape
    if b.shape != a.shape:
        raise ValueError(f"a {tuple(a.shape)} and b {tuple(b.shape)} must match")
    g = torch.empty(num_tokens, num_heads, dtype=a.dtype, device=a.device)
    beta_out = torch.empty(num_tokens, num_heads, dtype=a.dtype, device=a.device)
    _lib.call("hmx_gdn_gating",
              _lib.ptr(A_log), _lib.dtype_code(A_log),
              _lib.ptr(a), a.stride(0), a.stride(1),
              _lib.ptr(b), b.stride(0), b.stride(1), _lib.dtype_code(a),
              _lib.ptr(dt_bias), _lib.dtype_code(dt_bias),
              _lib.ptr(g), _lib.ptr(beta_out), _lib.dtype_code(g),
              num_tokens, num_heads, float(beta), float(threshold), _lib.stream_of(a))
    return g.unsqueeze(0), beta_out.unsqueeze(0)


def fused_recurrent_gated_delta_rule_gqa(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    g: torch.Tensor,
    beta: torch.Tensor | None = None,
    scale: float | None = None,
    initial_state: torch.Tensor | None = None,
    inplace_final_state: bool = True,
    cu_seqlens: torch.Tensor | None = None,
    ssm_state_indices: torch.Tensor | None = None,
    num_accepted_tokens: torch.Tensor | None = None,
    use_qk_l2norm_in_kernel: bool = False,
    *,
    o_norm_weight: torch.Tensor | None = None,
    o_norm_gate: torch.Tensor | None = None,
    o_norm_eps: float = 1e-5,
    out: torch.Tensor | None = None,
    gates: ProjGates | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """GQA-native fused recurrent gated delta rule (decode).

    q [B,T,H,K]; k [B,T,HKV,K]; v [B,T,HKV,V]; g [B,T,H]; beta [B,T,H] or
    [B,T,H,V].  With ``inplace_final_state`` the state pool ``initial_state``
    [slots,H,K,V] is updated in place at ``ssm_state_indices`` and returned;
    otherwise a new [B,T,H,K,V] tensor holds sequence n's final state in flat
    row bos_n (its first token's row over B*T, as fused_recurrent_gqa.py:137-139
    stores it); the other rows are left unwritten.  Returns (o [B,T,H,V],
    final_state)  (fused_recurrent_gqa.py:227-277).

    Keyword-only extension (no reference counterpart): ``o_norm_weight`` [V] (and
    optionally ``o_norm_gate`` [B,T,H,V], q.dtype) returns the layer's gated
    RMSNorm ``o_norm(o, z)`` (primed_gdn_layer.py:621-626) instead of o, fused into
    the kernel's output for V <= 128 (a separate hmx.rms_norm_gated call otherwise).
    ``out`` [B,T,H,V] (q.dtype, contiguous) receives o when given.  ``gates``
    (hmx.ProjGates) forms g and beta in the kernel from the layer's raw
    projections, in place of the gate tensors (g and beta are then ignored).
    """
    if cu_seqlens is not None and q.shape[0] != 1:
        raise ValueError(f"Batch size expected to be 1 with cu_seqlens, got {q.shape[0]}")
    if scale is None:
        scale = k.shape[-1] ** -0.5
    if gates is not None:
        gates.check(q.shape[0] * q.shape[1], q.shape[2], gka=False)
        g = beta = None
    elif beta is None:
        beta = torch.ones_like(g)
    _lib.require_gpu(q, k, v, g, beta, initial_state, cu_seqlens, ssm_state_indices,
                     num_accepted_tokens)
    if gates is None:
        g, beta = g.contiguous(), beta.contiguous()
    (q, q_ts), (k, k_ts), (v, v_ts) = (_token_rows(x, 4) for x in (q, k, v))
    if not (q.dtype == k.dtype == v.dtype):
        raise AssertionError("q, k, v must share a dtype")
    B, T, H, K = q.shape
    HKV, V = k.shape[2], v.shape[-1]
    if k.shape != (B, T, HKV, K) or v.shape[:3] != (B, T, HKV) or H % HKV != 0:
        raise ValueError(f"bad GQA shapes q{tuple(q.shape)} k{tuple(k.shape)} v{tuple(v.shape)}")
    N = B if cu_seqlens is None else len(cu_seqlens) - 1
    beta_headwise = beta is not None and beta.dim() == q.dim()
    if inplace_final_state:
        if initial_state is None or ssm_state_indices is None:
            raise ValueError("inplace_final_state=True needs initial_state (the state pool) "
                             "and ssm_state_indices")
        final_state = initial_state
    else:
        sdt = torch.float32 if initial_state is None else initial_state.dtype
        final_state = q.new_empty(B, T, H, K, V, dtype=sdt)
    if initial_state is not None:
        if tuple(initial_state.shape[1:]) != (H, K, V) or not initial_state[0].is_contiguous():
            raise ValueError(f"initial_state must be [rows,{H},{K},{V}] with contiguous rows, "
                             f"got {tuple(initial_state.shape)}")
        if initial_state.dtype != final_state.dtype:
            raise AssertionError("state dtypes differ")
    idx = _i32(ssm_state_indices)
    idx_stride = 0 if idx is None else idx.stride(0)
    if out is not None:
        _lib.require_gpu(out)
        if (tuple(out.shape) != (B, T, H, V) or out.dtype != q.dtype or not out.is_contiguous()
                or out.data_ptr() % 16):
            raise ValueError(f"out must be a contiguous [{B},{T},{H},{V}] {q.dtype} tensor")
        o = out
    else:
        o = q.new_empty(B, T, H, V)
    state_dt = _lib.dtype_code(final_state)
    onorm, norm_after = None, False
    if o_norm_weight is not None:
        _lib.require_gpu(o_norm_weight, o_norm_gate)
        z = None if o_norm_gate is None else _gate_rows(o_norm_gate, (B, T, H, V), q.dtype)
        if V <= 128:
            onorm = _lib.gated_norm(z, o_norm_weight, o_norm_eps, V)
        else:
            norm_after = True
    elif o_norm_gate is not None:
        raise ValueError("o_norm_gate needs o_norm_weight")
    _lib.call("hmx_gdn_recurrent_fwd",
              _lib.ptr(q), q_ts, _lib.ptr(k), k_ts, _lib.ptr(v), v_ts, _lib.dtype_code(q),
              _lib.ptr(g), 0 if g is None else _lib.dtype_code(g),
              _lib.ptr(beta), 0 if beta is None else _lib.dtype_code(beta), int(beta_headwise),
              _lib.ptr(o),
              _lib.ptr(initial_state), 0 if initial_state is None else initial_state.stride(0),
              _lib.ptr(final_state), final_state.stride(0) if inplace_final_state else H * K * V,
              state_dt,
              _lib.ptr(_i32(cu_seqlens)), _lib.ptr(idx), idx_stride,
              _lib.ptr(_i32(num_accepted_tokens)),
              B, T, N, H, HKV, K, V, float(scale), int(bool(use_qk_l2norm_in_kernel)),
              int(bool(inplace_final_state)), onorm, _lib.gate_proj(gates), _lib.stream_of(q))
    if norm_after:
        from .norm import rms_norm_gated
        normed = rms_norm_gated(o, o_norm_gate, o_norm_weight, eps=o_norm_eps)
        if out is None:
            o = normed
        else:
            o.copy_(normed)
    return o, final_state


def fused_recurrent_gated_delta_rule(q, k, v, g, beta=None, scale=None, initial_state=None,
                                     output_final_state=False, cu_seqlens=None,
                                     use_qk_l2norm_in_kernel=False):
    """fla-style decode entry (training/src/hmf/.../gated_deltanet/gdn.py:478-489).

    k, v already carry H heads.  ``initial_state`` [N,H,K,V] is read, never
    written; returns (o, final_state [N,H,K,V] fp32 or None).
    """
    B, T, H, K = q.shape
    V = v.shape[-1]
    N = B if cu_seqlens is None else len(cu_seqlens) - 1
    if cu_seqlens is not None and B != 1:
        raise ValueError(f"Batch size expected to be 1 with cu_seqlens, got {B}")
    if initial_state is None:
        pool = torch.zeros(N, H, K, V, dtype=torch.float32, device=q.device)
    else:
        pool = initial_state.to(torch.float32).clone()
    idx = torch.arange(N, dtype=torch.int32, device=q.device)
    if cu_seqlens is None:
        cu_seqlens = torch.arange(0, (B + 1) * T, T, dtype=torch.int32, device=q.device)[:B + 1]
        qf, kf, vf = (x.reshape(1, B * T, *x.shape[2:]) for x in (q, k, v))
        gf = g.reshape(1, B * T, H)
        bf = None if beta is None else beta.reshape(1, B * T, *beta.shape[2:])
    else:
        qf, kf, vf, gf, bf = q, k, v, g, beta
    o, _ = fused_recurrent_gated_delta_rule_gqa(
        qf, kf, vf, gf, bf, scale, pool, True, cu_seqlens, idx, None, use_qk_l2norm_in_kernel)
    return o.reshape(B, T, H, V), (pool if output_final_state else None)


# Segmented chunk-scan planning.  A segment is a run of CHUNK-token chunks of one
# sequence that one workgroup walks serially; more segments give more parallelism
# at the cost of a short warm-up (or the exact scan) per segment boundary.  The
# segment table comes from the library's host planner (hmx_plan_segments_bounds).
CHUNK = 32               # the kernel's chunk length
MAX_WARM_CHUNKS = 16
# A warm-up start drops history bounded by exp(-20) ~ 2e-9 of the state's norm at
# the warm-up start: below fp32 rounding, and far below the fp16 operand rounding
DECAY_THRESHOLD = 20.0
_CU_COUNT: dict[int, int] = {}


def _cu_count(device: torch.device) -> int:
    idx = device.index if device.index is not None else torch.cuda.current_device()
    if idx not in _CU_COUNT:
        _CU_COUNT[idx] = torch.cuda.get_device_properties(idx).multi_processor_count
    return _CU_COUNT[idx]


_SEG_CACHE: "collections.OrderedDict[tuple, torch.Tensor]" = collections.OrderedDict()
_SEG_CACHE_SIZE = 64


def seq_bounds(cu_seqlens: torch.Tensor | None, B: int, T: int) -> list[tuple[int, int]]:
    """(bos, eos) of every sequence over the B*T flattened tokens: the B rows, or the
    cu_seqlens runs (B == 1).  Rejects cu_seqlens that do not start at 0, decrease,
    or end past the tokens (ValueError), so no kernel reads or writes past them.
    The kernels never read cu_seqlens itself: a host (CPU) tensor, such as vLLM's
    query_start_loc_cpu, plans the call without a device-to-host copy; a device
    tensor is read back once here."""
    if cu_seqlens is None:
        return [(n * T, n * T + T) for n in range(B)]
    cs = [int(x) for x in cu_seqlens.tolist()]
    bounds = [(cs[n], cs[n + 1]) for n in range(len(cs) - 1)]
    if not cs or cs[0] != 0 or cs[-1] > B * T or any(b < a for a, b in bounds):
        raise ValueError(f"cu_seqlens must be non-decreasing from 0 to <= {B * T}: {cs}")
    return bounds


def _device_table(rows, device) -> torch.Tensor:
    """An int32 host table (segment rows) as a device tensor, without blocking the host.

    A copy from pageable memory waits for the stream to drain, which leaves the
    GPU idle for the host's per-call work; the table is therefore staged in
    pinned memory (the copy is then asynchronous), and the device copies of the
    last few distinct tables are kept, so a repeated batch shape uploads nothing.
    Kernels only read the table."""
    arr = np.ascontiguousarray(np.asarray(rows, dtype=np.int32))
    key = (str(device), arr.shape, arr.tobytes())
    t = _SEG_CACHE.get(key)
    if t is not None:
        _SEG_CACHE.move_to_end(key)
        return t
    host = torch.from_numpy(arr.copy()).pin_memory()
    t = host.to(device, non_blocking=True)
    _SEG_CACHE[key] = t
    if len(_SEG_CACHE) > _SEG_CACHE_SIZE:
        _SEG_CACHE.popitem(last=False)
    return t


def _segment_table(op: int, bounds: list[tuple[int, int]], tokens: int, H: int,
                   device: torch.device, segment_chunks: int | None = None):
    """The segment table (int32 [rows, 8]: n, bos, eos, c_start, c_end, seg_idx,
    first_seg, nseg) and the total chunk count for prefill ``op`` on ``device``,
    from the library's host planner.  With ``segment_chunks`` every sequence is cut
    into equal segments of at most that many chunks (tests)."""
    return _lib.plan_segments(op, bounds, tokens, H, _cu_count(device), segment_chunks)


def chunk_gated_delta_rule_gqa(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    g: torch.Tensor,
    beta: torch.Tensor,
    scale: float | None = None,
    initial_state: torch.Tensor | None = None,
    output_final_state: bool = False,
    cu_seqlens: torch.Tensor | None = None,
    use_qk_l2norm_in_kernel: bool = False,
    *,
    o_norm_weight: torch.Tensor | None = None,
    o_norm_gate: torch.Tensor | None = None,
    o_norm_eps: float = 1e-5,
    ssm_state_indices: torch.Tensor | None = None,
    has_initial_state: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
    gates: ProjGates | None = None,
    _segment_chunks: int | None = None,
) -> tuple[torch.Tensor, torch.Tensor | None]:
    """GQA-native chunked gated delta rule (prefill).

    q [B,T,H,K]; k, v [B,T,HKV,K|V] (bf16; k/v NOT expanded); g, beta [B,T,H];
    initial_state [N,H,K,V]; cu_seqlens [N+1] with B == 1.  Returns
    (o [B,T,H,V] in q.dtype, final_state [N,H,K,V] fp32 or None)
    (chunk_gqa.py:15-83).  ``_segment_chunks`` overrides the parallel
    decomposition (tests); results do not depend on it beyond fp32 rounding.
    
    Keyword-only extensions (no reference counterpart):

    - ``o_norm_weight`` [V] (and optionally ``o_norm_gate`` [B,T,H,V], q.dtype)
      returns the layer's ``o_norm(o, z)`` (gated RMSNorm, norm before gate, eps
      ``o_norm_eps``; primed_gdn_layer.py:621-626) computed in the kernel's output
      epilogue instead of o.
    - ``ssm_state_indices`` [N]: ``initial_state`` is the layer's state pool
      [slots,H,K,V] (fp32 or bf16); sequence n starts from slot
      ``ssm_state_indices[n]`` and, with ``output_final_state``, its end state is
      written back into that slot in place; the pool is returned as the final
      state.  This replaces the layer's gather / zero / scatter around the op
      (primed_gdn_layer.py:868-879).  A negative slot starts from zero and writes
      nothing.
    - ``has_initial_state`` [N] bool: sequences with False start from zero.
    - ``out`` [B,T,H,V] (q.dtype, contiguous): o is written there.
    - ``gates`` (hmx.ProjGates): g and beta are formed in the kernel from the
      layer's raw projections (A_log, dt_bias, a, b) instead of the gate tensors,
      which are then ignored (fused_gdn_gating.py:79-125 and its launch fused away).

    q, k and v may be the column slices of one fused projection (token stride
    larger than heads x dim): they are read in place.
    """
    assert q.dtype == k.dtype == v.dtype
    assert q.dtype != torch.float32, "Does not support float32. Use bfloat16."
    if gates is not None:
        gates.check(q.shape[0] * q.shape[1], q.shape[2], gka=False)
        g = beta = None
    assert beta is None or len(beta.shape) == 3, "beta must be [B, T, H]"
    if cu_seqlens is not None and q.shape[0] != 1:
        raise ValueError(f"Batch size expected to be 1 with cu_seqlens, got {q.shape[0]}")
    if cu_seqlens is not None and initial_state is not None and ssm_state_indices is None:
        if initial_state.shape[0] != len(cu_seqlens) - 1:
            raise ValueError(f"Initial states count mismatch: {initial_state.shape[0]} vs "
                             f"{len(cu_seqlens) - 1}")
    if scale is None:
        scale = k.shape[-1] ** -0.5
    _lib.require_gpu(q, k, v, g, beta, initial_state)    # cu_seqlens: host or device
    B, T, H, K = q.shape
    HKV, V = k.shape[2], v.shape[-1]
    if k.shape != (B, T, HKV, K) or v.shape[:3] != (B, T, HKV) or H % HKV != 0:
        raise ValueError(f"bad GQA shapes q{tuple(q.shape)} k{tuple(k.shape)} v{tuple(v.shape)}")
    if gates is None and (g.shape != (B, T, H) or beta.shape != (B, T, H)):
        raise ValueError(f"g {tuple(g.shape)} and beta {tuple(beta.shape)} must be [B,T,H]")
    bounds = seq_bounds(cu_seqlens, B, T)
    N = len(bounds)
    _lib.require_gpu(ssm_state_indices, has_initial_state, out)
    idx = None
    if ssm_state_indices is not None:
        if initial_state is None:
            raise ValueError("ssm_state_indices needs initial_state (the state pool)")
        idx = _i32(ssm_state_indices)
        if idx.shape != (N,):
            raise ValueError(f"ssm_state_indices must hold {N} slots, got {tuple(idx.shape)}")
        pool = initial_state
        if (pool.dim() != 4 or tuple(pool.shape[1:]) != (H, K, V) or not pool[0].is_contiguous()
                or pool.dtype not in (torch.float32, torch.bfloat16)):
            raise ValueError(f"the state pool must be [slots,{H},{K},{V}] fp32/bf16 with "
                             f"contiguous slots, got {tuple(pool.shape)} {pool.dtype}")
        h0, ht = pool, (pool if output_final_state else None)
        st_ss, st_dt = pool.stride(0), _lib.dtype_code(pool)
    else:
        if initial_state is not None and tuple(initial_state.shape) != (N, H, K, V):
            raise ValueError(f"initial_state must be [{N},{H},{K},{V}], "
                             f"got {tuple(initial_state.shape)}")
        h0 = None if initial_state is None else initial_state.to(torch.float32).contiguous()
        ht = (torch.empty(N, H, K, V, dtype=torch.float32, device=q.device)
              if output_final_state else None)
        st_ss, st_dt = H * K * V, _lib.HMX_F32
    hinit = None
    if has_initial_state is not None:
        if has_initial_state.shape != (N,):
            raise ValueError(f"has_initial_state must be [{N}], got {tuple(has_initial_state.shape)}")
        hinit = has_initial_state.to(torch.uint8).contiguous()
    if gates is None:
        g, beta = g.contiguous(), beta.contiguous()
    (q, q_ts), (k, k_ts), (v, v_ts) = (_token_rows(x, 8) for x in (q, k, v))
    if k_ts != v_ts:    # the prefill kernels read k and v at one token stride
        (k, k_ts), (v, v_ts) = _token_rows(k.contiguous(), 8), _token_rows(v.contiguous(), 8)
    if out is not None:
        if (tuple(out.shape) != (B, T, H, V) or out.dtype != q.dtype or not out.is_contiguous()
                or out.data_ptr() % 16):
            raise ValueError(f"out must be a contiguous [{B},{T},{H},{V}] {q.dtype} tensor")
        o = out
    else:
        o = torch.empty(B, T, H, V, dtype=q.dtype, device=q.device)
    if cu_seqlens is not None and bounds and bounds[-1][1] < T:
        o[:, bounds[-1][1]:].zero_()  # tokens past the last sequence are not computed
    rows, _ = _segment_table(_lib.PLAN_GDN, bounds, B * T, H, q.device, _segment_chunks)
    seg = _device_table(rows, q.device)
    lib = _lib.load()
    ws_bytes = int(lib.hmx_gdn_chunk_workspace_bytes(len(rows), N, H, int(idx is not None)))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=q.device)
    onorm = None
    if o_norm_weight is not None:
        _lib.require_gpu(o_norm_weight, o_norm_gate)
        z = None if o_norm_gate is None else _gate_rows(o_norm_gate, (B, T, H, V), q.dtype)
        onorm = _lib.gated_norm(z, o_norm_weight, o_norm_eps, V)
    elif o_norm_gate is not None:
        raise ValueError("o_norm_gate needs o_norm_weight")
    _lib.call("hmx_gdn_chunk_fwd",
              _lib.ptr(q), q_ts, _lib.ptr(k), k_ts, _lib.ptr(v), v_ts, _lib.dtype_code(q),
              _lib.ptr(g), 0 if g is None else _lib.dtype_code(g),
              _lib.ptr(beta), 0 if beta is None else _lib.dtype_code(beta),
              _lib.ptr(o), _lib.ptr(h0), _lib.ptr(ht), st_ss, st_dt, _lib.ptr(idx),
              _lib.ptr(hinit), _lib.ptr(seg), len(rows), N, H, HKV, K, V, float(scale),
              int(bool(use_qk_l2norm_in_kernel)), MAX_WARM_CHUNKS, DECAY_THRESHOLD,
              _lib.ptr(ws), ws.numel(), onorm, _lib.gate_proj(gates), _lib.stream_of(q))
    return o, ht


def _gate_rows(z: torch.Tensor, shape: tuple, dtype: torch.dtype) -> torch.Tensor:
    """The output-norm gate as a [tokens, H, V] view with V contiguous and 16-byte
    aligned rows (copied only when no such view exists)."""
    if tuple(z.shape) != tuple(shape) or z.dtype != dtype:
        raise ValueError(f"o_norm_gate must be {tuple(shape)} {dtype}, got {tuple(z.shape)} {z.dtype}")
    zz = z.reshape(-1, shape[-2], shape[-1]) if z.dim() == 4 else z
    if (zz.stride(-1) != 1 or zz.stride(0) % 8 or zz.stride(1) % 8 or zz.data_ptr() % 16):
        zz = zz.contiguous()
    return zz


def chunk_gated_delta_rule(q, k, v, g, beta, scale=None, initial_state=None,
                           output_final_state=False, cu_seqlens=None,
                           use_qk_l2norm_in_kernel=False):
    """fla-style prefill entry (training/src/hmf/.../gated_deltanet/gdn.py:462-476):
    the GQA op with k, v already expanded to H heads.  Returns (o, final_state
    [N,H,K,V] fp32 or None).

    The training layer passes q, k, v in the model's dtype.  bf16/fp16 inputs run
    the chunked kernel; fp32 inputs (which the chunked kernel's bf16 MFMA products
    would round) run the fp32 recurrent kernel over the same tokens, so an fp32
    model gets fp32 arithmetic throughout.

    With autograd recording and an input that requires a gradient, bf16 inputs go
    through hmx.ChunkGatedDeltaRule (the same forward, with the chunked backward);
    fp32 inputs have no backward here and raise NotImplementedError."""
    ins = (q, k, v, g, beta, initial_state)
    if torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in ins):
        if q.dtype == torch.float32:
            raise NotImplementedError("hmx chunk_gated_delta_rule: the backward needs bfloat16 "
                                      "q, k, v")
        from .gdn_train import ChunkGatedDeltaRule
        return ChunkGatedDeltaRule.apply(q, k, v, g, beta, scale, initial_state,
                                         output_final_state, cu_seqlens,
                                         use_qk_l2norm_in_kernel, None)
    if q.dtype == torch.float32:
        return fused_recurrent_gated_delta_rule(q, k, v, g, beta, scale, initial_state,
                                                output_final_state, cu_seqlens,
                                                use_qk_l2norm_in_kernel)
    return chunk_gated_delta_rule_gqa(q, k, v, g, beta, scale, initial_state, output_final_state,
                                      cu_seqlens, use_qk_l2norm_in_kernel)
