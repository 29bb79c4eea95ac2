"""Gated KalmaNet (GKA) ops — the reference's Python signatures over libhmx.

Entry points (reference paths relative to the reference repository root):

- ``fused_gka_gating`` — vllm-inference/src/primed_vllm/primed_gka_layer.py:303-358
- ``chebyshev_iteration_gqa`` — .../gka/ops/chebyshev_iteration_gqa.py:173-238
- ``gka_chebyshev_gla_decode`` — .../gka/gka_forward.py:248-326
- ``gka_chebyshev_gla_prefill`` — .../gka/gka_forward.py:161-242

Differences from the reference, by design: q and k are L2-normalised inside the
kernels instead of in place on the caller's tensors (gka_forward.py:149-159
mutates them); the results are the same.
"""
from __future__ import annotations

import logging

import torch

from .. import _lib
from .gates import ProjGates
from .gdn import (_cu_count, _device_table, _gate_rows, _i32, _segment_table, _token_rows,
                  seq_bounds)

GKA_BLOCK = 64              # tokens per block: the solve kernel's unit and the planner's chunk
_warned_num_iter_zero = False


def _check_sketching_constraints(gka, num_sketches_per_head, func_name):
    """Sketching is unsupported, as in gka_forward.py:23-34."""
    if gka is not None:
        raise NotImplementedError(
            f"{func_name}: gka projection is not supported. Set parallel_latent_sketch=False in config. ")
    if num_sketches_per_head != 1:
        raise NotImplementedError(
            f"{func_name}: num_sketches_per_head={num_sketches_per_head} is not supported. "
            "Must be 1 due to numerical instability in gating kernel. ")


def fused_gka_gating(A_log: torch.Tensor, a: torch.Tensor, alpha_in: torch.Tensor,
                     b: torch.Tensor | None, dt_bias: torch.Tensor, beta: float = 1.0,
                     threshold: float = 20.0):
    """g = -exp(A_log) softplus(a + dt_bias), alpha = sigmoid(alpha_in), beta = sigmoid(b).

    Returns (g, alpha, beta or None), each [1, num_tokens, num_heads] in a.dtype
    (primed_gka_layer.py:303-358).
    """
    _lib.require_gpu(A_log, a, alpha_in, b, dt_bias)
    num_tokens, num_heads = a.shape
    g = torch.empty(num_tokens, num_heads, dtype=a.dtype, device=a.device)
    alpha = torch.empty_like(g)
    beta_out = torch.empty_like(g) if b is not None else None
    if alpha_in.dtype != a.dtype or (b is not None and b.dtype != a.dtype):
        raise ValueError("a, alpha_in and b must share a dtype")
    _lib.call("hmx_gka_gating",
              _lib.ptr(A_log), _lib.dtype_code(A_log),
              _lib.ptr(a), a.stride(0), a.stride(1),
              _lib.ptr(alpha_in), alpha_in.stride(0), alpha_in.stride(1),
              _lib.ptr(b), 0 if b is None else b.stride(0), 0 if b is None else b.stride(1),
              _lib.dtype_code(a), _lib.ptr(dt_bias), _lib.dtype_code(dt_bias),
              _lib.ptr(g), _lib.ptr(alpha), _lib.ptr(beta_out), _lib.dtype_code(g),
              num_tokens, num_heads, float(beta), float(threshold), _lib.stream_of(a))
    return (g.unsqueeze(0), alpha.unsqueeze(0),
            beta_out.unsqueeze(0) if beta_out is not None else None)


def chebyshev_iteration_gqa(k, q, v, alpha, gk=None, beta=None, num_iter: int = 15,
                            scale: float | None = None, ridge_ratio: float = 0.1,
                            initial_state_kk=None, initial_state_kv=None,
                            output_final_state: bool = True, inplace_final_state: bool = True,
                            cu_seqlens=None, ssm_state_indices=None, *,
                            o_norm_weight=None, o_norm_gate=None, o_norm_eps: float = 1e-6,
                            out=None, gates: ProjGates | None = None):
    """Fused GKA decode step (chebyshev_iteration_gqa.py:173-238).

    k [B,T,HKV,D]; q [B,T,H,D]; v [B,T,HKV,V]; alpha, gk, beta [B,T,H].
    States [N,H,D,D] / [N,H,D,V] (slot pools with ssm_state_indices), updated in
    place when ``inplace_final_state``.  Only the first token of each sequence
    is processed.  Returns (o, h_kk_out, h_kv_out).

    Keyword-only extension (no reference counterpart): ``o_norm_weight`` [V] (and
    optionally ``o_norm_gate`` [B,T,H,V], q.dtype) returns the layer's gated
    RMSNorm ``o_norm(o, z)`` (primed_gka_layer.py:944-949) fused into the kernel's
    output instead of o; ``out`` [B,T,H,V] (q.dtype, contiguous) receives o;
    ``gates`` (hmx.ProjGates) forms alpha, gk and beta in the kernel from the
    layer's raw projections (the gate tensors are then ignored).
    """
    if gates is not None:
        gates.check(q.shape[0] * q.shape[1], q.shape[2], gka=True)
        alpha = gk = beta = None
    if cu_seqlens is not None and q.shape[0] != 1:
        raise ValueError(f"Batch size must be 1 when using cu_seqlens, got {q.shape[0]}.")
    B, T, H, D = q.shape
    HKV, V = k.shape[2], v.shape[-1]
    N = B if cu_seqlens is None else len(cu_seqlens) - 1
    if scale is None:
        scale = D ** -0.5
    if initial_state_kk is None:
        initial_state_kk = q.new_zeros(N, H, D, D, dtype=torch.float32)
    if initial_state_kv is None:
        initial_state_kv = q.new_zeros(N, H, D, V, dtype=torch.float32)
    _lib.require_gpu(q, k, v, alpha, gk, beta, initial_state_kk, initial_state_kv, cu_seqlens,
                     ssm_state_indices)
    if initial_state_kk.dtype != torch.float32:
        raise NotImplementedError("h_kk state must be float32 (primed_gka_layer.py:424-430)")
    for st, last in ((initial_state_kk, D), (initial_state_kv, V)):
        if tuple(st.shape[1:]) != (H, D, last) or not st[0].is_contiguous():
            raise ValueError(f"state must be [rows,{H},{D},{last}] with contiguous rows, "
                             f"got {tuple(st.shape)}")
    alpha = None if alpha is None else alpha.contiguous()
    (q, q_ts), (k, k_ts), (v, v_ts) = (_token_rows(x, 4) for x in (q, k, v))
    gk = None if gk is None else gk.contiguous()
    beta = None if beta is None else beta.contiguous()
    if inplace_final_state:
        hkk, hkv = initial_state_kk, initial_state_kv
    else:
        hkk, hkv = initial_state_kk.clone(), initial_state_kv.clone()
    idx = _i32(ssm_state_indices)
    if out is not None:
        _lib.require_gpu(out)
        if (tuple(out.shape) != (B, T, H, V) or out.dtype != q.dtype or not out.is_contiguous()
                or out.data_ptr() % 16):
            raise ValueError(f"out must be a contiguous [{B},{T},{H},{V}] {q.dtype} tensor")
        o = out
    else:
        o = q.new_empty(B, T, H, V)
    onorm = _onorm(o_norm_weight, o_norm_gate, o_norm_eps, (B, T, H, V), q.dtype)
    _lib.call("hmx_gka_decode_fwd",
              _lib.ptr(q), q_ts, _lib.ptr(k), k_ts, _lib.ptr(v), v_ts, _lib.dtype_code(q),
              _lib.ptr(alpha), 0 if alpha is None else _lib.dtype_code(alpha),
              _lib.ptr(gk), 0 if gk is None else _lib.dtype_code(gk),
              _lib.ptr(beta), 0 if beta is None else _lib.dtype_code(beta),
              _lib.ptr(o),
              _lib.ptr(hkk), hkk.stride(0), _lib.ptr(hkk), hkk.stride(0),
              _lib.ptr(hkv), hkv.stride(0), _lib.ptr(hkv), hkv.stride(0), _lib.dtype_code(hkv),
              _lib.ptr(_i32(cu_seqlens)), _lib.ptr(idx), 0 if idx is None else idx.stride(0),
              B, T, N, H, HKV, D, V, int(num_iter), float(ridge_ratio), float(scale),
              onorm, _lib.gate_proj(gates), _lib.stream_of(q))
    if not output_final_state:
        return o, None, None
    if not inplace_final_state and idx is not None:
        # the reference writes sequence n's new state to row n (chebyshev_iteration_gqa.py:106)
        hkk, hkv = hkk[idx.long()], hkv[idx.long()]
    return o, hkk, hkv


def gka_chebyshev_gla_decode(q, k, v, alpha, g, gk, beta, gla_scale: float,
                             ridge_ratio: float = 0.02, num_sketches_per_head: int = 1,
                             num_iter: int = 30, gka=None, h_kk=None, h_kv=None,
                             cu_seqlens=None, ssm_state_indices=None, *,
                             o_norm_weight=None, o_norm_gate=None, o_norm_eps: float = 1e-6,
                             out=None, gates: ProjGates | None = None):
    """Single-token GKA decode (gka_forward.py:248-326).  ``o_norm_*``, ``out`` and
    ``gates``: see chebyshev_iteration_gqa."""
    global _warned_num_iter_zero
    _check_sketching_constraints(gka, num_sketches_per_head, "gka_chebyshev_gla_decode")
    if num_iter == 0:
        if not _warned_num_iter_zero:
            logging.warning("gka_chebyshev_gla_decode: num_iter=0, running 1 Chebyshev iteration. "
                            "Ensure alpha is zeroed out by the caller to skip query correction.")
            _warned_num_iter_zero = True
        num_iter = 1
    if gates is None:
        assert g is gk, "GLA gate g not equal to GKA gate gk is not supported for decoding."
    elif not gates.gk_from_g and gates.A_log is not None:
        raise AssertionError("GLA gate g not equal to GKA gate gk is not supported for decoding.")
    return chebyshev_iteration_gqa(k=k, q=q, v=v, alpha=alpha, gk=gk, beta=beta,
                                   num_iter=num_iter, scale=gla_scale, ridge_ratio=ridge_ratio,
                                   initial_state_kk=h_kk, initial_state_kv=h_kv,
                                   output_final_state=True, inplace_final_state=True,
                                   cu_seqlens=cu_seqlens, ssm_state_indices=ssm_state_indices,
                                   o_norm_weight=o_norm_weight, o_norm_gate=o_norm_gate,
                                   o_norm_eps=o_norm_eps, out=out, gates=gates)


def gka_chebyshev_gla_prefill(q, k, v, alpha, g, gk, beta, gla_scale: float,
                              ridge_ratio: float = 0.02, num_sketches_per_head: int = 1,
                              num_iter: int = 30, gka=None, h_kk_initial=None, h_kv_initial=None,
                              output_final_state: bool = True, cu_seqlens=None, *,
                              o_norm_weight=None, o_norm_gate=None, o_norm_eps: float = 1e-6,
                              ssm_state_indices=None, has_initial_state=None, out=None,
                              gates: ProjGates | None = None,
                              _segment_chunks: int | None = None):
    """Full GKA prefill: Chebyshev query refinement + beta^2 simple GLA
    (gka_forward.py:161-242).  Returns (o, h_kk_final, h_kv_final); h_kk_final is
    None when num_iter == 0 or not output_final_state.

    Keyword-only extensions (no reference counterpart):

    - ``o_norm_weight`` [V] (and optionally ``o_norm_gate`` [B,T,H,V], q.dtype)
      returns the layer's gated RMSNorm ``o_norm(o, z)`` (primed_gka_layer.py:944-949)
      computed in the kernel's output epilogue instead of o.
    - ``ssm_state_indices`` [N]: ``h_kk_initial`` / ``h_kv_initial`` are the layer's
      state pools [slots,H,D,D] (fp32 or bf16); sequence n starts from slot
      ``ssm_state_indices[n]`` and, with ``output_final_state``, its end states are
      written back into that slot in place (the pools are returned).  This replaces
      the layer's gather / zero / scatter (primed_gka_layer.py:1245-1266); with
      num_iter == 0 a sequence without an initial state clears its h_kk slot, as
      that update does.  A negative slot starts from zero and writes nothing.
    - ``has_initial_state`` [N] bool: sequences with False start from zero.
    - ``out`` [B,T,H,V] (q.dtype, contiguous): o is written there.
    - ``gates`` (hmx.ProjGates): alpha, g, gk and beta are formed in the kernels
      from the layer's raw projections (primed_gka_layer.py:224-358, :1138-1153)
      instead of the gate tensors, which are then ignored.

    q, k and v may be the column slices of one fused projection: they are read in
    place."""
    _check_sketching_constraints(gka, num_sketches_per_head, "gka_chebyshev_gla_prefill")
    if cu_seqlens is not None and q.shape[0] != 1:
        raise ValueError(f"Batch size must be 1 when using cu_seqlens, got {q.shape[0]}")
    if gates is not None:
        gates.check(q.shape[0] * q.shape[1], q.shape[2], gka=True)
        alpha = g = gk = beta = None
    elif g is None:   # no GLA decay (the layer without a forgetting gate): e^0 = 1
        g = torch.zeros(q.shape[:3], dtype=torch.float32, device=q.device)
    return _gka_prefill(q, k, v, alpha, g, gk, beta, gla_scale, ridge_ratio, num_iter,
                        h_kk_initial, h_kv_initial, output_final_state, cu_seqlens, True,
                        _segment_chunks, (o_norm_weight, o_norm_gate, o_norm_eps),
                        ssm_state_indices, has_initial_state, out, gates)


def _onorm(weight, gate, eps, shape, dtype):
    """hmx_gated_norm pointer for the optional output norm (None: not requested)."""
    if weight is None:
        if gate is not None:
            raise ValueError("o_norm_gate needs o_norm_weight")
        return None
    _lib.require_gpu(weight, gate)
    z = None if gate is None else _gate_rows(gate, shape, dtype)
    return _lib.gated_norm(z, weight, eps, shape[-1])


def _gka_prefill(q, k, v, alpha, g, gk, beta, gla_scale, ridge_ratio, num_iter, h_kk_initial,
                 h_kv_initial, output_final_state, cu_seqlens, l2norm, segment_chunks=None,
                 o_norm=(None, None, 1e-6), state_indices=None, has_initial_state=None, out=None,
                 gates=None):
    _lib.require_gpu(q, k, v, alpha, g, gk, beta, h_kk_initial, h_kv_initial,
                     state_indices, has_initial_state, out)   # cu_seqlens: host or device
    B, T, H, D = q.shape
    HKV, V = k.shape[2], v.shape[-1]
    bounds = seq_bounds(cu_seqlens, B, T)
    N = len(bounds)
    idx = None
    if state_indices is not None:
        idx = _i32(state_indices)
        if idx.shape != (N,):
            raise ValueError(f"ssm_state_indices must hold {N} slots, got {tuple(idx.shape)}")
        pools = []
        for st, last, name in ((h_kk_initial, D, "h_kk_initial"),
                               (h_kv_initial, V, "h_kv_initial")):
            if (st is None or st.dim() != 4 or tuple(st.shape[1:]) != (H, D, last)
                    or not st[0].is_contiguous() or st.dtype not in (torch.float32, torch.bfloat16)):
                raise ValueError(f"{name} must be the state pool [slots,{H},{D},{last}] fp32/bf16 "
                                 f"with contiguous slots")
            pools.append(st)
        hkk0, hkv0 = pools
        hkk_t = hkk0 if output_final_state else None
        hkv_t = hkv0 if output_final_state else None
        ss_kk, dt_kk = hkk0.stride(0), _lib.dtype_code(hkk0)
        ss_kv, dt_kv = hkv0.stride(0), _lib.dtype_code(hkv0)
    else:
        for st, last, name in ((h_kk_initial, D, "h_kk_initial"),
                               (h_kv_initial, V, "h_kv_initial")):
            if st is not None and tuple(st.shape) != (N, H, D, last):
                raise ValueError(f"{name} must be [{N},{H},{D},{last}], got {tuple(st.shape)}")
        hkk0 = None if h_kk_initial is None else h_kk_initial.to(torch.float32).contiguous()
        hkv0 = None if h_kv_initial is None else h_kv_initial.to(torch.float32).contiguous()
        hkk_t = (torch.empty(N, H, D, D, dtype=torch.float32, device=q.device)
                 if output_final_state and num_iter > 0 else None)
        hkv_t = (torch.empty(N, H, D, V, dtype=torch.float32, device=q.device)
                 if output_final_state else None)
        ss_kk, dt_kk, ss_kv, dt_kv = H * D * D, _lib.HMX_F32, H * D * V, _lib.HMX_F32
    hinit = None
    if has_initial_state is not None:
        if has_initial_state.shape != (N,):
            raise ValueError(f"has_initial_state must be [{N}], got {tuple(has_initial_state.shape)}")
        hinit = has_initial_state.to(torch.uint8).contiguous()
    if gates is None:
        alpha, g = alpha.contiguous(), g.contiguous()
    (q, q_ts), (k, k_ts), (v, v_ts) = (_token_rows(x, 8) for x in (q, k, v))
    if k_ts != v_ts:    # the prefill kernels read k and v at one token stride
        (k, k_ts), (v, v_ts) = _token_rows(k.contiguous(), 8), _token_rows(v.contiguous(), 8)
    gk = None if gk is None else gk.contiguous()
    beta = None if beta is None else beta.contiguous()
    if out is not None:
        if (tuple(out.shape) != (B, T, H, V) or out.dtype != q.dtype or not out.is_contiguous()
                or out.data_ptr() % 16):
            raise ValueError(f"out must be a contiguous [{B},{T},{H},{V}] {q.dtype} tensor")
        o = out
    else:
        o = torch.empty(B, T, H, V, dtype=q.dtype, device=q.device)
    if cu_seqlens is not None and bounds and bounds[-1][1] < T:
        o[:, bounds[-1][1]:].zero_()
    rows, nblk = _segment_table(_lib.PLAN_GKA, bounds, B * T, H, q.device, segment_chunks)
    seg = _device_table(rows, q.device)
    lib = _lib.load()
    ws_bytes = int(lib.hmx_gka_chunk_workspace_bytes(len(rows), nblk, N, H))
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=q.device)
    _lib.call("hmx_gka_chunk_fwd",
              _lib.ptr(q), q_ts, _lib.ptr(k), k_ts, _lib.ptr(v), v_ts, _lib.dtype_code(q),
              _lib.ptr(alpha), 0 if alpha is None else _lib.dtype_code(alpha),
              _lib.ptr(g), 0 if g is None else _lib.dtype_code(g),
              _lib.ptr(gk), 0 if gk is None else _lib.dtype_code(gk),
              _lib.ptr(beta), 0 if beta is None else _lib.dtype_code(beta),
              _lib.ptr(o), _lib.ptr(hkk0), _lib.ptr(hkk_t), ss_kk, dt_kk,
              _lib.ptr(hkv0), _lib.ptr(hkv_t), ss_kv, dt_kv, _lib.ptr(idx), _lib.ptr(hinit),
              _lib.ptr(seg), len(rows), nblk, N, H, HKV, D, V, int(num_iter), float(ridge_ratio),
              float(gla_scale), int(bool(l2norm)), _lib.ptr(ws), ws.numel(),
              _onorm(*o_norm, tuple(o.shape), q.dtype), _lib.gate_proj(gates),
              _lib.stream_of(q))
    if idx is not None and num_iter == 0:
        return o, None, hkv_t
    return o, hkk_t, hkv_t


def gka_chebyshev_gla(q, k, v, alpha, g, gk, gla_scale, ridge_strength: float = 0.02,
                      solver_type: str = "chebyshev", num_iter: int = 30, bp_lambda: bool = True,
                      chunk_size: int = 64):
    """Training-form GKA forward (layers/gated_kalmanet/ops/chebyshev/
    gka_chebyshev_solve.py:107-164): q, k, v [B,L,H,D] with heads expanded, q and k
    already normalised and beta already applied to k and v by the layer
    (gka.py:477-490), no initial state.  ridge_strength is the ratio to |H_t|_F.
    Returns (o, kk_final [B,H,D,D] fp32 or None when num_iter == 0, kv_final).
    When a gradient is needed (grad mode on and an input requires it) the call runs
    through GkaChebyshevGla (hmx.ops.gka_train), whose backward follows the
    reference's (bp_lambda as there); chunk_size only tiles the reference's kernels."""
    if solver_type != "chebyshev":
        raise ValueError(f"Unknown GKA solver type: {solver_type}")
    if g is None:
        g = torch.zeros(q.shape[:3], dtype=torch.float32, device=q.device)
    if torch.is_grad_enabled() and any(t is not None and t.requires_grad
                                       for t in (q, k, v, alpha, g, gk)):
        from .gka_train import GkaChebyshevGla
        return GkaChebyshevGla.apply(q, k, v, alpha, g, gk, gla_scale, ridge_strength,
                                     num_iter, bp_lambda)
    return _gka_prefill(q, k, v, alpha, g, gk, None, gla_scale, ridge_strength, num_iter,
                        None, None, True, None, False)


def torch_decoding_one_step(q, k, v, alpha, g, gk, gla_scale: float, ridge_strength: float,
                            solver_type: str, num_iter: int, prev_h_kk, prev_h_kv):
    """Training-form single-token GKA step (gka_chebyshev_solve.py:324-397): q, k, v
    [B,1,H,D] or [1,H,D] (normalised, beta applied by the layer); separate gates g
    (h_kv) and gk (h_kk); prev_h_kk / prev_h_kv [B,H,D,D] or None.  Returns
    (o [B,1,H,D], h_kk or None when num_iter == 0, h_kv)."""
    if solver_type != "chebyshev":
        raise ValueError(f"Unknown GKA solver type: {solver_type}")
    if q.dim() < 4:
        q, k, v = q[None], k[None], v[None]
        alpha = alpha[None]
        g = None if g is None else g[None]
        gk = None if gk is None else gk[None]
    if g is None:
        g = torch.zeros(q.shape[:3], dtype=torch.float32, device=q.device)
    if num_iter > 0 and prev_h_kk is None:
        prev_h_kk = torch.zeros(q.shape[0], q.shape[2], q.shape[3], q.shape[3],
                                dtype=torch.float32, device=q.device)
    o, hkk, hkv = _gka_prefill(q, k, v, alpha, g, gk, None, gla_scale, ridge_strength, num_iter,
                               prev_h_kk if num_iter > 0 else None, prev_h_kv, True, None, False)
    return o, hkk, hkv


__all__ = ["fused_gka_gating", "chebyshev_iteration_gqa", "gka_chebyshev_gla_decode",
           "gka_chebyshev_gla_prefill", "gka_chebyshev_gla", "torch_decoding_one_step"]
