"""torch.library registrations of the hmx mixer ops (namespace ``hmx``).

vLLM runs each mixer inside a registered custom op that torch.compile treats
as opaque and CUDA graphs capture (vllm-inference/src/primed_vllm/
primed_gdn_layer.py:85-90), and the training mixers call the kernels under
autograd.  These registrations give every hmx op a schema, a fake (meta)
implementation for tracing, declared mutations for the in-place state pools,
and, for the functional (prefill / scan) ops, an autograd rule: these serving
kernels are forward-only, so a backward through them raises NotImplementedError
instead of silently returning no gradient.  The in-place decode ops declare their
mutations; torch refuses autograd through them by itself.  The training GKA op
with its backward is the autograd function behind ``hmx.gka_chebyshev_gla`` and
``hmx.ChebyshevIteration`` (hmx.ops.gka_train).

``torch.ops.hmx.<name>`` is the registered op; the functions of the same name
in this module wrap it with the reference's Python signature (optional
outputs come back as None).  The plain ``hmx.<name>`` functions call the
library directly and skip the dispatcher.
"""
from __future__ import annotations

from typing import Optional

import torch
from torch import Tensor

from . import ops

_FORWARD_ONLY = ("hmx kernels are forward-only: no backward is implemented for {}")


def _empty_like_none(t: Tensor | None, ref: Tensor) -> Tensor:
    return t if t is not None else ref.new_empty(0, dtype=torch.float32)


def _forward_only(op, name: str):
    def backward(ctx, *grads):
        raise NotImplementedError(_FORWARD_ONLY.format(name))

    def setup_context(ctx, inputs, output):
        return None

    op.register_autograd(backward, setup_context=setup_context)


def _n_seqs(B: int, cu_seqlens: Tensor | None) -> int:
    return B if cu_seqlens is None else cu_seqlens.shape[0] - 1


# --------------------------------------------------------------------------- GDN
@torch.library.custom_op("hmx::fused_gdn_gating", mutates_args=())
def _gdn_gating(A_log: Tensor, a: Tensor, b: Tensor, dt_bias: Tensor, beta: float,
                threshold: float) -> tuple[Tensor, Tensor]:
    g, be = ops.fused_gdn_gating(A_log, a, b, dt_bias, beta, threshold)
    return g, be


@_gdn_gating.register_fake
def _(A_log, a, b, dt_bias, beta, threshold):
    return a.new_empty(1, *a.shape), a.new_empty(1, *a.shape)


@torch.library.custom_op("hmx::chunk_gated_delta_rule_gqa", mutates_args=())
def _chunk_gdn(q: Tensor, k: Tensor, v: Tensor, g: Tensor, beta: Tensor, scale: float,
               initial_state: Optional[Tensor], output_final_state: bool,
               cu_seqlens: Optional[Tensor], use_qk_l2norm_in_kernel: bool) -> tuple[Tensor, Tensor]:
    o, s = ops.chunk_gated_delta_rule_gqa(q, k, v, g, beta, scale, initial_state,
                                          output_final_state, cu_seqlens, use_qk_l2norm_in_kernel)
    return o, _empty_like_none(s, q)


@_chunk_gdn.register_fake
def _(q, k, v, g, beta, scale, initial_state, output_final_state, cu_seqlens,
      use_qk_l2norm_in_kernel):
    B, T, H, K = q.shape
    V = v.shape[-1]
    o = q.new_empty(B, T, H, V)
    s = (q.new_empty(_n_seqs(B, cu_seqlens), H, K, V, dtype=torch.float32) if output_final_state
         else q.new_empty(0, dtype=torch.float32))
    return o, s


_forward_only(_chunk_gdn, "chunk_gated_delta_rule_gqa")


@torch.library.custom_op("hmx::fused_recurrent_gated_delta_rule_gqa",
                         mutates_args=("initial_state",))
def _recurrent_gdn(q: Tensor, k: Tensor, v: Tensor, g: Tensor, beta: Optional[Tensor],
                   scale: Optional[float], initial_state: Optional[Tensor],
                   inplace_final_state: bool, cu_seqlens: Optional[Tensor],
                   ssm_state_indices: Optional[Tensor], num_accepted_tokens: Optional[Tensor],
                   use_qk_l2norm_in_kernel: bool) -> tuple[Tensor, Tensor]:
    o, s = ops.fused_recurrent_gated_delta_rule_gqa(
        q, k, v, g, beta, scale, initial_state, inplace_final_state, cu_seqlens,
        ssm_state_indices, num_accepted_tokens, use_qk_l2norm_in_kernel)
    # the in-place pool is the caller's own tensor: return an empty marker instead
    return o, (q.new_empty(0, dtype=torch.float32) if inplace_final_state else s)


@_recurrent_gdn.register_fake
def _(q, k, v, g, beta, scale, initial_state, inplace_final_state, cu_seqlens,
      ssm_state_indices, num_accepted_tokens, use_qk_l2norm_in_kernel):
    B, T, H, K = q.shape
    V = v.shape[-1]
    o = q.new_empty(B, T, H, V)
    if inplace_final_state:
        return o, q.new_empty(0, dtype=torch.float32)
    sdt = torch.float32 if initial_state is None else initial_state.dtype
    return o, q.new_empty(B, T, H, K, V, dtype=sdt)




# --------------------------------------------------------------------------- GKA
@torch.library.custom_op("hmx::gka_chebyshev_gla_prefill", mutates_args=())
def _gka_prefill(q: Tensor, k: Tensor, v: Tensor, alpha: Tensor, g: Tensor, gk: Optional[Tensor],
                 beta: Optional[Tensor], gla_scale: float, ridge_ratio: float, num_iter: int,
                 h_kk_initial: Optional[Tensor], h_kv_initial: Optional[Tensor],
                 output_final_state: bool,
                 cu_seqlens: Optional[Tensor]) -> tuple[Tensor, Tensor, Tensor]:
    o, hkk, hkv = ops.gka_chebyshev_gla_prefill(
        q, k, v, alpha, g, gk, beta, gla_scale, ridge_ratio=ridge_ratio, num_iter=num_iter,
        h_kk_initial=h_kk_initial, h_kv_initial=h_kv_initial,
        output_final_state=output_final_state, cu_seqlens=cu_seqlens)
    return o, _empty_like_none(hkk, q), _empty_like_none(hkv, q)


@_gka_prefill.register_fake
def _(q, k, v, alpha, g, gk, beta, gla_scale, ridge_ratio, num_iter, h_kk_initial,
      h_kv_initial, output_final_state, cu_seqlens):
    B, T, H, D = q.shape
    V = v.shape[-1]
    N = _n_seqs(B, cu_seqlens)
    e = q.new_empty(0, dtype=torch.float32)
    hkk = q.new_empty(N, H, D, D, dtype=torch.float32) if output_final_state and num_iter > 0 else e
    hkv = q.new_empty(N, H, D, V, dtype=torch.float32) if output_final_state else e
    return q.new_empty(B, T, H, V), hkk, hkv


_forward_only(_gka_prefill, "gka_chebyshev_gla_prefill")


@torch.library.custom_op("hmx::gka_chebyshev_gla_decode", mutates_args=("h_kk", "h_kv"))
def _gka_decode(q: Tensor, k: Tensor, v: Tensor, alpha: Tensor, gk: Optional[Tensor],
                beta: Optional[Tensor], gla_scale: float, ridge_ratio: float, num_iter: int,
                h_kk: Tensor, h_kv: Tensor, cu_seqlens: Optional[Tensor],
                ssm_state_indices: Optional[Tensor]) -> Tensor:
    o, _, _ = ops.gka_chebyshev_gla_decode(q, k, v, alpha, gk, gk, beta, gla_scale,
                                           ridge_ratio=ridge_ratio, num_iter=num_iter,
                                           h_kk=h_kk, h_kv=h_kv, cu_seqlens=cu_seqlens,
                                           ssm_state_indices=ssm_state_indices)
    return o


@_gka_decode.register_fake
def _(q, k, v, alpha, gk, beta, gla_scale, ridge_ratio, num_iter, h_kk, h_kv, cu_seqlens,
      ssm_state_indices):
    B, T, H, _ = q.shape
    return q.new_empty(B, T, H, v.shape[-1])




# --------------------------------------------------------------------------- SSD
@torch.library.custom_op("hmx::mamba_chunk_scan_combined", mutates_args=())
def _ssd_scan(x: Tensor, dt: Tensor, A: Tensor, B: Tensor, C: Tensor, chunk_size: int,
              D: Optional[Tensor], z: Optional[Tensor], dt_bias: Optional[Tensor],
              initial_states: Optional[Tensor], seq_idx: Optional[Tensor],
              dt_softplus: bool, dt_min: float, dt_max: float) -> tuple[Tensor, Tensor]:
    y, fin = ops.mamba_chunk_scan_combined(x, dt, A, B, C, chunk_size, D=D, z=z, dt_bias=dt_bias,
                                           initial_states=initial_states, seq_idx=seq_idx,
                                           dt_softplus=dt_softplus, dt_limit=(dt_min, dt_max),
                                           return_final_states=True)
    return y, fin


@_ssd_scan.register_fake
def _(x, dt, A, B, C, chunk_size, D, z, dt_bias, initial_states, seq_idx, dt_softplus, dt_min,
      dt_max):
    b, l, H, P = x.shape
    return x.new_empty(b, l, H, P), x.new_empty(b, H, P, B.shape[-1], dtype=torch.float32)


_forward_only(_ssd_scan, "mamba_chunk_scan_combined")


@torch.library.custom_op("hmx::mamba_chunk_scan_combined_varlen", mutates_args=("out",))
def _ssd_varlen(x: Tensor, dt: Tensor, A: Tensor, B: Tensor, C: Tensor, chunk_size: int,
                cu_seqlens: Tensor, out: Tensor, D: Optional[Tensor], z: Optional[Tensor],
                dt_bias: Optional[Tensor], initial_states: Optional[Tensor], dt_softplus: bool,
                dt_min: float, dt_max: float) -> Tensor:
    return ops.mamba_chunk_scan_combined_varlen(
        x, dt, A, B, C, chunk_size, cu_seqlens, out=out, D=D, z=z, dt_bias=dt_bias,
        initial_states=initial_states, dt_softplus=dt_softplus, dt_limit=(dt_min, dt_max))


@_ssd_varlen.register_fake
def _(x, dt, A, B, C, chunk_size, cu_seqlens, out, D, z, dt_bias, initial_states, dt_softplus,
      dt_min, dt_max):
    H, P = dt.shape[1], x.shape[2]
    return x.new_empty(cu_seqlens.shape[0] - 1, H, P, B.shape[-1], dtype=torch.float32)


@torch.library.custom_op("hmx::mamba_chunk_scan_combined_varlen_chunks", mutates_args=("out",))
def _ssd_varlen_chunks(x: Tensor, dt: Tensor, A: Tensor, B: Tensor, C: Tensor, chunk_size: int,
                       cu_seqlens: Tensor, cu_chunk_seqlens: Tensor, seq_idx: Tensor, out: Tensor,
                       D: Optional[Tensor], z: Optional[Tensor], dt_bias: Optional[Tensor],
                       initial_states: Optional[Tensor], dt_softplus: bool, dt_min: float,
                       dt_max: float) -> Tensor:
    """The varlen scan returning the state after every chunk (prefix caching)."""
    return ops.mamba_chunk_scan_combined_varlen(
        x, dt, A, B, C, chunk_size, cu_seqlens, cu_chunk_seqlens=cu_chunk_seqlens,
        seq_idx=seq_idx, out=out, D=D, z=z, dt_bias=dt_bias, initial_states=initial_states,
        dt_softplus=dt_softplus, dt_limit=(dt_min, dt_max), return_intermediate_states=True)


@_ssd_varlen_chunks.register_fake
def _(x, dt, A, B, C, chunk_size, cu_seqlens, cu_chunk_seqlens, seq_idx, out, D, z, dt_bias,
      initial_states, dt_softplus, dt_min, dt_max):
    H, P = dt.shape[1], x.shape[2]
    return x.new_empty(cu_chunk_seqlens.shape[0] - 1, H, P, B.shape[-1], dtype=torch.float32)




@torch.library.custom_op("hmx::selective_state_update", mutates_args=("state", "out"))
def _ssd_update(state: Tensor, x: Tensor, dt: Tensor, A: Tensor, B: Tensor, C: Tensor,
                D: Optional[Tensor], z: Optional[Tensor], dt_bias: Optional[Tensor],
                dt_softplus: bool, state_batch_indices: Optional[Tensor],
                dst_state_batch_indices: Optional[Tensor], pad_slot_id: int, out: Tensor) -> None:
    ops.selective_state_update(state, x, dt, A, B, C, D, z, dt_bias, dt_softplus,
                               state_batch_indices, dst_state_batch_indices, pad_slot_id, out)


@_ssd_update.register_fake
def _(state, x, dt, A, B, C, D, z, dt_bias, dt_softplus, state_batch_indices,
      dst_state_batch_indices, pad_slot_id, out):
    return None




# ------------------------------------------------------- conv1d and the output norm
@torch.library.custom_op("hmx::causal_conv1d_fn", mutates_args=("conv_states",))
def _conv_fwd(x: Tensor, weight: Tensor, bias: Optional[Tensor], conv_states: Optional[Tensor],
              query_start_loc: Optional[Tensor], cache_indices: Optional[Tensor],
              has_initial_state: Optional[Tensor], activation: Optional[str],
              pad_slot_id: int, initial_state_idx: Optional[Tensor] = None,
              block_idx_first_scheduled_token: Optional[Tensor] = None,
              block_idx_last_scheduled_token: Optional[Tensor] = None,
              num_computed_tokens: Optional[Tensor] = None,
              block_size_to_align: int = 0) -> Tensor:
    blocks = ops.conv.block_args(initial_state_idx, block_idx_first_scheduled_token,
                                 block_idx_last_scheduled_token, num_computed_tokens,
                                 block_size_to_align)
    return ops.conv.conv_fwd_rows(x, weight, bias, conv_states, query_start_loc, cache_indices,
                                  has_initial_state, activation, pad_slot_id, blocks=blocks)


@_conv_fwd.register_fake
def _(x, weight, bias, conv_states, query_start_loc, cache_indices, has_initial_state, activation,
      pad_slot_id, initial_state_idx=None, block_idx_first_scheduled_token=None,
      block_idx_last_scheduled_token=None, num_computed_tokens=None, block_size_to_align=0):
    return x.new_empty(x.shape[1], x.shape[0])


@torch.library.custom_op("hmx::causal_conv1d_update", mutates_args=("conv_state",))
def _conv_update(x: Tensor, conv_state: Tensor, weight: Tensor, bias: Optional[Tensor],
                 activation: Optional[str], conv_state_indices: Optional[Tensor],
                 pad_slot_id: int, num_accepted_tokens: Optional[Tensor] = None,
                 query_start_loc: Optional[Tensor] = None,
                 block_idx_last_scheduled_token: Optional[Tensor] = None,
                 initial_state_idx: Optional[Tensor] = None) -> Tensor:
    return ops.causal_conv1d_update(x, conv_state, weight, bias, activation, conv_state_indices,
                                    num_accepted_tokens, query_start_loc, pad_slot_id=pad_slot_id,
                                    block_idx_last_scheduled_token=block_idx_last_scheduled_token,
                                    initial_state_idx=initial_state_idx)


@_conv_update.register_fake
def _(x, conv_state, weight, bias, activation, conv_state_indices, pad_slot_id,
      num_accepted_tokens=None, query_start_loc=None, block_idx_last_scheduled_token=None,
      initial_state_idx=None):
    return x.new_empty(x.shape)


@torch.library.custom_op("hmx::rms_norm_gated", mutates_args=())
def _norm(x: Tensor, z: Optional[Tensor], weight: Tensor, eps: float,
          norm_before_gate: bool) -> Tensor:
    return ops.rms_norm_gated(x, z, weight, eps, norm_before_gate)


@_norm.register_fake
def _(x, z, weight, eps, norm_before_gate):
    return torch.empty_like(x)


_forward_only(_norm, "rms_norm_gated")


# ------------------------------------------------------- reference-signature wrappers
def chunk_gated_delta_rule_gqa(q, k, v, g, beta, scale=None, initial_state=None,
                               output_final_state=False, cu_seqlens=None,
                               use_qk_l2norm_in_kernel=False):
    """``torch.ops.hmx.chunk_gated_delta_rule_gqa`` with the reference signature
    (chunk_gqa.py:15-26)."""
    scale = k.shape[-1] ** -0.5 if scale is None else scale
    o, s = torch.ops.hmx.chunk_gated_delta_rule_gqa(q, k, v, g, beta, float(scale), initial_state,
                                                    output_final_state, cu_seqlens,
                                                    use_qk_l2norm_in_kernel)
    return o, (s if output_final_state else None)


def fused_recurrent_gated_delta_rule_gqa(q, k, v, g, beta=None, scale=None, initial_state=None,
                                         inplace_final_state=True, cu_seqlens=None,
                                         ssm_state_indices=None, num_accepted_tokens=None,
                                         use_qk_l2norm_in_kernel=False):
    """``torch.ops.hmx.fused_recurrent_gated_delta_rule_gqa`` with the reference signature
    (fused_recurrent_gqa.py:227-240); the in-place pool is returned as the final state."""
    o, s = torch.ops.hmx.fused_recurrent_gated_delta_rule_gqa(
        q, k, v, g, beta, scale, initial_state, inplace_final_state, cu_seqlens,
        ssm_state_indices, num_accepted_tokens, use_qk_l2norm_in_kernel)
    return o, (initial_state if inplace_final_state else s)


def gka_chebyshev_gla_prefill(q, k, v, alpha, g, gk, beta, gla_scale, ridge_ratio=0.02,
                              num_sketches_per_head=1, num_iter=30, gka=None, h_kk_initial=None,
                              h_kv_initial=None, output_final_state=True, cu_seqlens=None):
    """``torch.ops.hmx.gka_chebyshev_gla_prefill`` with the reference signature
    (gka_forward.py:161-178)."""
    ops.gka._check_sketching_constraints(gka, num_sketches_per_head, "gka_chebyshev_gla_prefill")
    o, hkk, hkv = torch.ops.hmx.gka_chebyshev_gla_prefill(
        q, k, v, alpha, g, gk, beta, float(gla_scale), float(ridge_ratio), int(num_iter),
        h_kk_initial, h_kv_initial, output_final_state, cu_seqlens)
    if not output_final_state:
        return o, None, None
    return o, (hkk if num_iter > 0 else None), hkv


def gka_chebyshev_gla_decode(q, k, v, alpha, g, gk, beta, gla_scale, ridge_ratio=0.02,
                             num_sketches_per_head=1, num_iter=30, gka=None, h_kk=None,
                             h_kv=None, cu_seqlens=None, ssm_state_indices=None):
    """``torch.ops.hmx.gka_chebyshev_gla_decode`` with the reference signature
    (gka_forward.py:248-264); the pools are updated in place and returned."""
    ops.gka._check_sketching_constraints(gka, num_sketches_per_head, "gka_chebyshev_gla_decode")
    assert g is gk, "GLA gate g not equal to GKA gate gk is not supported for decoding."
    o = torch.ops.hmx.gka_chebyshev_gla_decode(q, k, v, alpha, gk, beta, float(gla_scale),
                                               float(ridge_ratio), int(num_iter), h_kk, h_kv,
                                               cu_seqlens, ssm_state_indices)
    return o, h_kk, h_kv


def mamba_chunk_scan_combined_varlen(x, dt, A, B, C, chunk_size, cu_seqlens, cu_chunk_seqlens=None,
                                     last_chunk_indices=None, seq_idx=None, out=None, D=None,
                                     z=None, dt_bias=None, initial_states=None, dt_softplus=False,
                                     dt_limit=(0.0, float("inf")),
                                     return_intermediate_states=False, state_dtype=None):
    """``torch.ops.hmx.mamba_chunk_scan_combined_varlen`` with vLLM's signature
    (return_intermediate_states through the ``_chunks`` op)."""
    if out is None:
        out = x.new_empty(x.shape[0], dt.shape[1], x.shape[2])
    if return_intermediate_states:
        st = torch.ops.hmx.mamba_chunk_scan_combined_varlen_chunks(
            x, dt, A, B, C, int(chunk_size), cu_seqlens, cu_chunk_seqlens, seq_idx, out, D, z,
            dt_bias, initial_states, bool(dt_softplus), float(dt_limit[0]), float(dt_limit[1]))
        return st if state_dtype in (None, torch.float32) else st.to(state_dtype)
    st = torch.ops.hmx.mamba_chunk_scan_combined_varlen(
        x, dt, A, B, C, int(chunk_size), cu_seqlens, out, D, z, dt_bias, initial_states,
        bool(dt_softplus), float(dt_limit[0]), float(dt_limit[1]))
    return st if state_dtype in (None, torch.float32) else st.to(state_dtype)


def selective_state_update(state, x, dt, A, B, C, D=None, z=None, dt_bias=None,
                           dt_softplus=False, state_batch_indices=None,
                           dst_state_batch_indices=None, pad_slot_id=-1, out=None):
    """``torch.ops.hmx.selective_state_update``; returns ``out``."""
    if out is None:
        out = x.new_empty(dt.shape)
    torch.ops.hmx.selective_state_update(state, x, dt, A, B, C, D, z, dt_bias, bool(dt_softplus),
                                         state_batch_indices, dst_state_batch_indices,
                                         int(pad_slot_id), out)
    return out


def _act_name(activation):
    if activation is True:
        return "silu"
    return None if activation in (None, False) else activation


def causal_conv1d_fn(x, weight, bias=None, conv_states=None, query_start_loc=None,
                     cache_indices=None, has_initial_state=None, activation="silu",
                     pad_slot_id=-1, metadata=None, validate_data=False,
                     block_idx_first_scheduled_token=None, block_idx_last_scheduled_token=None,
                     initial_state_idx=None, num_computed_tokens=None, block_size_to_align=0):
    """``torch.ops.hmx.causal_conv1d_fn`` with vLLM's signature (called at
    primed_gdn_layer.py:747-757, primed_mamba2_layer.py:782-793 with the prefix-cache
    block arguments); returns the [dim, total] view."""
    return torch.ops.hmx.causal_conv1d_fn(x, weight, bias, conv_states, query_start_loc,
                                          cache_indices, has_initial_state,
                                          _act_name(activation), int(pad_slot_id),
                                          initial_state_idx, block_idx_first_scheduled_token,
                                          block_idx_last_scheduled_token, num_computed_tokens,
                                          int(block_size_to_align or 0)).t()


def causal_conv1d_update(x, conv_state, weight, bias=None, activation=None,
                         conv_state_indices=None, num_accepted_tokens=None, query_start_loc=None,
                         max_query_len=-1, pad_slot_id=-1, validate_data=False,
                         block_idx_last_scheduled_token=None, initial_state_idx=None):
    """``torch.ops.hmx.causal_conv1d_update`` with vLLM's signature (called at
    primed_gdn_layer.py:775-785, :700-712 in the speculative form, and
    primed_mamba2_layer.py:964-973 with the prefix-cache block arguments); the state
    pool is updated in place."""
    return torch.ops.hmx.causal_conv1d_update(x, conv_state, weight, bias, _act_name(activation),
                                              conv_state_indices, int(pad_slot_id),
                                              num_accepted_tokens, query_start_loc,
                                              block_idx_last_scheduled_token, initial_state_idx)


def rms_norm_gated(x, z, weight, eps=1e-5, norm_before_gate=True):
    """``torch.ops.hmx.rms_norm_gated``: the layers' output norm ``o_norm(o, z)``."""
    return torch.ops.hmx.rms_norm_gated(x, z, weight, float(eps), bool(norm_before_gate))


__all__ = ["chunk_gated_delta_rule_gqa", "fused_recurrent_gated_delta_rule_gqa",
           "gka_chebyshev_gla_prefill", "gka_chebyshev_gla_decode",
           "mamba_chunk_scan_combined_varlen", "selective_state_update", "causal_conv1d_fn",
           "causal_conv1d_update", "rms_norm_gated"]
