"""The GDN layer's decode conv and recurrent step in one launch.

A GDN layer's decode tokens go through the short causal conv (vLLM's
``causal_conv1d_update``, vllm-inference/src/primed_vllm/primed_gdn_layer.py:775-785)
and then the fused recurrent gated delta rule on q, k, v views of the conv output
(:805-823).  ``gdn_conv_decode`` does both in the recurrent kernel
(``hmx_gdn_conv_recurrent_fwd``): each (sequence, head) workgroup forms its head's
q, k and v channels of the conv in LDS, with the conv op's arithmetic and bf16
rounding, so outputs, the state pool and the conv state pool equal those of
``causal_conv1d_update`` followed by ``fused_recurrent_gated_delta_rule_gqa``
bit for bit, and the conv output never reaches HBM.  No reference counterpart:
an hmx extension used by ``hmx.serving.gdn_forward_core``.
"""
from __future__ import annotations

import torch

from .. import _lib
from . import conv as _conv
from .gates import ProjGates
from .gdn import _gate_rows, _i32


def gdn_conv_decode(x: torch.Tensor, conv_weight: torch.Tensor, conv_bias: torch.Tensor | None,
                    conv_state: torch.Tensor, activation, state: torch.Tensor,
                    state_indices: torch.Tensor, H: int, HKV: int, scale: float | None = None,
                    use_qk_l2norm_in_kernel: bool = True, *, gates: ProjGates,
                    out: torch.Tensor | None = None, o_norm_weight: torch.Tensor | None = None,
                    o_norm_gate: torch.Tensor | None = None,
                    o_norm_eps: float = 1e-5) -> torch.Tensor:
    """One decode token per sequence: x [N, conv_dim] bf16 projection rows (q H*128 |
    k HKV*128 | v HKV*128 channels), conv_weight [conv_dim, width], conv_state the
    [slots, conv_dim, state_len] pool view (channels contiguous, as the layers pass
    it), state the [slots, H, 128, 128] recurrent pool; both pools are updated in
    place at ``state_indices`` [N] (entries < 0 are skipped).  ``gates`` forms g
    and beta from the layer's raw projections.  Returns o [1, N, H, 128] (``out`` when
    given; the layer's output norm applied with ``o_norm_weight``).  With HKV < H the
    k / v channels' conv state, shared by the heads of a group, shifts in a second
    launch (the conv update over those channels) after the kernel has read it."""
    _lib.require_gpu(x, conv_weight, conv_bias, conv_state, state, state_indices, o_norm_weight,
                     o_norm_gate, out)
    if x.dim() != 2 or x.dtype != torch.bfloat16:
        raise ValueError(f"x must be [N, conv_dim] bf16 rows, got {tuple(x.shape)} {x.dtype}")
    N, dim = x.shape
    K = V = 128
    if dim != H * K + 2 * HKV * K or H % HKV:
        raise ValueError(f"conv_dim {dim} must be H*128 + 2*HKV*128 (H={H}, HKV={HKV})")
    W = conv_weight.shape[-1]
    if conv_weight.shape != (dim, W):
        raise ValueError(f"conv_weight must be [{dim}, width], got {tuple(conv_weight.shape)}")
    st_len, sst, srs = _conv._pool(conv_state, dim, x.dtype, "conv_state")
    if (state.dim() != 4 or tuple(state.shape[1:]) != (H, K, V) or not state[0].is_contiguous()
            or state.dtype not in (torch.float32, torch.bfloat16)):
        raise ValueError(f"state must be the [slots,{H},{K},{V}] fp32/bf16 pool")
    if state_indices.numel() != N:
        raise ValueError(f"state_indices must hold {N} slots")
    gates.check(N, H, gka=False)
    if scale is None:
        scale = K ** -0.5
    if x.stride(-1) != 1 or x.stride(0) % 8 or x.data_ptr() % 16:
        x = x.contiguous()
    if out is None:
        out = x.new_empty(1, N, H, V)
    elif (tuple(out.shape) != (1, N, H, V) or out.dtype != x.dtype or not out.is_contiguous()
          or out.data_ptr() % 16):
        raise ValueError(f"out must be a contiguous [1,{N},{H},{V}] bf16 tensor")
    onorm = None
    if o_norm_weight is not None:
        z = None if o_norm_gate is None else _gate_rows(o_norm_gate, (1, N, H, V), x.dtype)
        onorm = _lib.gated_norm(z, o_norm_weight, o_norm_eps, V)
    elif o_norm_gate is not None:
        raise ValueError("o_norm_gate needs o_norm_weight")
    w, b = _conv._aligned(conv_weight), _conv._aligned(conv_bias)
    idx = _i32(state_indices)
    _lib.call("hmx_gdn_conv_recurrent_fwd", _lib.ptr(x), x.stride(0), _lib.dtype_code(x),
              _lib.ptr(w), _lib.dtype_code(w), W, _lib.ptr(b),
              0 if b is None else _lib.dtype_code(b), _lib.ptr(conv_state), sst, srs, st_len,
              _conv._act(activation), None, 0, None, 0, _lib.ptr(out), _lib.ptr(state),
              state.stride(0), _lib.dtype_code(state), _lib.ptr(idx), N, H, HKV, K, V,
              float(scale), int(bool(use_qk_l2norm_in_kernel)), onorm, _lib.gate_proj(gates),
              _lib.stream_of(x))
    if HKV < H:   # the group-shared k / v channels' conv state: shift after the kernel read it
        c0 = H * K
        _conv.causal_conv1d_update(x[:, c0:], conv_state[:, c0:], conv_weight[c0:],
                                   None if conv_bias is None else conv_bias[c0:], activation,
                                   conv_state_indices=state_indices,
                                   out=torch.empty_like(x[:, c0:]))
    return out
