"""Gated RMSNorm: the GDN / GKA output norm ``o_norm(core_attn_out, z)``.

vLLM's ``RMSNormGated(head_v_dim, eps, group_size=None, norm_before_gate=True)``
(constructed at vllm-inference/src/primed_vllm/primed_gdn_layer.py:443-450 and
primed_gka_layer.py:736-743, called at primed_gdn_layer.py:626 and
primed_gka_layer.py:949) and fla's ``FusedRMSNormGated`` in the training layers
compute, over the last dim in fp32 with one final rounding:

    norm_before_gate:  out = x / sqrt(mean(x^2) + eps) * weight * silu(z)
    otherwise:         u = x * silu(z); out = u / sqrt(mean(u^2) + eps) * weight
"""
from __future__ import annotations

import torch

from .. import _lib


def _rows(t: torch.Tensor, D: int) -> torch.Tensor:
    """[rows, D] view with unit element stride (copies only when no such view exists)."""
    if t.stride(-1) != 1:
        t = t.contiguous()
    r = t.reshape(-1, D)
    if r.stride(-1) != 1 or (r.shape[0] > 1 and r.stride(0) % (16 // t.element_size()) != 0) \
            or r.data_ptr() % 16 != 0:
        r = r.contiguous()
    return r


def rms_norm_gated(x: torch.Tensor, z: torch.Tensor | None, weight: torch.Tensor,
                   eps: float = 1e-5, norm_before_gate: bool = True) -> torch.Tensor:
    """Gated RMSNorm over the last dim of ``x`` ([..., D], D in {64, 128, 256});
    ``z`` None or x's shape and dtype; ``weight`` [D].  Returns x's shape and dtype."""
    _lib.require_gpu(x, z, weight)
    D = x.shape[-1]
    if z is not None and (z.shape != x.shape or z.dtype != x.dtype):
        raise ValueError(f"gate {tuple(z.shape)}/{z.dtype} must match x {tuple(x.shape)}/{x.dtype}")
    if weight.numel() != D:
        raise ValueError(f"weight has {weight.numel()} elements, expected {D}")
    xr = _rows(x, D)
    zr = None if z is None else _rows(z, D)
    w = weight.contiguous()
    out = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    orows = out.view(-1, D)
    _lib.call("hmx_rms_norm_gated", _lib.ptr(xr), xr.stride(0), _lib.ptr(zr),
              0 if zr is None else zr.stride(0), _lib.dtype_code(x), _lib.ptr(w),
              _lib.dtype_code(w), _lib.ptr(orows), orows.stride(0), xr.shape[0], D, float(eps),
              int(bool(norm_before_gate)), _lib.stream_of(x))
    return out
