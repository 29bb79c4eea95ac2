"""Gated RMSNorm CPU oracle — test infrastructure only (see package doc).

The output norm of the GDN and GKA layers, ``o_norm(core_attn_out, z)``:
  vllm-inference/src/primed_vllm/primed_gdn_layer.py:443-450 (construction,
  eps 1e-5 for GDN, :312) and :621-626 (call); primed_gka_layer.py:736-743, :944-949;
  the training layers use fla's FusedRMSNormGated (layers/gated_deltanet/gdn.py:201,
  layers/gated_kalmanet/gka.py:233).
Both are external to the reference (vLLM's RMSNormGated, fla's
FusedRMSNormGated).  Their published semantics, with group_size None:

    u   = x * silu(z)                 (only when not norm_before_gate)
    out = u / sqrt(mean(u^2) + eps) * weight
    out = out * silu(z)               (only when norm_before_gate)

computed in fp32 from the upcast inputs and rounded once to x's dtype.  The
reference's own torch form, Qwen3_5MoeRMSNormGated
(training/src/hmf/model/hybrid_zoo/models/qwen3_5_moe_hmf/modeling_qwen3_5_moe_hmf.py:271-286),
is the norm_before_gate case; it equals this one exactly for fp32 inputs (its
intermediate casts to the input dtype are then no-ops), which the tests check.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

DEFAULT = torch.float64


def rms_norm_gated(x: torch.Tensor, z: torch.Tensor | None, weight: torch.Tensor,
                   eps: float = 1e-5, norm_before_gate: bool = True,
                   dtype=DEFAULT) -> torch.Tensor:
    """Gated RMSNorm over the last dim in ``dtype``; returns ``dtype`` values."""
    u = x.to(dtype)
    w = weight.to(dtype)
    g = None if z is None else F.silu(z.to(dtype))
    if g is not None and not norm_before_gate:
        u = u * g
    out = u * torch.rsqrt((u * u).mean(-1, keepdim=True) + eps) * w
    if g is not None and norm_before_gate:
        out = out * g
    return out
