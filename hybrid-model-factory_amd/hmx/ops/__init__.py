"""Mixer ops with the reference's names, argument order, defaults and returns."""
from .gdn import (chunk_gated_delta_rule, chunk_gated_delta_rule_gqa, fused_gdn_gating,
                  fused_recurrent_gated_delta_rule, fused_recurrent_gated_delta_rule_gqa)

__all__ = [
    "fused_gdn_gating",
    "fused_recurrent_gated_delta_rule_gqa",
    "fused_recurrent_gated_delta_rule",
    "chunk_gated_delta_rule_gqa",
    "chunk_gated_delta_rule",
]
