"""Mixer ops with the reference's names, argument order, defaults and returns."""
from .gdn import (chunk_gated_delta_rule, chunk_gated_delta_rule_gqa, fused_gdn_gating,
                  fused_recurrent_gated_delta_rule, fused_recurrent_gated_delta_rule_gqa)
from .gka import (chebyshev_iteration_gqa, fused_gka_gating, gka_chebyshev_gla,
                  gka_chebyshev_gla_decode, gka_chebyshev_gla_prefill, torch_decoding_one_step)
from .conv import causal_conv1d_fn, causal_conv1d_update
from .gates import ProjGates
from .gdn_train import ChunkGatedDeltaRule
from .gka_train import ChebyshevIteration, GkaChebyshevGla, latent_chebyshev
from .ssd_train import MambaChunkScanCombined
from .norm import rms_norm_gated
from .ssd import (mamba_chunk_scan_combined, mamba_chunk_scan_combined_varlen,
                  selective_state_update)

__all__ = [
    "ProjGates",
    "fused_gdn_gating",
    "fused_recurrent_gated_delta_rule_gqa",
    "fused_recurrent_gated_delta_rule",
    "chunk_gated_delta_rule_gqa",
    "chunk_gated_delta_rule",
    "fused_gka_gating",
    "chebyshev_iteration_gqa",
    "gka_chebyshev_gla_decode",
    "gka_chebyshev_gla_prefill",
    "gka_chebyshev_gla",
    "torch_decoding_one_step",
    "ChunkGatedDeltaRule",
    "ChebyshevIteration",
    "MambaChunkScanCombined",
    "GkaChebyshevGla",
    "latent_chebyshev",
    "mamba_chunk_scan_combined",
    "mamba_chunk_scan_combined_varlen",
    "selective_state_update",
    "rms_norm_gated",
    "causal_conv1d_fn",
    "causal_conv1d_update",
]
