"""Gates formed from a layer's raw projections inside the mixer ops' loads.

The layers compute their gates in a separate elementwise launch and hand the
[tokens, H] gate tensors to the mixer op: GDN's fused_gdn_gating
(vllm-inference/src/primed_vllm/gdn/ops/fused_gdn_gating.py:79-125, then
``beta * 2`` for negative eigenvalues, primed_gdn_layer.py:798-802) and GKA's
fused_gka_gating with the alpha post-processing (primed_gka_layer.py:224-358,
:1138-1153).  Passing a ``ProjGates`` as ``gates=`` to
``chunk_gated_delta_rule_gqa``, ``fused_recurrent_gated_delta_rule_gqa``,
``gka_chebyshev_gla_prefill`` or ``gka_chebyshev_gla_decode`` has the kernels form
the same gates per token from A_log, dt_bias and the raw a / b / alpha_in
projections (each rounded to the projections' dtype, as the reference stores
them), with no gating launch and no gate tensors.
"""
from __future__ import annotations

from dataclasses import dataclass, replace

import torch


@dataclass
class ProjGates:
    """Raw gate projections of one op call; ``a``, ``b``, ``alpha_in`` are
    [tokens, H] (any strides, one dtype), indexed by the op's flattened tokens.

    g = -exp(A_log) * softplus(a + dt_bias) (0 when A_log is None); beta =
    sigmoid(b) * beta_scale (no beta gate when b is None); GKA: alpha =
    sigmoid(alpha_in) + alpha_add, or 0 with alpha_zero; gk = g when gk_from_g."""
    A_log: torch.Tensor | None
    dt_bias: torch.Tensor | None
    a: torch.Tensor | None
    b: torch.Tensor | None = None
    alpha_in: torch.Tensor | None = None
    softplus_beta: float = 1.0
    softplus_threshold: float = 20.0
    beta_scale: float = 1.0
    alpha_add: float = 0.0
    alpha_zero: bool = False
    gk_from_g: bool = False

    def tokens(self, lo: int, hi: int) -> "ProjGates":
        """The gates of tokens [lo, hi) (views of the projections)."""
        cut = lambda t: None if t is None else t[lo:hi]
        return replace(self, a=cut(self.a), b=cut(self.b), alpha_in=cut(self.alpha_in))

    def check(self, tokens: int, H: int, gka: bool) -> None:
        for name in ("a", "b", "alpha_in"):
            t = getattr(self, name)
            if t is not None and tuple(t.shape) != (tokens, H):
                raise ValueError(f"gates.{name} must be [{tokens}, {H}], got {tuple(t.shape)}")
        if self.A_log is not None and (self.a is None or self.dt_bias is None):
            raise ValueError("gates.A_log needs gates.a and gates.dt_bias")
        if not gka and (self.A_log is None or self.b is None):
            raise ValueError("GDN gates need A_log, dt_bias, a and b")
        if gka and self.alpha_in is None and not self.alpha_zero:
            raise ValueError("GKA gates need alpha_in (or alpha_zero)")
