"""Pins the gated RMSNorm oracle (oracle/norm.py) with closed forms and
identities (vLLM's RMSNormGated and fla's FusedRMSNormGated are un-vendored and
ship no vectors):
  - a hand-computed row (mean, not sum, of squares; silu, not sigmoid, gate);
  - eps inside the square root (a tiny row where eps dominates);
  - unit RMS of the normalised row (closed form mean(x^2)/(mean(x^2)+eps));
  - the gate after the norm (norm_before_gate) is an elementwise silu(z) factor,
    and before the norm it equals normalising x silu(z);
  - linearity in the weight and invariance under positive scaling of x.
"""
import math

import torch

from oracle import norm as ref

D64 = torch.float64


def test_hand_row():
    x = torch.tensor([[3.0, 4.0]], dtype=D64)
    w = torch.ones(2, dtype=D64)
    out = ref.rms_norm_gated(x, None, w, eps=0.0)
    r = 1.0 / math.sqrt((9.0 + 16.0) / 2.0)
    assert torch.allclose(out, torch.tensor([[3.0 * r, 4.0 * r]], dtype=D64), rtol=0, atol=1e-15)
    z = torch.tensor([[0.0, 2.0]], dtype=D64)
    silu2 = 2.0 / (1.0 + math.exp(-2.0))
    out = ref.rms_norm_gated(x, z, w, eps=0.0)
    assert torch.allclose(out, torch.tensor([[0.0, 4.0 * r * silu2]], dtype=D64), rtol=0, atol=1e-15)


def test_eps_inside_sqrt():
    x = torch.full((1, 4), 1e-3, dtype=D64)
    out = ref.rms_norm_gated(x, None, torch.ones(4, dtype=D64), eps=1e-5)
    expect = 1e-3 / math.sqrt(1e-6 + 1e-5)
    assert torch.allclose(out, torch.full_like(x, expect), rtol=1e-14, atol=0)


def test_unit_rms_closed_form():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(64, 128, generator=g, dtype=D64) * 3.0
    eps = 1e-5
    out = ref.rms_norm_gated(x, None, torch.ones(128, dtype=D64), eps=eps)
    ms = (x * x).mean(-1)
    assert torch.allclose((out * out).mean(-1), ms / (ms + eps), rtol=1e-12, atol=0)


def test_gate_placement():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(32, 128, generator=g, dtype=D64)
    z = torch.randn(32, 128, generator=g, dtype=D64) * 2.0
    w = torch.rand(128, generator=g, dtype=D64) + 0.5
    plain = ref.rms_norm_gated(x, None, w, eps=1e-6)
    after = ref.rms_norm_gated(x, z, w, eps=1e-6, norm_before_gate=True)
    silu = z / (1.0 + torch.exp(-z))
    assert torch.allclose(after, plain * silu, rtol=1e-13, atol=1e-15)
    before = ref.rms_norm_gated(x, z, w, eps=1e-6, norm_before_gate=False)
    assert torch.allclose(before, ref.rms_norm_gated(x * silu, None, w, eps=1e-6), rtol=1e-13, atol=1e-15)
    assert not torch.allclose(before, after)


def test_weight_linear_and_scale_invariant():
    g = torch.Generator().manual_seed(2)
    x = torch.randn(16, 64, generator=g, dtype=D64)
    z = torch.randn(16, 64, generator=g, dtype=D64)
    w = torch.rand(64, generator=g, dtype=D64) + 0.5
    one = ref.rms_norm_gated(x, z, torch.ones(64, dtype=D64), eps=0.0)
    assert torch.allclose(ref.rms_norm_gated(x, z, w, eps=0.0), one * w, rtol=1e-13, atol=1e-15)
    assert torch.allclose(ref.rms_norm_gated(x * 7.5, z, w, eps=0.0),
                          ref.rms_norm_gated(x, z, w, eps=0.0), rtol=1e-13, atol=1e-15)
