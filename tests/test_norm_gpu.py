"""GPU parity: hmx.rms_norm_gated (the GDN/GKA output norm) vs the CPU oracle.

Covers bf16 / fp16 / fp32 rows, D in {64, 128, 256}, the gate before and after the
norm, no gate, a strided gate (a view of a fused projection), bf16 and fp32
weights, row counts off the workgroup tiling, and zero rows.  The kernel computes in
fp32 and rounds once, so nearly every element must equal the oracle rounded to the
output dtype; the rest differ by one unit in the last place.
"""
import pytest
import torch

import hmx
from oracle import norm as ref
from util import assert_out_close, half_ulp

pytestmark = pytest.mark.gpu


def _check(out, expect):
    r = expect.to(out.dtype).double()
    o = out.double().cpu()
    assert torch.isfinite(o).all()
    exact = (o == r).double().mean().item()
    assert exact >= 0.99, f"only {exact:.4f} of elements round like the oracle"
    # the others within one unit in the last place
    assert ((o - r).abs() <= 2 * half_ulp(r, out.dtype) + 1e-30).all()


@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("before", [True, False])
def test_bf16_gated(dev, D, before):
    g = torch.Generator().manual_seed(D + before)
    rows = 1003
    x = (torch.randn(rows, D, generator=g) * 2.0).bfloat16()
    z = (torch.randn(rows, D, generator=g) * 1.5).bfloat16()
    w = torch.rand(D, generator=g) + 0.5
    out = hmx.rms_norm_gated(x.to(dev), z.to(dev), w.to(dev), eps=1e-5, norm_before_gate=before)
    torch.cuda.synchronize()
    assert out.dtype == torch.bfloat16 and out.shape == x.shape
    _check(out.cpu(), ref.rms_norm_gated(x, z, w, eps=1e-5, norm_before_gate=before))


def test_no_gate_and_head_layout(dev):
    """[tokens, heads, 128] as in the layers, eps 1e-6 (GKA), no gate."""
    g = torch.Generator().manual_seed(7)
    x = torch.randn(77, 16, 128, generator=g).bfloat16()
    w = (torch.rand(128, generator=g) + 0.5).bfloat16()
    out = hmx.rms_norm_gated(x.to(dev), None, w.to(dev), eps=1e-6)
    torch.cuda.synchronize()
    _check(out.cpu(), ref.rms_norm_gated(x, None, w, eps=1e-6))


def test_strided_gate(dev):
    """z as a slice of a fused projection output (row stride 3 * H * D)."""
    g = torch.Generator().manual_seed(8)
    T, H, D = 130, 8, 128
    proj = torch.randn(T, 3 * H * D, generator=g).bfloat16().to(dev)
    z = proj[:, H * D:2 * H * D].view(T, H, D)
    x = torch.randn(T, H, D, generator=g).bfloat16().to(dev)
    w = torch.rand(D, generator=g).to(dev) + 0.5
    out = hmx.rms_norm_gated(x, z, w)
    torch.cuda.synchronize()
    _check(out.cpu(), ref.rms_norm_gated(x.cpu(), z.cpu(), w.cpu(), eps=1e-5))


@pytest.mark.parametrize("dt", [torch.float16, torch.float32])
def test_other_dtypes(dev, dt):
    g = torch.Generator().manual_seed(9)
    x = torch.randn(300, 128, generator=g).to(dt)
    z = torch.randn(300, 128, generator=g).to(dt)
    w = torch.rand(128, generator=g) + 0.5
    out = hmx.rms_norm_gated(x.to(dev), z.to(dev), w.to(dev))
    torch.cuda.synchronize()
    e = ref.rms_norm_gated(x, z, w, eps=1e-5)
    if dt == torch.float32:
        assert_out_close(out.cpu(), e, max_abs_tol=1e-5, rel_tol=1e-6)
    else:
        _check(out.cpu(), e)


def test_zero_rows(dev):
    x = torch.empty(0, 128, dtype=torch.bfloat16, device=dev)
    out = hmx.rms_norm_gated(x, x, torch.ones(128, device=dev))
    assert out.shape == (0, 128)
