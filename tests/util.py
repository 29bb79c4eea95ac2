"""Shared tolerances and comparison helpers for the parity tests.

Tolerances (north star): bf16/f16 outputs max-abs <= 2e-2 and norm-wise
relative <= 1e-2 against an fp64/fp32 recurrence; fp32 final states
norm-wise relative <= 1e-3.

The max-abs bound is applied to the error beyond the unavoidable rounding of
the result to the output dtype: each element may additionally differ by half a
unit in the last place of the reference value in that dtype (2^-9 |ref| for
bf16).  Without this allowance an exact answer rounded to bf16 would fail the
bound wherever |ref| >= 5 (e.g. Mamba2 outputs with D x and z gating).
"""
import torch

OUT_MAX_ABS = 2e-2
OUT_REL = 1e-2
STATE_REL = 1e-3


def rel_err(a: torch.Tensor, b: torch.Tensor) -> float:
    a = a.detach().double().cpu()
    b = b.detach().double().cpu()
    den = b.norm().item()
    num = (a - b).norm().item()
    return num / den if den > 0 else num


def max_abs(a: torch.Tensor, b: torch.Tensor) -> float:
    return (a.detach().double().cpu() - b.detach().double().cpu()).abs().max().item() if a.numel() else 0.0


_SIGNIFICAND_BITS = {torch.bfloat16: 8, torch.float16: 11}


def half_ulp(ref: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """Half a unit in the last place of ``ref`` in ``dtype`` (0 for fp32/fp64 outputs)."""
    bits = _SIGNIFICAND_BITS.get(dtype)
    if bits is None:
        return torch.zeros_like(ref)
    _, e = torch.frexp(ref)                       # |ref| in [2^(e-1), 2^e)
    return torch.ldexp(torch.ones_like(ref), e - bits - 1) * (ref != 0)


def max_abs_beyond_rounding(out: torch.Tensor, ref: torch.Tensor) -> float:
    """max(|out - ref| - half_ulp(ref, out.dtype)), floored at 0."""
    if not out.numel():
        return 0.0
    r = ref.detach().double().cpu()
    err = (out.detach().double().cpu() - r).abs() - half_ulp(r, out.dtype)
    return max(0.0, err.max().item())


def assert_out_close(out, ref, max_abs_tol=OUT_MAX_ABS, rel_tol=OUT_REL, what="o"):
    ma, re = max_abs_beyond_rounding(out, ref), rel_err(out, ref)
    assert torch.isfinite(out.detach().float()).all(), f"{what}: non-finite values"
    assert ma <= max_abs_tol and re <= rel_tol, f"{what}: max_abs={ma:.3e} rel={re:.3e}"
    return ma, re


def assert_state_close(st, ref, rel_tol=STATE_REL, what="state"):
    re = rel_err(st, ref)
    assert torch.isfinite(st.detach().float()).all(), f"{what}: non-finite values"
    assert re <= rel_tol, f"{what}: rel={re:.3e}"
    return re
