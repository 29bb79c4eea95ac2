"""Shared tolerances and comparison helpers for the parity tests.

Tolerances (north star): bf16/f16 outputs max-abs <= 2e-2 and norm-wise
relative <= 1e-2 against an fp64/fp32 recurrence; fp32 final states
norm-wise relative <= 1e-3.
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


def assert_out_close(out, ref, max_abs_tol=OUT_MAX_ABS, rel_tol=OUT_REL, what="o"):
    ma, re = max_abs(out, ref), rel_err(out, ref)
    assert torch.isfinite(out.detach().float()).all(), f"{what}: non-finite values"
    assert ma <= max_abs_tol and re <= rel_tol, f"{what}: max_abs={ma:.3e} rel={re:.3e}"
    return ma, re


def assert_state_close(st, ref, rel_tol=STATE_REL, what="state"):
    re = rel_err(st, ref)
    assert torch.isfinite(st.detach().float()).all(), f"{what}: non-finite values"
    assert re <= rel_tol, f"{what}: rel={re:.3e}"
    return re
