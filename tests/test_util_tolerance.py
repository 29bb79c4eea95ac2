"""The output comparison allows exactly the rounding of the result to its dtype."""
import torch

from util import half_ulp, max_abs_beyond_rounding


def test_exact_bf16_rounding_is_free_and_one_more_ulp_is_not():
    ref = torch.linspace(-40, 40, 10001, dtype=torch.float64)
    exact = ref.to(torch.bfloat16)
    assert max_abs_beyond_rounding(exact, ref) == 0.0
    # moving every element by one full ulp exceeds the allowance by about half an ulp
    one_up = (exact.double() + 2 * half_ulp(ref, torch.bfloat16) * torch.sign(ref)).to(torch.bfloat16)
    assert max_abs_beyond_rounding(one_up, ref) > 0.05


def test_fp32_outputs_get_no_allowance():
    ref = torch.tensor([1.0, 10.0], dtype=torch.float64)
    assert torch.equal(half_ulp(ref, torch.float32), torch.zeros(2, dtype=torch.float64))
    assert abs(max_abs_beyond_rounding(ref.float() + 0.01, ref) - 0.01) < 1e-6


def test_half_ulp_values():
    r = torch.tensor([1.0, 1.5, 4.0, 0.0], dtype=torch.float64)
    assert torch.equal(half_ulp(r, torch.bfloat16), torch.tensor([2.0 ** -8, 2.0 ** -8, 2.0 ** -6, 0.0],
                                                                  dtype=torch.float64))
