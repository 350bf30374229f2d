"""GPU parity of oscar_rotate_rows (x @ R on MFMA for rows of 256 features),
which replaces the prefill route's fp32 rotations (oscar_ascend/backend.py:
392-413: q / k / v `x.float() @ rk` before the attention, `out.float() @
rv.t()` after it).  Reference: the same product in float64 on the host.

Stated bounds: R enters as bf16 high + low parts (each entry to 2^-17 of
itself), fp32 input as bf16 high + low parts (to 2^-17), products accumulate
in fp32; so |got - ref| <= 2^-14 * (|x| @ |R|) for fp32 output, and bf16
output adds its rounding to nearest even (at most 2^-8 of |ref|: 8 significant bits).
"""
import pytest
import torch

from oscar_amd.kernels import quant
from oscar_amd import synthetic

pytestmark = pytest.mark.gpu

D = 256


def reference(x, R):
    return x.double().cpu() @ R.double().cpu()


def bound(x, R):
    return 2.0 ** -14 * (x.double().abs().cpu() @ R.double().abs().cpu())


@pytest.mark.parametrize("rows", [1, 127, 128, 300, 4099])
def test_bf16_rows_to_fp32(device, rows):
    g = torch.Generator().manual_seed(rows)
    R, _ = synthetic.rotations(D, 11)
    x = (torch.randn(rows, D, generator=g) * 3.0).bfloat16()
    op = quant.rotation_operand(R.to(device))
    got = quant.rotate_rows(x.to(device), op).cpu().double()
    err = (got - reference(x, R)).abs()
    assert (err <= bound(x, R)).all(), f"max excess {(err - bound(x, R)).max().item():.3e}"


@pytest.mark.parametrize("rows", [5, 333])
def test_fp32_rows_to_bf16_in_place(device, rows):
    g = torch.Generator().manual_seed(100 + rows)
    R, _ = synthetic.rotations(D, 12)
    x = torch.randn(rows, D, generator=g) * torch.logspace(-3, 3, D)      # wide dynamic range per row
    op = quant.rotation_operand(R.to(device))
    out = torch.full((rows, D), float("nan"), dtype=torch.bfloat16, device=device)
    quant.rotate_rows(x.to(device), op, torch.bfloat16, out=out)
    ref = reference(x, R)
    got = out.cpu().double()
    assert torch.isfinite(got).all()
    err = (got - ref).abs()
    assert (err <= 2.0 ** -8 * ref.abs() + bound(x, R)).all()
    # rounding of a value within 2^-14 of the exact product: almost always the exact product's rounding
    assert (got == ref.float().bfloat16().double()).float().mean().item() >= 0.99


def test_head_strided_rows_and_shapes(device):
    """[tokens, heads, D] views: the rows of a token slice of a larger tensor."""
    g = torch.Generator().manual_seed(7)
    R, _ = synthetic.rotations(D, 13)
    full = torch.randn(50, 6, D, generator=g).bfloat16().to(device)
    x = full[10:37]
    op = quant.rotation_operand(R.to(device))
    got = quant.rotate_rows(x, op)
    assert got.shape == x.shape and got.dtype == torch.float32
    err = (got.cpu().double() - reference(x.reshape(-1, D), R).reshape(x.shape)).abs()
    assert (err <= bound(x.reshape(-1, D), R).reshape(x.shape)).all()


def test_empty_and_invalid(device):
    R, _ = synthetic.rotations(D, 14)
    op = quant.rotation_operand(R.to(device))
    assert quant.rotate_rows(torch.empty(0, D, dtype=torch.bfloat16, device=device), op).shape == (0, D)
    with pytest.raises(ValueError):
        quant.rotate_rows(torch.zeros(4, D, dtype=torch.float16, device=device), op)
