"""Error measure shared by the GPU parity tests.

A bf16 result cannot sit closer to the exact value than half the bf16 spacing at that value
(2^-9 relative, 0.0156 at |x| in [4, 8)), so in bf16 mode the north-star bar (max-abs 2e-2) applies
to the error beyond that rounding: max(|a - ref| - ulp_bf16(ref) / 2).  fp32 results are compared
plainly, max |a - ref|."""

import torch


def half_ulp_bf16(ref: torch.Tensor) -> torch.Tensor:
    _, e = torch.frexp(ref.abs())          # |ref| in [2^(e-1), 2^e): bf16 spacing 2^(e-8)
    return torch.where(ref == 0, torch.zeros_like(ref), torch.ldexp(torch.ones_like(ref), e - 9))


def err(a: torch.Tensor, ref: torch.Tensor) -> float:
    """max-abs error of ``a`` against ``ref``, net of ``a``'s own bf16 rounding when ``a`` is bf16."""
    d = (a.detach().double().cpu() - ref.detach().double().cpu()).abs()
    if a.dtype == torch.bfloat16:
        d = d - half_ulp_bf16(ref.detach().double().cpu())
    return max(d.max().item(), 0.0) if d.numel() else 0.0
