"""Error measures shared by the GPU parity tests.

``err`` is the raw max-abs difference |a - ref| against the oracle: the north-star bar (2e-2 in
bf16 mode, 1e-5 in fp32 mode) applies to it directly.  ``err_net`` is the same difference net of
the result's own rounding to bf16, max(|a - ref| - ulp_bf16(ref) / 2): a bf16 number cannot sit
closer to the exact value than half the bf16 spacing at that value (2^-9 relative, 0.0156 at |x| in
[4, 8)).  It is reported beside the raw figure and asserted only where a test names the element
whose magnitude puts the raw bar out of reach of any bf16 result."""

import torch

# (name, raw, net) of every comparison made in this process, printed by the tests that want them
RECORD = []


def half_ulp_bf16(ref: torch.Tensor) -> torch.Tensor:
    _, e = torch.frexp(ref.abs())          # |ref| in [2^(e-1), 2^e): bf16 spacing 2^(e-8)
    return torch.where(ref == 0, torch.zeros_like(ref), torch.ldexp(torch.ones_like(ref), e - 9))


def err_both(a: torch.Tensor, ref: torch.Tensor):
    """(raw, net) max-abs errors of ``a`` against ``ref``; net == raw unless ``a`` is bf16."""
    ad, rd = a.detach().double().cpu(), ref.detach().double().cpu()
    d = (ad - rd).abs()
    if not d.numel():
        return 0.0, 0.0
    raw = d.max().item()
    if a.dtype == torch.bfloat16:
        net = max((d - half_ulp_bf16(rd)).max().item(), 0.0)
    else:
        net = raw
    return raw, net


def err(a: torch.Tensor, ref: torch.Tensor, name: str = "") -> float:
    """Raw max-abs error of ``a`` against ``ref`` (the bar the parity tests assert)."""
    raw, net = err_both(a, ref)
    RECORD.append((name, raw, net))
    return raw


def err_net(a: torch.Tensor, ref: torch.Tensor, name: str = "") -> float:
    """Max-abs error net of ``a``'s own bf16 rounding (see the module docstring)."""
    raw, net = err_both(a, ref)
    RECORD.append((name, raw, net))
    return net


def argmax_err(a: torch.Tensor, ref: torch.Tensor):
    """(index, |ref| there, |a - ref| there) of the largest raw difference, for messages."""
    d = (a.detach().double().cpu() - ref.detach().double().cpu()).abs()
    i = int(d.argmax())
    idx = tuple(int(x) for x in torch.unravel_index(torch.tensor(i), d.shape))
    return idx, ref.detach().double().cpu().reshape(-1)[i].abs().item(), d.reshape(-1)[i].item()
