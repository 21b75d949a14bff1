"""RMSNorm and QKNorm, same parameters and semantics as src/model/normalization.py.

RMSNorm: x * rsqrt(mean(x^2) + eps) in fp32, cast back to x's dtype, times the weight (which
promotes the result to fp32 when the weight is fp32, the precision the PoPE transform then sees).
When no gradient is needed and the tensor is on the GPU it runs the library's one-pass HIP kernel
(pe_rmsnorm_fwd); in training it is the reference's torch expression, whose autograd gives the
backward.  On the position projections of the PoPE attention, inference skips the module
altogether: the norm is fused into the attention's transform kernel.  QKNorm is fused into the
attention kernel for the RoPE / no-PE modules (qk_l2norm); the module form here serves direct
callers.
"""

import torch
import torch.nn as nn

from .functional import rms_norm as _hip_rms_norm

_HIP_NORM_MAX = 8192


class RMSNorm(nn.Module):
    def __init__(self, dim: int, eps: float = 1e-6):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))

    def _norm(self, x: torch.Tensor) -> torch.Tensor:
        return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + self.eps)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        n = x.shape[-1]
        if (x.is_cuda and not torch.is_grad_enabled() and n % 8 == 0 and n <= _HIP_NORM_MAX
                and x.dtype in (torch.bfloat16, torch.float32)
                and self.weight.dtype in (torch.bfloat16, torch.float32)):
            return _hip_rms_norm(x, self.weight, self.eps)
        return self._norm(x.float()).type_as(x) * self.weight


class QKNorm(nn.Module):
    """q / (||q|| + eps), k / (||k|| + eps) over the head dim (eps added to the norm)."""

    def __init__(self, head_dim: int, eps: float = 1e-6):
        super().__init__()
        self.eps = eps
        self.head_dim = head_dim

    def forward(self, q: torch.Tensor, k: torch.Tensor):
        return q / (q.norm(dim=-1, keepdim=True) + self.eps), k / (k.norm(dim=-1, keepdim=True) + self.eps)
