"""RMSNorm and QKNorm, same parameters and semantics as src/model/normalization.py.

RMSNorm runs upstream of the kernel on the position projections (src/model/fpope_attention.py:
135-137) and stays a torch op: x * rsqrt(mean(x^2) + eps) in fp32, cast back, times the weight
(which promotes the result to fp32, the precision the PoPE transform then sees).  QKNorm is fused
into the attention kernel for the RoPE / no-PE modules (qk_l2norm); the module form here serves
direct callers.
"""

import torch
import torch.nn as nn


class RMSNorm(nn.Module):
    def __init__(self, dim: int, eps: float = 1e-6):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))

    def _norm(self, x: torch.Tensor) -> torch.Tensor:
        return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + self.eps)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self._norm(x.float()).type_as(x) * self.weight


class QKNorm(nn.Module):
    """q / (||q|| + eps), k / (||k|| + eps) over the head dim (eps added to the norm)."""

    def __init__(self, head_dim: int, eps: float = 1e-6):
        super().__init__()
        self.eps = eps
        self.head_dim = head_dim

    def forward(self, q: torch.Tensor, k: torch.Tensor):
        return q / (q.norm(dim=-1, keepdim=True) + self.eps), k / (k.norm(dim=-1, keepdim=True) + self.eps)
