"""Drop-ins for src/model/ffn.py: SwiGLU and the three-projection FeedForward.

Same parameter names (w1, w2, w3) and the same gating as the reference: the activation is called
as ``activation(w1(x), w3(x))`` and returns ``silu(gate) * x``, so w3 is the gate
(src/model/ffn.py:17-27,53-68).  The projections are plain hipBLASLt GEMMs through torch.  When no
gradient is needed, bf16 SwiGLU on the GPU runs the library's one-pass kernel (pe_swiglu_fwd),
bitwise equal to torch's two ops; in training it is the reference's torch expression.
"""

from __future__ import annotations

from typing import Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from .functional import swiglu as _hip_swiglu


class SwiGLU(nn.Module):
    """silu(gate) * x (src/model/ffn.py:8-27)."""

    def forward(self, x: torch.Tensor, gate: torch.Tensor) -> torch.Tensor:
        if (x.is_cuda and not torch.is_grad_enabled() and x.dtype == torch.bfloat16
                and gate.dtype == torch.bfloat16 and x.shape == gate.shape):
            return _hip_swiglu(x, gate)
        return F.silu(gate) * x


class FeedForward(nn.Module):
    """w2(silu(w3 x) * w1 x); hidden size ``ffn_dim`` or 4*hidden*2/3 rounded up to ``multiple_of``
    (src/model/ffn.py:30-68)."""

    def __init__(self, hidden_dim: int, ffn_dim: Optional[int] = None, multiple_of: int = 256):
        super().__init__()
        if ffn_dim is None:
            ffn_dim = int(4 * hidden_dim * 2 / 3)
            ffn_dim = multiple_of * ((ffn_dim + multiple_of - 1) // multiple_of)
        self.w1 = nn.Linear(hidden_dim, ffn_dim, bias=False)
        self.w2 = nn.Linear(ffn_dim, hidden_dim, bias=False)
        self.w3 = nn.Linear(hidden_dim, ffn_dim, bias=False)
        self.activation = SwiGLU()

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.w2(self.activation(self.w1(x), self.w3(x)))
