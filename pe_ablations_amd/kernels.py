"""The removed fused-kernel API of the reference (src/model/kernels/fpope_attention.py, known from
its call sites tests/test_fpope.py:18-23,222-226,1612-1615 and scripts/diagnose_kernel.py:180-188),
served by the HIP library.

Semantics of that API: q, k, v (B, H, S, D); softplus magnitudes inside; phase
(s - t) * freqs + phase_bias with no clamp; scale 1/sqrt(D) unless given; causal top-left.  The
kernel evaluates it in the factorised form q~ = mu [cos t w, sin t w], k~ = mu [cos(s w + b),
sin(s w + b)], whose dot product is the same sum.  GPU tensors only; there is no PyTorch
fallback (the CPU restatement lives in oracle/ as a test checker).
"""

from __future__ import annotations

import math
from typing import Optional

import torch

from . import _lib
from .functional import pe_attention

HAS_HIP_KERNEL = _lib.available()
HAS_TRITON = False          # no Triton in this build
HAS_CUDA_KERNEL = False     # no CUDA in this build


def fpope_attention_forward(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, freqs: torch.Tensor,
                            phase_bias: torch.Tensor, start_pos: int = 0, causal: bool = True,
                            scale: Optional[float] = None, use_triton: Optional[bool] = None) -> torch.Tensor:
    """Fused PoPE attention -> (B, H, S, D).  Differentiable w.r.t. q, k, v, freqs, phase_bias.
    ``use_triton`` is accepted for the legacy call sites and ignored."""
    D = q.shape[-1]
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    return pe_attention(q, k, v, mode="pope", freqs=freqs, delta=phase_bias, scale=scale,
                        causal=bool(causal), start_pos_q=start_pos, start_pos_k=start_pos)


def hip_fpope_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, freqs: torch.Tensor,
                        bias: torch.Tensor, start_pos: int = 0, return_lse: bool = False,
                        causal: bool = True, scale: Optional[float] = None):
    """Counterpart of triton_fpope_attention(q, k, v, freqs, bias, start_pos, return_lse)
    (scripts/diagnose_kernel.py:180-195): returns out, or (out, lse) with lse shaped (B*H, S)."""
    D = q.shape[-1]
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    out, lse = pe_attention(q, k, v, mode="pope", freqs=freqs, delta=bias, scale=scale, causal=bool(causal),
                            start_pos_q=start_pos, start_pos_k=start_pos, return_lse=True)
    if return_lse:
        return out, lse.reshape(-1, lse.shape[-1])
    return out
