"""Pure PoPE embedding, drop-in for src/model/pope.py:PoPEEmbedding.

Same constructor, buffers and parameter (``freqs``, ``effective_freqs``, ``base_angles``,
``phase_bias``) so reference checkpoints load unchanged (src/model/pope.py:47-97).  The attention
modules do not call ``forward_query`` / ``forward_key``: they hand the raw position projections,
``kernel_freqs()`` and ``kernel_delta()`` to the fused HIP attention, which applies the transform
in-kernel.  The standalone transforms run the library's HIP transform kernel (forward and
backward); there is no eager path.
"""

from __future__ import annotations

import math
from typing import Literal

import torch
import torch.nn as nn

from .transform import pe_transform


class PoPEEmbedding(nn.Module):
    """Polar position encoding: magnitude softplus(x), phase pos*theta (+ clamp(delta) on keys).

    Args mirror src/model/pope.py:47-55: dim, max_seq_len, theta, training_length, use_floor,
    delta_init ("zero" or "uniform" = U(-2pi, 0))."""

    def __init__(self, dim: int, max_seq_len: int = 2048, theta: float = 10000.0,
                 training_length: int = 512, use_floor: bool = False,
                 delta_init: Literal["zero", "uniform"] = "zero"):
        super().__init__()
        self.dim = dim
        self.n_freq = dim
        self.max_seq_len = max_seq_len
        self.theta_base = theta
        self.training_length = training_length
        self.use_floor = use_floor
        self.delta_init = delta_init
        self.floor_freq = 2 * math.pi / training_length
        freqs = theta ** (-(torch.arange(0, dim, dtype=torch.float32) / dim))
        self.register_buffer("freqs", freqs)
        eff = torch.where(freqs < self.floor_freq, torch.zeros_like(freqs), freqs) if use_floor else freqs
        self.register_buffer("effective_freqs", eff)
        pos = torch.arange(max_seq_len, dtype=torch.float32)
        self.register_buffer("base_angles", torch.outer(pos, self.effective_freqs))
        if delta_init == "zero":
            phase_bias = torch.zeros(dim)
        else:
            phase_bias = torch.rand(dim) * 2 * math.pi - 2 * math.pi
        self.phase_bias = nn.Parameter(phase_bias)

    # --- what the fused attention consumes -------------------------------------------------
    def kernel_freqs(self) -> torch.Tensor:
        """Per-dim frequency the kernel multiplies by the position (fp32, (dim,))."""
        return self.effective_freqs

    def kernel_delta(self) -> torch.Tensor:
        """Key phase bias as used: clamp(delta, -2pi, 0) (src/model/pope.py:172), differentiable."""
        return self.phase_bias.clamp(-2 * math.pi, 0.0)

    # --- reference interface ---------------------------------------------------------------
    def extend_seq_len(self, new_max_seq_len: int) -> None:
        """Extend the angle cache (src/model/pope.py:106-122); the kernels compute fl(pos*theta)
        directly, which is bit-identical to the cached table."""
        if new_max_seq_len <= self.max_seq_len:
            return
        pos = torch.arange(new_max_seq_len, dtype=torch.float32, device=self.freqs.device)
        self.register_buffer("base_angles", torch.outer(pos, self.effective_freqs), persistent=False)
        self.max_seq_len = new_max_seq_len

    def forward_query(self, x: torch.Tensor, start_pos: int = 0) -> torch.Tensor:
        """(B, S, H, D) -> (B, S, H, 2D) [mu cos(t theta), mu sin(t theta)] (src/model/pope.py:124-149)."""
        return pe_transform(x, self.kernel_freqs(), None, start_pos=start_pos, is_key=False)

    def forward_key(self, x: torch.Tensor, start_pos: int = 0) -> torch.Tensor:
        """(B, S, H, D) -> (B, S, H, 2D) with phase s theta + clamp(delta) (src/model/pope.py:151-183)."""
        return pe_transform(x, self.kernel_freqs(), self.kernel_delta(), start_pos=start_pos, is_key=True)

    def forward(self, x: torch.Tensor, apply_delta: bool = True, start_pos: int = 0) -> torch.Tensor:
        return self.forward_key(x, start_pos) if apply_delta else self.forward_query(x, start_pos)
