"""FoPE + PoPE embedding, drop-in for src/model/fpope.py:FoPEPoPEEmbedding.

Same constructor, buffers and parameters (``base_freqs``, ``fourier_coeffs``, ``fourier_indices``,
``phase_bias``, ``positions``; src/model/fpope.py:44-105).  FoPE collapses to one effective
frequency per dim (src/model/fpope.py:107-146), computed here with torch ops so that autograd
carries the kernel's frequency gradient into ``fourier_coeffs``; the fused HIP attention then
runs exactly the PoPE kernel with freqs = omega.
"""

from __future__ import annotations

import math
from typing import Literal, Optional

import torch
import torch.nn as nn

from .transform import pe_transform


class FoPEPoPEEmbedding(nn.Module):
    def __init__(self, dim: int, max_seq_len: int = 2048, theta: float = 10000.0,
                 num_fourier_terms: int = 64, fourier_sigma: float = 0.4,
                 training_length: int = 512, delta_init: Literal["zero", "uniform"] = "zero",
                 freeze_coeffs: bool = False, use_ceiling: bool = False,
                 normalize_coeffs: bool = True, freq_table: Optional[torch.Tensor] = None):
        """Args mirror src/model/fpope.py:44-56.  ``freq_table`` (dim, M), optional: replaces the
        harmonic table base_freqs[c] * j with an arbitrary per-dim table (the build's benchmark
        configuration draws the extra frequencies at random); None keeps the reference."""
        super().__init__()
        self.dim = dim
        self.max_seq_len = max_seq_len
        self.theta = theta
        self.num_fourier_terms = num_fourier_terms
        self.fourier_sigma = fourier_sigma
        self.training_length = training_length
        self.delta_init = delta_init
        self.floor_freq = 2 * math.pi / training_length
        self.use_ceiling = use_ceiling
        self.ceiling_freq = 2 * math.pi
        self.normalize_coeffs = normalize_coeffs
        base_freqs = theta ** (-torch.arange(0, dim, dtype=torch.float32) / dim)
        self.register_buffer("base_freqs", base_freqs)
        coeffs = torch.randn(dim, num_fourier_terms) * fourier_sigma
        self.fourier_coeffs = nn.Parameter(coeffs, requires_grad=not freeze_coeffs)
        self.register_buffer("fourier_indices", torch.arange(1, num_fourier_terms + 1, dtype=torch.float32))
        if freq_table is not None:
            if tuple(freq_table.shape) != (dim, num_fourier_terms):
                raise ValueError("freq_table must be (dim, num_fourier_terms)")
            self.register_buffer("freq_table", freq_table.float().clone(), persistent=False)
        else:
            self.freq_table = None
        if delta_init == "zero":
            phase_bias = torch.zeros(dim)
        else:
            phase_bias = torch.rand(dim) * 2 * math.pi - math.pi
        self.phase_bias = nn.Parameter(phase_bias)
        self.register_buffer("positions", torch.arange(max_seq_len, dtype=torch.float32))

    def _compute_effective_freqs(self) -> torch.Tensor:
        """omega = theta + sum_j a_hat_cj * f_cj, floor clip, optional ceiling clamp
        (src/model/fpope.py:107-146); f_cj = theta_c * j unless a freq_table was given."""
        if self.normalize_coeffs:
            a = self.fourier_coeffs / (self.fourier_coeffs.abs().sum(dim=1, keepdim=True) + 1e-8)
        else:
            a = self.fourier_coeffs
        table = self.freq_table
        if table is None:
            table = self.base_freqs.unsqueeze(1) * self.fourier_indices.unsqueeze(0)
        eff = (a * table).sum(dim=1) + self.base_freqs
        eff = torch.where(eff.abs() < self.floor_freq, torch.zeros_like(eff), eff)
        if self.use_ceiling:
            eff = eff.clamp(-self.ceiling_freq, self.ceiling_freq)
        return eff

    def kernel_freqs(self) -> torch.Tensor:
        return self._compute_effective_freqs()

    def kernel_delta(self) -> torch.Tensor:
        return self.phase_bias.clamp(-2 * math.pi, 0.0)

    def get_frequencies_and_phases(self, seq_len: int, start_pos: int = 0):
        """(effective_freqs, positions[start:start+seq_len], phase_bias) (src/model/fpope.py:148-167)."""
        return self._compute_effective_freqs(), self.positions[start_pos:start_pos + seq_len], self.phase_bias

    def forward(self, q: torch.Tensor, k: torch.Tensor, start_pos: int = 0):
        """(mu_q, mu_k, effective_freqs, positions, phase_bias) (src/model/fpope.py:169-206)."""
        freqs, pos, bias = self.get_frequencies_and_phases(q.shape[1], start_pos)
        return torch.nn.functional.softplus(q), torch.nn.functional.softplus(k), freqs, pos, bias

    def compute_attention_phases(self, seq_len_q: int, seq_len_k: int, start_pos: int = 0,
                                 device: Optional[torch.device] = None) -> torch.Tensor:
        """(s - t) * omega + delta, shape (Sq, Sk, dim) (src/model/fpope.py:208-244)."""
        device = self.base_freqs.device if device is None else device
        eff = self._compute_effective_freqs()
        pq = torch.arange(start_pos, start_pos + seq_len_q, device=device)
        pk = torch.arange(start_pos, start_pos + seq_len_k, device=device)
        return (pk.unsqueeze(0) - pq.unsqueeze(1)).unsqueeze(-1) * eff + self.phase_bias

    def extend_seq_len(self, new_max_seq_len: int) -> None:
        if new_max_seq_len <= self.max_seq_len:
            return
        self.register_buffer("positions", torch.arange(new_max_seq_len, dtype=torch.float32,
                                                        device=self.positions.device), persistent=False)
        self.max_seq_len = new_max_seq_len

    # the reference builds the positions of forward_query / forward_key with
    # torch.arange(..., dtype=x.dtype) (src/model/fpope.py:285,322): rounded to bf16 for a bf16 x
    positions_in_input_dtype = True

    def forward_query(self, x: torch.Tensor, start_pos: int = 0) -> torch.Tensor:
        return pe_transform(x, self.kernel_freqs(), None, start_pos=start_pos, is_key=False,
                            position_dtype=x.dtype)

    def forward_key(self, x: torch.Tensor, start_pos: int = 0) -> torch.Tensor:
        return pe_transform(x, self.kernel_freqs(), self.kernel_delta(), start_pos=start_pos, is_key=True,
                            position_dtype=x.dtype)
