"""RoPE / NTK / YaRN embeddings, drop-ins for src/model/rope.py.

Constructors, the ``freqs_cis`` buffer (non-persistent, (max_seq_len, dim/2) complex64),
``extend_seq_len`` and ``forward(xq, xk, start_pos)`` follow src/model/rope.py:60-217.  The
rotation itself (interleaved pairs (x0,x1),(x2,x3)... by angle fl(t * w_i), times YaRN's mscale)
runs in the HIP library: inside the fused attention (GroupedQueryAttention) or, for a direct
``forward`` call, through the standalone HIP transform.  ``inv_freq`` holds the per-pair inverse
frequency the kernels use; ``freqs_cis`` is kept for checkpoint / API compatibility.
"""

from __future__ import annotations

import math

import torch
import torch.nn as nn

from .transform import pe_transform


def precompute_freqs_cis(dim: int, max_seq_len: int, theta: float = 10000.0, device=None) -> torch.Tensor:
    """polar(1, outer(t, 1/theta^(2i/dim))), (max_seq_len, dim/2) complex64 (src/model/rope.py:11-32)."""
    freqs = 1.0 / (theta ** (torch.arange(0, dim, 2, device=device).float() / dim))
    t = torch.arange(max_seq_len, device=device)
    freqs = torch.outer(t, freqs)
    return torch.polar(torch.ones_like(freqs), freqs)


def rope_inv_freq(dim: int, theta: float, device=None) -> torch.Tensor:
    return 1.0 / (theta ** (torch.arange(0, dim, 2, device=device).float() / dim))


class RotaryEmbedding(nn.Module):
    def __init__(self, dim: int, max_seq_len: int = 2048, theta: float = 10000.0):
        super().__init__()
        self.dim = dim
        self.max_seq_len = max_seq_len
        self.theta = theta
        self.register_buffer("freqs_cis", precompute_freqs_cis(dim, max_seq_len, theta), persistent=False)
        self.register_buffer("inv_freq", rope_inv_freq(dim, theta), persistent=False)

    def kernel_inv_freq(self) -> torch.Tensor:
        return self.inv_freq

    def kernel_mscale(self) -> float:
        return 1.0

    def forward(self, xq: torch.Tensor, xk: torch.Tensor, start_pos: int = 0):
        """(B, S, H, D) query / key -> rotated, same dtype as the inputs (src/model/rope.py:83-101)."""
        ms = self.kernel_mscale()
        rq = pe_transform(xq, self.inv_freq, None, start_pos=start_pos, mode="rope", mscale=ms)
        rk = pe_transform(xk, self.inv_freq, None, start_pos=start_pos, mode="rope", mscale=ms)
        return rq.to(xq.dtype), rk.to(xk.dtype)

    def extend_seq_len(self, new_max_seq_len: int) -> None:
        """Rebuild the standard table from self.theta (src/model/rope.py:103-119).  Inherited by
        YaRN unchanged, so YaRN reverts to the plain RoPE frequencies past max_seq_len while its
        mscale stays, exactly as the reference behaves."""
        if new_max_seq_len <= self.max_seq_len:
            return
        dev = self.freqs_cis.device
        self.register_buffer("freqs_cis", precompute_freqs_cis(self.dim, new_max_seq_len, self.theta, dev),
                             persistent=False)
        self.register_buffer("inv_freq", rope_inv_freq(self.dim, self.theta, dev), persistent=False)
        self.max_seq_len = new_max_seq_len


class NTKAwareRotaryEmbedding(RotaryEmbedding):
    """theta' = theta * scale^(dim/(dim-2)) (src/model/rope.py:122-140)."""

    def __init__(self, dim: int, max_seq_len: int = 2048, theta: float = 10000.0, scale: float = 1.0):
        self.scale = scale
        super().__init__(dim, max_seq_len, theta * (scale ** (dim / (dim - 2))))


class YaRNRotaryEmbedding(RotaryEmbedding):
    """Ramp between extrapolated and interpolated inverse frequencies, bounds low/high without the
    paper's /2, mscale = 0.1 ln(scale) + 1 on q and k (src/model/rope.py:143-217)."""

    def __init__(self, dim: int, max_seq_len: int = 2048, theta: float = 10000.0, scale: float = 1.0,
                 original_max_seq_len: int = 512, beta_fast: float = 32.0, beta_slow: float = 1.0):
        super().__init__(dim, max_seq_len, theta)
        self.scale = scale
        self.original_max_seq_len = original_max_seq_len
        self.beta_fast = beta_fast
        self.beta_slow = beta_slow
        self._compute_yarn_freqs()

    def _compute_yarn_freqs(self) -> None:
        dim, theta, scale = self.dim, self.theta, self.scale
        pos_freqs = theta ** (torch.arange(0, dim, 2).float() / dim)
        extra = 1.0 / pos_freqs
        inter = 1.0 / (scale * pos_freqs)
        low = max(int(math.floor(dim * math.log(self.original_max_seq_len / (self.beta_fast * 2 * math.pi))
                                 / math.log(theta))), 0)
        high = min(int(math.ceil(dim * math.log(self.original_max_seq_len / (self.beta_slow * 2 * math.pi))
                                 / math.log(theta))), dim - 1)
        inv = inter.clone()
        inv[:low] = extra[:low]
        if low < high:
            smooth = (torch.arange(low, high + 1).float() - low) / (high - low)
            inv[low:high + 1] = (1 - smooth) * extra[low:high + 1] + smooth * inter[low:high + 1]
        self.low, self.high = low, high
        t = torch.arange(self.max_seq_len)
        ang = torch.outer(t, inv)
        self.register_buffer("freqs_cis", torch.polar(torch.ones_like(ang), ang), persistent=False)
        self.register_buffer("inv_freq", inv, persistent=False)
        self.register_buffer("mscale", torch.tensor(0.1 * math.log(scale) + 1.0), persistent=False)

    def kernel_mscale(self) -> float:
        return float(self.mscale)
