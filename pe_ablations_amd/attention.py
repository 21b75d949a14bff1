"""Drop-in for src/model/attention.py:GroupedQueryAttention (pe_mode "rope" and "nope").

Same constructor, submodules (wq, wk, wv, wo, qk_norm, rope) and forward.  The span
RoPE rotation -> QKNorm -> GQA repeat_interleave -> causal SDPA (src/model/attention.py:77-96) is
one fused HIP forward / backward: the kernel rotates the interleaved pairs by fl(t * w_i) (times
YaRN's mscale), applies QKNorm x / (||x|| + 1e-6) when the module has one, and uses the
reference's scale 1/sqrt(head_dim).
"""

from __future__ import annotations

from typing import Optional

import torch
import torch.nn as nn

from .fpope_attention import KVCache, cached_attention
from .functional import pe_attention
from .normalization import QKNorm


class GroupedQueryAttention(nn.Module):
    def __init__(self, hidden_dim: int, num_heads: int, num_kv_heads: int, head_dim: Optional[int] = None,
                 use_qk_norm: bool = True, rope: Optional[nn.Module] = None):
        super().__init__()
        self.hidden_dim = hidden_dim
        self.num_heads = num_heads
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim or (hidden_dim // num_heads)
        self.num_groups = num_heads // num_kv_heads
        assert num_heads % num_kv_heads == 0, "num_heads must be divisible by num_kv_heads"
        self.wq = nn.Linear(hidden_dim, num_heads * self.head_dim, bias=False)
        self.wk = nn.Linear(hidden_dim, num_kv_heads * self.head_dim, bias=False)
        self.wv = nn.Linear(hidden_dim, num_kv_heads * self.head_dim, bias=False)
        self.wo = nn.Linear(num_heads * self.head_dim, hidden_dim, bias=False)
        self.qk_norm = QKNorm(self.head_dim) if use_qk_norm else None
        self.rope = rope
        # KV cache for generation (an addition: the reference's RoPE / no-PE module has no cache and
        # its generate re-runs the whole sequence, src/model/transformer.py:389-446)
        self.max_cache_len = 2048
        self.cache = KVCache()

    def reset_cache(self) -> None:
        self.cache.reset()

    def forward(self, x: torch.Tensor, mask: Optional[torch.Tensor] = None, start_pos: int = 0,
                use_cache: bool = False) -> torch.Tensor:
        """``mask``: None for the causal path; else SDPA's attn_mask, bool (True = attend) or float
        (added to the scaled scores), broadcastable to (B, num_heads, S, S), applied without the
        causal mask as the reference does (is_causal=(mask is None), src/model/attention.py:91-96).
        ``use_cache`` keeps the rotated, normalised keys of earlier calls (with gradients, their
        autograd history too) and attends the new queries to all of them under the bottom-right
        causal mask; it takes no explicit mask."""
        if mask is not None and use_cache:
            raise NotImplementedError("GroupedQueryAttention: use_cache takes no explicit mask")
        B, S, _ = x.shape
        q = self.wq(x).view(B, S, self.num_heads, self.head_dim).transpose(1, 2)
        k = self.wk(x).view(B, S, self.num_kv_heads, self.head_dim).transpose(1, 2)
        v = self.wv(x).view(B, S, self.num_kv_heads, self.head_dim).transpose(1, 2)
        norm = self.qk_norm is not None
        if use_cache:
            rope = {} if self.rope is None else dict(freqs=self.rope.kernel_inv_freq(),
                                                     rope_mscale=self.rope.kernel_mscale())
            out = cached_attention(self.cache, self.max_cache_len, start_pos, q=q, k=k, v=v,
                                   mode="rope" if self.rope is not None else "none", qk_norm=norm,
                                   scale=1.0 / (self.head_dim ** 0.5), d_v=self.head_dim, **rope)
            out = out.transpose(1, 2).reshape(B, S, -1)
            return self.wo(out if torch.is_autocast_enabled() else out.to(x.dtype))
        causal = mask is None
        if self.rope is not None:
            out = pe_attention(q, k, v, mode="rope", freqs=self.rope.kernel_inv_freq(),
                               rope_mscale=self.rope.kernel_mscale(), qk_norm=norm,
                               scale=1.0 / (self.head_dim ** 0.5), causal=causal,
                               start_pos_q=start_pos, start_pos_k=start_pos, mask=mask)
        else:
            out = pe_attention(q, k, v, mode="none", qk_norm=norm, scale=1.0 / (self.head_dim ** 0.5),
                               causal=causal, start_pos_q=start_pos, start_pos_k=start_pos, mask=mask)
        return self.wo(out.transpose(1, 2).reshape(B, S, -1))
