"""Drop-ins for src/model/fpope_attention.py: FPoPEGroupedQueryAttention and its KV-cache variant.

Same constructor arguments, submodule / parameter names (wq_c, wk_c, wq_r, wk_r, qr_norm, kr_norm,
wv, wo, fpope) and forward signature as the reference (src/model/fpope_attention.py:57-181,
191-327), so reference checkpoints load and TransformerBlock uses them unchanged.  The span
PoPE/FoPE transform -> [content | position] concat -> GQA repeat_interleave -> causal SDPA
(src/model/fpope_attention.py:145-177) is one fused HIP forward and one HIP backward
(pe_ablations_amd.functional.pe_attention): the projections go in as (B, H, S, d) views of the
linear outputs, the kernel applies the transform in registers and maps query head h to kv head
h // (H / Hkv), and the output comes back as a (B, H, S, Dv) view of a (B, S, H, Dv) buffer.
"""

from __future__ import annotations

from typing import Optional

import torch
import torch.nn as nn

from .functional import pe_attention
from .normalization import RMSNorm


class FPoPEGroupedQueryAttention(nn.Module):
    def __init__(self, hidden_dim: int, num_heads: int, num_kv_heads: int, head_dim: int = 64,
                 d_rope: int = 32, use_qk_norm: bool = True, fpope: Optional[nn.Module] = None,
                 use_triton: Optional[bool] = None, d_content: Optional[int] = None):
        """``fpope``: a PoPEEmbedding or FoPEPoPEEmbedding (anything with kernel_freqs() /
        kernel_delta()), or None for the reference's no-PE fallback that duplicates the position
        projection.  ``use_triton`` is accepted for the legacy call sites and ignored: the HIP
        kernel is the only implementation.

        ``d_content`` (an addition; default None = ``head_dim``, the reference's split form) set
        to 0 gives the fused form of the legacy API, every head dim PoPE-encoded: no ``wq_c`` /
        ``wk_c``, ``d_rope`` must equal ``head_dim``, and the scale is that API's 1/sqrt(head_dim)
        (tests/test_fpope.py:222-226)."""
        super().__init__()
        assert num_heads % num_kv_heads == 0, "num_heads must be divisible by num_kv_heads"
        self.hidden_dim = hidden_dim
        self.num_heads = num_heads
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.d_rope = d_rope
        self.d_content = head_dim if d_content is None else int(d_content)
        if self.d_content not in (0, head_dim):
            raise ValueError(f"d_content must be head_dim ({head_dim}) or 0, got {d_content}")
        if self.d_content == 0 and d_rope != head_dim:
            raise ValueError(f"the fused form (d_content=0) needs d_rope == head_dim, got {d_rope} != {head_dim}")
        self.num_groups = num_heads // num_kv_heads
        if self.d_content:
            self.wq_c = nn.Linear(hidden_dim, num_heads * self.d_content, bias=False)
            self.wk_c = nn.Linear(hidden_dim, num_kv_heads * self.d_content, bias=False)
        else:
            self.wq_c = None
            self.wk_c = None
        self.wq_r = nn.Linear(hidden_dim, num_heads * d_rope, bias=False)
        self.wk_r = nn.Linear(hidden_dim, num_kv_heads * d_rope, bias=False)
        if use_qk_norm:
            self.qr_norm = RMSNorm(num_heads * d_rope)
            self.kr_norm = RMSNorm(num_kv_heads * d_rope)
        else:
            self.qr_norm = None
            self.kr_norm = None
        self.wv = nn.Linear(hidden_dim, num_kv_heads * head_dim, bias=False)
        self.wo = nn.Linear(num_heads * head_dim, hidden_dim, bias=False)
        self.fpope = fpope
        self.scale = (self.d_content + d_rope * 2) ** -0.5 if self.d_content else head_dim ** -0.5

    def _fuse_norm(self, x: torch.Tensor) -> bool:
        """Inference with PoPE / FoPE and QK RMSNorm on the GPU: the norm runs inside the
        transform kernel (pe_attn_fwd_normed) instead of as a separate op."""
        return (x.is_cuda and self.qr_norm is not None and self.fpope is not None
                and not torch.is_grad_enabled() and self.qr_norm.eps == self.kr_norm.eps
                and self.qr_norm.weight.dtype == self.kr_norm.weight.dtype)

    def _project(self, x: torch.Tensor, fuse_norm: bool = False):
        B, S, _ = x.shape
        if self.d_content:
            q_c = self.wq_c(x).view(B, S, self.num_heads, self.d_content).transpose(1, 2)
            k_c = self.wk_c(x).view(B, S, self.num_kv_heads, self.d_content).transpose(1, 2)
        else:
            q_c = k_c = None
        q_r = self.wq_r(x)
        k_r = self.wk_r(x)
        if self.qr_norm is not None and not fuse_norm:
            q_r = self.qr_norm(q_r)
            k_r = self.kr_norm(k_r)
        q_r = q_r.view(B, S, self.num_heads, self.d_rope).transpose(1, 2)
        k_r = k_r.view(B, S, self.num_kv_heads, self.d_rope).transpose(1, 2)
        v = self.wv(x).view(B, S, self.num_kv_heads, self.head_dim).transpose(1, 2)
        return q_c, k_c, q_r, k_r, v

    def _attend(self, q_c, k_c, q_r, k_r, v, start_q: int, start_k: int, causal,
                fuse_norm: bool = False) -> torch.Tensor:
        if self.fpope is None:
            # reference fallback: q = [q_c | q_r | q_r] without any transform (:148-151)
            dt = v.dtype
            qc = torch.cat(([q_c] if q_c is not None else []) + [q_r.to(dt), q_r.to(dt)], dim=-1)
            kc = torch.cat(([k_c] if k_c is not None else []) + [k_r.to(dt), k_r.to(dt)], dim=-1)
            return pe_attention(qc, kc, v, mode="none", scale=self.scale, causal=causal,
                                start_pos_q=start_q, start_pos_k=start_k)
        norm = {}
        if fuse_norm:
            norm = dict(qr_norm_weight=self.qr_norm.weight, kr_norm_weight=self.kr_norm.weight,
                        norm_eps=self.qr_norm.eps)
        return pe_attention(q_r, k_r, v, mode="pope", q_c=q_c, k_c=k_c, freqs=self.fpope.kernel_freqs(),
                            delta=self.fpope.kernel_delta(), scale=self.scale, causal=causal,
                            start_pos_q=start_q, start_pos_k=start_k, **norm)

    def forward(self, x: torch.Tensor, mask: Optional[torch.Tensor] = None, start_pos: int = 0) -> torch.Tensor:
        """(B, S, hidden) -> (B, S, hidden); ``mask`` is ignored (causal always, as the reference)."""
        B, S, _ = x.shape
        fuse = self._fuse_norm(x)
        q_c, k_c, q_r, k_r, v = self._project(x, fuse)
        out = self._attend(q_c, k_c, q_r, k_r, v, start_pos, start_pos, True, fuse)
        return self.wo(out.transpose(1, 2).reshape(B, S, -1))


class FPoPEGroupedQueryAttentionWithCache(FPoPEGroupedQueryAttention):
    """KV-cache variant (src/model/fpope_attention.py:184-327).  The cache holds the raw content
    keys, normalised position keys and values; the kernel re-applies the key transform with
    absolute positions 0..L-1, which reproduces the reference's cached [k_c | PoPE(k_r)] exactly,
    and masks bottom-right (query i sees keys <= L - S + i)."""

    def __init__(self, hidden_dim: int, num_heads: int, num_kv_heads: int, head_dim: int = 64,
                 d_rope: int = 32, use_qk_norm: bool = True, fpope: Optional[nn.Module] = None,
                 max_cache_len: int = 2048, use_triton: Optional[bool] = None, d_content: Optional[int] = None):
        super().__init__(hidden_dim, num_heads, num_kv_heads, head_dim, d_rope, use_qk_norm, fpope,
                         d_content=d_content)
        self.max_cache_len = max_cache_len
        self.register_buffer("k_cache", None, persistent=False)
        self.register_buffer("v_cache", None, persistent=False)
        self.kr_cache: Optional[torch.Tensor] = None
        self.cache_len = 0

    def reset_cache(self) -> None:
        self.k_cache = None
        self.v_cache = None
        self.kr_cache = None
        self.cache_len = 0

    def forward(self, x: torch.Tensor, mask: Optional[torch.Tensor] = None, start_pos: int = 0,
                use_cache: bool = False) -> torch.Tensor:
        if not use_cache:
            return super().forward(x, mask, start_pos)
        B, S, _ = x.shape
        q_c, k_c, q_r, k_r, v = self._project(x)
        if self.kr_cache is None:
            if k_c is not None:
                self.k_cache = torch.zeros(B, self.num_kv_heads, self.max_cache_len, self.d_content,
                                           dtype=k_c.dtype, device=x.device)
            self.kr_cache = torch.zeros(B, self.num_kv_heads, self.max_cache_len, self.d_rope,
                                        dtype=k_r.dtype, device=x.device)
            self.v_cache = torch.zeros(B, self.num_kv_heads, self.max_cache_len, self.head_dim,
                                       dtype=v.dtype, device=x.device)
        if k_c is not None:
            self.k_cache[:, :, start_pos:start_pos + S] = k_c
        self.kr_cache[:, :, start_pos:start_pos + S] = k_r
        self.v_cache[:, :, start_pos:start_pos + S] = v
        self.cache_len = start_pos + S
        L = self.cache_len
        k_c_all = self.k_cache[:, :, :L] if k_c is not None else None
        out = self._attend(q_c, k_c_all, q_r, self.kr_cache[:, :, :L], self.v_cache[:, :, :L],
                           start_pos, 0, "bottom_right")
        return self.wo(out.transpose(1, 2).reshape(B, S, -1))
