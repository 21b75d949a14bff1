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

from .functional import cache_widths, norm_out_dtype, pe_attention, pe_attention_decode, pe_cache_append
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
        """PoPE / FoPE with QK RMSNorm on the GPU: the norm runs inside the transform kernel
        (pe_attn_fwd_normed) instead of as a separate op; in training its backward follows the
        attention backward (pe_rmsnorm_bwd), with the same gradients for the projections and the
        norm weights as the module's RMSNorm under autograd."""
        return (x.is_cuda and self.qr_norm is not None and self.fpope is not None
                and self.qr_norm.eps == self.kr_norm.eps
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
        x_dtype = q_r.dtype  # what the reference's forward_query / forward_key receive
        if fuse_norm:
            norm = dict(qr_norm_weight=self.qr_norm.weight, kr_norm_weight=self.kr_norm.weight,
                        norm_eps=self.qr_norm.eps)
            # RMSNorm's output dtype: the 16-bit type when the projection and the weight share it
            x_dtype = norm_out_dtype(q_r.dtype, self.qr_norm.weight.dtype)
        return pe_attention(q_r, k_r, v, mode="pope", q_c=q_c, k_c=k_c, freqs=self.fpope.kernel_freqs(),
                            delta=self.fpope.kernel_delta(), scale=self.scale, causal=causal,
                            start_pos_q=start_q, start_pos_k=start_k,
                            position_dtype=kernel_position_dtype(self.fpope, x_dtype), **norm)

    def forward(self, x: torch.Tensor, mask: Optional[torch.Tensor] = None, start_pos: int = 0) -> torch.Tensor:
        """(B, S, hidden) -> (B, S, hidden); ``mask`` is ignored (causal always, as the reference)."""
        B, S, _ = x.shape
        fuse = self._fuse_norm(x)
        q_c, k_c, q_r, k_r, v = self._project(x, fuse)
        out = self._attend(q_c, k_c, q_r, k_r, v, start_pos, start_pos, True, fuse)
        return self.wo(out.transpose(1, 2).reshape(B, S, -1))


class KVCache:
    """Per-layer cache of transformed keys and values for the decode path.

    ``k_cache`` (B, Hkv, capacity, Wk) holds the library's operand rows [content | transform | zero
    pad] in the compute dtype (its first Dc + 2*Dr columns are the reference's cached
    [k_c | PoPE(k_r)], src/model/fpope_attention.py:283-296); ``v_cache`` (B, Hkv, capacity, Wv)
    the zero-padded values.  New rows are transformed once, when appended; every later step reads
    them as they are."""

    def __init__(self):
        self.k = None
        self.v = None
        self.length = 0
        # (k rows, v rows) carrying the autograd history of the calls that wrote them with gradients
        # on, or None; set by _cached_attention_autograd, cleared by any write without gradients
        self.hist = None

    def ensure(self, B: int, Hkv: int, capacity: int, wk: int, wv: int, dtype, device, keep: int = 0) -> None:
        """Buffers of this shape, dtype and device.  When they have to be replaced, the first ``keep``
        rows (those a chunk at start_pos = keep still attends to) are carried over into the new ones;
        a change of batch, heads or row widths cannot keep them and raises."""
        shape_k, shape_v = (B, Hkv, capacity, wk), (B, Hkv, capacity, wv)
        if (self.k is not None and tuple(self.k.shape) == shape_k and tuple(self.v.shape) == shape_v
                and self.k.dtype == dtype and self.k.device == device):
            return
        old_k, old_v = self.k, self.v
        keep = min(keep, self.length)
        if keep > 0 and (old_k is None or old_k.shape[:2] != (B, Hkv) or old_k.shape[3] != wk
                         or old_v.shape[3] != wv or keep > capacity):
            raise ValueError(f"the cache holds {self.length} rows for another batch / head / width layout; "
                             "start over at start_pos = 0")
        self.k = torch.zeros(shape_k, dtype=dtype, device=device)
        self.v = torch.zeros(shape_v, dtype=dtype, device=device)
        if keep > 0:
            self.k[:, :, :keep] = old_k[:, :, :keep].to(device=device, dtype=dtype)
            self.v[:, :, :keep] = old_v[:, :, :keep].to(device=device, dtype=dtype)

    def reset(self) -> None:
        self.k = None
        self.v = None
        self.length = 0
        self.hist = None


def cache_compute_dtype(x: torch.Tensor) -> torch.dtype:
    """Autocast's dtype under autocast, the activations' 16-bit type, else fp32 (as pe_attention
    decides)."""
    if torch.is_autocast_enabled():
        return torch.get_autocast_dtype("cuda")
    if x.dtype in (torch.bfloat16, torch.float16):
        return x.dtype
    return torch.float32


def kernel_position_dtype(embedding, x_dtype):
    """The dtype the embedding's phase product takes positions in for an input of x_dtype: FoPE
    builds them with torch.arange(..., dtype=x.dtype) (src/model/fpope.py:285,322), PoPE in fp32
    (src/model/pope.py:110-119).  None means exact positions."""
    if getattr(embedding, "positions_in_input_dtype", False) and x_dtype in (torch.bfloat16, torch.float16):
        return x_dtype
    return None


def cached_attention(cache: KVCache, capacity: int, start_pos: int, *, q, k, v, q_c=None, k_c=None, mode: str,
                     freqs=None, delta=None, scale: float, rope_mscale: float = 1.0, qk_norm: bool = False,
                     d_v: int, position_dtype=None) -> torch.Tensor:
    """Append the new key / value rows at ``start_pos`` and attend the new queries to every cached
    row with the bottom-right causal mask (src/model/fpope_attention.py:294-324).  Without
    gradients the first chunk (start_pos 0) runs the regular causal forward on the same operands
    and later chunks the split-key decode kernel over the cache.  With gradients (grad mode on and
    an operand that requires one) the chunk runs _cached_attention_autograd.  Returns
    (B, Hq, S, d_v)."""
    B, Hkv, S = k.shape[0], k.shape[1], k.shape[2]
    if start_pos < 0 or start_pos + S > capacity:
        raise ValueError(f"cache rows {start_pos}..{start_pos + S - 1} exceed max_cache_len {capacity}")
    cdt = cache_compute_dtype(k)
    wk, wv = cache_widths(mode=mode, d_content=0 if k_c is None else k_c.shape[-1], d_pe=k.shape[-1], d_v=d_v)
    if start_pos > cache.length:
        raise ValueError(f"the cache holds {cache.length} rows; a chunk at {start_pos} would leave a gap "
                         "(start at or before the cached length)")
    cache.ensure(B, Hkv, capacity, wk, wv, cdt, k.device, keep=start_pos)
    if torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in (q, k, v, q_c, k_c, freqs, delta)):
        return _cached_attention_autograd(cache, start_pos, q=q, k=k, v=v, q_c=q_c, k_c=k_c, mode=mode, freqs=freqs,
                                          delta=delta, scale=scale, rope_mscale=rope_mscale, qk_norm=qk_norm,
                                          position_dtype=position_dtype, cdt=cdt)
    cache.hist = None
    # a chunk at start_pos <= length overwrites rows start_pos.. and ends the cache after itself, as
    # the reference's cache update does (src/model/fpope_attention.py:296-302)
    cache.length = start_pos
    pe_cache_append(k, v, cache.k, cache.v, start_pos=start_pos, mode=mode, k_c=k_c, freqs=freqs, delta=delta,
                    rope_mscale=rope_mscale, qk_norm=qk_norm, position_dtype=position_dtype)
    cache.length = start_pos + S
    if start_pos == 0:
        return pe_attention(q, k, v, mode=mode, q_c=q_c, k_c=k_c, freqs=freqs, delta=delta, scale=scale, causal=True,
                            rope_mscale=rope_mscale, qk_norm=qk_norm, compute_dtype=cdt,
                            position_dtype=position_dtype)
    return pe_attention_decode(q, cache.k, cache.v, cache.length, d_v=d_v, mode=mode, q_c=q_c, freqs=freqs,
                               scale=scale, causal="bottom_right", start_pos_q=start_pos, rope_mscale=rope_mscale,
                               qk_norm=qk_norm, position_dtype=position_dtype)


def _l2norm(x: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """QKNorm's x / (||x|| + eps) over the head dim (src/model/normalization.py:54-55)."""
    return x / (x.norm(dim=-1, keepdim=True) + eps)


def _cached_attention_autograd(cache: KVCache, start_pos: int, *, q, k, v, q_c, k_c, mode: str, freqs, delta,
                               scale: float, rope_mscale: float, qk_norm: bool, position_dtype, cdt) -> torch.Tensor:
    """The cache path with gradients.  The reference writes the new rows into its cache buffers by
    slice assignment, which carries their autograd history into the buffer, and runs SDPA over
    cache[:, :, :start_pos + S] (src/model/fpope_attention.py:294-324); gradients reach the
    queries, the new keys and values and, through the buffer's history, the rows that earlier calls
    wrote with gradients on.  Here the same graph is built without writing in place: the new rows
    are transformed by the differentiable transform (pe_transform), rounded to the cache's dtype and
    appended to the earlier rows, those of earlier calls made with gradients keeping their history
    (KVCache.hist), and the queries attend to them through the fused attention kernels on the
    transformed operands (no-PE mode, bottom-right causal mask).  The cache buffers also receive
    the new rows' values for later decode steps.  Unlike the reference, whose later writes into the
    buffer invalidate the saved tensors of earlier calls, the outputs of several chunks can be
    differentiated together.  Each chunk copies the earlier rows into its own operand, so a run of
    n chunks with gradients holds and copies O(n L) rows where the reference's in-place buffer holds
    O(L); generation without gradients takes the decode path and copies nothing."""
    from .transform import pe_transform

    S = k.shape[2]

    def rows(x, is_key):  # (B, H, S, D) -> the operand rows [content | transform] of the chunk
        if mode in ("pope", "rope"):
            x = pe_transform(x.transpose(1, 2), freqs, delta if is_key else None, start_pos=start_pos, is_key=is_key,
                             mode=mode, mscale=rope_mscale, position_dtype=position_dtype).transpose(1, 2)
        if qk_norm:
            x = _l2norm(x.float())
        c = k_c if is_key else q_c
        if c is not None:
            dt = torch.promote_types(c.dtype, x.dtype)
            x = torch.cat([c.to(dt), x.to(dt)], dim=-1)
        return x

    kt, vt = rows(k, True).to(cdt), v.to(cdt)
    qt = rows(q, False)
    w, dv = kt.shape[-1], vt.shape[-1]
    hist = cache.hist
    if hist is not None and hist[0].shape[2] >= start_pos and hist[0].shape[-1] == w and hist[0].dtype == cdt:
        k_prev, v_prev = hist[0][:, :, :start_pos], hist[1][:, :, :start_pos]
    else:  # rows written without gradients: constants of this graph
        k_prev, v_prev = cache.k[:, :, :start_pos, :w], cache.v[:, :, :start_pos, :dv]
    k_all = torch.cat([k_prev, kt], dim=2)
    v_all = torch.cat([v_prev, vt], dim=2)
    with torch.no_grad():
        cache.k[:, :, start_pos:start_pos + S, :w] = kt
        cache.v[:, :, start_pos:start_pos + S, :dv] = vt
    cache.length = start_pos + S
    cache.hist = (k_all, v_all)
    return pe_attention(qt, k_all, v_all, mode="none", scale=scale, causal="bottom_right", compute_dtype=cdt)


class FPoPEGroupedQueryAttentionWithCache(FPoPEGroupedQueryAttention):
    """KV-cache variant (src/model/fpope_attention.py:184-327): same constructor, ``k_cache`` /
    ``v_cache`` / ``cache_len`` / ``reset_cache`` and ``forward(x, mask, start_pos, use_cache)``.
    With ``use_cache`` the new keys are transformed once into the cache (pe_attn_cache_append) and
    the new queries attend to all ``cache_len`` cached rows under the bottom-right mask
    (pe_attn_decode).  With gradients the chunk runs the differentiable form of the same graph
    (_cached_attention_autograd).  A chunk may start at any start_pos up to the current cache length
    (the length after it is start_pos + S, so an earlier start_pos rewinds); a later one would
    leave a gap of rows never written and raises."""

    def __init__(self, hidden_dim: int, num_heads: int, num_kv_heads: int, head_dim: int = 64,
                 d_rope: int = 32, use_qk_norm: bool = True, fpope: Optional[nn.Module] = None,
                 max_cache_len: int = 2048, use_triton: Optional[bool] = None, d_content: Optional[int] = None):
        super().__init__(hidden_dim, num_heads, num_kv_heads, head_dim, d_rope, use_qk_norm, fpope,
                         d_content=d_content)
        self.max_cache_len = max_cache_len
        self.cache = KVCache()

    @property
    def k_cache(self) -> Optional[torch.Tensor]:
        return self.cache.k

    @property
    def v_cache(self) -> Optional[torch.Tensor]:
        return self.cache.v

    @property
    def cache_len(self) -> int:
        return self.cache.length

    def reset_cache(self) -> None:
        self.cache.reset()

    def forward(self, x: torch.Tensor, mask: Optional[torch.Tensor] = None, start_pos: int = 0,
                use_cache: bool = False) -> torch.Tensor:
        if not use_cache:
            return super().forward(x, mask, start_pos)
        B, S, _ = x.shape
        q_c, k_c, q_r, k_r, v = self._project(x)
        if self.fpope is None:
            # the reference's no-PE fallback keys [k_c | k_r | k_r] (:148-151), untransformed
            dt = v.dtype
            qa = torch.cat(([q_c] if q_c is not None else []) + [q_r.to(dt), q_r.to(dt)], dim=-1)
            ka = torch.cat(([k_c] if k_c is not None else []) + [k_r.to(dt), k_r.to(dt)], dim=-1)
            out = cached_attention(self.cache, self.max_cache_len, start_pos, q=qa, k=ka, v=v, mode="none",
                                   scale=self.scale, d_v=self.head_dim)
        else:
            out = cached_attention(self.cache, self.max_cache_len, start_pos, q=q_r, k=k_r, v=v, q_c=q_c, k_c=k_c,
                                   mode="pope", freqs=self.fpope.kernel_freqs(), delta=self.fpope.kernel_delta(),
                                   scale=self.scale, d_v=self.head_dim,
                                   position_dtype=kernel_position_dtype(self.fpope, q_r.dtype))
        out = out.transpose(1, 2).reshape(B, S, -1)
        return self.wo(out if torch.is_autocast_enabled() else out.to(x.dtype))
