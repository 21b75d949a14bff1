"""KV-cache decode on the GPU: pe_cache_append + pe_attention_decode (the split-key decode kernel)
against the oracle and against the full causal forward.

The reference's cache path (src/model/fpope_attention.py:226-327) caches [k_c | PoPE(k_r)] and
runs SDPA of the new queries over the cached rows with a bottom-right mask; the oracle restates
that as pope_attention_chunked with Sq < Sk (bottom-right alignment), transforms in fp32, operands
rounded to bf16 in bf16 mode.  Bars: raw max-abs 2e-2 in bf16, 1e-5 in fp32 (north star).
"""

import math

import pytest
import torch

from oracle import pe_oracle as O
from pe_ablations_amd import _lib
from pe_ablations_amd.functional import cache_widths, pe_attention, pe_attention_decode, pe_cache_append
from tests._cmp import err

pytestmark = pytest.mark.gpu


def rnd(*shape, seed):
    return torch.randn(*shape, generator=torch.Generator().manual_seed(seed))


def fill_cache(cuda, k, v, freqs, delta, cap, dtype, chunks, k_c=None, mode="pope", **kw):
    """Append the keys of k (B, Hkv, L, Dr) / v in the given chunk lengths; returns the caches."""
    B, Hkv, L, Dr = k.shape
    Dc = 0 if k_c is None else k_c.shape[-1]
    wk, wv = cache_widths(mode=mode, d_content=Dc, d_pe=Dr, d_v=v.shape[-1])
    kc = torch.zeros(B, Hkv, cap, wk, dtype=dtype, device=cuda)
    vc = torch.zeros(B, Hkv, cap, wv, dtype=dtype, device=cuda)
    pos = 0
    for n in chunks:
        sl = slice(pos, pos + n)
        pe_cache_append(k[:, :, sl].to(cuda), v[:, :, sl].to(cuda), kc, vc, start_pos=pos, mode=mode,
                        k_c=None if k_c is None else k_c[:, :, sl].to(cuda),
                        freqs=None if freqs is None else freqs.to(cuda),
                        delta=None if delta is None else delta.to(cuda), **kw)
        pos += n
    assert pos == L
    return kc, vc


@pytest.mark.parametrize("L, Sq", [(1000, 1), (1000, 5), (16384, 1), (16384, 4)])
@torch.no_grad()
def test_decode_fused_pope_bf16_long_context(cuda, L, Sq):
    """The 1B shape (16 heads of D = 128, every dim PoPE-encoded, per-head delta) decoding Sq
    tokens against L cached keys: equal to the oracle and to the full forward's last rows."""
    B, H, D = 1, 16, 128
    q, k, v = rnd(B, H, L, D, seed=L + Sq), rnd(B, H, L, D, seed=L + Sq + 1), rnd(B, H, L, D, seed=L + Sq + 2)
    q, k, v = (t.to(torch.bfloat16) for t in (q, k, v))
    freqs = O.pope_freqs(D)
    delta = -torch.rand(H, D, generator=torch.Generator().manual_seed(3)) * 2 * math.pi
    scale = 1 / math.sqrt(D)
    kc, vc = fill_cache(cuda, k, v, freqs, delta, L + 64, torch.bfloat16, [L - Sq, Sq])
    qn = q[:, :, L - Sq:]
    out, lse = pe_attention_decode(qn.to(cuda), kc, vc, L, d_v=D, freqs=freqs.to(cuda), scale=scale,
                                   return_lse=True)
    full = pe_attention(q.to(cuda), k.to(cuda), v.to(cuda), freqs=freqs.to(cuda), delta=delta.to(cuda), scale=scale)
    assert err(out, full[:, :, L - Sq:]) < 2e-2
    for h in (0, 9):
        ref = O.pope_attention_chunked(qn[0, h].float(), k[0, h].float(), v[0, h].float(), freqs, delta[h],
                                       scale=scale, start_q=L - Sq, operand_dtype=torch.bfloat16, chunk=4096)
        assert err(out[0, h], ref["out"]) < 2e-2, h
        assert err(lse[0, h], ref["lse"]) < 2e-3, h


@torch.no_grad()
def test_decode_split_form_gqa_bf16(cuda):
    """The reference module's split form ([q_c (64) | PoPE (2 x 32)], V 64, GQA 8 -> 4, scale
    (64 + 64)^-1/2): each kv head's 2 query heads x 3 new queries share one 32-row tile."""
    B, Hq, Hkv, L, Sq, Dc, Dr, Dv = 2, 8, 4, 700, 3, 64, 32, 64
    qr, kr = rnd(B, Hq, Sq, Dr, seed=1), rnd(B, Hkv, L, Dr, seed=2)
    qc, kc_ = rnd(B, Hq, Sq, Dc, seed=3), rnd(B, Hkv, L, Dc, seed=4)
    v = rnd(B, Hkv, L, Dv, seed=5)
    qr, kr, qc, kc_, v = (t.to(torch.bfloat16) for t in (qr, kr, qc, kc_, v))
    freqs = O.pope_freqs(Dr)
    delta = -torch.rand(Dr, generator=torch.Generator().manual_seed(6)) * 6
    scale = (Dc + 2 * Dr) ** -0.5
    kcache, vcache = fill_cache(cuda, kr, v, freqs, delta, 1024, torch.bfloat16, [512, 100, 88], k_c=kc_)
    out = pe_attention_decode(qr.to(cuda), kcache, vcache, L, d_v=Dv, q_c=qc.to(cuda), freqs=freqs.to(cuda),
                              scale=scale)
    tq = torch.cat([qc.float(), O.pope_transform(qr, freqs, L - Sq)], -1)
    tk = torch.cat([kc_.float(), O.pope_transform(kr, freqs, 0, delta)], -1)
    tq, tk, vv = (t.to(torch.bfloat16).float() for t in (tq, tk, v))
    ref, _ = O.attention(tq, tk, vv, scale, causal=True)   # GQA by repeat_interleave, bottom-right mask
    assert err(out, ref) < 2e-2


@torch.no_grad()
def test_decode_rope_qknorm_and_fp32(cuda):
    """RoPE with QKNorm (GroupedQueryAttention's path) in bf16, and PoPE in fp32 at 1e-5."""
    B, H, L, Sq, D = 1, 4, 300, 2, 64
    q, k, v = rnd(B, H, Sq, D, seed=7), rnd(B, H, L, D, seed=8), rnd(B, H, L, D, seed=9)
    inv = O.rope_inv_freq(D)
    kc, vc = fill_cache(cuda, k.to(torch.bfloat16), v.to(torch.bfloat16), inv, None, 320, torch.bfloat16, [L],
                        mode="rope", qk_norm=True)
    out = pe_attention_decode(q.to(torch.bfloat16).to(cuda), kc, vc, L, d_v=D, mode="rope", freqs=inv.to(cuda),
                              qk_norm=True, scale=D ** -0.5)
    tq = O.qk_l2norm(O.rope_rotate(q.to(torch.bfloat16), inv, L - Sq))
    tk = O.qk_l2norm(O.rope_rotate(k.to(torch.bfloat16), inv, 0))
    ref, _ = O.attention(tq.to(torch.bfloat16).float(), tk.to(torch.bfloat16).float(),
                         v.to(torch.bfloat16).float(), D ** -0.5, causal=True)
    assert err(out, ref) < 2e-2

    freqs = O.pope_freqs(D)
    delta = -torch.rand(H, D, generator=torch.Generator().manual_seed(10)) * 6
    kc, vc = fill_cache(cuda, k, v, freqs, delta, 300, torch.float32, [200, 100])
    out, lse = pe_attention_decode(q.to(cuda), kc, vc, L, d_v=D, freqs=freqs.to(cuda), scale=0.1, return_lse=True)
    for h in range(H):
        ref = O.pope_attention_chunked(q[0, h], k[0, h], v[0, h], freqs, delta[h], scale=0.1, start_q=L - Sq,
                                       core_dtype=torch.float64)
        assert err(out[0, h], ref["out"]) < 1e-5 and err(lse[0, h], ref["lse"]) < 1e-5, h


@torch.no_grad()
def test_decode_bitwise_reproducible_and_nonfull_rows(cuda):
    """Two identical calls agree bit for bit (fixed-order merge, no atomics); a cache with more
    capacity than rows ignores the rows past cache_len."""
    B, H, L, D = 1, 2, 333, 64
    k, v, q = rnd(B, H, L, D, seed=11), rnd(B, H, L, D, seed=12), rnd(B, H, 1, D, seed=13)
    freqs = O.pope_freqs(D)
    kc, vc = fill_cache(cuda, k.bfloat16(), v.bfloat16(), freqs, None, 1000, torch.bfloat16, [L])
    kc[:, :, L:] = 1e4
    vc[:, :, L:] = float("nan")
    a = pe_attention_decode(q.bfloat16().to(cuda), kc, vc, L, d_v=D, freqs=freqs.to(cuda))
    b = pe_attention_decode(q.bfloat16().to(cuda), kc, vc, L, d_v=D, freqs=freqs.to(cuda))
    assert torch.equal(a, b) and bool(torch.isfinite(a).all())


@torch.no_grad()
def test_decode_in_kernel_query_transform_matches_prologue(cuda):
    """A tile of at most 8 query rows (here GQA 2 x 1 token) has its PoPE transform done inside the
    split kernel; 2 x 5 rows go through the prologue launch.  With no mask and the same query
    positions, the first token's output and lse agree bit for bit between the two paths, and both
    match the oracle."""
    B, Hq, Hkv, L, D = 2, 4, 2, 777, 64
    k, v = rnd(B, Hkv, L, D, seed=21).bfloat16(), rnd(B, Hkv, L, D, seed=22).bfloat16()
    q5 = rnd(B, Hq, 5, D, seed=23).bfloat16()
    freqs = O.pope_freqs(D)
    delta = -torch.rand(Hkv, D, generator=torch.Generator().manual_seed(24)) * 6
    kc, vc = fill_cache(cuda, k, v, freqs, delta, 800, torch.bfloat16, [L])
    kw = dict(d_v=D, freqs=freqs.to(cuda), scale=0.125, causal="none", start_pos_q=L - 5, return_lse=True)
    o5, l5 = pe_attention_decode(q5.to(cuda), kc, vc, L, **kw)
    o1, l1 = pe_attention_decode(q5[:, :, :1].contiguous().to(cuda), kc, vc, L, **kw)
    assert torch.equal(o1, o5[:, :, :1]) and torch.equal(l1, l5[:, :, :1])
    for b, h in ((0, 0), (1, 3)):
        ref = O.pope_attention_chunked(q5[b, h, :1].float(), k[b, h // 2].float(), v[b, h // 2].float(), freqs,
                                       delta[h // 2], scale=0.125, start_q=L - 5, causal=False,
                                       operand_dtype=torch.bfloat16, chunk=1024)
        assert err(o1[b, h], ref["out"]) < 2e-2 and err(l1[b, h], ref["lse"]) < 2e-3, (b, h)


@torch.no_grad()
def test_small_appends_match_bulk_append_bitwise(cuda):
    """A few rows per call (here one token of 2 kv heads) take the one-thread-per-element append
    kernel, a long chunk the vectorised one; the caches they fill agree bit for bit, including the
    content part, the operand rows' zero padding (width 96 -> 128) and value rows narrower than
    the cache (48 -> 64)."""
    B, Hkv, L, Dc, Dr, Dv = 1, 2, 300, 32, 32, 48
    g = torch.Generator().manual_seed(31)
    kr, kc_ = rnd(B, Hkv, L, Dr, seed=32).bfloat16(), rnd(B, Hkv, L, Dc, seed=33).bfloat16()
    v = rnd(B, Hkv, L, Dv, seed=34).bfloat16()
    freqs = O.pope_freqs(Dr)
    delta = -torch.rand(Hkv, Dr, generator=g) * 6
    bulk = fill_cache(cuda, kr, v, freqs, delta, 320, torch.bfloat16, [L], k_c=kc_)
    small = fill_cache(cuda, kr, v, freqs, delta, 320, torch.bfloat16, [1] * L, k_c=kc_)
    assert torch.equal(bulk[0], small[0]) and torch.equal(bulk[1], small[1])
    assert bool((bulk[0][:, :, :, Dc + 2 * Dr:] == 0).all()) and bool((bulk[1][:, :, :, Dv:] == 0).all())


@torch.no_grad()
def test_decode_argument_errors(cuda):
    B, H, D = 1, 2, 64
    freqs = O.pope_freqs(D).to(cuda)
    wk, wv = cache_widths(d_pe=D, d_v=D)
    kc = torch.zeros(B, H, 64, wk, dtype=torch.bfloat16, device=cuda)
    vc = torch.zeros(B, H, 64, wv, dtype=torch.bfloat16, device=cuda)
    k = torch.zeros(B, H, 8, D, dtype=torch.bfloat16, device=cuda)
    with pytest.raises(ValueError, match="capacity"):
        pe_cache_append(k, k, kc, vc, start_pos=60, freqs=freqs)
    with pytest.raises(ValueError, match="k_cache"):
        pe_cache_append(k, k, kc[..., :64], vc, start_pos=0, freqs=freqs)
    with pytest.raises(ValueError, match="capacity"):
        pe_attention_decode(k[:, :, :1], kc, vc, 65, d_v=D, freqs=freqs)
    with torch.enable_grad(), pytest.raises(RuntimeError, match="inference"):
        pe_attention_decode(k[:, :, :1].float().requires_grad_(True), kc, vc, 8, d_v=D, freqs=freqs)
    assert _lib.lib().pe_attn_decode_workspace_bytes(None) == 0
