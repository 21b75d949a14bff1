"""A seeded random sweep of the KV-cache decode path (pe_cache_append + pe_attention_decode)
against the oracle.

Each seed draws a mode (PoPE fused or with a content part, RoPE with or without QKNorm, no PE), a
dtype, batch, kv heads and GQA group (up to 8), a cache length in [1, 3000] filled in 1-3
appends, a cache capacity above it, Sq new queries (the tiles of at most 8 query rows take the
split kernel's own query transform, larger ones the prologue launch), widths, the mask
(bottom-right or none) and the phase-bias layout.  The oracle transforms the queries at positions
cache_len - Sq .. and the keys at 0 .. cache_len - 1 as the reference's cache path does
(src/model/fpope_attention.py:283-324), rounds the operands to bf16 in bf16 mode and runs the
attention in fp64.  Bars: 2e-2 (bf16) / 1e-5 (fp32) max-abs on out, scaled by max|ref| / 4 above
4, and 2e-3 / 1e-5 on lse.
"""

import math
import random

import pytest
import torch

from oracle import pe_oracle as O
from pe_ablations_amd.functional import cache_widths, pe_attention_decode, pe_cache_append
from tests._cmp import err

pytestmark = pytest.mark.gpu


def draw(seed):
    r = random.Random(seed)
    mode = r.choices(["pope", "rope", "none"], [6, 2, 2])[0]
    dtype = r.choices(["bf16", "fp32"], [8, 2])[0]
    B, Hkv, grp = r.choice([1, 2]), r.choice([1, 2, 3, 4]), r.choice([1, 2, 4, 8])
    L = r.randint(1, 3000)
    Sq = min(L, r.choice([1, 1, 1, 2, 3, 5, 8, 16]))
    if mode == "pope":
        Dr = r.choice([16, 32, 64, 128])
        Dc = r.choice([0, 0, 32, 64]) if 2 * Dr + 64 <= 256 else 0
    elif mode == "rope":
        Dr, Dc = r.choice([32, 64, 128]), 0
    else:
        Dr, Dc = r.choice([32, 64, 128]), 0
    Dv = r.choice([32, 64, 128])
    nch = r.choice([1, 2, 3])
    cuts = sorted(r.sample(range(1, L), min(nch - 1, L - 1))) if L > 1 else []
    chunks = [b - a for a, b in zip([0] + cuts, cuts + [L])]
    return dict(mode=mode, dtype=dtype, B=B, Hkv=Hkv, Hq=Hkv * grp, L=L, Sq=Sq, Dr=Dr, Dc=Dc, Dv=Dv,
                chunks=chunks, cap=L + r.randint(0, 64), causal=r.choice(["bottom_right", "bottom_right", "none"]),
                per_head=r.choice([True, False]), qk_norm=r.choice([True, False]))


def check(cuda, seed):
    c = draw(seed)
    g = torch.Generator().manual_seed(seed)
    dt = torch.bfloat16 if c["dtype"] == "bf16" else torch.float32
    B, Hq, Hkv, L, Sq, Dr, Dc, Dv = (c[k] for k in ("B", "Hq", "Hkv", "L", "Sq", "Dr", "Dc", "Dv"))
    mode = c["mode"]
    k = torch.randn(B, Hkv, L, Dr, generator=g).to(dt)
    v = torch.randn(B, Hkv, L, Dv, generator=g).to(dt)
    q = torch.randn(B, Hq, Sq, Dr, generator=g).to(dt)
    kc = torch.randn(B, Hkv, L, Dc, generator=g).to(dt) if Dc else None
    qc = torch.randn(B, Hq, Sq, Dc, generator=g).to(dt) if Dc else None
    freqs = delta = None
    if mode == "pope":
        freqs = O.pope_freqs(Dr)
        delta = torch.rand((Hkv, Dr) if c["per_head"] else (Dr,), generator=g) * (-2 * math.pi)
    elif mode == "rope":
        freqs = O.rope_inv_freq(Dr)
    kw = dict(qk_norm=c["qk_norm"]) if mode == "rope" else {}
    wk, wv = cache_widths(mode=mode, d_content=Dc, d_pe=Dr, d_v=Dv)
    kcache = torch.zeros(B, Hkv, c["cap"], wk, dtype=dt, device=cuda)
    vcache = torch.zeros(B, Hkv, c["cap"], wv, dtype=dt, device=cuda)
    on = (lambda t: None if t is None else t.to(cuda))
    pos = 0
    for n in c["chunks"]:
        sl = slice(pos, pos + n)
        pe_cache_append(k[:, :, sl].to(cuda), v[:, :, sl].to(cuda), kcache, vcache, start_pos=pos, mode=mode,
                        k_c=None if kc is None else kc[:, :, sl].to(cuda), freqs=on(freqs), delta=on(delta), **kw)
        pos += n
    with torch.no_grad():
        out, lse = pe_attention_decode(q.to(cuda), kcache, vcache, L, d_v=Dv, mode=mode, q_c=on(qc), freqs=on(freqs),
                                       causal=c["causal"], return_lse=True, **kw)
    # oracle: transformed operands, rounded as the cache stores them, then the fp64 attention
    if mode == "pope":
        tq = O.pope_transform(q, freqs, L - Sq)
        tk = O.pope_transform(k, freqs, 0, delta)
        if Dc:
            tq, tk = torch.cat([qc.float(), tq], -1), torch.cat([kc.float(), tk], -1)
        scale = (Dc + 2 * Dr) ** -0.5
    elif mode == "rope":
        tq, tk = O.rope_rotate(q, freqs, L - Sq), O.rope_rotate(k, freqs, 0)
        if c["qk_norm"]:
            tq, tk = O.qk_l2norm(tq), O.qk_l2norm(tk)
        scale = Dr ** -0.5
    else:
        tq, tk, scale = q.float(), k.float(), Dr ** -0.5
    rd = (lambda t: t.to(torch.bfloat16).float()) if dt == torch.bfloat16 else (lambda t: t.float())
    ref, rlse = O.attention(rd(tq), rd(tk), rd(v), scale, causal=c["causal"] != "none")
    base = 2e-2 if dt == torch.bfloat16 else 1e-5
    bar = base * max(1.0, ref.abs().max().item() / 4)
    assert err(out, ref) < bar, (seed, c, "out", err(out, ref), bar)
    assert err(lse, rlse) < (2e-3 if dt == torch.bfloat16 else 1e-5), (seed, c, "lse", err(lse, rlse))
    return c


@pytest.mark.parametrize("seed", range(24))
def test_random_decode_matches_oracle(cuda, seed):
    check(cuda, seed)
