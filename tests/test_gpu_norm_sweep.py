"""A seeded random sweep of the PoPE forward with the position projections' RMSNorm fused into the
transform kernel (pe_attention with qr_norm_weight / kr_norm_weight -> pe_attn_fwd_normed), the
evaluation and generation path of the reference modules (src/model/fpope_attention.py:128-177 with
qr_norm / kr_norm applied to the raw position projections, src/model/normalization.py:22-27).

Each seed draws batch, kv heads and GQA group, length, start positions, Dr (H * Dr up to 2048
features per token), an optional content part, the layout of the raw projections (the modules'
(B, S, H, D) buffer seen through transpose(1, 2), or a contiguous (B, H, S, D) tensor), the dtype
and the norm weights' dtype.  The oracle applies the reference's RMSNorm over each token's H * Dr
features (oracle.rms_norm, with its type_as rounding), then the PoPE attention in fp64 with the
operands rounded to bf16 in bf16 mode.  Bars: 2e-2 (bf16) / 1e-5 (fp32) on out and 2e-3 / 1e-5 on
lse; in bf16 with bf16 weights the norm's two roundings move some operands by one bf16 ulp, which
the attention bar absorbs.
"""

import math
import random

import pytest
import torch

from oracle import pe_oracle as O
from pe_ablations_amd.functional import pe_attention
from tests._cmp import err

pytestmark = pytest.mark.gpu


def draw(seed):
    r = random.Random(seed)
    B, Hkv, grp = r.choice([1, 2]), r.choice([1, 2, 4]), r.choice([1, 2, 4])
    Dr = r.choice([16, 32, 64, 128])
    while Hkv * grp * Dr > 2048:
        grp //= 2
    return dict(B=B, Hkv=Hkv, Hq=Hkv * grp, S=r.randint(1, 700), Dr=Dr,
                Dc=r.choice([0, 0, 32]) if 2 * Dr + 32 <= 256 else 0, Dv=r.choice([32, 64, 128]),
                start=r.choice([0, 0, 17, 4000]), dtype=r.choice(["bf16", "bf16", "fp32"]),
                wdtype=r.choice(["fp32", "bf16"]), module_layout=r.choice([True, False]),
                per_head=r.choice([True, False]), causal=r.choice([True, True, False]))


def check(cuda, seed):
    c = draw(seed)
    g = torch.Generator().manual_seed(seed)
    dt = torch.bfloat16 if c["dtype"] == "bf16" else torch.float32
    wdt = torch.bfloat16 if c["wdtype"] == "bf16" else torch.float32
    if dt == torch.float32:
        wdt = torch.float32
    B, Hq, Hkv, S, Dr, Dc, Dv = (c[k] for k in ("B", "Hq", "Hkv", "S", "Dr", "Dc", "Dv"))

    def proj(H, D, amp=1.0):   # raw projection rows of H heads
        if c["module_layout"]:
            return (torch.randn(B, S, H, D, generator=g) * amp).to(dt).transpose(1, 2)
        return (torch.randn(B, H, S, D, generator=g) * amp).to(dt)

    # the position projections at 3x the unit scale, which the norm takes out
    qr, kr, v = proj(Hq, Dr, 3.0), proj(Hkv, Dr, 3.0), proj(Hkv, Dv)
    qc, kc = (proj(Hq, Dc), proj(Hkv, Dc)) if Dc else (None, None)
    wq = (0.5 + torch.rand(Hq * Dr, generator=g)).to(wdt)
    wk = (0.5 + torch.rand(Hkv * Dr, generator=g)).to(wdt)
    freqs = O.pope_freqs(Dr)
    delta = torch.rand((Hkv, Dr) if c["per_head"] else (Dr,), generator=g) * (-2 * math.pi)
    scale = (Dc + 2 * Dr) ** -0.5
    on = (lambda t: None if t is None else t.to(cuda))
    with torch.no_grad():
        out, lse = pe_attention(on(qr), on(kr), on(v), mode="pope", q_c=on(qc), k_c=on(kc), freqs=on(freqs),
                                delta=on(delta), scale=scale, causal=c["causal"], start_pos_q=c["start"],
                                start_pos_k=c["start"], qr_norm_weight=on(wq), kr_norm_weight=on(wk),
                                return_lse=True)

    def normed(x, w, H):   # the module's RMSNorm over each token's H * Dr features
        y = O.rms_norm(x.transpose(1, 2).reshape(B, S, H * Dr), w)
        return y.reshape(B, S, H, Dr).transpose(1, 2)

    qn, kn = normed(qr, wq, Hq), normed(kr, wk, Hkv)
    tq = O.pope_transform(qn, freqs, c["start"])
    tk = O.pope_transform(kn, freqs, c["start"], delta)
    if Dc:
        tq, tk = torch.cat([qc.float(), tq], -1), torch.cat([kc.float(), tk], -1)
    rd = (lambda t: t.to(torch.bfloat16).float()) if dt == torch.bfloat16 else (lambda t: t.float())
    ref, rlse = O.attention(rd(tq), rd(tk), rd(v), scale, causal=c["causal"])
    assert err(out, ref) < (2e-2 if dt == torch.bfloat16 else 1e-5), (seed, c, "out", err(out, ref))
    assert err(lse, rlse) < (2e-3 if dt == torch.bfloat16 else 1e-5), (seed, c, "lse", err(lse, rlse))
    return c


@pytest.mark.parametrize("seed", range(16))
def test_random_fused_norm_forward_matches_oracle(cuda, seed):
    check(cuda, seed)
