"""A seeded random sweep of fused attention fwd+bwd configurations against the oracle.

Each seed draws a mode (PoPE fused or split form, RoPE with or without QKNorm, no PE), a dtype, a
batch, kv heads and GQA group, a sequence length in [1, 600], widths (Dr, Dc, Dv), the causal flag
and a shared or per-head phase bias, and compares out, the input gradients and dδ with the oracle
(the reference's expressions: oracle.pope_attention, split_pope_attention, rope_attention,
attention; fp64 core, operands rounded to the 16-bit type in bf16 and fp16 mode).

Bars.  The same graph is also evaluated with the reference path's own attention core: in bf16 mode
the rounding points of the bf16 fused SDPA the reference calls under autocast
(oracle.attention_bf16_path: P rounded to bf16 before PV and dV, dS rounded to bf16 before dQ and
dK, every result rounded to bf16), in fp32 mode the core in float32.  Each result is held to the
north-star bar (2e-2 bf16, 1e-5 fp32, raw max-abs) wherever the reference path meets it, and to
1.25 times the reference path's own error where the path itself misses it (bf16 results of
magnitude above about 4, where one bf16 spacing is already 0.03); dδ relative to its own scale
(2e-2 bf16, 1e-4 fp32).  Over seeds 0-299 and the long seeds 1000-1023: the reference path missed
2e-2 in 66 bf16 results; there the kernel's error was at most 1.19 times the path's (seed 257 dv
0.034 against 0.029) and equal to it in most.  Elsewhere the tightest bf16 result was seed 56's dK
(kernel 0.0199, path 0.0188), and fp32 stayed within 4.8e-6 (path 3.6e-6).  Seed 288 (no PE, D =
32, |dK| 6.8: kernel and path both 0.026) is kept; four long configurations are kept.

fp16 draws (the same configurations on fp16 operands) take the fp16 path core
(oracle.attention_fp16_path) and the bf16 bar over 8 (fp16 carries three more mantissa bits),
2.5e-3; dδ 2e-3 relative.  fp16_rows gives the exemption for results above magnitude 4.
"""

import math
import random

import pytest
import torch

from oracle import pe_oracle as O
from pe_ablations_amd.functional import pe_attention
from tests._cmp import err

pytestmark = pytest.mark.gpu


def draw(seed, long=False):
    """A configuration; ``long`` draws lengths in [1024, 6000] (where the forward takes 96-key tiles
    from 2048 on) with at most 4 heads, so the dense fp64 oracle stays small."""
    r = random.Random(seed)
    mode = r.choices(["pope", "rope", "none"], [6, 2, 2])[0]
    dtype = r.choices(["bf16", "fp32"], [7, 3])[0]
    B, Hkv, grp = r.choice([1, 2, 3]), r.choice([1, 2, 3]), r.choice([1, 2, 4])
    S = r.randint(1, 600) if not long else r.randint(1024, 6000)
    if long:
        B, Hkv, grp = 1, r.choice([1, 2]), r.choice([1, 2])
    if mode == "pope":
        Dr = r.choice([16, 32, 48, 64, 96, 128])
        Dc = r.choice([0, 0, 32, 64]) if 2 * Dr + 64 <= 256 else 0
    elif mode == "rope":
        Dr, Dc = r.choice([32, 64, 96, 128]), 0
    else:
        Dr, Dc = r.choice([32, 64, 128]), 0
    Dv = r.choice([32, 64, 96, 128])
    return dict(mode=mode, dtype=dtype, B=B, Hkv=Hkv, Hq=Hkv * grp, S=S, Dr=Dr, Dc=Dc, Dv=Dv,
                causal=r.choice([True, False]), per_head=r.choice([True, False]), qk_norm=r.choice([True, False]))


@pytest.mark.parametrize("seed", list(range(30)) + [288])
def test_random_config_matches_oracle(cuda, seed):
    check(cuda, seed)


@pytest.mark.parametrize("seed", range(2000, 2024))
def test_random_fp16_config_matches_oracle(cuda, seed):
    """The same draws in fp16 (the reference trainer's mixed_precision fp16): every mode on fp16
    operands, against the fp16 reference path (bars in fp16_rows).  Over seeds 2000-2199 the largest
    error beyond one fp16 spacing was 0.88 of its bar (seed 2059 dqc, equal to the path's), and the
    largest mean error 1.04 times the path's (out, from the forward).  With P handed from the dK/dV
    kernel's score wave to its dS wave in fp16, as on bf16 operands, dq's and dk's mean errors were
    1.24-1.26 times the path's on every seed; the kernel hands P over in fp32 on fp16 operands."""
    check(cuda, seed, dtype="fp16")


@pytest.mark.parametrize("seed", [1001, 1007, 1014, 1022])
def test_random_long_fp16_config_matches_oracle(cuda, seed):
    """The long draws in fp16 (lengths 1024-6000: the forward's 96-key tiles from 2048 on).  Seeds
    1000-1023 all passed, the worst at 0.78 of its bar (seed 1000, out's mean error, equal to the
    reference path's); the four of the bf16 / fp32 long set are committed."""
    check(cuda, seed, long=True, dtype="fp16")


@pytest.mark.parametrize("seed", [1001, 1007, 1014, 1022])
def test_random_long_config_matches_oracle(cuda, seed):
    """RoPE bf16 at 4114 (GQA 2), no PE fp32 at 2476, split PoPE bf16 at 2444 (GQA 2, per-head
    delta) and split PoPE fp32 at 5482 (24 long seeds ran without a failure)."""
    check(cuda, seed, long=True)


def oracle_run(c, x, dout, delta, core=None):
    """The oracle's graph for configuration ``c`` on fresh float leaves of the inputs ``x`` (and the
    phase bias ``delta`` in PoPE mode), with the attention core replaced by ``core`` when given;
    returns {name: result} for out, the input gradients and ddelta."""
    dt = x["qr"].dtype
    B, Hq, Hkv, S, Dr, Dc, Dv = c["B"], c["Hq"], c["Hkv"], c["S"], c["Dr"], c["Dc"], c["Dv"]
    od = dt if dt in (torch.bfloat16, torch.float16) else None
    ox = {n: t.float().clone().requires_grad_(True) for n, t in x.items()}
    res = {}
    if c["mode"] == "pope":
        freqs = O.pope_freqs(Dr)
        od_delta = delta.clone().requires_grad_(True)
        scale = (Dc + 2 * Dr) ** -0.5
        if Dc:
            ref, _ = O.split_pope_attention(ox["qc"], ox["kc"], ox["qr"], ox["kr"], ox["v"], freqs, od_delta,
                                            scale=scale, causal=c["causal"], operand_dtype=od, core=core)
        else:
            ref, _ = O.pope_attention(ox["qr"], ox["kr"], ox["v"], freqs, od_delta, scale=scale,
                                      causal=c["causal"], clamp=False, operand_dtype=od, core=core)
        res["_pope"] = (freqs, delta, scale)
    elif c["mode"] == "rope":
        inv = O.rope_inv_freq(Dr)
        ref, _ = O.rope_attention(ox["qr"], ox["kr"], ox["v"], inv, qk_norm=c["qk_norm"], causal=c["causal"],
                                  operand_dtype=od, core=core)
        res["_rope"] = inv
    else:
        ref, _ = (core or O.attention)(O.round_ste(ox["qr"], od), O.round_ste(ox["kr"], od),
                                       O.round_ste(ox["v"], od), Dr ** -0.5, c["causal"])
    ref.backward(dout.double() if core is None else dout.to(ref.dtype))
    res["out"] = ref.detach()
    for n in x:
        res["d" + n] = ox[n].grad
    if c["mode"] == "pope":
        res["ddelta"] = od_delta.grad
    return res


def fp32_core(q, k, v, scale, causal):
    """The reference's fp32 attention core: the same expression evaluated in float32."""
    return O.attention(q, k, v, scale, causal, dtype=torch.float32)


DTYPES = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}
PATH_CORES = {torch.bfloat16: O.attention_bf16_path, torch.float16: O.attention_fp16_path}
# The north-star bar per dtype (raw max-abs) and dδ's bar relative to its own scale.  fp16 carries
# three more mantissa bits than bf16, so its bar is the bf16 one over 8.
BASE = {torch.bfloat16: 2e-2, torch.float16: 2.5e-3, torch.float32: 1e-5}
DDELTA = {torch.bfloat16: 2e-2, torch.float16: 2e-3, torch.float32: 1e-4}


def measure(cuda, seed, long=False, dtype=None):
    """Kernel results, the oracle (fp64 core) and the reference path (bf16 / fp16 mode: the core with
    the 16-bit fused SDPA's rounding points, oracle.attention_bf16_path / attention_fp16_path, and
    every result rounded to the 16-bit type as the reference returns it for such inputs; fp32 mode:
    the core in float32) for one seed; ``dtype`` overrides the drawn dtype.  Returns
    (config, [(name, kernel error, reference-path error, bar)])."""
    c = draw(seed, long)
    if dtype is not None:
        c["dtype"] = dtype
    g = torch.Generator().manual_seed(seed)
    dt = DTYPES[c["dtype"]]
    B, Hq, Hkv, S, Dr, Dc, Dv = c["B"], c["Hq"], c["Hkv"], c["S"], c["Dr"], c["Dc"], c["Dv"]
    names = ["qr", "kr", "v"] + (["qc", "kc"] if Dc else [])
    shapes = {"qr": (B, Hq, S, Dr), "kr": (B, Hkv, S, Dr), "v": (B, Hkv, S, Dv), "qc": (B, Hq, S, Dc),
              "kc": (B, Hkv, S, Dc)}
    x = {n: torch.randn(*shapes[n], generator=g).to(dt) for n in names}
    dout = torch.randn(B, Hq, S, Dv, generator=g).to(dt)
    delta = None
    if c["mode"] == "pope":
        delta = torch.rand((Hkv, Dr) if c["per_head"] else (Dr,), generator=g) * (-2 * math.pi)
    exact = oracle_run(c, x, dout, delta)
    path = oracle_run(c, x, dout, delta, core=PATH_CORES.get(dt, fp32_core))
    gx = {n: t.to(cuda).requires_grad_(True) for n, t in x.items()}
    if c["mode"] == "pope":
        freqs, delta, scale = exact["_pope"]
        gd = delta.to(cuda).requires_grad_(True)
        out = pe_attention(gx["qr"], gx["kr"], gx["v"], mode="pope", q_c=gx.get("qc"), k_c=gx.get("kc"),
                           freqs=freqs.to(cuda), delta=gd, scale=scale, causal=c["causal"])
    elif c["mode"] == "rope":
        out = pe_attention(gx["qr"], gx["kr"], gx["v"], mode="rope", freqs=exact["_rope"].to(cuda),
                           qk_norm=c["qk_norm"], causal=c["causal"])
    else:
        out = pe_attention(gx["qr"], gx["kr"], gx["v"], mode="none", causal=c["causal"])
    out.backward(dout.to(cuda))
    torch.cuda.synchronize()
    kern = {"out": out} | {"d" + n: gx[n].grad for n in names}
    rows = []
    for n, a in kern.items():
        assert a.dtype == dt, (n, a.dtype)
        pe = err(path[n].to(dt), exact[n], f"path {n}")
        if dt == torch.float16:
            rows += fp16_rows(n, a, path[n].to(dt), exact[n], pe)
        else:
            rows.append((n, err(a, exact[n], n), pe, bar_for(pe, BASE[dt])))
    if c["mode"] == "pope":
        b = exact["ddelta"]
        rel = err(gd.grad, b) / max(1.0, b.abs().max().item())
        rows.append(("ddelta", rel, None, DDELTA[dt]))
    return c, rows


# Where the reference path meets the north-star bar the kernel is held to it.  Where the reference
# path itself misses it (bf16 results of magnitude above about 4, where one bf16 spacing is 0.03),
# the kernel is held to 1.25 times the reference path's own error at the same elements.
PATH_FACTOR = 1.25


def bar_for(path_err, base):
    return base if path_err < base else PATH_FACTOR * path_err


def spacing_f16(ref: torch.Tensor) -> torch.Tensor:
    """fp16's spacing at |ref| (2^-24 below the normal range)."""
    _, e = torch.frexp(ref.abs())  # |ref| in [2^(e-1), 2^e): spacing 2^(e-11)
    e = torch.where(ref == 0, torch.full_like(e, -13), e)
    return torch.ldexp(torch.ones_like(ref), torch.clamp(e - 11, min=-24))


def fp16_rows(n, a, p, ex, pe):
    """fp16 results.  The bar (2.5e-3, or 1.25 times the path's error where the path misses it) is
    below one fp16 spacing for results of magnitude 4 and above (3.9e-3), where the kernel and the
    path each land on one of the two fp16 neighbours of the exact value, not always the same one.
    Elements within one fp16 spacing of the exact value are therefore exempt from the max-abs bar,
    and the mean error must stay within 1.25 times the path's (plus 1e-6, one fp16 spacing at 1e-3,
    for results the path gets exactly, such as the vanishing dS of a one-key row), so a systematic
    error cannot hide under the exemption."""
    ad, pd, ed = a.detach().double().cpu(), p.double(), ex.double()
    d = (ad - ed).abs()
    if not d.numel():
        return [(n, 0.0, pe, 1.0)]
    beyond = torch.where(d > spacing_f16(ed), d, torch.zeros_like(d)).max().item()
    mk, mp = d.mean().item(), (pd - ed).abs().mean().item()
    return [(n + " beyond one fp16 spacing", beyond, pe, bar_for(pe, BASE[torch.float16])),
            (n + " mean", mk, mp, PATH_FACTOR * mp + 1e-6)]


def check(cuda, seed, long=False, dtype=None):
    c, rows = measure(cuda, seed, long, dtype)
    for n, ke, pe, bar in rows:
        assert ke < bar, (seed, c, n, "kernel", ke, "reference path", pe, "bar", bar)
