"""Explicit attention masks on the GPU: F.scaled_dot_product_attention(attn_mask=mask) of the
reference's GroupedQueryAttention (src/model/attention.py:91-96), through pe_attn_fwd_masked /
pe_attn_bwd_masked and the generic kernels' mask instantiations.

Each case runs fwd+bwd against the oracle graph of its mode (oracle.pope_attention,
split_pope_attention, rope_attention or the plain core) with the mask handed to the attention core
(oracle.attention(mask=...), pinned against torch's SDPA in tests/test_oracle.py).  Bars are those
of the random sweep (tests/test_gpu_sweep.py): the north-star bar (2e-2 bf16, 1e-5 fp32, 2.5e-3
fp16) wherever the reference path (the core with the 16-bit fused SDPA's rounding points, or the
fp32 core) meets it, else 1.25 times that path's error; fp16 with its one-spacing exemption and
mean-error check.  The masks: bool (Sq, Sk) with a fully masked row, float (B, 1, Sq, Sk) with -inf
entries and a fully -inf row, per-head bool (B, Hq, Sq, Sk), key padding (B, 1, 1, Sk) (one read per
step in the dK/dV kernel), bf16 and fp16 float masks, a transposed bool view (unit stride along the
queries: per-score reads) and a float mask together with the causal flag; Sq != Sk where the flag is
off.  16-bit operands run the tuned kernels' mask instantiations (the forward's 8-key vector reads
where the view allows them), fp32 and QK width 64 the generic kernels.
"""

import functools
import math
import random

import pytest
import torch

from oracle import pe_oracle as O
from pe_ablations_amd.attention import GroupedQueryAttention
from pe_ablations_amd.functional import pe_attention
from pe_ablations_amd.rope import RotaryEmbedding
from tests._cmp import err
from tests.test_gpu_sweep import BASE, DDELTA, DTYPES, bar_for, draw, fp16_rows

pytestmark = pytest.mark.gpu

CASES = [
    dict(mode="none", dt="bf16", B=2, Hq=4, Hkv=2, Sq=130, Sk=130, Dr=64, Dc=0, Dv=64, mask="bool2d", causal=False),
    dict(mode="rope", dt="fp32", B=1, Hq=4, Hkv=4, Sq=97, Sk=161, Dr=64, Dc=0, Dv=128, mask="float_b1", causal=False),
    dict(mode="pope", dt="bf16", B=2, Hq=2, Hkv=1, Sq=200, Sk=200, Dr=64, Dc=0, Dv=64, mask="perhead", causal=False),
    dict(mode="pope", dt="fp16", B=1, Hq=8, Hkv=4, Sq=256, Sk=256, Dr=32, Dc=64, Dv=64, mask="float_b1", causal=True),
    dict(mode="pope", dt="fp32", B=2, Hq=2, Hkv=2, Sq=64, Sk=300, Dr=128, Dc=0, Dv=128, mask="keypad", causal=False),
    dict(mode="none", dt="fp16", B=1, Hq=2, Hkv=1, Sq=180, Sk=180, Dr=128, Dc=0, Dv=128, mask="bool2d", causal=True),
    dict(mode="rope", dt="bf16", B=2, Hq=4, Hkv=1, Sq=150, Sk=150, Dr=128, Dc=0, Dv=128, mask="bf16_b1", causal=False),
    dict(mode="pope", dt="bf16", B=1, Hq=4, Hkv=2, Sq=333, Sk=333, Dr=128, Dc=0, Dv=128, mask="bool2d", causal=False),
    # a transposed view (unit stride along the queries): the per-score reads of the forward
    dict(mode="rope", dt="bf16", B=2, Hq=4, Hkv=2, Sq=200, Sk=232, Dr=64, Dc=0, Dv=64, mask="transposed", causal=False),
    # an fp16 float mask whose rows take the forward's 8-key vector reads (Sk % 8 == 0)
    dict(mode="pope", dt="fp16", B=2, Hq=4, Hkv=4, Sq=256, Sk=256, Dr=64, Dc=0, Dv=64, mask="f16_b1", causal=False),
]


def make_mask(kind, B, Hq, Sq, Sk, seed):
    g = torch.Generator().manual_seed(seed)
    if kind == "bool2d":
        m = torch.rand(Sq, Sk, generator=g) > 0.3
        if Sq > 3:
            m[3] = False
        return m
    if kind in ("float_b1", "bf16_b1", "f16_b1"):
        m = torch.randn(B, 1, Sq, Sk, generator=g) * 2
        m = m.masked_fill(torch.rand(B, 1, Sq, Sk, generator=g) > 0.8, float("-inf"))
        if Sq > 5:
            m[0, 0, 5] = float("-inf")
        return m.to({"bf16_b1": torch.bfloat16, "f16_b1": torch.float16}.get(kind, torch.float32))
    if kind == "transposed":
        return (torch.rand(B, 1, Sk, Sq, generator=g) > 0.3).transpose(-1, -2)
    if kind == "perhead":
        return torch.rand(B, Hq, Sq, Sk, generator=g) > 0.5
    if kind == "keypad":
        lens = [Sk - 50, Sk // 3][:B] + [Sk] * max(0, B - 2)
        return (torch.arange(Sk).view(1, Sk) < torch.tensor(lens).view(B, 1)).view(B, 1, 1, Sk)
    raise ValueError(kind)


def oracle_run(c, x, dout, delta, mask, core):
    """Out, input gradients and ddelta of the oracle graph of case ``c`` with ``core`` (the mask
    bound into it) as its attention core."""
    dt = x["qr"].dtype
    od = dt if dt in (torch.bfloat16, torch.float16) else None
    ox = {n: t.float().clone().requires_grad_(True) for n, t in x.items()}
    res = {}
    Dr, Dc = c["Dr"], c["Dc"]
    if c["mode"] == "pope":
        freqs = O.pope_freqs(Dr)
        od_delta = delta.clone().requires_grad_(True)
        scale = (Dc + 2 * Dr) ** -0.5
        if Dc:
            ref, _ = O.split_pope_attention(ox["qc"], ox["kc"], ox["qr"], ox["kr"], ox["v"], freqs, od_delta, scale=scale,
                                            causal=c["causal"], operand_dtype=od, core=core)
        else:
            ref, _ = O.pope_attention(ox["qr"], ox["kr"], ox["v"], freqs, od_delta, scale=scale, causal=c["causal"],
                                      clamp=False, operand_dtype=od, core=core)
        res["_pope"] = (freqs, scale)
    elif c["mode"] == "rope":
        inv = O.rope_inv_freq(Dr)
        ref, _ = O.rope_attention(ox["qr"], ox["kr"], ox["v"], inv, qk_norm=True, causal=c["causal"],
                                  operand_dtype=od, core=core)
        res["_rope"] = inv
    else:
        ref, _ = core(O.round_ste(ox["qr"], od), O.round_ste(ox["kr"], od), O.round_ste(ox["v"], od), Dr ** -0.5,
                      c["causal"])
    ref.backward(dout.to(ref.dtype))
    res["out"] = ref.detach()
    for n in x:
        res["d" + n] = ox[n].grad
    if c["mode"] == "pope":
        res["ddelta"] = od_delta.grad
    return res


@pytest.mark.parametrize("i", range(len(CASES)))
def test_masked_fwd_bwd_matches_oracle(cuda, i):
    check_case(cuda, CASES[i], i)


def check_case(cuda, c, i):
    """Case ``c`` (seeded by ``i``) against the oracle and the reference path (see the module
    docstring); returns the rows (name, kernel error, path error, bar)."""
    print(f"masked fwd+bwd case {i}: {c}", flush=True)
    dt = DTYPES[c["dt"]]
    B, Hq, Hkv, Sq, Sk, Dr, Dc, Dv = (c[k] for k in ("B", "Hq", "Hkv", "Sq", "Sk", "Dr", "Dc", "Dv"))
    g = torch.Generator().manual_seed(100 + i)
    shapes = {"qr": (B, Hq, Sq, Dr), "kr": (B, Hkv, Sk, Dr), "v": (B, Hkv, Sk, Dv), "qc": (B, Hq, Sq, Dc),
              "kc": (B, Hkv, Sk, Dc)}
    names = ["qr", "kr", "v"] + (["qc", "kc"] if Dc else [])
    x = {n: torch.randn(*shapes[n], generator=g).to(dt) for n in names}
    dout = torch.randn(B, Hq, Sq, Dv, generator=g).to(dt)
    delta = torch.rand(Hkv, Dr, generator=g) * (-2 * math.pi) if c["mode"] == "pope" else None
    mask = make_mask(c["mask"], B, Hq, Sq, Sk, 200 + i)
    exact = oracle_run(c, x, dout, delta, mask, functools.partial(O.attention, mask=mask))
    if dt == torch.float32:
        path_core = functools.partial(O.attention, dtype=torch.float32, mask=mask)
    else:
        path_core = functools.partial(O.attention_bf16_path if dt == torch.bfloat16 else O.attention_fp16_path,
                                      mask=mask)
    path = oracle_run(c, x, dout, delta, mask, path_core)

    gx = {n: t.to(cuda).requires_grad_(True) for n, t in x.items()}
    gm = mask.to(cuda)
    if c["mode"] == "pope":
        freqs, scale = exact["_pope"]
        gd = delta.to(cuda).requires_grad_(True)
        out = pe_attention(gx["qr"], gx["kr"], gx["v"], mode="pope", q_c=gx.get("qc"), k_c=gx.get("kc"),
                           freqs=freqs.to(cuda), delta=gd, scale=scale, causal=c["causal"], mask=gm)
    elif c["mode"] == "rope":
        out = pe_attention(gx["qr"], gx["kr"], gx["v"], mode="rope", freqs=exact["_rope"].to(cuda), qk_norm=True,
                           causal=c["causal"], mask=gm)
    else:
        out = pe_attention(gx["qr"], gx["kr"], gx["v"], mode="none", causal=c["causal"], mask=gm)
    out.backward(dout.to(cuda))
    torch.cuda.synchronize()
    kern = {"out": out} | {"d" + n: gx[n].grad for n in names}
    all_rows = []
    for n, a in kern.items():
        assert a.dtype == dt, (n, a.dtype)
        assert torch.isfinite(a).all(), n
        pe = err(path[n].to(dt), exact[n], f"path {n}")
        rows = fp16_rows(n, a, path[n].to(dt), exact[n], pe) if dt == torch.float16 else \
            [(n, err(a, exact[n], n), pe, bar_for(pe, BASE[dt]))]
        for name, ke, pe_, bar in rows:
            assert ke < bar, (i, name, "kernel", ke, "reference path", pe_, "bar", bar)
        all_rows += rows
    r = {"bool2d": 3, "float_b1": 5, "bf16_b1": 5, "f16_b1": 5}.get(c["mask"])
    if r is not None and r < Sq:  # the fully masked row: zeros, as SDPA returns
        assert (out[0, :, r] == 0).all() and (gx["qr"].grad[0, :, r] == 0).all()
    if c["mode"] == "pope":
        b = exact["ddelta"]
        rel = err(gd.grad, b) / max(1.0, b.abs().max().item())
        assert rel < DDELTA[dt], (i, "ddelta", rel)
        all_rows.append(("ddelta", rel, None, DDELTA[dt]))
    return all_rows


def draw_masked(seed):
    """A masked case from the random sweep's draw (tests/test_gpu_sweep.py): mode, dtype (fp16 too),
    batch, heads, widths and length, plus a mask kind, the causal flag (with a mask both apply) and,
    without it, a key length that may differ from the query length."""
    c = draw(seed)
    r = random.Random(10_000 + seed)
    c["dt"] = r.choice(["bf16", "bf16", "fp32", "fp16"])
    c["mask"] = r.choice(["bool2d", "float_b1", "bf16_b1", "perhead", "keypad"])
    c["Sq"] = c["S"]
    c["Sk"] = c["S"] if c["causal"] else r.randint(1, 600)
    if c["mask"] == "keypad" and c["Sk"] < 60:
        c["mask"] = "bool2d"
    return c


@pytest.mark.parametrize("seed", range(16))
def test_random_masked_config_matches_oracle(cuda, seed):
    """Seeds 0-199 were scanned on an MI355X under these bars.  199 passed, the tightest at 0.95 of
    the bar (seed 2, fp16 dk, equal to the reference path's error) and 0.93 (seed 197, bf16 dv, equal
    to the path's).  Seed 174 (no PE, D = 32, bf16, causal with a bf16 float mask) missed by 4 %:
    dk 0.0208 against 2e-2, where the path's error is 0.0179.  The element has |dk| = 4.04, where
    one bf16 spacing is 0.031, and the kernel and the path round to different neighbours of the exact
    value.  Net of that rounding the errors are 0.0112 (kernel) and 0.0104 (path), and the kernel's
    mean dk error is below the path's (1.16e-3 against 1.32e-3).  The first 16 seeds are committed."""
    check_case(cuda, draw_masked(seed), 300 + seed)


def test_grouped_query_attention_with_mask(cuda):
    """GroupedQueryAttention(mask=key padding), RoPE + QKNorm, fp32: the module's output and the
    gradients of x and of the four projections against the reference's forward restated on the
    oracle (its own projections in fp64, rope_attention with the mask and is_causal=False)."""
    torch.manual_seed(7)
    B, S, Hd, H, Hkv, D = 2, 96, 128, 4, 2, 32
    m = GroupedQueryAttention(Hd, H, Hkv, D, use_qk_norm=True, rope=RotaryEmbedding(D, 256)).to(cuda)
    x = torch.randn(B, S, Hd, device=cuda, requires_grad=True)
    mask = (torch.arange(S).view(1, S) < torch.tensor([S, 50]).view(B, 1)).view(B, 1, 1, S).to(cuda)
    dout = torch.randn(B, S, Hd, device=cuda)
    out = m(x, mask)
    out.backward(dout)
    W = {n: getattr(m, n).weight.detach().double().cpu().requires_grad_(True) for n in ("wq", "wk", "wv", "wo")}
    xc = x.detach().double().cpu().requires_grad_(True)
    q = (xc @ W["wq"].T).view(B, S, H, D).transpose(1, 2)
    k = (xc @ W["wk"].T).view(B, S, Hkv, D).transpose(1, 2)
    v = (xc @ W["wv"].T).view(B, S, Hkv, D).transpose(1, 2)
    core = functools.partial(O.attention, mask=mask.cpu())
    o, _ = O.rope_attention(q, k, v, m.rope.kernel_inv_freq().cpu(), qk_norm=True, causal=False, core=core)
    ref = o.transpose(1, 2).reshape(B, S, H * D) @ W["wo"].T
    ref.backward(dout.double().cpu())
    assert err(out, ref) < 1e-5
    assert err(x.grad, xc.grad) < 1e-5
    for n in W:
        assert err(getattr(m, n).weight.grad, W[n].grad) < 1e-4, n


def test_mask_argument_errors(cuda):
    q = torch.randn(1, 2, 16, 32, device=cuda)
    with pytest.raises(ValueError, match="broadcast"):
        pe_attention(q, q, q, mode="none", causal=False, mask=torch.ones(3, 16, dtype=torch.bool, device=cuda))
    with pytest.raises(TypeError, match="bool or floating"):
        pe_attention(q, q, q, mode="none", causal=False, mask=torch.ones(16, 16, dtype=torch.int32, device=cuda))
    with pytest.raises(NotImplementedError, match="no gradient"):
        pe_attention(q, q, q, mode="none", causal=False, mask=torch.zeros(16, 16, device=cuda, requires_grad=True))
    with pytest.raises(ValueError, match="mask is on cpu"):
        pe_attention(q, q, q, mode="none", causal=False, mask=torch.ones(16, 16, dtype=torch.bool))


def test_masked_module_under_bf16_autocast(cuda):
    """GroupedQueryAttention(mask) under bf16 autocast: the float mask is rounded to bf16 as autocast
    rounds SDPA's inputs, and the output and gradients stay within the bf16 scale of the fp32
    module's (the masked kernels run on bf16 operands)."""
    torch.manual_seed(8)
    B, S = 2, 80
    m = GroupedQueryAttention(256, 4, 2, 64, use_qk_norm=True, rope=RotaryEmbedding(64, 256)).to(cuda)
    x = torch.randn(B, S, 256, device=cuda)
    mask = torch.randn(B, 1, S, S, device=cuda).masked_fill(torch.rand(B, 1, S, S, device=cuda) > 0.7, float("-inf"))
    dout = torch.randn(B, S, 256, device=cuda)
    res = []
    for ac in (False, True):
        xg = x.clone().requires_grad_(True)
        with torch.autocast("cuda", dtype=torch.bfloat16, enabled=ac):
            out = m(xg, mask)
        if ac:
            assert out.dtype == torch.bfloat16
        out.float().backward(dout)
        res.append([out.float()] + [xg.grad] + [p.grad.clone() for p in m.parameters()])
        m.zero_grad()
    for i, (a, b) in enumerate(zip(res[1], res[0])):
        scale = max(1.0, b.abs().max().item())
        assert torch.isfinite(a).all() and (a - b).abs().max().item() < 3e-2 * scale, (i, (a - b).abs().max().item())
