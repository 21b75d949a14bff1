"""fp16 compute (the reference trainer's mixed_precision fp16, src/training/trainer.py:343-347) on
the GPU: fp16 inputs and torch.autocast(dtype=torch.float16) run the matrix-core kernels on fp16
operands (v_mfma_f32_32x32x16_f16, fp32 accumulation), where the reference's SDPA runs fp16.

Bars.  The oracle graph is evaluated with the exact (fp64) core and with the reference path's fp16
core (oracle.attention_fp16_path: P and dS rounded to fp16 before their products, results rounded
to fp16).  Every result is held to 1.25 times the fp16 reference path's own error at the same
elements (plus 1e-4); out, dq and dk must also be well inside the bf16 reference path's error, so a
kernel that narrowed fp16 to bf16 fails.
"""

import copy
import math

import pytest
import torch

from oracle import pe_oracle as O
from pe_ablations_amd.fpope_attention import FPoPEGroupedQueryAttention, FPoPEGroupedQueryAttentionWithCache
from pe_ablations_amd.functional import pe_attention, rms_norm, rms_norm_backward
from pe_ablations_amd.pope import PoPEEmbedding
from pe_ablations_amd.transform import pe_transform
from tests._cmp import err

pytestmark = pytest.mark.gpu


def rnd(*shape, seed, scale=1.0):
    return torch.randn(*shape, generator=torch.Generator().manual_seed(seed)) * scale


def oracle_graph(x, dout, freqs, delta, scale, causal, Dc, rd, core=None):
    """Oracle out and input gradients for the PoPE call (split form when Dc), operands rounded to
    ``rd``; ``core`` replaces the exact attention core."""
    ox = {n: t.float().clone().requires_grad_(True) for n, t in x.items()}
    od = delta.clone().requires_grad_(True)
    if Dc:
        ref, _ = O.split_pope_attention(ox["qc"], ox["kc"], ox["qr"], ox["kr"], ox["v"], freqs, od, scale=scale,
                                        causal=causal, operand_dtype=rd, core=core)
    else:
        ref, _ = O.pope_attention(ox["qr"], ox["kr"], ox["v"], freqs, od, scale=scale, causal=causal, clamp=False,
                                  operand_dtype=rd, core=core)
    ref.backward(dout.to(ref.dtype))
    return {"out": ref.detach()} | {"d" + n: t.grad for n, t in ox.items()} | {"ddelta": od.grad}


@pytest.mark.parametrize("cfg", [
    dict(B=2, Hq=4, Hkv=4, S=300, Dr=64, Dc=0, Dv=64),        # fused PoPE, QK width 128
    dict(B=1, Hq=2, Hkv=2, S=700, Dr=128, Dc=0, Dv=128),      # the headline's widths
    dict(B=2, Hq=8, Hkv=4, S=256, Dr=32, Dc=64, Dv=64),       # the reference module's split form, GQA
    dict(B=1, Hq=2, Hkv=1, S=2100, Dr=64, Dc=0, Dv=128),      # 96-key forward tiles, GQA
])
def test_fp16_fwd_bwd_matches_oracle(cuda, cfg):
    B, Hq, Hkv, S, Dr, Dc, Dv = (cfg[k] for k in ("B", "Hq", "Hkv", "S", "Dr", "Dc", "Dv"))
    seed = S + Dr
    x = {"qr": rnd(B, Hq, S, Dr, seed=seed), "kr": rnd(B, Hkv, S, Dr, seed=seed + 1), "v": rnd(B, Hkv, S, Dv, seed=seed + 2)}
    if Dc:
        x["qc"], x["kc"] = rnd(B, Hq, S, Dc, seed=seed + 3), rnd(B, Hkv, S, Dc, seed=seed + 4)
    x = {n: t.half() for n, t in x.items()}
    dout = rnd(B, Hq, S, Dv, seed=seed + 5).half()
    freqs = O.pope_freqs(Dr)
    delta = -torch.rand(Hkv, Dr, generator=torch.Generator().manual_seed(seed + 6)) * 6
    scale = (Dc + 2 * Dr) ** -0.5
    print(f"fp16 fwd+bwd {cfg}", flush=True)
    exact = oracle_graph(x, dout, freqs, delta, scale, True, Dc, torch.float16)
    path16 = oracle_graph(x, dout, freqs, delta, scale, True, Dc, torch.float16, O.attention_fp16_path)
    path_bf = oracle_graph(x, dout, freqs, delta, scale, True, Dc, torch.bfloat16, O.attention_bf16_path)
    gx = {n: t.to(cuda).requires_grad_(True) for n, t in x.items()}
    gd = delta.to(cuda).requires_grad_(True)
    out = pe_attention(gx["qr"], gx["kr"], gx["v"], mode="pope", q_c=gx.get("qc"), k_c=gx.get("kc"),
                       freqs=freqs.to(cuda), delta=gd, scale=scale)
    assert out.dtype == torch.float16
    out.backward(dout.to(cuda))
    torch.cuda.synchronize()
    kern = {"out": out} | {"d" + n: t.grad for n, t in gx.items()}
    for n, a in kern.items():
        assert a.dtype == torch.float16, n
        ke = err(a, exact[n], n)
        p16 = err(path16[n].half(), exact[n], "fp16 path " + n)
        pbf = err(path_bf[n].bfloat16(), exact[n], "bf16 path " + n)
        assert ke < 1.25 * p16 + 1e-4, (n, "kernel", ke, "fp16 path", p16)
        if n in ("out", "dqr", "dkr"):
            assert ke < 0.5 * pbf, (n, "kernel", ke, "bf16 path", pbf)
    rel = err(gd.grad, exact["ddelta"]) / max(1.0, exact["ddelta"].abs().max().item())
    assert rel < 2e-3, rel


def test_fp16_autocast_runs_fp16_operands(cuda):
    """fp32 inputs under torch.autocast(dtype=torch.float16): the transformed operands are rounded to
    fp16 (as autocast rounds them on their way into SDPA) and the output is fp16, against the oracle
    with fp16 operand rounding."""
    B, H, S, D = 1, 4, 400, 64
    x = {"qr": rnd(B, H, S, D, seed=1), "kr": rnd(B, H, S, D, seed=2), "v": rnd(B, H, S, D, seed=3)}
    dout = rnd(B, H, S, D, seed=4).half()
    freqs, delta, scale = O.pope_freqs(D), -torch.rand(D, generator=torch.Generator().manual_seed(5)) * 6, D ** -0.5
    exact = oracle_graph(x, dout, freqs, delta, scale, True, 0, torch.float16)
    path16 = oracle_graph(x, dout, freqs, delta, scale, True, 0, torch.float16, O.attention_fp16_path)
    gx = {n: t.to(cuda).requires_grad_(True) for n, t in x.items()}
    with torch.autocast("cuda", dtype=torch.float16):
        out = pe_attention(gx["qr"], gx["kr"], gx["v"], mode="pope", freqs=freqs.to(cuda), delta=delta.to(cuda),
                           scale=scale)
    assert out.dtype == torch.float16
    out.backward(dout.to(cuda))
    for n, a in {"out": out, "dqr": gx["qr"].grad, "dkr": gx["kr"].grad, "dv": gx["v"].grad}.items():
        p16 = err(path16[n].to(a.dtype), exact[n])
        assert err(a, exact[n]) < 1.25 * p16 + 1e-4, (n, err(a, exact[n]), p16)


def test_fp16_autocast_module_training(cuda):
    """The split-form module under fp16 autocast with the fused norm, one training step: every
    gradient within the fp16 scale of the fp32 module's, and closer to it than the bf16-autocast
    step's."""
    torch.manual_seed(21)
    pe = PoPEEmbedding(32, 1024, delta_init="uniform")
    m = FPoPEGroupedQueryAttention(256, 8, 4, 64, 32, fpope=pe)
    x = torch.randn(2, 300, 256)
    dout = torch.randn(2, 300, 256)
    res = {}
    for name, dt in (("fp32", None), ("fp16", torch.float16), ("bf16", torch.bfloat16)):
        mod = copy.deepcopy(m).to(cuda)
        xg = x.to(cuda).requires_grad_(True)
        if dt is None:
            out = mod(xg)
        else:
            with torch.autocast("cuda", dtype=dt):
                out = mod(xg)
        out.float().backward(dout.to(cuda))
        res[name] = {"out": out.float().cpu(), "x": xg.grad.cpu()} | \
            {n: p.grad.float().cpu() for n, p in mod.named_parameters() if p.grad is not None}
    for n in res["fp32"]:
        scale = max(1.0, res["fp32"][n].abs().max().item())
        e16 = (res["fp16"][n] - res["fp32"][n]).abs().max().item()
        ebf = (res["bf16"][n] - res["fp32"][n]).abs().max().item()
        assert math.isfinite(e16) and e16 < 5e-3 * scale, (n, e16)
        assert e16 < ebf or e16 < 1e-4 * scale, (n, e16, ebf)


@torch.no_grad()
def test_fp16_kv_cache_decode_matches_full_forward(cuda):
    """The KV-cache path in fp16 (fp16 caches, the decode kernel on fp16 operands): prefill plus
    decoded tokens equal the full fp16 forward's rows to fp16 rounding."""
    torch.manual_seed(22)
    pe = PoPEEmbedding(32, 512, delta_init="uniform")
    m = FPoPEGroupedQueryAttentionWithCache(128, 4, 2, 32, 32, fpope=pe, max_cache_len=96).to(cuda).half()
    x = torch.randn(1, 40, 128, device=cuda).half()
    full = m(x)
    outs = [m(x[:, :33], use_cache=True)] + [m(x[:, t:t + 1], start_pos=t, use_cache=True) for t in range(33, 40)]
    assert m.k_cache.dtype == torch.float16
    d = (torch.cat(outs, 1).float() - full.float()).abs().max().item()
    assert d < 2e-3 * max(1.0, full.float().abs().max().item()), d


@pytest.mark.parametrize("xd,wd", [("fp16", "fp16"), ("fp16", "fp32"), ("bf16", "fp16")])
def test_fp16_rmsnorm_forward_and_backward(cuda, xd, wd):
    """RMSNorm with fp16 x and / or weight: y's dtype by torch's promotion (fp16 only when both are
    fp16; bf16 * fp16 is fp32), forward and backward against the reference expression's autograd on
    the CPU in the same dtypes, to one spacing of the rounded results."""
    DT = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}
    g = torch.Generator().manual_seed(23)
    x = (torch.randn(300, 512, generator=g) * 3).to(DT[xd])
    w = (0.5 + torch.rand(512, generator=g)).to(DT[wd])
    xr, wr = x.clone().requires_grad_(True), w.clone().requires_grad_(True)
    y_ref = O.rms_norm(xr, wr)
    dy = torch.randn(300, 512, generator=g).to(y_ref.dtype)
    y_ref.backward(dy)
    y = rms_norm(x.to(cuda), w.to(cuda))
    dx, dw = rms_norm_backward(x.to(cuda), w.to(cuda), dy.to(cuda))
    assert y.dtype == y_ref.dtype and dx.dtype == x.dtype and dw.dtype == w.dtype

    def spacing(t, dtype):
        bits = {torch.float16: 10, torch.bfloat16: 7, torch.float32: 23}[dtype]
        return torch.pow(2.0, torch.floor(torch.log2(t.double().abs().clamp_min(1e-30))) - bits)

    # the normalised value is rounded to x's dtype: a last-bit difference in the fp32 statistics can
    # move it by one spacing of that type, times the weight; plus one spacing of y when y is 16-bit
    n_ref = O.rms_norm(x, torch.ones(512, dtype=x.dtype)).double()
    tol = spacing(n_ref, x.dtype) * w.double().abs() * 1.01 + spacing(y_ref, y_ref.dtype) + 1e-7
    assert ((y.double().cpu() - y_ref.double()).abs() <= tol).all()
    assert ((dx.double().cpu() - xr.grad.double()).abs() <= 2 * spacing(xr.grad, x.dtype) +
            1e-5 * xr.grad.double().abs().max()).all()
    assert ((dw.double().cpu() - wr.grad.double()).abs() <= 1e-3 * wr.grad.double().abs().max()).all()


@pytest.mark.parametrize("mode", ["pope", "rope"])
def test_fp16_standalone_transform_keeps_fp16(cuda, mode):
    """forward_query / forward_key (src/model/pope.py:124-183, src/model/rope.py:35-57) as the
    standalone transform on fp16 input: the output stays fp16 (not narrowed to bf16) and equals the
    oracle's fp32 transform to fp16 rounding; the input gradient likewise."""
    g = torch.Generator().manual_seed(24)
    x = (torch.randn(2, 40, 3, 64, generator=g) * 2).half()
    if mode == "pope":
        freqs, delta = O.pope_freqs(64), O.clamp_delta(-torch.rand(3, 64, generator=g) * 6)
    else:
        freqs, delta = O.rope_inv_freq(64), None
    xo = x.float().requires_grad_(True)
    if mode == "pope":
        ref = O.pope_transform(xo.transpose(1, 2), freqs, 5, delta).transpose(1, 2)
    else:
        ref = O.rope_rotate(xo.transpose(1, 2), freqs, 5).transpose(1, 2)
    gout = torch.randn(ref.shape, generator=g)
    ref.backward(gout)
    xg = x.to(cuda).requires_grad_(True)
    out = pe_transform(xg, freqs.to(cuda), None if delta is None else delta.to(cuda), start_pos=5,
                       is_key=delta is not None, mode=mode)
    assert out.dtype == torch.float16
    out.backward(gout.to(cuda).half())
    torch.cuda.synchronize()
    assert xg.grad.dtype == torch.float16

    def spacing(t):  # fp16 spacing at each element's magnitude
        return torch.pow(2.0, torch.floor(torch.log2(t.double().abs().clamp_min(2.0 ** -14))) - 10)

    assert ((out.double().cpu() - ref.double()).abs() <= spacing(ref) + 1e-6).all()
    # the gradient of the fp16-rounded output: gout is rounded to fp16 first
    dref = xo.grad.double()
    assert ((xg.grad.double().cpu() - dref).abs() <= 2 * spacing(dref) + 2e-3 * gout.abs().max()).all()
