"""GPU parity of every mode of the fused kernel (through the C ABI) against the CPU oracle.

Covers FoPE (gradient into the effective frequencies), RoPE / NTK / YaRN with and without the
fused QKNorm, no-PE, the reference module's split form (content 64 | PoPE 2x32, value 64), GQA,
bottom-right (KV-cache) and non-causal masks, start positions, fp32 and bf16.  Tolerances: 1e-5
max-abs in fp32 mode and 2e-2 in bf16 mode for out / dq / dk / dv (raw
max-abs including the result's own rounding to bf16, tests/_cmp.py); the
frequency and phase-bias gradients are sums over B*H*S rows and are compared relative to their
largest entry.
"""

import math

import pytest
import torch

from oracle import pe_oracle as O
from tests._cmp import argmax_err, err
from tests.test_gpu_sweep import bar_for, fp32_core
from pe_ablations_amd.functional import pe_attention

pytestmark = pytest.mark.gpu
f64 = torch.float64


def rnd(*shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g) * scale


def md(a, b):
    return err(a, b)


def oracle_operands(mode, qc, kc, qr, kr, freqs, delta, start_q, start_k, mscale, qk_norm, pos_dtype=None):
    """[content | transform] operands in fp32 the way the reference builds them."""
    if mode == "pope":
        tq = O.pope_transform(qr, freqs, start_q, pos_dtype=pos_dtype)
        tk = O.pope_transform(kr, freqs, start_k, delta, pos_dtype=pos_dtype)
    elif mode == "rope":
        tq = O.rope_rotate(qr, freqs, start_q) * mscale
        tk = O.rope_rotate(kr, freqs, start_k) * mscale
    else:
        tq, tk = qr.float(), kr.float()
    if qk_norm:
        tq, tk = O.qk_l2norm(tq), O.qk_l2norm(tk)
    if qc is not None:
        tq = torch.cat([qc.float(), tq], -1)
        tk = torch.cat([kc.float(), tk], -1)
    return tq, tk


def run_case(cuda, *, mode="pope", B=1, Hq=2, Hkv=2, Sq=128, Sk=None, Dr=64, Dv=64, Dc=0,
             dtype=torch.bfloat16, causal=True, freqs=None, delta=None, scale=None, mscale=1.0,
             qk_norm=False, start_q=0, start_k=0, seed=0, grad_freqs=False, grad_delta=True,
             path_names=(), pos_dtype=None):
    """One case through pe_attention against the oracle.  Every listed error is the raw max-abs.
    Each result is held to the raw bar (1e-5 fp32, 2e-2 bf16) wherever the reference path meets it
    at the same elements, else to PATH_FACTOR times the reference path's own error (bar_for);
    ``path_names`` lists the results for which the test expects the latter (it asserts that the
    reference path does miss the raw bar there)."""
    Sk = Sq if Sk is None else Sk
    tol = 2e-2 if dtype == torch.bfloat16 else 1e-5
    qr, kr = rnd(B, Hq, Sq, Dr, seed=seed), rnd(B, Hkv, Sk, Dr, seed=seed + 1)
    v = rnd(B, Hkv, Sk, Dv, seed=seed + 2)
    dout = rnd(B, Hq, Sq, Dv, seed=seed + 3)
    qc = rnd(B, Hq, Sq, Dc, seed=seed + 4) if Dc else None
    kc = rnd(B, Hkv, Sk, Dc, seed=seed + 5) if Dc else None
    ins = [t if t is None else t.to(dtype) for t in (qr, kr, v, qc, kc)]
    dout = dout.to(dtype)
    if scale is None:
        scale = (Dc + (2 * Dr if mode == "pope" else Dr)) ** -0.5
    causal_flag = ("bottom_right" if Sq != Sk else True) if causal else False

    # oracle: fp32 transforms, fp64 core, bf16 operand rounding in bf16 mode; the same graph with
    # the reference path's core (bf16: a bf16 fused SDPA's rounding points; fp32: float32 math)
    # gives the reference path's own error at every element
    rd = torch.bfloat16 if dtype == torch.bfloat16 else None

    def oracle_graph(core=None):
        o_in = [None if t is None else t.float().clone().requires_grad_(True) for t in ins]
        of = None if freqs is None else freqs.clone().requires_grad_(grad_freqs)
        od = None if delta is None else delta.clone().requires_grad_(grad_delta)
        tq, tk = oracle_operands(mode, o_in[3], o_in[4], o_in[0], o_in[1], of, od, start_q, start_k, mscale,
                                 qk_norm, pos_dtype)
        tq, tk, vv = O.round_ste(tq, rd), O.round_ste(tk, rd), O.round_ste(o_in[2].float(), rd)
        if core is None:
            ref, ref_lse = O.attention(tq, tk, vv, scale, causal=bool(causal))
        else:
            ref, ref_lse = core(tq, tk, vv, scale, bool(causal))
        ref.backward(dout.to(ref.dtype))
        return o_in, of, od, ref, ref_lse, vv

    o_in, of, od, ref, ref_lse, vv = oracle_graph()
    p_in, _, _, pref, _, _ = oracle_graph(O.attention_bf16_path if rd is not None else fp32_core)

    g_in = [None if t is None else t.to(cuda).requires_grad_(True) for t in ins]
    gf = None if freqs is None else freqs.to(cuda).requires_grad_(grad_freqs)
    gd = None if delta is None else delta.to(cuda).requires_grad_(grad_delta)
    out, lse = pe_attention(g_in[0], g_in[1], g_in[2], mode=mode, q_c=g_in[3], k_c=g_in[4], freqs=gf, delta=gd,
                            scale=scale, causal=causal_flag, start_pos_q=start_q, start_pos_k=start_k,
                            rope_mscale=mscale, qk_norm=qk_norm, return_lse=True, position_dtype=pos_dtype)
    out.backward(dout.to(cuda))
    torch.cuda.synchronize()
    errs = {"out": md(out, ref), "lse": md(lse, ref_lse)}
    path = {"out": err(pref.to(dtype), ref, "path out")}
    pairs = {"out": (out, ref)}
    for name, a, b, p in zip(("dq", "dk", "dv", "dqc", "dkc"), g_in, o_in, p_in):
        if a is not None:
            errs[name] = md(a.grad, b.grad)
            path[name] = err(p.grad.to(dtype), b.grad, "path " + name)
            pairs[name] = (a.grad, b.grad)
    print(f"run_case errors {errs} reference path {path}", flush=True)
    for name, e in errs.items():
        bar = bar_for(path[name], tol) if name in path else tol
        if name in path_names:  # the reference path itself misses the raw bar here (named by the test)
            assert path[name] >= tol, (name, "reference path meets the raw bar", path[name], errs)
        assert e < bar, (name, e, "bar", bar, "reference path", path.get(name),
                         "at (index, |ref|, err)", argmax_err(*pairs[name]) if name in pairs else None, errs)
    for name, a, b in (("dfreqs", gf, of), ("ddelta", gd, od)):
        if a is not None and a.requires_grad:
            rel = md(a.grad, b.grad) / max(1.0, b.grad.abs().max().item())
            assert rel < (2e-2 if dtype == torch.bfloat16 else 1e-4), (name, rel, errs)
    if pos_dtype is not None:
        # not vacuous: with exact positions the oracle's output is far from the kernel's
        eq, ek = oracle_operands(mode, *(None if t is None else t.detach() for t in (o_in[3], o_in[4], o_in[0], o_in[1])),
                                 freqs, None if delta is None else delta, start_q, start_k, mscale, qk_norm)
        exact, _ = O.attention(O.round_ste(eq, rd), O.round_ste(ek, rd), vv.detach(), scale, causal=bool(causal))
        errs["vs_exact_positions"] = md(out, exact)
        assert errs["vs_exact_positions"] > 5 * tol, errs
    return errs


# ------------------------------------------------------------------------------------- PoPE / FoPE

def test_fope_bf16_frequency_gradient(cuda):
    """FoPE = PoPE kernel with freqs = omega (src/model/fpope.py:107-146); d omega flows back.
    omega from 4 Fourier terms over random extra frequencies, floor 2pi/2048 (BASELINE config 3
    in miniature: D=128)."""
    D, M = 128, 4
    base = O.pope_freqs(D)
    table = torch.cat([base.unsqueeze(1), torch.rand(D, M - 1, generator=torch.Generator().manual_seed(9)) * float(base[0])], 1)
    coeffs = rnd(D, M, seed=10, scale=0.1)
    omega = O.fope_effective_freqs(base, coeffs, freq_table=table, training_length=2048).detach()
    delta = -torch.rand(2, D, generator=torch.Generator().manual_seed(11)) * 2 * math.pi
    run_case(cuda, Dr=D, Dv=D, Sq=320, freqs=omega, delta=delta, grad_freqs=True, seed=20)


def test_fope_fp32_frequency_gradient(cuda):
    D = 32
    omega = O.fope_effective_freqs(O.pope_freqs(D), rnd(D, 4, seed=12, scale=0.4)).detach()
    run_case(cuda, Dr=D, Dv=64, Sq=200, B=2, dtype=torch.float32, freqs=omega,
             delta=-torch.rand(D) * 6, grad_freqs=True, seed=30)


def test_pope_shared_delta_start_pos_fp32(cuda):
    """Reference layout: delta (D,) shared by heads, start_pos > 0 (cached-angle offset)."""
    run_case(cuda, Dr=64, Dv=64, Sq=150, Hq=3, Hkv=3, dtype=torch.float32, freqs=O.pope_freqs(64),
             delta=-torch.rand(64) * 6, start_q=77, start_k=77, seed=40)


def test_split_form_reference_module_shape(cuda):
    """The reference module's contraction: [q_c (64) | PoPE(q_r) (2x32)], V 64, GQA 8 -> 4,
    scale (64 + 64)^-1/2 (src/model/fpope_attention.py:107,166-177).

    dv sums two query heads' gradients per key and reaches |dv| ~ 7 here, where the bf16 spacing
    is 2^-5.  The reference path (bf16 SDPA rounding points) misses the raw 2e-2 bar on dv itself
    (0.0249), so dv is held to 1.25 times that path's own error; the kernel's measured 0.0168."""
    run_case(cuda, Dc=64, Dr=32, Dv=64, Hq=8, Hkv=4, Sq=256, B=2, freqs=O.pope_freqs(32),
             delta=-torch.rand(32) * 6, seed=50, path_names=("dv",))


def test_split_form_fp32(cuda):
    run_case(cuda, Dc=64, Dr=32, Dv=64, Hq=4, Hkv=2, Sq=130, dtype=torch.float32, freqs=O.pope_freqs(32),
             delta=-torch.rand(32) * 6, seed=60)


def test_pope_bottom_right_decode(cuda):
    """KV-cache shapes: Sq < Sk with the bottom-right mask (src/model/fpope_attention.py:313-317)."""
    run_case(cuda, Dr=64, Dv=64, Sq=3, Sk=300, Hq=4, Hkv=2, freqs=O.pope_freqs(64),
             delta=-torch.rand(2, 64) * 6, start_q=297, start_k=0, seed=70)
    run_case(cuda, Dr=64, Dv=64, Sq=64, Sk=200, dtype=torch.float32, freqs=O.pope_freqs(64),
             delta=-torch.rand(2, 64) * 6, start_q=136, start_k=0, seed=71)


def test_pope_non_causal(cuda):
    run_case(cuda, Dr=64, Dv=128, Sq=100, Sk=150, causal=False, freqs=O.pope_freqs(64),
             delta=-torch.rand(2, 64) * 6, seed=80)


def test_pope_odd_width_padding(cuda):
    """D = 48 (transformed width 96, padded to 128 inside the library), V = 40."""
    run_case(cuda, Dr=48, Dv=40, Sq=90, freqs=O.pope_freqs(48), delta=-torch.rand(2, 48) * 6, seed=85)


# ------------------------------------------------------------------------------------- RoPE / none

@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_rope_qknorm(cuda, dtype):
    """RoPE (interleaved pairs) + QKNorm, scale 1/sqrt(D), GQA (src/model/attention.py:77-96)."""
    run_case(cuda, mode="rope", Dr=64, Dv=64, Hq=4, Hkv=2, Sq=200, B=2, dtype=dtype,
             freqs=O.rope_inv_freq(64), qk_norm=True, scale=1 / 8, seed=90)


def test_rope_ntk_no_norm(cuda):
    run_case(cuda, mode="rope", Dr=128, Dv=128, Sq=160, freqs=O.rope_inv_freq(128, O.ntk_theta(128, 10000.0, 4.0)),
             qk_norm=False, scale=128 ** -0.5, start_q=11, start_k=11, seed=100)


def test_yarn_mscale(cuda):
    """YaRN inverse frequencies and mscale on both q and k (src/model/rope.py:206-217), no QKNorm
    (with QKNorm the mscale cancels)."""
    inv, ms, _, _ = O.yarn_inv_freq(64, 10000.0, 8.0)
    run_case(cuda, mode="rope", Dr=64, Dv=64, Sq=140, dtype=torch.float32, freqs=inv, mscale=ms,
             qk_norm=False, scale=1 / 8, seed=110)


def test_nope_qknorm(cuda):
    run_case(cuda, mode="none", Dr=64, Dv=64, Hq=4, Hkv=4, Sq=96, qk_norm=True, scale=1 / 8, seed=120)


@pytest.mark.parametrize("mode,Dr,qk_norm,dtype,mscale", [
    ("rope", 64, True, torch.bfloat16, 1.0),
    ("rope", 128, False, torch.bfloat16, 1.25),
    ("rope", 32, True, torch.float16, 1.0),
    ("rope", 64, True, torch.float16, 1.25),
    ("rope", 64, True, torch.float32, 1.0),
    ("none", 64, True, torch.bfloat16, 1.0),
    ("none", 128, False, torch.bfloat16, 1.0)])
def test_rope_vector_prologue_matches_row_kernels(cuda, mode, Dr, qk_norm, dtype, mscale):
    """RoPE / no-PE operands whose rows take 16-byte accesses go through the vectorised prologue and
    gradient kernels (8 elements per thread); at width 64 in 16-bit the gradient runs in the dQ GEMM's
    and the dK/dV kernel's epilogues instead, on their staged rows.  q and k views that start one
    element off alignment go through the one-wave-per-row kernels.  All of them evaluate the same
    per-pair arithmetic and add QKNorm's row sums in the same order (chunks of 4 pairs, then an xor
    butterfly over the chunks), so the outputs and every gradient agree bit for bit."""
    B, Hq, Hkv, S, Dv = 2, 4, 2, 300, 64
    g = torch.Generator().manual_seed(130 + Dr)
    mk = lambda h, d: torch.randn(B, h, S, d, generator=g).to(dtype)
    q, k, v, do = mk(Hq, Dr), mk(Hkv, Dr), mk(Hkv, Dv), mk(Hq, Dv)
    freqs = O.rope_inv_freq(Dr).to(cuda) if mode == "rope" else None

    def off(t):  # the same values in a view one element past a 16-byte boundary
        wide = torch.zeros(*t.shape[:-1], t.shape[-1] + 1, dtype=t.dtype, device=cuda)
        wide[..., 1:] = t.to(cuda)
        return wide[..., 1:]

    def run(unaligned):
        qv, kv = (off(q), off(k)) if unaligned else (q.to(cuda), k.to(cuda))
        leaves = [qv.requires_grad_(True), kv.requires_grad_(True), v.to(cuda).requires_grad_(True)]
        out = pe_attention(*leaves, mode=mode, freqs=freqs, qk_norm=qk_norm, rope_mscale=mscale,
                           scale=Dr ** -0.5)
        grads = torch.autograd.grad(out, leaves, do.to(cuda))
        torch.cuda.synchronize()
        return [out] + list(grads)

    vec, rows = run(False), run(True)
    for n, a, b in zip(["out", "dq", "dk", "dv"], vec, rows):
        assert torch.equal(a, b), (mode, Dr, n, md(a, b))


# ------------------------------------------------------------- FoPE positions in the input dtype

def test_fope_positions_bf16_fused(cuda):
    """FoPE without QK norm under bf16 autocast builds its positions with
    torch.arange(..., dtype=bf16) (src/model/fpope.py:285,322): above 256 they are rounded (to
    multiples of 4 in 512..1023).  The fused bf16 path (prologue, dK/dV and dQ epilogues, query
    phase table, frequency gradient) with position_dtype=bf16 against the oracle built the same
    way, positions 300..1019."""
    D = 64
    omega = O.fope_effective_freqs(O.pope_freqs(D), rnd(D, 4, seed=40, scale=0.4)).detach()
    delta = -torch.rand(2, D, generator=torch.Generator().manual_seed(41)) * 2 * math.pi
    run_case(cuda, Dr=D, Dv=D, Sq=720, freqs=omega, delta=delta, grad_freqs=True, start_q=300, start_k=300,
             pos_dtype=torch.bfloat16, seed=42)


def test_fope_positions_bf16_split_form_gqa(cuda):
    """The same rounding through the split form (content 64 | PoPE 2 x 32, GQA 4 -> 2), whose
    backward takes the stand-alone inverse-transform kernels."""
    D = 32
    omega = O.fope_effective_freqs(O.pope_freqs(D), rnd(D, 4, seed=43, scale=0.4)).detach()
    run_case(cuda, Dr=D, Dv=64, Dc=64, Hq=4, Hkv=2, Sq=600, freqs=omega, delta=-torch.rand(D) * 6,
             grad_freqs=True, start_q=400, start_k=400, pos_dtype=torch.bfloat16, seed=44)


def test_positions_fp16_fp32_mode(cuda):
    """fp16 rounding (fp16 autocast; spacing 4 between 4096 and 8191) checked at the fp32 bar, so
    every phase must match the oracle's to fp32 accuracy."""
    D = 32
    omega = O.fope_effective_freqs(O.pope_freqs(D), rnd(D, 4, seed=45, scale=0.4)).detach()
    run_case(cuda, Dr=D, Dv=64, Sq=160, dtype=torch.float32, freqs=omega, delta=-torch.rand(D) * 6,
             grad_freqs=True, start_q=5000, start_k=5000, pos_dtype=torch.float16, seed=46)


def test_split_form_fused_epilogue_matches_unfused_path(cuda):
    """The split form [content 64 | PoPE 2 x 32] in bf16 applies its inverse transform and copies
    the content gradient in the gradient kernels' epilogues when every view is 16-byte aligned.
    The same call with a q_c view that starts 2 bytes off alignment takes the stand-alone inverse
    kernels instead.  Both evaluate the same per-element function on the same fp32 gradients, so
    every gradient agrees bit for bit; the phase-gradient partial sums run over different blocks."""
    B, Hq, Hkv, S, Dc, Dr, Dv = 2, 8, 4, 700, 64, 32, 64
    g = torch.Generator().manual_seed(60)
    mk = lambda h, d: torch.randn(B, h, S, d, generator=g).to(torch.bfloat16)
    qr, kr, qc, kc, v, do = mk(Hq, Dr), mk(Hkv, Dr), mk(Hq, Dc), mk(Hkv, Dc), mk(Hkv, Dv), mk(Hq, Dv)
    freqs = O.fope_effective_freqs(O.pope_freqs(Dr), rnd(Dr, 4, seed=61, scale=0.4)).detach()
    delta = -torch.rand(Dr, generator=g) * 6

    def run(unaligned):
        wide = torch.zeros(B, Hq, S, Dc + 1, dtype=torch.bfloat16)
        wide[..., 1:] = qc
        qcv = wide.to(cuda)[..., 1:] if unaligned else qc.to(cuda)
        ins = [t.to(cuda) for t in (qr, kr, v, kc)]
        leaves = [ins[0], ins[1], ins[2], qcv, ins[3]]
        for t in leaves:
            t.requires_grad_(True)
        f, d = freqs.to(cuda).requires_grad_(True), delta.to(cuda).requires_grad_(True)
        out = pe_attention(ins[0], ins[1], ins[2], mode="pope", q_c=qcv, k_c=ins[3], freqs=f, delta=d)
        grads = torch.autograd.grad(out, leaves + [f, d], do.to(cuda))
        torch.cuda.synchronize()
        return [out] + list(grads)

    fused, plain = run(False), run(True)
    names = ["out", "dqr", "dkr", "dv", "dqc", "dkc", "dfreqs", "ddelta"]
    for n, a, b in zip(names, fused, plain):
        if n in ("dfreqs", "ddelta"):
            assert md(a, b) / max(1.0, b.abs().max().item()) < 1e-5, n
        else:
            assert torch.equal(a, b), (n, md(a, b))
    # and the fused path against the oracle (the reference module's contraction, fp64 core)
    o = [t.float().requires_grad_(True) for t in (qc, kc, qr, kr, v)]
    of, od = freqs.clone().requires_grad_(True), delta.clone().requires_grad_(True)
    ref, _ = O.split_pope_attention(o[0], o[1], o[2], o[3], o[4], of, od, operand_dtype=torch.bfloat16)
    rg = torch.autograd.grad(ref, [o[2], o[3], o[4], o[0], o[1], of, od], do.double())
    for n, a, b in zip(names, fused, [ref] + list(rg)):
        if n in ("dfreqs", "ddelta"):
            assert md(a, b) / max(1.0, b.abs().max().item()) < 2e-2, n
        else:
            assert md(a, b) < 2e-2, n
