"""GPU parity of the HIP PE-attention path (libpe_attn.so through its C ABI) against the CPU oracle.

Tolerances (north star): max-abs 1e-5 in fp32 mode, 2e-2 in bf16 mode for the output and
dQ/dK/dV (raw max-abs, a bf16 result including its own rounding to bf16, tests/_cmp.py); the
phase-bias / frequency gradients are sums over B*H*S rows and are compared relative
to their own scale.  The oracle computes the transforms in fp32 exactly as the reference orders
them and the attention core in fp64; in bf16 mode it rounds the transformed operands to bf16 the
way autocast hands them to SDPA.
"""

import math

import pytest
import torch

from oracle import pe_oracle as O
from tests._cmp import err
from pe_ablations_amd.functional import pe_attention

pytestmark = pytest.mark.gpu


def _inputs(B, Hq, Hkv, S, D, Dv=None, dtype=torch.float32, seed=0, delta_per_head=True, Sk=None):
    g = torch.Generator().manual_seed(seed)
    Sk = S if Sk is None else Sk
    Dv = D if Dv is None else Dv
    q = torch.randn(B, Hq, S, D, generator=g).to(dtype)
    k = torch.randn(B, Hkv, Sk, D, generator=g).to(dtype)
    v = torch.randn(B, Hkv, Sk, Dv, generator=g).to(dtype)
    freqs = O.pope_freqs(D)
    shape = (Hkv, D) if delta_per_head else (D,)
    delta = torch.rand(shape, generator=g) * (-2 * math.pi)
    return q, k, v, freqs, delta


def _maxdiff(a, b):
    return err(a, b)


def _gpu(*ts, dev):
    return [None if t is None else t.to(dev) for t in ts]


@pytest.mark.parametrize("delta_per_head", [True, False])
def test_config1_pope_fp32_forward(cuda, delta_per_head):
    """B=1, H=4, S=512, D=64, fp32 forward, seed 0 -> 1e-5."""
    q, k, v, freqs, delta = _inputs(1, 4, 4, 512, 64, seed=0, delta_per_head=delta_per_head)
    ref_out, ref_lse = O.pope_attention(q, k, v, freqs, delta, scale=1 / 8, clamp=False)
    qg, kg, vg, fg, dg = _gpu(q, k, v, freqs, delta, dev=cuda)
    out, lse = pe_attention(qg, kg, vg, mode="pope", freqs=fg, delta=dg, scale=1 / 8, return_lse=True)
    torch.cuda.synchronize()
    assert out.dtype == torch.float32
    assert _maxdiff(out, ref_out) < 1e-5
    assert _maxdiff(lse, ref_lse) < 1e-5


def _check_bwd(cuda, B, Hq, Hkv, S, D, dtype, tol, Dv=None, seed=1, scale=None, grad_tol=None):
    q, k, v, freqs, delta = _inputs(B, Hq, Hkv, S, D, Dv=Dv, dtype=dtype, seed=seed)
    g = torch.Generator().manual_seed(seed + 100)
    dout = torch.randn(B, Hq, S, v.shape[-1], generator=g).to(dtype)
    scale = scale if scale is not None else 1 / math.sqrt(D)
    # oracle with autograd (fp64 core, fp32 transforms, bf16 operand rounding in bf16 mode)
    qo, ko, vo = (t.detach().float().clone().requires_grad_(True) for t in (q, k, v))
    fo, do_ = freqs.clone().requires_grad_(True), delta.clone().requires_grad_(True)
    od = torch.bfloat16 if dtype == torch.bfloat16 else None
    ref_out, _ = O.pope_attention(qo, ko, vo, fo, do_, scale=scale, clamp=False, operand_dtype=od)
    ref_out.backward(dout.double())
    qg, kg, vg, fg, dg, dog = _gpu(q, k, v, freqs, delta, dout, dev=cuda)
    for t in (qg, kg, vg, fg, dg):
        t.requires_grad_(True)
    out = pe_attention(qg, kg, vg, mode="pope", freqs=fg, delta=dg, scale=scale)
    out.backward(dog)
    torch.cuda.synchronize()
    res = {"out": _maxdiff(out, ref_out), "dq": _maxdiff(qg.grad, qo.grad), "dk": _maxdiff(kg.grad, ko.grad),
           "dv": _maxdiff(vg.grad, vo.grad)}
    for name, val in res.items():
        assert val < tol, (name, res)
    gt = grad_tol if grad_tol is not None else tol
    for name, a, b in (("dfreqs", fg.grad, fo.grad), ("ddelta", dg.grad, do_.grad)):
        rel = _maxdiff(a, b) / max(1.0, b.abs().max().item())
        assert rel < gt, (name, rel, res)
    return res


def test_pope_bwd_fp32_small(cuda):
    _check_bwd(cuda, 2, 3, 3, 100, 32, torch.float32, 1e-5, grad_tol=1e-4)


def test_pope_bwd_fp32_d64(cuda):
    _check_bwd(cuda, 1, 2, 2, 256, 64, torch.float32, 1e-5, grad_tol=1e-4)


def test_pope_bwd_bf16_ragged(cuda):
    _check_bwd(cuda, 2, 3, 3, 300, 64, torch.bfloat16, 2e-2, grad_tol=2e-2)


def test_pope_bwd_bf16_d128(cuda):
    _check_bwd(cuda, 1, 2, 2, 384, 128, torch.bfloat16, 2e-2, grad_tol=2e-2)


def test_pope_bwd_bf16_gqa(cuda):
    _check_bwd(cuda, 1, 4, 2, 200, 64, torch.bfloat16, 2e-2, grad_tol=2e-2)


def test_pope_minimal_dims(cuda):
    """S=1, H=1, B=1, D=1 (tests/test_fpope.py:911-976): O = V for a single token."""
    q, k, v, freqs, delta = _inputs(1, 1, 1, 1, 1)
    qg, kg, vg, fg, dg = _gpu(q, k, v, freqs, delta, dev=cuda)
    out = pe_attention(qg, kg, vg, mode="pope", freqs=fg, delta=dg, scale=1.0)
    torch.cuda.synchronize()
    assert _maxdiff(out, v) < 1e-6


def test_zero_values_give_zero_output(cuda):
    """V = 0 -> O = 0 (tests/test_fpope.py:1033-1045)."""
    q, k, v, freqs, delta = _inputs(2, 4, 4, 16, 64)
    qg, kg, fg, dg = _gpu(q, k, freqs, delta, dev=cuda)
    out = pe_attention(qg, kg, torch.zeros_like(v, device=cuda), mode="pope", freqs=fg, delta=dg)
    torch.cuda.synchronize()
    assert out.abs().max().item() < 1e-6


def test_deterministic(cuda):
    q, k, v, freqs, delta = _inputs(1, 2, 2, 200, 64, dtype=torch.bfloat16)
    res = []
    for _ in range(2):
        qg, kg, vg, fg, dg = _gpu(q, k, v, freqs, delta, dev=cuda)
        for t in (qg, kg, vg, dg):
            t.requires_grad_(True)
        out = pe_attention(qg, kg, vg, mode="pope", freqs=fg, delta=dg)
        out.sum().backward()
        res.append([out.detach(), qg.grad, kg.grad, vg.grad, dg.grad])
    for a, b in zip(*res):
        assert torch.equal(a, b)


@pytest.mark.parametrize("D", [64, 128])
def test_unaligned_views_take_the_elementwise_epilogue(cuda, D):
    """bf16 fwd+bwd with q and k as views that start one element into a wider buffer.  The fused
    inverse transform in the gradient kernels cannot use 16-byte vectors on them and takes its
    element-by-element path; dq / dk must equal those of the vectorised path (same inputs in
    aligned tensors) bit for bit, since both apply the same per-element arithmetic, and the
    phase-gradient sums (reduced in another order) must agree with the oracle."""
    B, H, S = 1, 2, 384
    q, k, v, freqs, delta = _inputs(B, H, H, S, D, dtype=torch.bfloat16, seed=7)
    g = torch.Generator().manual_seed(77)
    dout = torch.randn(B, H, S, D, generator=g).to(torch.bfloat16).to(cuda)
    scale = 1 / math.sqrt(D)

    def run(qx, kx):
        vg, fg, dg = (t.to(cuda).requires_grad_(True) for t in (v, freqs, delta))
        out = pe_attention(qx, kx, vg, mode="pope", freqs=fg, delta=dg, scale=scale)
        out.backward(dout)
        torch.cuda.synchronize()
        return out.detach(), qx.grad, kx.grad, vg.grad, fg.grad, dg.grad

    def unaligned(t):
        wide = torch.zeros(*t.shape[:-1], t.shape[-1] + 8, dtype=t.dtype, device=cuda)
        wide[..., 1:1 + t.shape[-1]] = t.to(cuda)
        view = wide[..., 1:1 + t.shape[-1]].detach().requires_grad_(True)
        assert view.data_ptr() % 16 != 0
        return view

    ref = run(q.to(cuda).requires_grad_(True), k.to(cuda).requires_grad_(True))
    got = run(unaligned(q), unaligned(k))
    for name, a, b in zip(("out", "dq", "dk", "dv"), ref[:4], got[:4]):
        assert torch.equal(a, b), name
    qo, ko, vo = (t.detach().float().clone().requires_grad_(True) for t in (q, k, v))
    fo, do_ = freqs.clone().requires_grad_(True), delta.clone().requires_grad_(True)
    ref_out, _ = O.pope_attention(qo, ko, vo, fo, do_, scale=scale, clamp=False, operand_dtype=torch.bfloat16)
    ref_out.backward(dout.cpu().double())
    assert _maxdiff(got[1], qo.grad) < 2e-2 and _maxdiff(got[2], ko.grad) < 2e-2
    for a, b in ((got[4], fo.grad), (got[5], do_.grad), (ref[4], fo.grad), (ref[5], do_.grad)):
        assert _maxdiff(a, b) / max(1.0, b.abs().max().item()) < 2e-2
