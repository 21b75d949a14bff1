"""The fused SwiGLU kernel (pe_swiglu_fwd) against the reference's expression F.silu(gate) * x
(src/model/ffn.py:17-27).

The kernel evaluates both bf16 ops as torch's GPU kernels do (silu in fp32 as g / (1 + exp(-g)),
rounded to bf16, then the product in fp32, rounded to bf16), so it is compared bit for bit with
torch on the GPU.  Against the expression on the CPU, whose exp is another implementation, the bar
is one bf16 ulp of the silu, carried through the product, plus one ulp of the result.
"""

import pytest
import torch
import torch.nn.functional as F

from pe_ablations_amd.ffn import FeedForward, SwiGLU
from pe_ablations_amd.functional import swiglu

pytestmark = pytest.mark.gpu


def ulp_bf16(x):
    e = torch.floor(torch.log2(x.abs().clamp_min(1e-30)))
    return torch.pow(2.0, e - 7)


@pytest.mark.parametrize("shape", [(8,), (3, 77, 5632), (1, 16384, 64), (2, 5, 24), (3, 7)])
@torch.no_grad()
def test_swiglu_bitwise_torch_gpu(cuda, shape):
    g = torch.Generator().manual_seed(sum(shape))
    x = (torch.randn(*shape, generator=g) * 3).bfloat16().to(cuda)
    gate = (torch.randn(*shape, generator=g) * 4).bfloat16().to(cuda)
    out = swiglu(x, gate)
    ref = F.silu(gate) * x
    assert out.dtype == torch.bfloat16 and out.shape == x.shape
    assert torch.equal(out, ref)
    # the CPU expression, another exp: within one ulp of the silu (times |x|) and one of the result
    cref = (F.silu(gate.cpu()) * x.cpu()).float()
    sil = F.silu(gate.cpu().float())
    tol = ulp_bf16(sil) * x.cpu().float().abs() + ulp_bf16(cref)
    assert bool(((out.cpu().float() - cref).abs() <= tol).all())


@torch.no_grad()
def test_swiglu_special_values(cuda):
    gate = torch.tensor([-200.0, -88.0, -20.0, -1.0, -0.0, 0.0, 1.0, 20.0, 88.0, 3e38, -3e38,
                         float("inf"), float("-inf"), 1e-30, -1e-30, 7.5], dtype=torch.bfloat16, device=cuda)
    x = torch.tensor([1.0, -2.0, 3.0, -4.0, 5.0, -6.0, 7.0, -8.0, 9.0, 1.0, 1.0,
                      2.0, 2.0, 1e30, -1e30, 0.0], dtype=torch.bfloat16, device=cuda)
    out, ref = swiglu(x, gate), F.silu(gate) * x
    same = (out == ref) | (torch.isnan(out) & torch.isnan(ref))
    assert bool(same.all()), (out, ref)
    num = ~torch.isnan(ref)   # the sign of a NaN (gate = -inf: -inf / inf) carries no meaning
    assert torch.equal(torch.signbit(out)[num], torch.signbit(ref)[num])


@torch.no_grad()
def test_feedforward_module_takes_the_kernel_without_grad(cuda):
    torch.manual_seed(0)
    ff = FeedForward(256, ffn_dim=688).to(cuda).bfloat16()
    h = torch.randn(4, 33, 256, device=cuda).bfloat16()
    a, b = ff.w1(h), ff.w3(h)
    assert torch.equal(SwiGLU()(a, b), F.silu(b) * a)
    assert torch.equal(ff(h), ff.w2(F.silu(b) * a))
    with torch.enable_grad():   # training keeps the torch expression (autograd)
        hg = h.clone().requires_grad_(True)
        y = ff(hg)
        y.float().sum().backward()
        assert hg.grad is not None and bool(torch.isfinite(hg.grad.float()).all())


def test_swiglu_argument_errors(cuda):
    x = torch.zeros(16, dtype=torch.bfloat16, device=cuda)
    with pytest.raises(TypeError):
        swiglu(x, x.float())
    with pytest.raises(TypeError):
        swiglu(x, x[:8])
    with pytest.raises(RuntimeError):
        swiglu(x.cpu(), x.cpu())
