"""The RMSNorm kernels on the GPU: the stand-alone pe_rmsnorm_fwd against the oracle's RMSNorm
(oracle.rms_norm, the reference's expression on the CPU), and the PoPE prologue with the norm
fused in (pe_attn_fwd_normed) against the module's unfused path (torch-autograd RMSNorm followed
by pe_attn_fwd) and against the oracle.

Tolerances: fp32 results to 2e-6 relative (the sum of squares is reduced in another order than
torch's).  A last-bit difference in those fp32 statistics can move a bf16 rounding boundary: for
bf16 x the normalised value may differ by one bf16 ulp (times the weight in the result), and when
the weight is bf16 too the product is rounded again, which adds one ulp of the result.
"""

import pytest
import torch

from oracle import pe_oracle as O
from pe_ablations_amd.fpope import FoPEPoPEEmbedding
from pe_ablations_amd.fpope_attention import FPoPEGroupedQueryAttention
from pe_ablations_amd.functional import pe_attention, rms_norm
from pe_ablations_amd.normalization import RMSNorm
from pe_ablations_amd.pope import PoPEEmbedding

pytestmark = pytest.mark.gpu

DT = {"bf16": torch.bfloat16, "fp32": torch.float32}


def ulp_bf16(x):
    e = torch.floor(torch.log2(x.abs().clamp_min(1e-30)))
    return torch.pow(2.0, e - 7)


@pytest.mark.parametrize("xd,wd", [("bf16", "bf16"), ("bf16", "fp32"), ("fp32", "fp32"), ("fp32", "bf16")])
@pytest.mark.parametrize("rows,n", [(1, 64), (37, 2048), (5, 4096), (513, 8192), (9, 1000)])
def test_rmsnorm_matches_oracle(cuda, xd, wd, rows, n):
    g = torch.Generator().manual_seed(rows * 7 + n)
    x = (torch.randn(rows, n, generator=g) * 3).to(DT[xd])
    w = (0.5 + torch.rand(n, generator=g)).to(DT[wd])
    print(f"rmsnorm x={xd} w={wd} rows={rows} n={n}", flush=True)
    y = rms_norm(x.to(cuda), w.to(cuda), 1e-6)
    ref = O.rms_norm(x, w, 1e-6)
    assert y.dtype == ref.dtype
    d = (y.double().cpu() - ref.double()).abs()
    if x.dtype == torch.bfloat16:
        # the normalised value is rounded to bf16: one ulp of it, scaled by the weight, plus one ulp
        # of the result when the product is rounded to bf16 as well
        n_ref = O.rms_norm(x, torch.ones(n, dtype=torch.bfloat16), 1e-6).double()
        tol = ulp_bf16(n_ref) * w.double().abs() * 1.01
        if y.dtype == torch.bfloat16:
            tol = tol + ulp_bf16(ref.double())
        assert (d <= tol).all()
    else:
        assert (d <= 2e-6 * ref.double().abs() + 1e-30).all()


def test_rmsnorm_strided_rows_and_batch_dims(cuda):
    g = torch.Generator().manual_seed(3)
    base = torch.randn(4, 50, 3 * 256, generator=g)
    x = base[..., 256:512]                      # row stride 768, offset 256 elements
    w = 0.5 + torch.rand(256, generator=g)
    y = rms_norm(x.to(cuda), w.to(cuda))
    assert y.shape == x.shape
    assert (y.cpu() - O.rms_norm(x, w)).abs().max().item() < 2e-6 * x.abs().max().item() * 10


def test_rmsnorm_module_switches_to_kernel_only_without_grad(cuda):
    m = RMSNorm(512).to(cuda)
    with torch.no_grad():
        m.weight.copy_(0.5 + torch.rand(512))
    x = torch.randn(3, 11, 512, device=cuda)
    with torch.no_grad():
        a = m(x)
    b = m(x)                                    # autograd path: the reference's expression
    assert b.requires_grad and not a.requires_grad
    assert (a - b).abs().max().item() < 2e-6 * b.abs().max().item()


def _module(kind, dr, seed=0, dtype=torch.float32):
    torch.manual_seed(seed)
    if kind == "fpope":
        pe = FoPEPoPEEmbedding(dr, 1024, num_fourier_terms=4, delta_init="uniform")
    else:
        pe = PoPEEmbedding(dr, 1024, delta_init="uniform")
    m = FPoPEGroupedQueryAttention(256, 8, 4, 64, dr, fpope=pe)
    with torch.no_grad():
        m.qr_norm.weight.copy_(0.5 + torch.rand(m.qr_norm.weight.shape))
        m.kr_norm.weight.copy_(0.5 + torch.rand(m.kr_norm.weight.shape))
    return m


@pytest.mark.parametrize("kind,dr", [("pope", 32), ("pope", 64), ("fpope", 32)])
def test_fused_norm_prologue_fp32_equals_unfused(cuda, kind, dr):
    """No-grad forward (norm inside the transform kernel) == grad-enabled forward (module RMSNorm,
    then the plain prologue) == the oracle on the CPU."""
    m = _module(kind, dr)
    x = torch.randn(2, 77, 256)
    from tests.test_gpu_modules import cpu_fpope_module
    ref = cpu_fpope_module(m, x, start_pos=9)
    g = m.to(cuda)
    xg = x.to(cuda)
    with torch.no_grad():
        assert g._fuse_norm(xg)
        fused = g(xg, start_pos=9)
    unfused = g(xg, start_pos=9).detach()
    assert (fused - unfused).abs().max().item() < 1e-5
    assert (fused.cpu().double() - ref.double()).abs().max().item() < 1e-4


def test_fused_norm_prologue_bf16(cuda):
    """bf16 weights and activations (the decoder's setting): the fused path and the module path
    differ only by where rounding boundaries fall; both stay within the bf16 attention tolerance
    of the fp32 result."""
    m = _module("pope", 64, seed=1)
    x = torch.randn(1, 300, 256)
    g32 = m.to(cuda)
    with torch.no_grad():
        ref = g32(x.to(cuda), start_pos=3).float()
    gb = _module("pope", 64, seed=1).to(cuda)
    for name, p in gb.named_parameters():
        if not name.startswith("fpope."):
            p.data = p.data.to(torch.bfloat16)
    xb = x.to(cuda).to(torch.bfloat16)
    with torch.no_grad():
        fused = gb(xb, start_pos=3)
    unfused = gb(xb, start_pos=3).detach()
    assert fused.dtype == torch.bfloat16
    assert (fused.float() - unfused.float()).abs().max().item() < 2e-2
    assert (fused.float() - ref).abs().max().item() < 5e-2


def test_fused_norm_refuses_grad(cuda):
    q = torch.randn(1, 2, 16, 32, device=cuda, requires_grad=True)
    k = torch.randn(1, 2, 16, 32, device=cuda)
    v = torch.randn(1, 2, 16, 32, device=cuda)
    w = torch.ones(64, device=cuda)
    with pytest.raises(RuntimeError, match="forward-only"):
        pe_attention(q, k, v, mode="pope", freqs=torch.ones(32, device=cuda), qr_norm_weight=w, kr_norm_weight=w)


def test_fused_norm_fused_form_decoder_shape(cuda):
    """Fused form at the 1B shape's head layout (16 heads x 128, H*Dr = 2048 features per token,
    one wave per token with four chunks per lane) against the oracle, fp32."""
    torch.manual_seed(5)
    pe = PoPEEmbedding(128, 512, delta_init="uniform")
    m = FPoPEGroupedQueryAttention(256, 16, 16, 128, 128, fpope=pe, d_content=0)
    with torch.no_grad():
        m.qr_norm.weight.copy_(0.5 + torch.rand(2048))
        m.kr_norm.weight.copy_(0.5 + torch.rand(2048))
    x = torch.randn(1, 130, 256)
    B, S = 1, 130
    qr = O.rms_norm(x @ m.wq_r.weight.T, m.qr_norm.weight).view(B, S, 16, 128).transpose(1, 2)
    kr = O.rms_norm(x @ m.wk_r.weight.T, m.kr_norm.weight).view(B, S, 16, 128).transpose(1, 2)
    v = (x @ m.wv.weight.T).view(B, S, 16, 128).transpose(1, 2)
    ref, _ = O.pope_attention(qr, kr, v, pe.effective_freqs, pe.phase_bias, scale=128 ** -0.5)
    ref = ref.float().transpose(1, 2).reshape(B, S, -1) @ m.wo.weight.T
    with torch.no_grad():
        out = m.to(cuda)(x.to(cuda))
    assert (out.cpu() - ref).abs().max().item() < 1e-4
