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
from pe_ablations_amd.functional import pe_attention, rms_norm, rms_norm_backward
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
    """Forward with the norm inside the transform kernel == the module's RMSNorm then the plain
    prologue == the oracle on the CPU."""
    m = _module(kind, dr)
    x = torch.randn(2, 77, 256)
    from tests.test_gpu_modules import cpu_fpope_module
    ref = cpu_fpope_module(m, x, start_pos=9)
    g = m.to(cuda)
    xg = x.to(cuda)
    with torch.no_grad():
        assert g._fuse_norm(xg)
        fused = g(xg, start_pos=9)
        unfused = _unfused(g)(xg, start_pos=9)
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
        unfused = _unfused(gb)(xb, start_pos=3)
    assert fused.dtype == torch.bfloat16
    assert (fused.float() - unfused.float()).abs().max().item() < 2e-2
    assert (fused.float() - ref).abs().max().item() < 5e-2


@pytest.mark.parametrize("xd,wd", [("bf16", "bf16"), ("bf16", "fp32"), ("fp32", "fp32"), ("fp32", "bf16")])
@pytest.mark.parametrize("rows,n", [(1, 64), (37, 2048), (700, 256), (513, 8192), (9, 1000), (4096, 128)])
def test_rmsnorm_backward_matches_autograd(cuda, xd, wd, rows, n):
    """pe_rmsnorm_bwd against torch autograd of the reference's expression (oracle.rms_norm, the
    module's forward, src/model/normalization.py:22-27) in the same dtypes on the CPU.  The kernel
    reduces its sums (the forward's sum of squares, the gradient's sum through r, dw over the rows)
    in another order than torch; fp32 results agree to 1e-5 of their scale, a bf16 dx to one bf16
    spacing (a last-bit difference can move a rounding boundary), and dw within the few spacings of
    the rounded normalised values that such a boundary can move."""
    g = torch.Generator().manual_seed(rows * 3 + n)
    x = (torch.randn(rows, n, generator=g) * 3).to(DT[xd])
    w = (0.5 + torch.rand(n, generator=g)).to(DT[wd])
    ydt = torch.bfloat16 if xd == "bf16" and wd == "bf16" else torch.float32
    dy = torch.randn(rows, n, generator=g).to(ydt)
    print(f"rmsnorm bwd x={xd} w={wd} rows={rows} n={n}", flush=True)
    xr, wr = x.clone().requires_grad_(True), w.clone().requires_grad_(True)
    y = O.rms_norm(xr, wr, 1e-6)
    assert y.dtype == ydt
    y.backward(dy)
    dx, dw = rms_norm_backward(x.to(cuda), w.to(cuda), dy.to(cuda), 1e-6)
    assert dx.dtype == x.dtype and dw.dtype == w.dtype and dw.shape == w.shape
    ddx = (dx.double().cpu() - xr.grad.double()).abs()
    if xd == "bf16":
        assert (ddx <= ulp_bf16(xr.grad.double()) + 1e-5 * xr.grad.double().abs().max()).all()
    else:
        assert ddx.max().item() <= 1e-5 * xr.grad.double().abs().max().item()
    nc = O.rms_norm(x, torch.ones(n, dtype=x.dtype), 1e-6).double()
    terms = (dy.double() * nc).abs()
    tol = 1e-5 * terms.sum(0)
    if xd == "bf16":
        tol = tol + 4 * ulp_bf16(nc).max() * dy.double().abs().max()
    if wd == "bf16":
        tol = tol + ulp_bf16(wr.grad.double())
    assert ((dw.double().cpu() - wr.grad.double()).abs() <= tol).all()


def test_rmsnorm_backward_is_reproducible(cuda):
    g = torch.Generator().manual_seed(8)
    x, dy = torch.randn(3000, 512, generator=g).to(cuda), torch.randn(3000, 512, generator=g).to(cuda)
    w = (0.5 + torch.rand(512, generator=g)).to(cuda)
    a, b = rms_norm_backward(x, w, dy), rms_norm_backward(x, w, dy)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def _unfused(m):
    m._fuse_norm = lambda x: False   # the module's RMSNorm under autograd, then pe_attention
    return m


@pytest.mark.parametrize("kind,dr", [("pope", 32), ("pope", 64), ("fpope", 32)])
def test_fused_norm_training_matches_module_autograd(cuda, kind, dr):
    """Training through the fused norm (pe_attn_fwd_normed, then pe_attn_bwd and pe_rmsnorm_bwd)
    against the module with its RMSNorm under torch autograd (the reference's expression) followed
    by the plain kernels, fp32: output, input gradient and every parameter gradient (projections,
    both norm weights, the PE parameters).  Also against the CPU oracle module's autograd."""
    import copy
    m = _module(kind, dr, seed=4)
    x = torch.randn(2, 77, 256)
    dout = torch.randn(2, 77, 256)
    runs = {}
    for name, mod in (("fused", copy.deepcopy(m).to(cuda)), ("unfused", _unfused(copy.deepcopy(m).to(cuda)))):
        xg = x.to(cuda).requires_grad_(True)
        assert mod._fuse_norm(xg) == (name == "fused")
        out = mod(xg, start_pos=9)
        out.backward(dout.to(cuda))
        runs[name] = {"out": out.detach().cpu(), "x": xg.grad.cpu()} | \
            {n: p.grad.cpu() for n, p in mod.named_parameters() if p.grad is not None}
    xc = x.clone().requires_grad_(True)
    mc = copy.deepcopy(m)
    ref = cpu_module_ref(mc, xc, dout)
    assert set(runs["fused"]) == set(runs["unfused"]) and "qr_norm.weight" in runs["fused"]
    for n in runs["fused"]:
        a, b, r = runs["fused"][n], runs["unfused"][n], ref[n]
        scale = max(1.0, r.abs().max().item())
        assert (a - b).abs().max().item() < 1e-5 * scale, (n, (a - b).abs().max().item())
        assert (a.double() - r.double()).abs().max().item() < 1e-4 * scale, (n, (a.double() - r.double()).abs().max())


def cpu_module_ref(m, x, dout):
    from tests.test_gpu_modules import cpu_fpope_module
    out = cpu_fpope_module(m, x, start_pos=9)
    out.backward(dout)
    return {"out": out.detach(), "x": x.grad} | {n: p.grad for n, p in m.named_parameters() if p.grad is not None}


def test_fused_norm_training_bf16_autocast(cuda):
    """The module in bf16 autocast (the reference trainer's setting): the fused-norm training step
    and the module-autograd one give gradients within the bf16 bar of each other."""
    import copy
    m = _module("pope", 32, seed=6)
    x = torch.randn(2, 300, 256)
    dout = torch.randn(2, 300, 256)
    res = []
    for mod in (copy.deepcopy(m).to(cuda), _unfused(copy.deepcopy(m).to(cuda))):
        xg = x.to(cuda).requires_grad_(True)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            out = mod(xg, start_pos=0)
        out.float().backward(dout.to(cuda))
        res.append({"out": out.float().cpu(), "x": xg.grad.cpu()} |
                   {n: p.grad.float().cpu() for n, p in mod.named_parameters() if p.grad is not None})
    for n in res[0]:
        scale = max(1.0, res[1][n].abs().max().item())
        assert (res[0][n] - res[1][n]).abs().max().item() < 2e-2 * scale, n


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
