"""The KV-cache path with gradients (FPoPEGroupedQueryAttentionWithCache.forward and
GroupedQueryAttention.forward with use_cache=True under autograd).

The reference writes each chunk's transformed keys and values into its cache buffers by slice
assignment and runs SDPA over cache[:, :, :start_pos + S] with the bottom-right mask
(src/model/fpope_attention.py:283-324).  The buffer then carries the chunks' autograd history, so
the gradient of a later chunk's output reaches the earlier chunks' inputs through their cached keys
and values.  The chunked outputs are the rows of the no-cache causal forward over the whole
sequence, so the gradients of a loss over the chunks' outputs must equal those of the same loss over
the full forward's rows: x, every projection weight, the PoPE phase bias and FoPE's Fourier
coefficients, in fp32 to 2e-5 of each
gradient's scale (the two sides run different kernels: the fused PoPE forward and backward, against
the stand-alone transform and the no-PE kernels on transformed operands).  A rewind (a chunk at a
start_pos inside the cached rows) must equal the full forward over the kept prefix and the new
chunk.
"""

import pytest
import torch

from pe_ablations_amd.attention import GroupedQueryAttention
from pe_ablations_amd.fpope import FoPEPoPEEmbedding
from pe_ablations_amd.fpope_attention import FPoPEGroupedQueryAttentionWithCache
from pe_ablations_amd.pope import PoPEEmbedding
from pe_ablations_amd.rope import RotaryEmbedding
from tests._cmp import err

pytestmark = pytest.mark.gpu


def rel(a, b):
    return err(a, b) / max(1.0, b.abs().max().item())


def fpope_module(cuda, fope=False):
    torch.manual_seed(11)
    if fope:  # Fourier frequencies: their coefficients get gradients through the transform's d(omega)
        pe = FoPEPoPEEmbedding(32, 512, num_fourier_terms=4, fourier_sigma=0.4, delta_init="uniform")
    else:
        pe = PoPEEmbedding(32, 512, delta_init="uniform")
    return FPoPEGroupedQueryAttentionWithCache(256, 4, 2, 64, 32, fpope=pe, max_cache_len=128).to(cuda)


def chunked(m, x, chunks):
    m.reset_cache()
    return torch.cat([m(x[:, a:b], start_pos=a, use_cache=True) for a, b in chunks], 1)


@pytest.mark.parametrize("which", ["fpope", "fope", "rope", "nope"])
def test_cached_chunk_gradients_equal_full_forward(cuda, which):
    print(f"cache grad {which}", flush=True)
    if which in ("fpope", "fope"):
        m = fpope_module(cuda, fope=which == "fope")
    else:
        torch.manual_seed(12)
        m = GroupedQueryAttention(256, 4, 2, 64, use_qk_norm=True,
                                  rope=RotaryEmbedding(64, 256) if which == "rope" else None).to(cuda)
    params = [p for p in m.parameters() if p.requires_grad]
    x = torch.randn(2, 64, 256, device=cuda)
    d = torch.randn(2, 64, 256, device=cuda)
    xf = x.clone().requires_grad_(True)
    full = m(xf)
    gf = torch.autograd.grad((full * d).sum(), [xf] + params)
    xc = x.clone().requires_grad_(True)
    out = chunked(m, xc, [(0, 40), (40, 63), (63, 64)])
    assert m.cache.length == 64
    assert rel(out, full) < 2e-5
    gc = torch.autograd.grad((out * d).sum(), [xc] + params)
    for i, (a, b) in enumerate(zip(gc, gf)):
        assert rel(a, b) < 2e-5, (which, i, rel(a, b))


def test_cached_rewind_gradients(cuda):
    """Prefill 40 rows with gradients, then a chunk of 10 at start_pos 30: its output and the
    gradients of a loss over it equal the full forward over x[:, :30] followed by the new chunk; the
    overwritten rows' inputs x[:, 30:40] get no gradient."""
    m = fpope_module(cuda)
    params = [p for p in m.parameters() if p.requires_grad]
    x1 = torch.randn(1, 40, 256, device=cuda, requires_grad=True)
    x2 = torch.randn(1, 10, 256, device=cuda, requires_grad=True)
    d = torch.randn(1, 10, 256, device=cuda)
    m.reset_cache()
    m(x1, start_pos=0, use_cache=True)
    o2 = m(x2, start_pos=30, use_cache=True)
    assert m.cache.length == 40
    g = torch.autograd.grad((o2 * d).sum(), [x1, x2] + params)
    xf = torch.cat([x1.detach()[:, :30], x2.detach()], 1).requires_grad_(True)
    full = m(xf)
    gf = torch.autograd.grad((full[:, 30:] * d).sum(), [xf] + params)
    assert rel(o2, full[:, 30:]) < 2e-5
    assert rel(g[0][:, :30], gf[0][:, :30]) < 2e-5 and (g[0][:, 30:] == 0).all()
    assert rel(g[1], gf[0][:, 30:]) < 2e-5
    for i, (a, b) in enumerate(zip(g[2:], gf[1:])):
        assert rel(a, b) < 2e-5, (i, rel(a, b))


def test_decode_after_a_prefill_with_gradients(cuda):
    """A prefill run with gradients fills the cache buffers too: the next token, decoded without
    gradients by the split-key decode kernel, equals the full forward's row."""
    m = fpope_module(cuda)
    x = torch.randn(1, 41, 256, device=cuda)
    m.reset_cache()
    m(x[:, :40].clone().requires_grad_(True), start_pos=0, use_cache=True)
    assert m.cache.hist is not None
    with torch.no_grad():
        step = m(x[:, 40:], start_pos=40, use_cache=True)
        full = m(x)
    assert m.cache.hist is None
    assert rel(step, full[:, 40:]) < 1e-5


def test_cached_gradients_under_bf16_autocast(cuda):
    """The same chunked loss under bf16 autocast: finite gradients within the bf16 scale of the
    full forward's (both compute in bf16, through different kernels)."""
    m = fpope_module(cuda)
    params = [p for p in m.parameters() if p.requires_grad]
    x = torch.randn(2, 64, 256, device=cuda)
    d = torch.randn(2, 64, 256, device=cuda)
    res = []
    for use_cache in (False, True):
        xg = x.clone().requires_grad_(True)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            out = chunked(m, xg, [(0, 40), (40, 64)]) if use_cache else m(xg)
        res.append(torch.autograd.grad((out.float() * d).sum(), [xg] + params))
    for i, (a, b) in enumerate(zip(*res)):
        assert torch.isfinite(a).all() and rel(a, b) < 5e-2, (i, rel(a, b))
