"""The drop-in modules on the GPU against a CPU re-computation of the reference module with the
same weights (projections and RMSNorm as torch CPU ops, the attention span through the oracle).

fp32 module outputs and parameter gradients are held to 1e-4 (the projections add fp32 GEMM
rounding of their own around the 1e-5 attention core); bf16 autocast runs are checked against the
fp32 result at 5e-2.
"""

import math

import pytest
import torch

from oracle import pe_oracle as O
from pe_ablations_amd.attention import GroupedQueryAttention
from pe_ablations_amd.fpope import FoPEPoPEEmbedding
from pe_ablations_amd.fpope_attention import FPoPEGroupedQueryAttention, FPoPEGroupedQueryAttentionWithCache
from pe_ablations_amd.kernels import fpope_attention_forward, hip_fpope_attention
from pe_ablations_amd.pope import PoPEEmbedding
from pe_ablations_amd.rope import NTKAwareRotaryEmbedding, RotaryEmbedding, YaRNRotaryEmbedding
from pe_ablations_amd.transform import pe_transform

pytestmark = pytest.mark.gpu


def md(a, b):
    return (a.detach().double().cpu() - b.detach().double().cpu()).abs().max().item()


def cpu_fpope_module(m, x, start_pos=0):
    """src/model/fpope_attention.py:109-181 on the CPU: torch projections + oracle attention."""
    B, S, _ = x.shape
    q_c = (x @ m.wq_c.weight.T).view(B, S, m.num_heads, m.d_content).transpose(1, 2)
    k_c = (x @ m.wk_c.weight.T).view(B, S, m.num_kv_heads, m.d_content).transpose(1, 2)
    q_r, k_r = x @ m.wq_r.weight.T, x @ m.wk_r.weight.T
    if m.qr_norm is not None:
        q_r = O.rms_norm(q_r, m.qr_norm.weight)
        k_r = O.rms_norm(k_r, m.kr_norm.weight)
    q_r = q_r.view(B, S, m.num_heads, m.d_rope).transpose(1, 2)
    k_r = k_r.view(B, S, m.num_kv_heads, m.d_rope).transpose(1, 2)
    v = (x @ m.wv.weight.T).view(B, S, m.num_kv_heads, m.head_dim).transpose(1, 2)
    pe = m.fpope
    if isinstance(pe, FoPEPoPEEmbedding):
        freqs = O.fope_effective_freqs(pe.base_freqs, pe.fourier_coeffs, pe.fourier_indices,
                                       training_length=pe.training_length, normalize=pe.normalize_coeffs,
                                       use_ceiling=pe.use_ceiling)
    else:
        freqs = pe.effective_freqs
    qt = torch.cat([q_c, O.pope_transform(q_r, freqs, start_pos)], -1)
    kt = torch.cat([k_c, O.pope_transform(k_r, freqs, start_pos, O.clamp_delta(pe.phase_bias))], -1)
    out, _ = O.attention(qt, kt, v, m.scale, causal=True)
    return out.float().transpose(1, 2).reshape(B, S, -1) @ m.wo.weight.T


def clone_to(m, dev):
    import copy
    c = copy.deepcopy(m)
    return c.to(dev)


@pytest.mark.parametrize("kind", ["pope", "pope_floor", "fpope"])
def test_fpope_module_fp32(cuda, kind):
    torch.manual_seed(0)
    if kind == "fpope":
        pe = FoPEPoPEEmbedding(32, 512, num_fourier_terms=8, delta_init="uniform")
    else:
        pe = PoPEEmbedding(32, 512, use_floor=(kind == "pope_floor"), delta_init="uniform")
    m = FPoPEGroupedQueryAttention(256, 8, 4, 64, 32, fpope=pe)
    g = clone_to(m, cuda)
    x = torch.randn(2, 96, 256)
    ref = cpu_fpope_module(m, x, start_pos=5)
    ref.sum().backward()
    out = g(x.to(cuda), start_pos=5)
    out.sum().backward()
    torch.cuda.synchronize()
    assert md(out, ref) < 1e-4
    for (n1, p1), (n2, p2) in zip(m.named_parameters(), g.named_parameters()):
        if p1.grad is not None:
            scale = max(1.0, p1.grad.abs().max().item())
            assert md(p2.grad, p1.grad) / scale < 1e-4, n1


def test_fpope_module_bf16_autocast_close_to_fp32(cuda):
    torch.manual_seed(1)
    pe = PoPEEmbedding(32, 2048, delta_init="uniform")
    m = FPoPEGroupedQueryAttention(512, 8, 4, 64, 32, fpope=pe).to(cuda)
    x = torch.randn(2, 512, 512, device=cuda)
    ref = m(x)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        out = m(x)
    assert out.dtype == torch.bfloat16
    assert md(out, ref) < 5e-2


def test_kv_cache_decode_equals_full_forward(cuda):
    """Prefill 40 tokens, decode 3 one at a time: each step equals the matching rows of the
    no-cache forward over the whole sequence (bottom-right mask, absolute key positions)."""
    torch.manual_seed(2)
    pe = PoPEEmbedding(32, 512, delta_init="uniform")
    m = FPoPEGroupedQueryAttentionWithCache(256, 4, 2, 64, 32, fpope=pe, max_cache_len=128).to(cuda)
    x = torch.randn(1, 43, 256, device=cuda)
    with torch.no_grad():
        full = m(x)
        outs = [m(x[:, :40], use_cache=True)]
        for t in range(40, 43):
            outs.append(m(x[:, t:t + 1], start_pos=t, use_cache=True))
    inc = torch.cat(outs, 1)
    assert m.cache_len == 43
    # the cache holds the transformed key rows [k_c | mu cos | mu sin] (width 64 + 2 * 32)
    assert tuple(m.k_cache.shape) == (1, 2, 128, 128) and tuple(m.v_cache.shape) == (1, 2, 128, 64)
    assert md(inc, full) < 1e-5
    m.reset_cache()
    assert m.k_cache is None and m.v_cache is None and m.cache_len == 0


@pytest.mark.parametrize("rope_kind", ["standard", "ntk", "yarn", "nope"])
def test_gqa_rope_module_fp32(cuda, rope_kind):
    torch.manual_seed(3)
    D = 64
    rope = {"standard": lambda: RotaryEmbedding(D, 512), "ntk": lambda: NTKAwareRotaryEmbedding(D, 512, scale=4.0),
            "yarn": lambda: YaRNRotaryEmbedding(D, 512, scale=4.0), "nope": lambda: None}[rope_kind]()
    m = GroupedQueryAttention(256, 4, 2, D, use_qk_norm=True, rope=rope)
    g = clone_to(m, cuda)
    x = torch.randn(2, 80, 256)
    B, S = 2, 80
    q = (x @ m.wq.weight.T).view(B, S, 4, D).transpose(1, 2)
    k = (x @ m.wk.weight.T).view(B, S, 2, D).transpose(1, 2)
    v = (x @ m.wv.weight.T).view(B, S, 2, D).transpose(1, 2)
    if rope is not None:
        ms = rope.kernel_mscale()
        q, k = O.rope_rotate(q, rope.inv_freq, 0) * ms, O.rope_rotate(k, rope.inv_freq, 0) * ms
    q, k = O.qk_l2norm(q), O.qk_l2norm(k)
    o, _ = O.attention(q, k, v, 1 / math.sqrt(D))
    ref = o.float().transpose(1, 2).reshape(B, S, -1) @ m.wo.weight.T
    ref.sum().backward()
    out = g(x.to(cuda))
    out.sum().backward()
    torch.cuda.synchronize()
    assert md(out, ref) < 1e-4
    for (n1, p1), (_, p2) in zip(m.named_parameters(), g.named_parameters()):
        assert md(p2.grad, p1.grad) / max(1.0, p1.grad.abs().max().item()) < 1e-4, n1


def test_standalone_transforms_and_gradients(cuda):
    """forward_query / forward_key (src/model/pope.py:124-183) through the HIP transform, and their
    backward, against the oracle transform and its autograd (fp32)."""
    torch.manual_seed(4)
    pe = FoPEPoPEEmbedding(48, 256, num_fourier_terms=4, delta_init="uniform")
    x = torch.randn(2, 30, 3, 48)
    for is_key in (False, True):
        pg = clone_to(pe, cuda)
        xo = x.clone().requires_grad_(True)
        freqs = O.fope_effective_freqs(pe.base_freqs, pe.fourier_coeffs, pe.fourier_indices)
        delta = O.clamp_delta(pe.phase_bias) if is_key else None
        ref = O.pope_transform(xo.transpose(1, 2), freqs, 7, delta).transpose(1, 2)
        gout = torch.randn_like(ref)
        ref.backward(gout)
        xg = x.to(cuda).requires_grad_(True)
        out = pg.forward_key(xg, 7) if is_key else pg.forward_query(xg, 7)
        out.backward(gout.to(cuda))
        torch.cuda.synchronize()
        assert out.shape == (2, 30, 3, 96)
        # fp32 bar (1e-5): omega itself is a torch reduction on each device, and one ulp of omega
        # moves the phase at position 36 by ~2e-6 rad
        assert md(out, ref) < 1e-5
        assert md(xg.grad, xo.grad) < 1e-5
        assert md(pg.fourier_coeffs.grad, pe.fourier_coeffs.grad) / max(1.0, pe.fourier_coeffs.grad.abs().max().item()) < 1e-4
        if is_key:
            assert md(pg.phase_bias.grad, pe.phase_bias.grad) / max(1.0, pe.phase_bias.grad.abs().max().item()) < 1e-4
        pe.zero_grad()


def test_rope_module_forward_rotates(cuda):
    rope = YaRNRotaryEmbedding(64, 128, scale=2.0)
    xq, xk = torch.randn(2, 10, 4, 64), torch.randn(2, 10, 2, 64)
    rq, rk = clone_to(rope, cuda)(xq.to(cuda), xk.to(cuda), 3)
    ms = float(rope.mscale)
    eq = O.rope_rotate(xq.transpose(1, 2), rope.inv_freq, 3).transpose(1, 2) * ms
    ek = O.rope_rotate(xk.transpose(1, 2), rope.inv_freq, 3).transpose(1, 2) * ms
    assert md(rq, eq) < 2e-6 and md(rk, ek) < 2e-6


@pytest.mark.parametrize("dim", [64, 96, 128])
def test_legacy_fused_api(cuda, dim):
    """fpope_attention_forward (tests/test_fpope.py:222-226): difference-form semantics, no clamp,
    random freqs / bias, fp32; forward 1e-3 and backward 1e-2 as the reference's own kernel tests
    (tests/test_fpope.py:249,356-360).  The factorised kernel rounds the absolute phases t*w, the
    difference form rounds (s - t)*w, so the two differ by phase rounding, not by formula."""
    torch.manual_seed(5)
    B, H, S = 2, 4, 64
    q, k, v = torch.randn(B, H, S, dim), torch.randn(B, H, S, dim), torch.randn(B, H, S, dim)
    freqs, bias = torch.randn(dim), torch.randn(dim)
    qo, ko, vo, fo, bo = (t.clone().requires_grad_(True) for t in (q, k, v, freqs, bias))
    ref, ref_lse = O.pope_attention_diff_form(qo, ko, vo, fo, bo)
    ref.sum().backward()
    qg, kg, vg, fg, bg = (t.to(cuda).requires_grad_(True) for t in (q, k, v, freqs, bias))
    out = fpope_attention_forward(qg, kg, vg, fg, bg, causal=True, use_triton=False)
    out.sum().backward()
    torch.cuda.synchronize()
    assert md(out, ref) < 1e-3
    for a, b in ((qg, qo), (kg, ko), (vg, vo)):
        assert md(a.grad, b.grad) < 1e-2
    for a, b in ((fg, fo), (bg, bo)):
        assert md(a.grad, b.grad) / max(1.0, b.grad.abs().max().item()) < 1e-2
    out2, lse = hip_fpope_attention(qg.detach(), kg.detach(), vg.detach(), fg.detach(), bg.detach(), return_lse=True)
    assert lse.shape == (B * H, S)
    assert md(lse, ref_lse.reshape(B * H, S)) < 1e-3
    assert torch.equal(out2, out.detach())


@pytest.mark.parametrize("start_pos", [0, 16000, 131040, 1_000_000])
def test_transform_phase_range(cuda, start_pos):
    """Phases fl(t * w) from 0 up to ~1e6 rad: the device sin/cos (Cody-Waite below 2^17 rad, the
    library routine above; start 131040 straddles the switch) against torch's float32 sin/cos in
    the oracle transform, forward and backward, PoPE keys with phase bias and RoPE."""
    torch.manual_seed(6)
    D = 128
    x = torch.randn(1, 64, 2, D)
    freqs = O.pope_freqs(D)
    delta = O.clamp_delta(torch.rand(2, D) * -7.0)
    xo = x.clone().requires_grad_(True)
    ref = O.pope_transform(xo.transpose(1, 2), freqs, start_pos, delta).transpose(1, 2)
    gout = torch.randn_like(ref)
    ref.backward(gout)
    xg = x.to(cuda).requires_grad_(True)
    out = pe_transform(xg, freqs.to(cuda), delta.to(cuda), start_pos=start_pos, is_key=True)
    out.backward(gout.to(cuda))
    torch.cuda.synchronize()
    assert md(out, ref) < 1e-5
    assert md(xg.grad, xo.grad) < 1e-5
    inv = O.rope_inv_freq(D)
    rr = O.rope_rotate(x.transpose(1, 2), inv, start_pos).transpose(1, 2)
    rg = pe_transform(x.to(cuda), inv.to(cuda), None, start_pos=start_pos, mode="rope")
    assert md(rg, rr) < 1e-5


# ------------------------------------------------------------- FoPE positions in the input dtype

def _fope(dim, max_len, seed):
    torch.manual_seed(seed)
    return FoPEPoPEEmbedding(dim, max_len, num_fourier_terms=4, fourier_sigma=0.4, delta_init="uniform")


def _omega(pe):
    return O.fope_effective_freqs(pe.base_freqs, pe.fourier_coeffs, pe.fourier_indices,
                                  training_length=pe.training_length, normalize=pe.normalize_coeffs,
                                  use_ceiling=pe.use_ceiling)


def test_fope_embedding_bf16_input_rounds_positions(cuda):
    """forward_query / forward_key on a bf16 x take positions in bf16, as the reference's
    torch.arange(..., dtype=x.dtype) (src/model/fpope.py:285,322): against the oracle transform
    with bf16 positions (forward and input gradient at the bf16 bar, coefficient gradient relative),
    and far from the exact-position transform.  PoPEEmbedding keeps exact positions."""
    pe = _fope(48, 1024, seed=50)
    x = torch.randn(2, 200, 3, 48).to(torch.bfloat16)
    for is_key in (False, True):
        pg = clone_to(pe, cuda)
        xo = x.float().requires_grad_(True)
        delta = O.clamp_delta(pe.phase_bias) if is_key else None
        ref = O.pope_transform(xo.transpose(1, 2), _omega(pe), 400, delta, pos_dtype=torch.bfloat16).transpose(1, 2)
        gout = torch.randn_like(ref)
        ref.backward(gout)
        xg = x.to(cuda).requires_grad_(True)
        out = pg.forward_key(xg, 400) if is_key else pg.forward_query(xg, 400)
        out.backward(gout.to(cuda).to(out.dtype))
        torch.cuda.synchronize()
        assert md(out, ref) < 2e-2
        assert md(xg.grad, xo.grad) / max(1.0, xo.grad.abs().max().item()) < 1e-2
        assert md(pg.fourier_coeffs.grad, pe.fourier_coeffs.grad) / max(1.0, pe.fourier_coeffs.grad.abs().max().item()) < 2e-2
        exact = O.pope_transform(x.float().transpose(1, 2), _omega(pe).detach(), 400,
                                 None if delta is None else delta.detach()).transpose(1, 2)
        assert md(out, exact) > 0.5
        pe.zero_grad()
    pp = PoPEEmbedding(48, 1024, delta_init="uniform").to(cuda)
    out = pp.forward_query(x.to(cuda), 400)
    assert md(out, O.pope_transform(x.float().transpose(1, 2), pp.effective_freqs.cpu(), 400).transpose(1, 2)) < 2e-2


@pytest.mark.parametrize("qk_norm", [False, True])
def test_fpope_module_autocast_position_dtype(cuda, qk_norm):
    """The FoPE module under bf16 autocast: without QK norm the position projections are bf16, so
    the reference's positions are bf16 (rounded past 256); with the norm its fp32 weight makes them
    fp32 and the positions stay exact.  The module's attention (before wo) against the oracle built
    each way, on the projections the module itself computed."""
    pe = _fope(32, 1024, seed=51)
    m = FPoPEGroupedQueryAttention(256, 8, 4, 64, 32, use_qk_norm=qk_norm, fpope=pe).to(cuda)
    # without the norm, larger inputs sharpen attention so that the positions visibly matter
    x = torch.randn(1, 640, 256, device=cuda) * (1 if qk_norm else 3)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        q_c, k_c, q_r, k_r, v = m._project(x)
        out = m._attend(q_c, k_c, q_r, k_r, v, 0, 0, True)
    assert q_r.dtype == (torch.float32 if qk_norm else torch.bfloat16)
    pos_dt = None if qk_norm else torch.bfloat16
    import copy
    pc = copy.deepcopy(m.fpope).cpu()
    omega, delta = _omega(pc).detach(), O.clamp_delta(pc.phase_bias).detach()
    c = [t.float().cpu() for t in (q_c, k_c, q_r, k_r, v)]

    def oracle(pd):
        tq = torch.cat([c[0], O.pope_transform(c[2], omega, 0, pos_dtype=pd)], -1).to(torch.bfloat16).float()
        tk = torch.cat([c[1], O.pope_transform(c[3], omega, 0, delta, pos_dtype=pd)], -1).to(torch.bfloat16).float()
        return O.attention(tq, tk, c[4].to(torch.bfloat16).float(), m.scale, causal=True)[0]

    e = md(out, oracle(pos_dt))
    assert e < 2e-2
    if not qk_norm:   # the kernel is far closer to the rounded positions than to exact ones
        assert md(out, oracle(None)) > max(4 * e, 0.02), (e, md(out, oracle(None)))


def test_fope_cache_decode_bf16_positions(cuda):
    """KV-cache decode with the FoPE module under bf16 autocast and no QK norm: keys appended and
    queries decoded at bf16-rounded positions agree with the full forward's last rows."""
    pe = _fope(32, 1024, seed=52)
    m = FPoPEGroupedQueryAttentionWithCache(256, 4, 2, 64, 32, use_qk_norm=False, fpope=pe,
                                            max_cache_len=640).to(cuda)
    x = torch.randn(1, 603, 256, device=cuda)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        full = m(x)
        outs = [m(x[:, :600], use_cache=True)]
        for t in range(600, 603):
            outs.append(m(x[:, t:t + 1], start_pos=t, use_cache=True))
    assert md(torch.cat(outs, 1), full) < 2e-2
