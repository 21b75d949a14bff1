"""Pins of the CPU oracle (oracle/pe_oracle.py) against checks that do not restate its formulas.

Each oracle function is held against something independent of its own code path: pure-Python
brute force, torch's SDPA in a special case the PoPE math reduces to, the reference's other
(difference-form) formulation, fp64 autograd and finite differences, closed forms the reference
fixes (frequency tables, YaRN bounds, floor-clip counts) and the known answers the reference's
tests assert (tests/test_fpope.py).  A plausible slip in the oracle (dropped delta, a sign in the
phase, transposed q/k, missing scale, wrong GQA mapping, rotate-half instead of interleaved pairs)
fails at least one of these.
"""

import math

import pytest
import torch
import torch.nn.functional as F

from oracle import pe_oracle as O

f64 = torch.float64


def rnd(*shape, seed=0, scale=1.0, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g, dtype=f64) * scale).to(dtype)


# ---------------------------------------------------------------------------------------------
# attention core
# ---------------------------------------------------------------------------------------------

@pytest.mark.parametrize("causal", [True, False])
def test_factorised_matches_brute_force(causal):
    """pope_attention (factorised [mu cos, mu sin] GEMM form) == triple Python loop over the
    difference form sum_c mu_q mu_k cos((s-t) theta_c + delta_c)."""
    S, D = 7, 6
    q, k, v = rnd(1, 1, S, D, seed=1), rnd(1, 1, S, D, seed=2), rnd(1, 1, S, D, seed=3)
    freqs = O.pope_freqs(D, 10.0)
    delta = -torch.rand(D, generator=torch.Generator().manual_seed(4)) * 2 * math.pi
    out, _ = O.pope_attention(q, k, v, freqs, delta, scale=0.3, causal=causal, clamp=False,
                              transform_dtype=f64)
    bf = torch.tensor(O.brute_force_pope(q[0, 0], k[0, 0], v[0, 0], freqs, delta, 0.3, causal), dtype=f64)
    assert (out[0, 0] - bf).abs().max().item() < 1e-12


def test_zero_freq_zero_delta_is_plain_sdpa():
    """theta = 0, delta = 0: q~.k~ = mu_q . mu_k, so PoPE attention is SDPA on softplus inputs."""
    B, H, S, D = 2, 3, 33, 16
    q, k, v = rnd(B, H, S, D, seed=5), rnd(B, H, S, D, seed=6), rnd(B, H, S, D, seed=7)
    out, _ = O.pope_attention(q, k, v, torch.zeros(D), torch.zeros(D), scale=0.25, clamp=False,
                              transform_dtype=f64)
    ref = F.scaled_dot_product_attention(F.softplus(q.double()), F.softplus(k.double()), v.double(),
                                         is_causal=True, scale=0.25)
    assert (out - ref).abs().max().item() < 1e-12


def test_attention_core_gqa_and_lse():
    """GQA maps query head h to kv head h // (Hq/Hkv) (repeat_interleave); lse = logsumexp."""
    q, k, v = rnd(1, 4, 9, 8, seed=8), rnd(1, 2, 9, 8, seed=9), rnd(1, 2, 9, 5, seed=10)
    out, lse = O.attention(q, k, v, 0.5, causal=True)
    for h in range(4):
        o1, l1 = O.attention(q[:, h:h + 1], k[:, h // 2:h // 2 + 1], v[:, h // 2:h // 2 + 1], 0.5)
        assert torch.allclose(out[:, h:h + 1], o1, atol=1e-13)
        assert torch.allclose(lse[:, h:h + 1], l1, atol=1e-13)
    s = torch.matmul(q.double(), k.double().repeat_interleave(2, 1).transpose(-1, -2)) * 0.5
    s = s.masked_fill(torch.triu(torch.ones(9, 9, dtype=torch.bool), 1), float("-inf"))
    assert torch.allclose(lse, torch.logsumexp(s, -1), atol=1e-12)


def test_bottom_right_mask_matches_reference_cache_mask():
    """Sq < Sk: mask = triu(ones(Sq, Sk), Sk - Sq + 1) as the cache path builds it
    (src/model/fpope_attention.py:313-317); the last query sees every key."""
    m = O.causal_mask(3, 7)
    assert m.tolist() == [[False] * 5 + [True] * 2, [False] * 6 + [True], [False] * 7]
    assert torch.equal(O.causal_mask(5, 5), torch.triu(torch.ones(5, 5, dtype=torch.bool), 1))


# ---------------------------------------------------------------------------------------------
# PoPE transform and known answers (tests/test_fpope.py)
# ---------------------------------------------------------------------------------------------

def test_factorised_equals_difference_form():
    """Factorised transform (what the module computes) == the eager difference form
    (src/model/fpope.py:341-418, tests/test_fpope.py:1539-1560), evaluated in fp64."""
    q, k, v = rnd(2, 3, 20, 8, seed=11), rnd(2, 3, 20, 8, seed=12), rnd(2, 3, 20, 8, seed=13)
    freqs = rnd(8, seed=14)            # arbitrary signs and sizes, like the legacy tests
    bias = rnd(8, seed=15)
    a, la = O.pope_attention(q, k, v, freqs, bias, clamp=False, transform_dtype=f64)
    b, lb = O.pope_attention_diff_form(q, k, v, freqs, bias)
    assert (a - b).abs().max().item() < 1e-10
    assert (la - lb).abs().max().item() < 1e-10


def test_fp32_transform_rounding_is_the_reference_order():
    """The fp32 phase is fl(fl(pos*theta) + delta): exactly torch.outer followed by an add, not a
    fused multiply-add (src/model/pope.py:88-90,175-176)."""
    freqs = O.pope_freqs(64)
    delta = -torch.rand(64, generator=torch.Generator().manual_seed(16)) * 2 * math.pi
    ph = O.pope_phases(4096, freqs, 0, delta)
    ref = torch.outer(torch.arange(4096, dtype=torch.float32), freqs) + delta
    assert torch.equal(ph, ref)
    fused = (torch.arange(4096, dtype=f64).unsqueeze(1) * freqs.double() + delta.double()).float()
    assert not torch.equal(ph, fused)  # the single-rounding form differs somewhere


def test_diagonal_phase_is_delta():
    """Query t and key s = t: phase difference is delta alone (tests/test_fpope.py:111-125)."""
    freqs = O.pope_freqs(16)
    delta = -torch.rand(16, generator=torch.Generator().manual_seed(17)) * 2 * math.pi
    phq = O.pope_phases(50, freqs, 0, dtype=f64)
    phk = O.pope_phases(50, freqs, 0, delta, dtype=f64)
    assert torch.allclose(phk - phq, delta.double().expand(50, 16), atol=1e-12)


def test_transform_shape_and_magnitude():
    """[mu cos, mu sin] halves: row norm per dim pair is softplus(x) > 0 (tests/test_fpope.py:98-109)."""
    x = rnd(2, 3, 10, 8, seed=18, scale=5.0)
    t = O.pope_transform(x, O.pope_freqs(8), 3, -torch.ones(3, 8))
    assert t.shape == (2, 3, 10, 16)
    mag = torch.sqrt(t[..., :8] ** 2 + t[..., 8:] ** 2)
    assert torch.allclose(mag, F.softplus(x), atol=1e-5)
    assert (F.softplus(x) > 0).all()


def test_softplus_threshold_20():
    x = torch.tensor([19.0, 20.0, 20.5, 30.0, -30.0])
    t = O.pope_transform(x.view(1, 1, 1, 5), torch.zeros(5))
    assert torch.equal(t[0, 0, 0, :5], torch.tensor([math.log1p(math.exp(19.0)), math.log1p(math.exp(20.0)),
                                                     20.5, 30.0, math.log1p(math.exp(-30.0))], dtype=torch.float32))


def test_known_answers():
    B, H, S, D = 2, 2, 12, 8
    q, k = rnd(B, H, S, D, seed=19), rnd(B, H, S, D, seed=20)
    freqs, delta = O.pope_freqs(D), -torch.rand(D) * 2 * math.pi
    # V = 0 -> O = 0 (tests/test_fpope.py:1033-1045)
    out, _ = O.pope_attention(q, k, torch.zeros(B, H, S, D), freqs, delta)
    assert out.abs().max().item() == 0.0
    # S = 1 -> O = V (single visible key)
    v1 = rnd(1, 1, 1, D, seed=21)
    o1, _ = O.pope_attention(q[:1, :1, :1], k[:1, :1, :1], v1, freqs, delta)
    assert torch.allclose(o1, v1.double(), atol=1e-15)
    # causal: the first query only sees key 0 -> O[0] = V[0]
    v = rnd(B, H, S, D, seed=22)
    o, _ = O.pope_attention(q, k, v, freqs, delta)
    assert torch.allclose(o[:, :, 0], v[:, :, 0].double(), atol=1e-15)


def test_start_pos_shift_invariance():
    """Equal-length q/k shifted together: scores depend on s - t only (up to fp rounding of the
    absolute phase), tests/test_fpope.py:563-594."""
    q, k, v = rnd(1, 2, 16, 8, seed=23), rnd(1, 2, 16, 8, seed=24), rnd(1, 2, 16, 8, seed=25)
    freqs, delta = O.pope_freqs(8), -torch.rand(8) * 2
    a, _ = O.pope_attention(q, k, v, freqs, delta, transform_dtype=f64)
    b, _ = O.pope_attention(q, k, v, freqs, delta, start_q=37, start_k=37, transform_dtype=f64)
    assert (a - b).abs().max().item() < 1e-10


def test_delta_clamp_keys_only():
    """clamp(delta, -2pi, 0) on keys (src/model/pope.py:172); queries carry no delta."""
    d = torch.tensor([-10.0, -1.0, 0.5, 3.0])
    assert torch.equal(O.clamp_delta(d), torch.tensor([-2 * math.pi, -1.0, 0.0, 0.0]))
    q, k, v = rnd(1, 1, 6, 4, seed=26), rnd(1, 1, 6, 4, seed=27), rnd(1, 1, 6, 4, seed=28)
    fr = O.pope_freqs(4)
    a, _ = O.pope_attention(q, k, v, fr, d, clamp=True)
    b, _ = O.pope_attention(q, k, v, fr, O.clamp_delta(d), clamp=False)
    assert torch.equal(a, b)


def test_extreme_inputs_finite():
    """x10, x1e-6, zeros, uniform, freqs x100, negative freqs: no NaN/Inf (tests/test_fpope.py:980-1097)."""
    base = rnd(1, 2, 16, 8, seed=29)
    fr = O.pope_freqs(8)
    for q, k, f in [(base * 10, base * 10, fr), (base * 1e-6, base * 1e-6, fr),
                    (torch.zeros_like(base), torch.zeros_like(base), fr),
                    (torch.ones_like(base), torch.ones_like(base), fr),
                    (base, base, fr * 100), (base, base, -fr)]:
        out, lse = O.pope_attention(q, k, base, f, -torch.ones(8))
        assert torch.isfinite(out).all() and torch.isfinite(lse).all()


# ---------------------------------------------------------------------------------------------
# backward
# ---------------------------------------------------------------------------------------------

@pytest.mark.parametrize("shape,causal", [((1, 2, 4, 8), True), ((2, 4, 8, 16), True), ((1, 2, 6, 8), False)])
def test_gradcheck_reference_shapes(shape, causal):
    """fp64 gradcheck at the reference's shapes and tolerances (tests/test_fpope.py:754-801:
    eps 1e-6, atol 1e-4, rtol 1e-3), gradients w.r.t. q, k, v, freqs and delta."""
    B, H, S, D = shape
    q, k, v = (rnd(*shape, seed=s, dtype=f64).requires_grad_(True) for s in (30, 31, 32))
    fr = (O.pope_freqs(D).double() * 0.5).requires_grad_(True)
    de = (-torch.rand(D, generator=torch.Generator().manual_seed(33), dtype=f64)).requires_grad_(True)

    def fn(q, k, v, fr, de):
        return O.pope_attention(q, k, v, fr, de, causal=causal, clamp=False, transform_dtype=f64)[0]

    assert torch.autograd.gradcheck(fn, (q, k, v, fr, de), eps=1e-6, atol=1e-4, rtol=1e-3)


@pytest.mark.parametrize("per_head", [False, True])
def test_closed_form_backward_matches_autograd(per_head):
    """The closed form the kernels implement (tests/test_fpope.py:1571-1602 extended with the
    factorised inverse transform) == fp64 autograd of the forward."""
    B, H, S, D = 2, 3, 10, 8
    q, k, v = (rnd(B, H, S, D, seed=s, dtype=f64).requires_grad_(True) for s in (34, 35, 36))
    fr = (O.pope_freqs(D).double()).requires_grad_(True)
    dshape = (H, D) if per_head else (D,)
    de = (-torch.rand(*dshape, generator=torch.Generator().manual_seed(37), dtype=f64) * 6).requires_grad_(True)
    dout = rnd(B, H, S, D, seed=38, dtype=f64)
    out, _ = O.pope_attention(q, k, v, fr, de, clamp=False, transform_dtype=f64, start_q=3, start_k=3)
    out.backward(dout)
    cf = O.pope_attention_backward_closed_form(q.detach(), k.detach(), v.detach(), fr.detach(),
                                               de.detach(), dout, start_q=3, start_k=3)
    assert (cf["out"] - out.detach()).abs().max().item() < 1e-12
    for name, g in (("dq", q.grad), ("dk", k.grad), ("dv", v.grad), ("dfreqs", fr.grad), ("ddelta", de.grad)):
        assert (cf[name] - g).abs().max().item() < 1e-10, name


# ---------------------------------------------------------------------------------------------
# frequency tables: PoPE / FoPE / RoPE / NTK / YaRN
# ---------------------------------------------------------------------------------------------

def test_pope_freq_table_and_floor_count():
    """theta_i = 10000^(-i/D) (src/model/pope.py:71); floor 2pi/L zeroes the slow dims."""
    f = O.pope_freqs(128)
    closed = torch.tensor([10000.0 ** (-(i / 128)) for i in range(128)], dtype=f64)
    assert (f.double() - closed).abs().max().item() <= 1.2e-7 * closed.abs().max().item()
    clipped = O.floor_clip(f, 2048)
    # theta_i < 2pi/2048 <=> i > 128 * ln(2048/(2pi)) / ln(10000) = 80.4: dims 81..127 clip
    assert (clipped == 0).sum().item() == 47
    assert (clipped[:81] > 0).all() and (clipped[81:] == 0).all()
    assert (O.floor_clip(O.pope_freqs(32), 512) == 0).sum().item() == sum(
        1 for i in range(32) if 10000.0 ** (-i / 32) < 2 * math.pi / 512)


def test_fope_effective_freqs():
    """omega_c = theta_c + sum_j a_hat_cj * j * theta_c, then floor clip / ceiling clamp
    (src/model/fpope.py:107-146), against an independent loop."""
    D, M = 16, 4
    base = O.pope_freqs(D)
    a = rnd(D, M, seed=39, scale=0.4)
    eff = O.fope_effective_freqs(base, a, training_length=512)
    for c in range(D):
        tot = sum(abs(float(a[c, j])) for j in range(M)) + 1e-8
        w = float(base[c]) + sum(float(a[c, j]) / tot * (j + 1) * float(base[c]) for j in range(M))
        w = 0.0 if abs(w) < 2 * math.pi / 512 else w
        assert abs(float(eff[c]) - w) <= 1e-6 * max(1.0, abs(w))
    # zero coefficients collapse to the base table
    assert torch.equal(O.fope_effective_freqs(base, torch.zeros(D, M), training_length=10 ** 9), base)
    # ceiling clamp at +-2pi
    big = O.fope_effective_freqs(base * 100, torch.zeros(D, M), training_length=512, use_ceiling=True)
    assert big.max().item() <= 2 * math.pi + 1e-6


def test_rope_rotation_forms_and_norm():
    """Interleaved pairs (x0,x1),(x2,x3) rotated by t*w_i (src/model/rope.py:28-57): the real-arith
    form == the complex-multiply form, rotation keeps the norm, and it is not rotate-half."""
    x = rnd(2, 3, 11, 16, seed=40)
    inv = O.rope_inv_freq(16)
    a = O.rope_rotate(x, inv, 5)
    b = O.rope_rotate_complex(x, inv, 5)
    assert (a - b).abs().max().item() < 1e-5
    assert torch.allclose(a.norm(dim=-1), x.norm(dim=-1), atol=1e-4)
    # position t rotates pair i by t * inv_freq[i]: check pair 1 of position 2 by hand
    t, i = 2 + 5, 1
    ang = t * float(inv[i])
    x0, x1 = float(x[0, 0, 2, 2 * i]), float(x[0, 0, 2, 2 * i + 1])
    assert abs(float(a[0, 0, 2, 2 * i]) - (x0 * math.cos(ang) - x1 * math.sin(ang))) < 1e-5
    assert abs(float(a[0, 0, 2, 2 * i + 1]) - (x0 * math.sin(ang) + x1 * math.cos(ang))) < 1e-5


def test_ntk_and_yarn_tables():
    """NTK theta' = theta * s^(D/(D-2)) (src/model/rope.py:139); YaRN bounds without the /2:
    D=64 -> (6, 31), D=128 -> (12, 62); ramp endpoints; mscale = 0.1 ln s + 1 (src/model/rope.py:170-207)."""
    assert abs(O.ntk_theta(64, 10000.0, 4.0) - 10000.0 * 4.0 ** (64 / 62)) < 1e-6
    for D, lo, hi in ((64, 6, 31), (128, 12, 62)):
        inv, ms, low, high = O.yarn_inv_freq(D, 10000.0, 8.0)
        assert (low, high) == (lo, hi)
        ext = O.rope_inv_freq(D)
        assert torch.allclose(inv[:low], ext[:low])
        assert abs(float(inv[low]) - float(ext[low])) < 1e-12            # smooth = 0
        if high < D // 2:
            assert abs(float(inv[high]) - float(ext[high]) / 8.0) < 1e-9  # smooth = 1
        assert abs(ms - (0.1 * math.log(8.0) + 1.0)) < 1e-12


def test_qknorm_and_rmsnorm():
    """QKNorm x/(||x||+eps) gives unit rows; RMSNorm gives RMS ~ 1 and promotes to fp32 through the
    weight (src/model/normalization.py:22-27,54-55; tests/test_model.py:21-26,43-51)."""
    x = rnd(3, 5, 32, seed=41, scale=3.0)
    n = O.qk_l2norm(x)
    assert torch.allclose(n.norm(dim=-1), torch.ones(3, 5), atol=1e-5)
    w = torch.ones(32)
    y = O.rms_norm(x.to(torch.bfloat16), w)
    assert y.dtype == torch.float32
    assert torch.allclose(y.float().pow(2).mean(-1).sqrt(), torch.ones(3, 5), atol=1e-2)


def test_split_form_reduces_to_fused_form():
    """Split module contraction [q_c | PoPE(q_r)] with zero content == fused PoPE at the same scale."""
    qr, kr, v = rnd(1, 2, 9, 8, seed=42), rnd(1, 2, 9, 8, seed=43), rnd(1, 2, 9, 8, seed=44)
    fr, de = O.pope_freqs(8), -torch.rand(2, 8) * 3
    z = torch.zeros(1, 2, 9, 4)
    a, _ = O.split_pope_attention(z, z, qr, kr, v, fr, de, scale=0.2)
    b, _ = O.pope_attention(qr, kr, v, fr, de, scale=0.2, clamp=False)
    assert (a - b).abs().max().item() < 1e-12


def test_chunked_oracle_matches_closed_form():
    """The row-chunked evaluator used for full-length GPU checks == the unchunked closed form."""
    S, D = 50, 8
    q, k, v, do = (rnd(S, D, seed=s) for s in (45, 46, 47, 48))
    fr, de = O.pope_freqs(D), -torch.rand(D, generator=torch.Generator().manual_seed(49)) * 6
    ch = O.pope_attention_chunked(q, k, v, fr, de, dout=do, scale=0.3, chunk=16, core_dtype=f64)
    cf = O.pope_attention_backward_closed_form(q.view(1, 1, S, D), k.view(1, 1, S, D), v.view(1, 1, S, D),
                                               fr, de, do.view(1, 1, S, D), scale=0.3)
    for name in ("out", "lse", "dq", "dk", "dv"):
        assert (ch[name] - cf[name][0, 0]).abs().max().item() < 1e-5, name
    for name in ("dfreqs", "ddelta"):
        assert (ch[name] - cf[name]).abs().max().item() < 1e-4 * max(1.0, cf[name].abs().max().item()), name
    # bottom-right alignment for Sq < Sk equals the tail rows of the full causal problem
    sub = O.pope_attention_chunked(q[30:], k, v, fr, de, scale=0.3, chunk=7, core_dtype=f64, start_q=30)
    assert (sub["out"] - ch["out"][30:]).abs().max().item() < 1e-5


def _round_to_bits(p: int, bits: int, max_finite: float) -> float:
    """p rounded to `bits` significant bits, ties to even, by integer arithmetic alone (inf past
    the type's largest finite value, rounding first): the value a bf16 (bits 8) or fp16 (bits 11)
    holds for the integer p."""
    if p == 0:
        return 0.0
    e = p.bit_length() - 1
    shift = e - (bits - 1)
    if shift <= 0:
        r = p
    else:
        q, rem = divmod(p, 1 << shift)
        half = 1 << (shift - 1)
        if rem > half or (rem == half and q % 2 == 1):
            q += 1
        r = q << shift
    return float("inf") if r > max_finite else float(r)


@pytest.mark.parametrize("dtype, bits, top", [(torch.bfloat16, 8, 3.3895313892515355e38), (torch.float16, 11, 65504.0)])
def test_positions_in_input_dtype(dtype, bits, top):
    """The oracle's FoPE positions (torch.arange(..., dtype=x.dtype), src/model/fpope.py:285,322)
    against round-to-nearest-even computed on integers: exact below 2^bits, then multiples of 2,
    4, ... with ties to the even multiple (257 -> 256, 259 -> 260 in bf16); fp16 overflows to inf
    from 65520 on."""
    for start, n in ((0, 600), (250, 20), (16370, 40), (65500, 40), (1 << 20, 50)):
        got = O.positions(n, start, dtype)
        want = torch.tensor([_round_to_bits(p, bits, top) for p in range(start, start + n)])
        assert torch.equal(got, want), (dtype, start)
    assert O.positions(3, 256, torch.bfloat16).tolist() == [256.0, 256.0, 258.0]
    assert O.positions(2, 259, torch.bfloat16).tolist() == [260.0, 260.0]
    assert torch.equal(O.positions(10, 7, None), torch.arange(7, 17, dtype=torch.float32))
    # the phases use the rounded positions, the frequency gradient too (pope_attention_chunked)
    f = O.pope_freqs(8)
    assert torch.equal(O.pope_phases(20, f, 300, pos_dtype=torch.bfloat16),
                       torch.outer(O.positions(20, 300, torch.bfloat16), f))


# ------------------------------------------------------------------ reference path (bf16 SDPA)

def _qkv(seed, B, Hq, Hkv, S, D, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(*s, generator=g).to(dtype) for s in
            ((B, Hq, S, D), (B, Hkv, S, D), (B, Hkv, S, D), (B, Hq, S, D))]


@pytest.mark.parametrize("causal", [True, False])
def test_bf16_path_without_rounding_is_the_exact_core(monkeypatch, causal):
    """With its rounding points switched off, attention_bf16_path is the fp64 core: the forward,
    lse and the hand-written backward (Di, dS, dQ, dK, dV and the GQA fold) equal autograd through
    oracle.attention.  A dropped term, a wrong sign or a transposed operand in the backward fails."""
    monkeypatch.setattr(O, "_bf16", lambda x: x)
    q, k, v, do = (t.double() for t in _qkv(3, 2, 4, 2, 37, 16, torch.float64))
    a = [t.clone().requires_grad_(True) for t in (q, k, v)]
    b = [t.clone().requires_grad_(True) for t in (q, k, v)]
    oa, la = O.attention(*a, 0.3, causal)
    ob, lb = O.attention_bf16_path(*b, 0.3, causal)
    oa.backward(do)
    ob.backward(do)
    assert torch.allclose(oa, ob, atol=1e-12) and torch.allclose(la, lb, atol=1e-12)
    for x, y in zip(a, b):
        assert torch.allclose(x.grad, y.grad, atol=1e-12)


def test_bf16_path_tracks_torch_bf16_sdpa():
    """The rounding points are those of a bf16 fused SDPA: against torch's own bf16
    F.scaled_dot_product_attention (CPU flash kernel), out and dQ agree to one bf16 spacing at their
    largest magnitude and
    have the same largest error to the exact core (within 25 %); dK / dV, which the fused GPU kernels accumulate
    in fp32 over every query block, carry at most torch's CPU error.  Both miss the 2e-2 bar on dv
    at |dv| ~ 5, which is why the GPU parity tests measure the path beside the kernel."""
    q, k, v, do = _qkv(0, 1, 2, 2, 300, 64)
    ts = [t.clone().requires_grad_(True) for t in (q, k, v)]
    o = F.scaled_dot_product_attention(*ts, is_causal=True)
    o.backward(do)
    ex = [t.double().requires_grad_(True) for t in (q, k, v)]
    oe, _ = O.attention(*ex, 64 ** -0.5, True)
    oe.backward(do.double())
    pa = [t.double().requires_grad_(True) for t in (q, k, v)]
    op, _ = O.attention_bf16_path(*pa, 64 ** -0.5, True)
    op.backward(do.double())
    ulp = lambda x: 2.0 ** (math.floor(math.log2(x)) - 7)  # bf16 spacing at magnitude x
    e_torch = {"out": o, "dq": ts[0].grad, "dk": ts[1].grad, "dv": ts[2].grad}
    e_path = {"out": op, "dq": pa[0].grad, "dk": pa[1].grad, "dv": pa[2].grad}
    e_ex = {"out": oe, "dq": ex[0].grad, "dk": ex[1].grad, "dv": ex[2].grad}
    for n in ("out", "dq"):
        d = (e_torch[n].double() - e_path[n].double()).abs().max().item()
        assert d <= ulp(e_ex[n].abs().max().item()), (n, d)
        et = (e_torch[n].double() - e_ex[n]).abs().max().item()
        ep = (e_path[n].double() - e_ex[n]).abs().max().item()
        assert 0.75 * et <= ep <= 1.25 * et, (n, et, ep)
    for n in ("dk", "dv"):
        et = (e_torch[n].double() - e_ex[n]).abs().max().item()
        ep = (e_path[n].double() - e_ex[n]).abs().max().item()
        assert 0 < ep <= et, (n, et, ep)
    assert (e_path["dv"].double() - e_ex["dv"]).abs().max().item() > 0.005
    assert (e_torch["dv"].double() - e_ex["dv"]).abs().max().item() > 2e-2


def test_bf16_path_gqa_fold():
    """GQA: per-head gradients are rounded to bf16 by the core, then summed over the kv head's query
    group (repeat_interleave backward), equal to running the expanded heads and summing."""
    q, k, v, do = (t.double() for t in _qkv(5, 1, 4, 2, 40, 16))
    a = [t.clone().requires_grad_(True) for t in (q, k, v)]
    o, _ = O.attention_bf16_path(*a, 0.25, True)
    o.backward(do)
    b = [q.clone().requires_grad_(True), k.repeat_interleave(2, 1).requires_grad_(True),
         v.repeat_interleave(2, 1).requires_grad_(True)]
    o2, _ = O.attention_bf16_path(*b, 0.25, True)
    o2.backward(do)
    assert torch.equal(o, o2) and torch.equal(a[0].grad, b[0].grad)
    assert torch.equal(a[1].grad, b[1].grad.view(1, 2, 2, 40, 16).sum(2))
    assert torch.equal(a[2].grad, b[2].grad.view(1, 2, 2, 40, 16).sum(2))


def test_rms_norm_gradient_rounds_once():
    """The reference casts x to fp32 once (self._norm(x.float()), src/model/normalization.py:25), so
    autograd sums the two paths of the gradient through x (x * r and r's dependence on x) in fp32
    and rounds to bf16 once.  Two separate casts would round each path before adding them, which
    for these inputs moves dx by a bf16 spacing (checked against that variant below)."""
    g = torch.Generator().manual_seed(1 * 3 + 64)
    x = (torch.randn(1, 64, generator=g) * 3).to(torch.bfloat16)
    w = (0.5 + torch.rand(64, generator=g)).to(torch.bfloat16)
    dy = torch.randn(1, 64, generator=g).to(torch.bfloat16)
    xr = x.clone().requires_grad_(True)
    O.rms_norm(xr, w).backward(dy)
    gc = (dy * w).float()                      # the gradient of the cast value, a bf16 product
    xf = x.float().requires_grad_(True)
    n = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6)
    once = torch.autograd.grad(n, xf, gc)[0].to(torch.bfloat16)
    assert torch.equal(xr.grad, once)
    xt = x.clone().requires_grad_(True)
    ((xt.float() * torch.rsqrt(xt.float().pow(2).mean(-1, keepdim=True) + 1e-6)).type_as(xt) * w).backward(dy)
    assert not torch.equal(xt.grad, once)     # the two-cast form differs here


def test_fp16_path_tracks_torch_fp16_sdpa():
    """The fp16 variant of the reference path against torch's own fp16
    F.scaled_dot_product_attention on the CPU: out and dQ agree to one fp16 spacing at their largest
    magnitude, with largest errors to the exact core within a factor 1.5 of torch's; dK / dV errors
    at most 1.5 times torch's."""
    q, k, v, do = _qkv(0, 1, 2, 2, 300, 64, torch.float16)
    ts = [t.clone().requires_grad_(True) for t in (q, k, v)]
    o = F.scaled_dot_product_attention(*ts, is_causal=True)
    o.backward(do)
    ex = [t.double().requires_grad_(True) for t in (q, k, v)]
    oe, _ = O.attention(*ex, 64 ** -0.5, True)
    oe.backward(do.double())
    pa = [t.double().requires_grad_(True) for t in (q, k, v)]
    op, _ = O.attention_fp16_path(*pa, 64 ** -0.5, True)
    op.backward(do.double())
    ulp = lambda x: 2.0 ** (math.floor(math.log2(x)) - 10)  # fp16 spacing at magnitude x
    res = {"out": (o, op, oe), "dq": (ts[0].grad, pa[0].grad, ex[0].grad),
           "dk": (ts[1].grad, pa[1].grad, ex[1].grad), "dv": (ts[2].grad, pa[2].grad, ex[2].grad)}
    for n, (t, pth, e) in res.items():
        et = (t.double() - e).abs().max().item()
        ep = (pth.double() - e).abs().max().item()
        assert 0 < ep <= 1.5 * et, (n, et, ep)
        if n in ("out", "dq"):
            assert (t.double() - pth.double()).abs().max().item() <= ulp(e.abs().max().item()), n
            assert ep >= et / 1.5, (n, et, ep)


# ---------------------------------------------------------------------------------------------
# explicit masks (SDPA's attn_mask, src/model/attention.py:91-96)
# ---------------------------------------------------------------------------------------------

def _masks(B, Hq, Sq, Sk, seed):
    """A bool (Sq, Sk) mask with one fully masked row, a float (B, 1, Sq, Sk) mask of finite values
    and -inf with one fully -inf row, and a per-head bool (B, Hq, Sq, Sk) mask."""
    g = torch.Generator().manual_seed(seed)
    mb = torch.rand(Sq, Sk, generator=g) > 0.4
    mb[1] = False
    mf = torch.randn(B, 1, Sq, Sk, generator=g, dtype=f64) * 2
    mf = mf.masked_fill(torch.rand(B, 1, Sq, Sk, generator=g) > 0.7, float("-inf"))
    mf[0, 0, 2] = float("-inf")
    mh = torch.rand(B, Hq, Sq, Sk, generator=g) > 0.5
    return [mb, mf, mh]


@pytest.mark.parametrize("which", [0, 1, 2])
def test_attention_mask_matches_torch_sdpa(which):
    """oracle.attention(mask=...) against torch's F.scaled_dot_product_attention(attn_mask=...) in
    fp64 after the reference's repeat_interleave (src/model/attention.py:86-96): out and the q / k / v
    gradients, GQA 4 -> 2, Sq != Sk, a fully masked row (zeros in both)."""
    B, Hq, Hkv, Sq, Sk, D = 2, 4, 2, 7, 11, 8
    mask = _masks(B, Hq, Sq, Sk, which)[which]
    q, k, v = rnd(B, Hq, Sq, D, seed=1, dtype=f64), rnd(B, Hkv, Sk, D, seed=2, dtype=f64), rnd(B, Hkv, Sk, D, seed=3, dtype=f64)
    do = rnd(B, Hq, Sq, D, seed=4, dtype=f64)
    a = [t.clone().requires_grad_(True) for t in (q, k, v)]
    b = [t.clone().requires_grad_(True) for t in (q, k, v)]
    oa, _ = O.attention(*a, 0.37, causal=False, mask=mask)
    ob = F.scaled_dot_product_attention(b[0], b[1].repeat_interleave(2, 1), b[2].repeat_interleave(2, 1),
                                        attn_mask=mask, scale=0.37)
    oa.backward(do)
    ob.backward(do)
    assert torch.allclose(oa, ob, atol=1e-12, rtol=0)
    for x, y in zip(a, b):
        assert torch.isfinite(x.grad).all()
        assert torch.allclose(x.grad, y.grad, atol=1e-12, rtol=0)
    if which in (0, 1):  # the fully masked row: zero output and zero query gradient
        r = 1 if which == 0 else 2
        assert (oa[0, :, r] == 0).all() and (a[0].grad[0, :, r] == 0).all()


def test_attention_mask_brute_force():
    """Plain Python loops on a tiny input: softmax over the keys of exp(q.k * scale + bias), bias 0
    / -inf from a bool mask or the float's value; a row with no key left gives 0."""
    B, Hq, Hkv, Sq, Sk, D = 1, 2, 1, 3, 4, 3
    q, k, v = rnd(B, Hq, Sq, D, seed=5, dtype=f64), rnd(B, Hkv, Sk, D, seed=6, dtype=f64), rnd(B, Hkv, Sk, D, seed=7, dtype=f64)
    mf = torch.tensor([[0.5, -1.0, float("-inf"), 2.0],
                       [float("-inf")] * 4,
                       [0.0, 0.0, 0.0, -3.0]], dtype=f64)
    for mask in (mf, ~torch.isneginf(mf)):
        out, _ = O.attention(q, k, v, 0.5, causal=False, mask=mask)
        for h in range(Hq):
            for i in range(Sq):
                bias = [(0.0 if mask[i][j] else -math.inf) if mask.dtype == torch.bool else mask[i][j].item()
                        for j in range(Sk)]
                e = [math.exp(0.5 * sum(q[0, h, i, d].item() * k[0, 0, j, d].item() for d in range(D)) + bias[j])
                     for j in range(Sk)]
                z = sum(e)
                for d in range(D):
                    want = 0.0 if z == 0 else sum(e[j] * v[0, 0, j, d].item() for j in range(Sk)) / z
                    assert abs(out[0, h, i, d].item() - want) < 1e-12


@pytest.mark.parametrize("which", [0, 1, 2])
def test_half_path_mask_without_rounding_is_the_exact_core(monkeypatch, which):
    """The 16-bit path core with a mask and its rounding points switched off equals the exact core
    with the same mask: forward, lse (-inf on the fully masked row) and the hand-written backward."""
    monkeypatch.setattr(O, "_bf16", lambda x: x)
    B, Hq, Hkv, Sq, Sk, D = 2, 4, 2, 7, 11, 8
    mask = _masks(B, Hq, Sq, Sk, 10 + which)[which]
    q, k, v = rnd(B, Hq, Sq, D, seed=8, dtype=f64), rnd(B, Hkv, Sk, D, seed=9, dtype=f64), rnd(B, Hkv, Sk, D, seed=10, dtype=f64)
    do = rnd(B, Hq, Sq, D, seed=11, dtype=f64)
    a = [t.clone().requires_grad_(True) for t in (q, k, v)]
    b = [t.clone().requires_grad_(True) for t in (q, k, v)]
    oa, la = O.attention(*a, 0.37, causal=False, mask=mask)
    ob, lb = O.attention_bf16_path(*b, 0.37, causal=False, mask=mask)
    oa.backward(do)
    ob.backward(do)
    assert torch.allclose(oa, ob, atol=1e-12) and torch.equal(torch.isneginf(la), torch.isneginf(lb))
    assert torch.allclose(la[torch.isfinite(la)], lb[torch.isfinite(lb)], atol=1e-12)
    for x, y in zip(a, b):
        assert torch.allclose(x.grad, y.grad, atol=1e-12)
