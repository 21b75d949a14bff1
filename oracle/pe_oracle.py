"""CPU oracle for the positional-encoding attention hot path (TEST INFRASTRUCTURE ONLY).

This module is the checker, never the product: only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it.  The product path (``pe_ablations_amd``) never
routes through it and raises when the HIP library is missing.

It restates, in plain PyTorch on the CPU, the reference's eager PE attention path of
shyampathak22/pe_ablations (all citations are files under the reference tree):

* PoPE frequencies, floor clip and angle cache ...... src/model/pope.py:67-90
* PoPE query / key transform ........................ src/model/pope.py:124-183
* FoPE effective-frequency collapse ................. src/model/fpope.py:107-146
* FoPE query / key transform ........................ src/model/fpope.py:266-338
* difference-form eager attention ................... src/model/fpope.py:208-244, 341-418
* RoPE / NTK / YaRN tables and interleaved rotation . src/model/rope.py:11-57, 122-217
* RMSNorm / QKNorm .................................. src/model/normalization.py:7-56
* split-form module contraction (content | PE) ...... src/model/fpope_attention.py:109-181
* RoPE module (rotate, QKNorm, SDPA) ................ src/model/attention.py:50-100
* closed-form backward .............................. tests/test_fpope.py:1571-1602
* whole decoder forward (embedding, blocks, head, CE) src/model/transformer.py:186-205,313-364

The transforms are computed in float32 exactly as the reference orders them (``fl(pos*theta)``
then ``+ delta``, no fused multiply-add) so that the fp32 kernel path can be held to 1e-5; the
attention core (softmax(QK^T * scale) V) is evaluated in float64 so the oracle's own rounding is
far below every tolerance it is used with.

Parity pins (each checked in ``tests/test_oracle.py``):
* attention core ............ brute-force Python loops on tiny inputs; torch SDPA special case
                               (freqs = 0, delta = 0 reduces PoPE to plain attention on softplus)
* explicit masks ............ torch's SDPA with attn_mask (bool, float with -inf, per head, fully
                               masked rows) in fp64, out and gradients; brute force on tiny inputs;
                               the 16-bit path core with its roundings off equals the exact core
* factorised PE transform ... equals the independent difference form (s-t)*theta + delta in fp64
* backward .................. closed form == fp64 autograd == fp64 finite differences (gradcheck)
* known answers ............. V = 0 -> O = 0, S = 1 -> O = V, diagonal phase = delta,
                               causal upper triangle = -inf, start_pos invariance, floor-clip counts
* RoPE ...................... complex-multiply formulation, norm preservation, NTK / YaRN closed forms
* whole decoder ............. S = 1 reduction to wo.wv (tests/test_decoder_host.py), zero layers,
                               causal prefix, loss at init; the SwiGLU gate order and the pre-norm
                               residuals by closed-form logit ratios of a hand-set one-token decoder
* reference vectors ......... PoPE / FoPE transforms bit for bit, and the RoPE family within one
                               float32 rounding, against outputs of the reference's own modules
                               (tests/golden/pe_transforms.npz, tests/test_golden.py)
"""

from __future__ import annotations

import math
from typing import Optional, Tuple

import torch
import torch.nn.functional as F

TWO_PI = 2.0 * math.pi


# --------------------------------------------------------------------------------------------
# frequency tables
# --------------------------------------------------------------------------------------------

def pope_freqs(dim: int, theta: float = 10000.0) -> torch.Tensor:
    """theta_i = theta ** (-(i / dim)), i < dim, float32 (src/model/pope.py:71)."""
    return theta ** (-(torch.arange(0, dim, dtype=torch.float32) / dim))


def floor_clip(freqs: torch.Tensor, training_length: int) -> torch.Tensor:
    """Zero frequencies below 2*pi/L (src/model/pope.py:67,75-82)."""
    floor = 2 * math.pi / training_length
    return torch.where(freqs < floor, torch.zeros_like(freqs), freqs)


def fope_effective_freqs(base_freqs: torch.Tensor, coeffs: torch.Tensor,
                         indices: Optional[torch.Tensor] = None, *,
                         training_length: int = 512, normalize: bool = True,
                         use_ceiling: bool = False,
                         freq_table: Optional[torch.Tensor] = None) -> torch.Tensor:
    """FoPE collapse to one effective frequency per dim (src/model/fpope.py:107-146).

    omega_c = theta_c + sum_j a_hat_cj * f_cj, with f_cj = theta_c * j (the reference's harmonics,
    ``indices`` = 1..M) or, when ``freq_table`` (D, M) is given, an arbitrary per-dim frequency
    table (BASELINE config 3 draws the extra frequencies from U(0, theta_0)).  Then the floor clip
    |omega| < 2*pi/L -> 0 and the optional +-2*pi ceiling clamp.
    """
    if normalize:
        a = coeffs / (coeffs.abs().sum(dim=1, keepdim=True) + 1e-8)
    else:
        a = coeffs
    if freq_table is None:
        if indices is None:
            indices = torch.arange(1, coeffs.shape[1] + 1, dtype=base_freqs.dtype)
        freq_table = base_freqs.unsqueeze(1) * indices.unsqueeze(0)
    eff = (a * freq_table).sum(dim=1) + base_freqs
    eff = torch.where(eff.abs() < 2 * math.pi / training_length, torch.zeros_like(eff), eff)
    if use_ceiling:
        eff = eff.clamp(-TWO_PI, TWO_PI)
    return eff


def rope_inv_freq(dim: int, theta: float = 10000.0) -> torch.Tensor:
    """1 / theta^(2i/dim), i < dim/2 (src/model/rope.py:28)."""
    return 1.0 / (theta ** (torch.arange(0, dim, 2).float() / dim))


def ntk_theta(dim: int, theta: float, scale: float) -> float:
    """theta * scale^(dim/(dim-2)) (src/model/rope.py:139)."""
    return theta * (scale ** (dim / (dim - 2)))


def yarn_inv_freq(dim: int, theta: float, scale: float, original_max_seq_len: int = 512,
                  beta_fast: float = 32.0, beta_slow: float = 1.0) -> Tuple[torch.Tensor, float, int, int]:
    """YaRN ramp between extrapolated and interpolated inverse frequencies and mscale
    (src/model/rope.py:170-207).  Note the reference's low/high bounds have no /2 and are
    indexed over the D/2 frequency slots.  Returns (inv_freq, mscale, low, high)."""
    pos_freqs = theta ** (torch.arange(0, dim, 2).float() / dim)
    extra = 1.0 / pos_freqs
    inter = 1.0 / (scale * pos_freqs)
    low = max(int(math.floor(dim * math.log(original_max_seq_len / (beta_fast * 2 * math.pi)) / math.log(theta))), 0)
    high = min(int(math.ceil(dim * math.log(original_max_seq_len / (beta_slow * 2 * math.pi)) / math.log(theta))), dim - 1)
    inv = inter.clone()
    inv[:low] = extra[:low]
    if low < high:
        smooth = (torch.arange(low, high + 1).float() - low) / (high - low)
        inv[low:high + 1] = (1 - smooth) * extra[low:high + 1] + smooth * inter[low:high + 1]
    mscale = float(0.1 * math.log(scale) + 1.0)
    return inv, mscale, low, high


# --------------------------------------------------------------------------------------------
# PE transforms (float32, reference operation order)
# --------------------------------------------------------------------------------------------

def positions(n: int, start: int = 0, pos_dtype=None) -> torch.Tensor:
    """start .. start + n - 1 as float32.  ``pos_dtype`` bf16 / fp16 builds them as the reference
    FoPE does on the GPU, torch.arange(..., dtype=x.dtype) (src/model/fpope.py:285,322): ATen's GPU
    arange forms each value start + i in fp32 and casts it to the dtype, so every position is
    rounded to nearest, ties to even (fp16: inf from 65520 on).  Torch's CPU arange for fp16 rounds
    the start first and differs, so the positions are cast here rather than built by a CPU arange
    of that dtype.  None keeps them exact (PoPE, src/model/pope.py:110-119)."""
    pos = torch.arange(start, start + n, dtype=torch.float32)
    if pos_dtype is None or pos_dtype == torch.float32:
        return pos
    return pos.to(pos_dtype).float()


def pope_phases(n: int, freqs: torch.Tensor, start: int = 0,
                delta: Optional[torch.Tensor] = None, dtype=torch.float32, pos_dtype=None) -> torch.Tensor:
    """phi = fl(pos * theta) (+ delta): torch.outer then add, float32 (src/model/pope.py:88-90,172-176).

    delta: None, (D,) shared, or (H, D) per head.  Returns (S, D) or (H, S, D).  ``dtype`` float64
    evaluates the same expression in double precision (used by gradient checks)."""
    ph = torch.outer(positions(n, start, pos_dtype).to(dtype), freqs.to(dtype))
    if delta is None:
        return ph
    delta = delta.to(dtype)
    if delta.dim() == 1:
        return ph + delta
    return ph.unsqueeze(0) + delta.unsqueeze(1)


def pope_transform(x: torch.Tensor, freqs: torch.Tensor, start: int = 0,
                   delta: Optional[torch.Tensor] = None, dtype=torch.float32, pos_dtype=None) -> torch.Tensor:
    """x (B, H, S, D) -> [mu cos phi, mu sin phi] (B, H, S, 2D), float32 math (or ``dtype``).

    Query: delta None (src/model/pope.py:124-149).  Key: delta already clamped by the caller
    (src/model/pope.py:151-183).  mu = softplus (beta 1, threshold 20)."""
    B, H, S, D = x.shape
    mu = F.softplus(x.to(dtype))
    ph = pope_phases(S, freqs, start, delta, dtype, pos_dtype)
    if ph.dim() == 2:
        ph = ph.view(1, 1, S, D)
    else:
        ph = ph.view(1, H, S, D)
    return torch.cat([mu * ph.cos(), mu * ph.sin()], dim=-1)


def clamp_delta(delta: torch.Tensor) -> torch.Tensor:
    """delta clamped to [-2pi, 0] on keys (src/model/pope.py:172, src/model/fpope.py:328)."""
    return delta.clamp(-2 * math.pi, 0.0)


def rope_rotate(x: torch.Tensor, inv_freq: torch.Tensor, start: int = 0) -> torch.Tensor:
    """Interleaved-pair rotation (x0,x1),(x2,x3)... by angle fl(t * w_i), float32
    (src/model/rope.py:28-32,50-57).  x: (B, H, S, D)."""
    B, H, S, D = x.shape
    ang = torch.outer(positions(S, start), inv_freq.float())  # (S, D/2)
    c, s = ang.cos().view(1, 1, S, D // 2), ang.sin().view(1, 1, S, D // 2)
    xf = x.float().reshape(B, H, S, D // 2, 2)
    a, b = xf[..., 0], xf[..., 1]
    return torch.stack([a * c - b * s, a * s + b * c], dim=-1).reshape(B, H, S, D)


def rope_rotate_complex(x: torch.Tensor, inv_freq: torch.Tensor, start: int = 0) -> torch.Tensor:
    """The same rotation through torch.polar / complex multiply (src/model/rope.py:31,50-56)."""
    B, H, S, D = x.shape
    ang = torch.outer(positions(S, start), inv_freq.float())
    cis = torch.polar(torch.ones_like(ang), ang).view(1, 1, S, D // 2)
    xc = torch.view_as_complex(x.float().reshape(B, H, S, D // 2, 2).contiguous())
    return torch.view_as_real(xc * cis).reshape(B, H, S, D)


def qk_l2norm(x: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """x / (||x|| + eps) over the last dim (src/model/normalization.py:54-55)."""
    return x / (x.norm(dim=-1, keepdim=True) + eps)


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """x * rsqrt(mean(x^2) + eps) in fp32, cast back, then * weight (src/model/normalization.py:22-27).
    One cast to fp32 feeds both uses of x, as in the reference's self._norm(x.float()), so that under
    autograd the two gradient parts are summed in fp32 and rounded to x's dtype once."""
    xf = x.float()
    out = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)).type_as(x)
    return out * weight


# --------------------------------------------------------------------------------------------
# attention core (float64)
# --------------------------------------------------------------------------------------------

def causal_mask(sq: int, sk: int) -> torch.Tensor:
    """True where masked.  Sq == Sk: SDPA is_causal top-left triu(1)
    (src/model/fpope_attention.py:171-177, src/model/fpope.py:378-383); Sq < Sk: the cache path's
    bottom-right alignment triu(Sk - Sq + 1) (src/model/fpope_attention.py:313-317)."""
    return torch.triu(torch.ones(sq, sk, dtype=torch.bool), diagonal=sk - sq + 1)


def mask_bias(mask: torch.Tensor, shape) -> torch.Tensor:
    """SDPA's attn_mask (src/model/attention.py:91-96) as an additive float64 bias broadcast to
    ``shape`` (B, Hq, Sq, Sk): a bool mask gives 0 where True (the key takes part) and -inf where
    False; a float mask is added as given."""
    if mask.dtype == torch.bool:
        b = torch.zeros(mask.shape, dtype=torch.float64).masked_fill(~mask, float("-inf"))
    else:
        b = mask.to(torch.float64)
    return b.expand(shape)


def softmax_rows(s: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """(p, lse) over the last axis.  A row whose every score is -inf gives p = 0 and lse = -inf, as
    torch's SDPA returns zeros for it, with no NaN in the forward or in autograd's backward (the
    row's scores are replaced by a constant before the logsumexp)."""
    dead = torch.isneginf(s).all(-1, keepdim=True)
    s = s.masked_fill(dead, 0.0)
    lse = torch.logsumexp(s, dim=-1, keepdim=True)
    p = torch.exp(s - lse).masked_fill(dead, 0.0)
    return p, lse.masked_fill(dead, float("-inf")).squeeze(-1)


def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float,
              causal: bool = True, dtype=torch.float64, mask: Optional[torch.Tensor] = None
              ) -> Tuple[torch.Tensor, torch.Tensor]:
    """softmax(q k^T * scale + mask, causal) v.  q (B,Hq,Sq,Dqk), k (B,Hkv,Sk,Dqk), v (B,Hkv,Sk,Dv).
    GQA: kv head = h // (Hq/Hkv) (repeat_interleave, src/model/fpope_attention.py:160-163).
    ``mask``: SDPA's attn_mask broadcastable to (B, Hq, Sq, Sk) (mask_bias).
    Returns (out (B,Hq,Sq,Dv), lse (B,Hq,Sq)) in ``dtype``."""
    B, Hq, Sq, _ = q.shape
    Hkv = k.shape[1]
    g = Hq // Hkv
    if g > 1:
        k = k.repeat_interleave(g, dim=1)
        v = v.repeat_interleave(g, dim=1)
    qd, kd, vd = q.to(dtype), k.to(dtype), v.to(dtype)
    s = torch.matmul(qd, kd.transpose(-2, -1)) * scale
    if mask is not None:
        s = s + mask_bias(mask, s.shape).to(dtype)
    if causal:
        s = s.masked_fill(causal_mask(Sq, k.shape[2]), float("-inf"))
    p, lse = softmax_rows(s)
    return torch.matmul(p, vd), lse


def round_ste(x: torch.Tensor, dtype) -> torch.Tensor:
    """Round to ``dtype`` in the forward, identity in the backward (autocast's cast semantics)."""
    if dtype is None:
        return x
    return x + (x.to(dtype).to(x.dtype) - x).detach()


def _round16(x: torch.Tensor, dtype) -> torch.Tensor:
    return x.to(dtype).to(x.dtype)


def _bf16(x: torch.Tensor) -> torch.Tensor:
    return _round16(x, torch.bfloat16)


class _SdpaHalfPath(torch.autograd.Function):
    """The attention core with the rounding points of a 16-bit fused SDPA (the kernel the reference
    reaches through F.scaled_dot_product_attention under bf16 or fp16 autocast,
    src/model/fpope_attention.py:171-177 and src/model/attention.py:91-96), not its exact value.

    Forward: scores and the row sums in full precision, the probabilities exp(s - max) rounded to
    the 16-bit type before the PV product, out = (sum p v) / sum p rounded to it.  Backward (the
    flash-attention recomputation): Di = rowsum(dO * out) over the rounded out, P = exp(s - lse),
    dV = P^T dO with P rounded, dS = P (dP - Di) rounded before dQ = dS K and dK = dS^T Q, every
    gradient rounded per query head; GQA sums the per-head dK / dV afterwards (the reference's
    repeat_interleave backward).  Inputs hold values of the 16-bit type; math is float64 between
    the rounding points.  Used only to measure the reference path's own error beside the kernel's."""

    @staticmethod
    def forward(ctx, q, k, v, scale, causal, dtype, mask=None):
        f64 = torch.float64
        r = (lambda x: _bf16(x)) if dtype == torch.bfloat16 else (lambda x: _round16(x, dtype))
        Hq, Hkv = q.shape[1], k.shape[1]
        g = Hq // Hkv
        kr, vr = k.to(f64).repeat_interleave(g, 1), v.to(f64).repeat_interleave(g, 1)
        qd = q.to(f64)
        s = torch.matmul(qd, kr.transpose(-2, -1)) * scale
        bias = None if mask is None else mask_bias(mask, s.shape)
        if bias is not None:
            s = s + bias
        if causal:
            s = s.masked_fill(causal_mask(q.shape[2], k.shape[2]), float("-inf"))
        m = s.amax(-1, keepdim=True).clamp_min(-1e300)
        pt = torch.exp(s - m)
        lsum = pt.sum(-1, keepdim=True)
        # a row with every key masked: out 0 and lse -inf (torch's SDPA returns zeros)
        out = r(torch.matmul(r(pt), vr) / lsum.masked_fill(lsum == 0, 1.0))
        lse = (m + torch.log(lsum)).squeeze(-1)
        ctx.save_for_backward(qd, kr, vr, out, lse)
        ctx.scale, ctx.causal, ctx.g, ctx.r, ctx.bias = scale, causal, g, r, bias
        return out.to(q.dtype), lse

    @staticmethod
    def backward(ctx, dout, dlse):
        qd, kr, vr, out, lse = ctx.saved_tensors
        scale, g, r = ctx.scale, ctx.g, ctx.r
        do = r(dout.to(torch.float64))
        di = (do * out).sum(-1, keepdim=True)
        s = torch.matmul(qd, kr.transpose(-2, -1)) * scale
        if ctx.bias is not None:
            s = s + ctx.bias
        if ctx.causal:
            s = s.masked_fill(causal_mask(qd.shape[2], kr.shape[2]), float("-inf"))
        p = torch.exp(s - lse.masked_fill(torch.isneginf(lse), 0.0).unsqueeze(-1))
        dv = r(torch.matmul(r(p).transpose(-2, -1), do))
        ds = r(p * (torch.matmul(do, vr.transpose(-2, -1)) - di))
        dq = r(torch.matmul(ds, kr) * scale)
        dk = r(torch.matmul(ds.transpose(-2, -1), qd) * scale)

        def fold(x):  # per-head gradients summed over each kv head's query group
            B, H, S, D = x.shape
            return x.view(B, H // g, g, S, D).sum(2)

        return dq, fold(dk), fold(dv), None, None, None, None


def attention_bf16_path(q, k, v, scale: float, causal: bool = True, mask: Optional[torch.Tensor] = None):
    """(out, lse) of ``attention`` with a bf16 fused SDPA's rounding points (_SdpaHalfPath);
    differentiable, so the transforms around it carry the path's gradients to the raw inputs."""
    return _SdpaHalfPath.apply(q, k, v, scale, bool(causal), torch.bfloat16, mask)


def attention_fp16_path(q, k, v, scale: float, causal: bool = True, mask: Optional[torch.Tensor] = None):
    """The same with an fp16 fused SDPA's rounding points (fp16 autocast)."""
    return _SdpaHalfPath.apply(q, k, v, scale, bool(causal), torch.float16, mask)


# --------------------------------------------------------------------------------------------
# fused-form PoPE attention (legacy fused API)
# --------------------------------------------------------------------------------------------

def pope_attention(q, k, v, freqs, delta, scale: Optional[float] = None, causal: bool = True,
                   start_q: int = 0, start_k: int = 0, clamp: bool = True,
                   operand_dtype=None, core_dtype=torch.float64, transform_dtype=torch.float32,
                   core=None):
    """Fused-form PoPE causal attention, factorised (what the reference module computes,
    src/model/pope.py:124-183 + src/model/fpope_attention.py:166-177 with d_content = 0).

    q (B,Hq,S,D), k/v (B,Hkv,S,D); freqs (D,); delta (D,) or (Hkv?,D) -- per head uses the key
    head index; ``clamp`` applies the module's [-2pi, 0] clamp.  ``operand_dtype`` rounds the
    transformed q~/k~ and v (e.g. torch.bfloat16, what SDPA sees under autocast).  ``core``
    replaces the attention core (signature of ``attention_bf16_path``).
    Differentiable (autograd) w.r.t. q, k, v, freqs, delta.  Returns (out, lse)."""
    D = q.shape[-1]
    scale = (1.0 / math.sqrt(D)) if scale is None else scale
    d = clamp_delta(delta) if clamp else delta
    qt = pope_transform(q, freqs, start_q, dtype=transform_dtype)
    kt = pope_transform(k, freqs, start_k, d, dtype=transform_dtype)
    qt = round_ste(qt, operand_dtype)
    kt = round_ste(kt, operand_dtype)
    vv = round_ste(v.to(transform_dtype), operand_dtype)
    if core is not None:
        return core(qt, kt, vv, scale, causal)
    return attention(qt, kt, vv, scale, causal, core_dtype)


def pope_attention_diff_form(q, k, v, freqs, phase_bias, scale=None, causal=True, dtype=torch.float64):
    """The eager difference form: score = sum_c mu_q mu_k cos((s-t) w_c + b_c)
    (src/model/fpope.py:208-244, 341-418; legacy pytorch restatement tests/test_fpope.py:1539-1560).
    No clamp.  O(S^2 D) memory: tiny inputs only."""
    q, k, v, freqs, phase_bias = (t.to(dtype) for t in (q, k, v, freqs, phase_bias))
    Sq, Sk, D = q.shape[2], k.shape[2], q.shape[3]
    scale = (1.0 / math.sqrt(D)) if scale is None else scale
    mu_q, mu_k = F.softplus(q), F.softplus(k)
    pos_q = torch.arange(Sq, dtype=dtype)
    pos_k = torch.arange(Sk, dtype=dtype)
    ph = (pos_k.unsqueeze(0) - pos_q.unsqueeze(1)).unsqueeze(-1) * freqs + phase_bias
    sc = (mu_q.unsqueeze(3) * mu_k.unsqueeze(2) * torch.cos(ph)).sum(-1) * scale
    if causal:
        sc = sc.masked_fill(causal_mask(Sq, Sk), float("-inf"))
    p = torch.softmax(sc, dim=-1)
    return torch.matmul(p, v), torch.logsumexp(sc, dim=-1)


def pope_attention_backward_closed_form(q, k, v, freqs, delta, dout, scale=None, causal=True,
                                        start_q: int = 0, start_k: int = 0):
    """Closed-form gradients of fused PoPE attention in float64 (no clamp applied here: ``delta``
    is the value the transform uses).  Follows tests/test_fpope.py:1571-1602 (dP = dO V^T,
    D_i = rowsum(P o dP), dS = P o (dP - D_i), d_raw = dS * scale) and extends it with the
    factorised inverse transform that the kernels implement:

        dq~ = d_raw k~,  dk~ = d_raw^T q~;  (g_c, g_s) = halves of dq~ / dk~
        dmu = g_c cos phi + g_s sin phi,    dphi = mu (g_s cos phi - g_c sin phi)
        dq = dmu_q sigmoid(q),  dk = dmu_k sigmoid(k)
        ddelta_c = sum_{b,h,s} dphi_k;  dfreqs_c = sum t dphi_q + sum s dphi_k

    Single kv head per query head (no GQA).  delta (D,) shared or (H, D) per head.
    Returns dict(out, lse, dq, dk, dv, dfreqs, ddelta)."""
    f64 = torch.float64
    q, k, v, dout = (t.to(f64) for t in (q, k, v, dout))
    freqs, delta = freqs.to(f64), delta.to(f64)
    B, H, S, D = q.shape
    Sk = k.shape[2]
    scale = (1.0 / math.sqrt(D)) if scale is None else scale
    tq = torch.arange(start_q, start_q + S, dtype=f64)
    tk = torch.arange(start_k, start_k + Sk, dtype=f64)
    phq = (tq.unsqueeze(1) * freqs).view(1, 1, S, D)
    if delta.dim() == 1:
        phk = (tk.unsqueeze(1) * freqs + delta).view(1, 1, Sk, D)
    else:
        phk = (tk.unsqueeze(1) * freqs).view(1, 1, Sk, D) + delta.view(1, H, 1, D)
    mq, mk = F.softplus(q), F.softplus(k)
    qt = torch.cat([mq * phq.cos(), mq * phq.sin()], -1)
    kt = torch.cat([mk * phk.cos(), mk * phk.sin()], -1)
    s = torch.matmul(qt, kt.transpose(-2, -1)) * scale
    if causal:
        s = s.masked_fill(causal_mask(S, Sk), float("-inf"))
    P = torch.softmax(s, -1)
    lse = torch.logsumexp(s, -1)
    out = torch.matmul(P, v)
    dP = torch.matmul(dout, v.transpose(-2, -1))
    Di = (P * dP).sum(-1, keepdim=True)
    dS = P * (dP - Di)
    draw = dS * scale
    dqt = torch.matmul(draw, kt)
    dkt = torch.matmul(draw.transpose(-2, -1), qt)
    dv = torch.matmul(P.transpose(-2, -1), dout)

    def inv(g, mu, ph):
        gc, gs = g[..., :D], g[..., D:]
        c, sn = ph.cos(), ph.sin()
        return gc * c + gs * sn, mu * (gs * c - gc * sn)

    dmq, dphq = inv(dqt, mq, phq)
    dmk, dphk = inv(dkt, mk, phk)
    dq = dmq * torch.sigmoid(q)
    dk = dmk * torch.sigmoid(k)
    if delta.dim() == 1:
        ddelta = dphk.sum(dim=(0, 1, 2))
    else:
        ddelta = dphk.sum(dim=(0, 2))
    dfreqs = (dphq * tq.view(1, 1, S, 1)).sum(dim=(0, 1, 2)) + (dphk * tk.view(1, 1, Sk, 1)).sum(dim=(0, 1, 2))
    return dict(out=out, lse=lse, dq=dq, dk=dk, dv=dv, dfreqs=dfreqs, ddelta=ddelta)


# --------------------------------------------------------------------------------------------
# split-form module attention and RoPE module attention
# --------------------------------------------------------------------------------------------

def split_pope_attention(qc, kc, qr, kr, v, freqs, delta, scale=None, causal=True, start: int = 0,
                         operand_dtype=None, core_dtype=torch.float64, core=None):
    """The reference module's contraction: Q = [q_c | PoPE(q_r)], K = [k_c | PoPE(k_r, delta)]
    (src/model/fpope_attention.py:128-177).  q_c/q_r (B,Hq,S,Dc/Dr), k_c/k_r/v (B,Hkv,S,.).
    delta is the (already clamped) key phase bias.  scale defaults to (Dc + 2 Dr)^-1/2
    (src/model/fpope_attention.py:107)."""
    Dc, Dr = qc.shape[-1], qr.shape[-1]
    scale = (Dc + 2 * Dr) ** -0.5 if scale is None else scale
    qt = torch.cat([qc.float(), pope_transform(qr, freqs, start)], -1)
    kt = torch.cat([kc.float(), pope_transform(kr, freqs, start, delta)], -1)
    qt, kt = round_ste(qt, operand_dtype), round_ste(kt, operand_dtype)
    vv = round_ste(v.float(), operand_dtype)
    if core is not None:
        return core(qt, kt, vv, scale, causal)
    return attention(qt, kt, vv, scale, causal, core_dtype)


def rope_attention(q, k, v, inv_freq, mscale: float = 1.0, qk_norm: bool = True, causal=True,
                   start: int = 0, scale=None, operand_dtype=None, core=None):
    """RoPE module path: interleaved rotation (x mscale for YaRN), QKNorm, SDPA with scale
    1/sqrt(D) (src/model/attention.py:69-96, src/model/rope.py:209-217).  (B,H,S,D) layout."""
    D = q.shape[-1]
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    qr = rope_rotate(q, inv_freq, start) * mscale
    kr = rope_rotate(k, inv_freq, start) * mscale
    if qk_norm:
        qr, kr = qk_l2norm(qr), qk_l2norm(kr)
    qr, kr = round_ste(qr, operand_dtype), round_ste(kr, operand_dtype)
    return (core or attention)(qr, kr, round_ste(v.float(), operand_dtype), scale, causal)


# --------------------------------------------------------------------------------------------
# brute force (pure Python, tiny inputs)
# --------------------------------------------------------------------------------------------

def brute_force_pope(q, k, v, freqs, delta, scale, causal=True):
    """Triple loop over (t, s, c) in Python floats: sum_c mu_q mu_k cos((s - t) theta_c + delta_c),
    softmax over s <= t, weighted sum of V.  Single (b, h); q/k/v (S, D) nested lists or tensors."""
    q, k, v = (t.tolist() if hasattr(t, "tolist") else t for t in (q, k, v))
    freqs = freqs.tolist() if hasattr(freqs, "tolist") else freqs
    delta = delta.tolist() if hasattr(delta, "tolist") else delta
    S, D = len(q), len(q[0])
    sp = lambda x: x if x > 20 else math.log1p(math.exp(x))
    out = []
    for t in range(S):
        sc = []
        for s in range(len(k)):
            if causal and s > t:
                continue
            acc = 0.0
            for c in range(D):
                acc += sp(q[t][c]) * sp(k[s][c]) * math.cos((s - t) * freqs[c] + delta[c])
            sc.append(acc * scale)
        m = max(sc)
        w = [math.exp(x - m) for x in sc]
        z = sum(w)
        out.append([sum(w[s] * v[s][j] for s in range(len(w))) / z for j in range(len(v[0]))])
    return out


# --------------------------------------------------------------------------------------------
# row-chunked closed form for long sequences (one head at S = 16384 fits in memory)
# --------------------------------------------------------------------------------------------

def pope_attention_chunked(q, k, v, freqs, delta, dout=None, scale=None, causal=True,
                           start_q: int = 0, start_k: int = 0, chunk: int = 1024,
                           core_dtype=torch.float32, operand_dtype=None, pos_dtype=None):
    """Fused-form PoPE attention forward (and, with ``dout``, the closed-form backward of
    pope_attention_backward_closed_form) evaluated in query-row chunks so the (S, S) score
    matrix never exists whole.  Single (b, h): q (Sq, D), k/v (Sk, D), delta (D,) as used.
    Transforms in fp32 in the reference order; ``operand_dtype`` rounds q~, k~, v as autocast
    would; the GEMMs run in ``core_dtype``.  Causal alignment: top-left when Sq == Sk, else
    bottom-right.  ``pos_dtype`` rounds the positions as in ``positions`` (FoPE's x.dtype), in the
    phases and in the frequency gradient.  Returns dict(out, lse[, dq, dk, dv, dfreqs, ddelta])."""
    Sq, D = q.shape
    Sk = k.shape[0]
    scale = (1.0 / math.sqrt(D)) if scale is None else scale
    ct = core_dtype
    qt = pope_transform(q.view(1, 1, Sq, D), freqs, start_q, pos_dtype=pos_dtype)[0, 0]
    kt = pope_transform(k.view(1, 1, Sk, D), freqs, start_k, delta, pos_dtype=pos_dtype)[0, 0]
    vv = v.float()
    if operand_dtype is not None:
        qt, kt, vv = (t.to(operand_dtype).float() for t in (qt, kt, vv))
    qt, kt, vv = qt.to(ct), kt.to(ct), vv.to(ct)
    off = Sk - Sq
    out = torch.empty(Sq, v.shape[1], dtype=ct)
    lse = torch.empty(Sq, dtype=ct)
    kpos = torch.arange(Sk)
    for r0 in range(0, Sq, chunk):
        r1 = min(Sq, r0 + chunk)
        s = (qt[r0:r1] @ kt.T) * scale
        if causal:
            s = s.masked_fill(kpos.view(1, -1) > (torch.arange(r0, r1) + off).view(-1, 1), float("-inf"))
        l = torch.logsumexp(s, -1)
        out[r0:r1] = torch.exp(s - l.unsqueeze(-1)) @ vv
        lse[r0:r1] = l
    res = dict(out=out, lse=lse)
    if dout is None:
        return res
    do = dout.to(ct)
    Di = (do * out).sum(-1)
    dqt = torch.zeros_like(qt)
    dkt = torch.zeros_like(kt)
    dv = torch.zeros(Sk, v.shape[1], dtype=ct)
    for r0 in range(0, Sq, chunk):
        r1 = min(Sq, r0 + chunk)
        s = (qt[r0:r1] @ kt.T) * scale
        if causal:
            s = s.masked_fill(kpos.view(1, -1) > (torch.arange(r0, r1) + off).view(-1, 1), float("-inf"))
        P = torch.exp(s - lse[r0:r1].unsqueeze(-1))
        dP = do[r0:r1] @ vv.T
        dS = P * (dP - Di[r0:r1].unsqueeze(-1)) * scale
        dqt[r0:r1] = dS @ kt
        dkt += dS.T @ qt[r0:r1]
        dv += P.T @ do[r0:r1]
    f64 = torch.float64
    tq = positions(Sq, start_q, pos_dtype).to(f64)
    tk = positions(Sk, start_k, pos_dtype).to(f64)
    phq = pope_phases(Sq, freqs, start_q, pos_dtype=pos_dtype).to(f64)
    phk = pope_phases(Sk, freqs, start_k, delta, pos_dtype=pos_dtype).to(f64)
    mq, mk = F.softplus(q.double()), F.softplus(k.double())

    def inv(g, mu, ph):
        g = g.double()
        gc, gs = g[:, :D], g[:, D:]
        c, sn = ph.cos(), ph.sin()
        return gc * c + gs * sn, mu * (gs * c - gc * sn)

    dmq, dphq = inv(dqt, mq, phq)
    dmk, dphk = inv(dkt, mk, phk)
    res.update(dq=dmq * torch.sigmoid(q.double()), dk=dmk * torch.sigmoid(k.double()), dv=dv,
               ddelta=dphk.sum(0), dfreqs=(dphq * tq.view(-1, 1)).sum(0) + (dphk * tk.view(-1, 1)).sum(0))
    return res


# --------------------------------------------------------------------------------------------
# whole decoder (the long-context evaluation and 1B-forward callers of the attention)
# --------------------------------------------------------------------------------------------

def decoder_forward(state: dict, cfg, input_ids: torch.Tensor, start: int = 0,
                    labels: Optional[torch.Tensor] = None, yarn_extended: bool = False) -> dict:
    """Transformer.forward of the reference (src/model/transformer.py:313-364) restated over a
    state dict: token embedding -> per layer x + attn(RMSNorm(x)), x + w2(silu(w3 h) * w1 h)
    (src/model/transformer.py:186-205, src/model/ffn.py:17-27,53-68) -> RMSNorm -> LM head ->
    shifted cross entropy (ignore_index -100).  Weights in float32, the attention core in float64.

    ``cfg`` has TransformerConfig's attributes.  The attention per pe_mode follows
    src/model/transformer.py:127-178: "pope" / "pope_floor" / "fpope" use the split module
    contraction (or, with ``cfg.pope_fused``, the fused form of the legacy API: every head dim
    PoPE-encoded, scale 1/sqrt(head_dim)); "rope" / "nope" use the RoPE module path.
    ``yarn_extended``: the YaRN module after extend_seq_len, which rebuilds the plain RoPE table
    from theta and keeps its mscale (src/model/rope.py:103-119 inherited, :209-217)."""
    w = {k: v.float() for k, v in state.items()}
    B, S = input_ids.shape
    H, Hkv, D, eps = cfg.num_heads, cfg.num_kv_heads, cfg.head_dim, cfg.norm_eps
    mode = cfg.pe_mode
    fused = bool(getattr(cfg, "pope_fused", False)) and mode in ("pope", "pope_floor")

    if mode in ("pope", "pope_floor"):
        freqs, delta = w["pope.effective_freqs"], clamp_delta(w["pope.phase_bias"])
    elif mode == "fpope":
        freqs = fope_effective_freqs(w["fpope.base_freqs"], w["fpope.fourier_coeffs"], w["fpope.fourier_indices"],
                                     training_length=cfg.fpope_training_length,
                                     normalize=cfg.fpope_normalize_coeffs, use_ceiling=cfg.fpope_use_ceiling)
        delta = clamp_delta(w["fpope.phase_bias"])
    elif mode == "rope":
        if cfg.rope_type == "yarn":
            inv_freq, mscale, _, _ = yarn_inv_freq(D, cfg.rope_theta, cfg.rope_scale, 512)
            if yarn_extended:
                inv_freq = rope_inv_freq(D, cfg.rope_theta)
        elif cfg.rope_type == "ntk":
            inv_freq, mscale = rope_inv_freq(D, ntk_theta(D, cfg.rope_theta, cfg.rope_scale)), 1.0
        else:
            inv_freq, mscale = rope_inv_freq(D, cfg.rope_theta), 1.0

    def heads(t, n, d):
        return t.view(B, S, n, d).transpose(1, 2)

    def attn(p, h):
        v = heads(F.linear(h, w[p + "wv.weight"]), Hkv, D)
        if mode in ("pope", "pope_floor", "fpope"):
            qr, kr = F.linear(h, w[p + "wq_r.weight"]), F.linear(h, w[p + "wk_r.weight"])
            if cfg.use_qk_norm:
                qr, kr = rms_norm(qr, w[p + "qr_norm.weight"]), rms_norm(kr, w[p + "kr_norm.weight"])
            dr = qr.shape[-1] // H
            qr, kr = heads(qr, H, dr), heads(kr, Hkv, dr)
            if fused:
                out, _ = pope_attention(qr, kr, v, freqs, delta, scale=D ** -0.5, start_q=start,
                                        start_k=start, clamp=False)
            else:
                qc = heads(F.linear(h, w[p + "wq_c.weight"]), H, D)
                kc = heads(F.linear(h, w[p + "wk_c.weight"]), Hkv, D)
                out, _ = split_pope_attention(qc, kc, qr, kr, v, freqs, delta, start=start)
        else:
            q = heads(F.linear(h, w[p + "wq.weight"]), H, D)
            k = heads(F.linear(h, w[p + "wk.weight"]), Hkv, D)
            if mode == "rope":
                out, _ = rope_attention(q, k, v, inv_freq, mscale, cfg.use_qk_norm, start=start)
            else:
                if cfg.use_qk_norm:
                    q, k = qk_l2norm(q), qk_l2norm(k)
                out, _ = attention(q, k, v, D ** -0.5)
        out = out.float().transpose(1, 2).reshape(B, S, H * v.shape[-1])
        return F.linear(out, w[p + "wo.weight"])

    x = F.embedding(input_ids, w["token_embedding.embedding.weight"])
    for i in range(cfg.num_layers):
        p = f"layers.{i}."
        x = x + attn(p + "attention.", rms_norm(x, w[p + "attention_norm.weight"], eps))
        h = rms_norm(x, w[p + "ffn_norm.weight"], eps)
        f = p + "feed_forward."
        x = x + F.linear(F.silu(F.linear(h, w[f + "w3.weight"])) * F.linear(h, w[f + "w1.weight"]), w[f + "w2.weight"])
    logits = F.linear(rms_norm(x, w["norm.weight"], eps), w["output.weight"])
    res = {"logits": logits}
    if labels is not None:
        res["loss"] = F.cross_entropy(logits[..., :-1, :].reshape(-1, logits.shape[-1]),
                                      labels[..., 1:].reshape(-1), ignore_index=-100)
    return res
