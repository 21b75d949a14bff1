"""Fused positional-encoding attention as a torch.autograd.Function over libpe_attn.so.

``pe_attention`` replaces, in one forward and one backward launch sequence, the span
PE transform -> content|position concat -> GQA repeat_interleave -> causal SDPA of the reference
modules (src/model/fpope_attention.py:145-177, src/model/attention.py:69-96).  Tensors are
(B, H, S, D) views with any strides whose last dimension is contiguous (e.g. the projections'
``view(B, S, H, D).transpose(1, 2)``); nothing is copied on the way in.  The output is a
(B, H, S, Dv) view of a (B, S, H, Dv) buffer, so the caller's ``transpose(1, 2).reshape`` is free.

Compute dtype: bf16 when autocast is on or any input is bf16/fp16, else fp32 (the reference's
autocast training path and its fp32 eval path).  Only GPU tensors are accepted.
"""

from __future__ import annotations

import contextlib
import ctypes
import math
import threading
from typing import Optional

import torch

from . import _lib

_MODES = {"pope": _lib.PE_MODE_POPE, "fope": _lib.PE_MODE_POPE, "rope": _lib.PE_MODE_ROPE,
          "none": _lib.PE_MODE_NONE, "nope": _lib.PE_MODE_NONE}
_CAUSAL = {False: _lib.PE_CAUSAL_NONE, True: _lib.PE_CAUSAL_TOP_LEFT,
           "none": _lib.PE_CAUSAL_NONE, "top_left": _lib.PE_CAUSAL_TOP_LEFT,
           "bottom_right": _lib.PE_CAUSAL_BOTTOM_RIGHT}


def _dtype_code(t: torch.dtype) -> int:
    if t == torch.bfloat16:
        return _lib.PE_DTYPE_BF16
    if t == torch.float32:
        return _lib.PE_DTYPE_FP32
    if t == torch.float16:
        return _lib.PE_DTYPE_FP16
    raise TypeError(f"pe_attention: unsupported tensor dtype {t}")


_TORCH_DTYPE = {_lib.PE_DTYPE_BF16: torch.bfloat16, _lib.PE_DTYPE_FP32: torch.float32,
                _lib.PE_DTYPE_FP16: torch.float16}
_HALF = (torch.bfloat16, torch.float16)


def norm_out_dtype(x_dtype: torch.dtype, w_dtype: torch.dtype) -> torch.dtype:
    """RMSNorm's output dtype, torch's promotion of (normalised value in x's dtype) * weight: the
    16-bit type when x and the weight share it, else fp32 (bf16 * fp16 promotes to fp32 too)."""
    return x_dtype if (x_dtype == w_dtype and x_dtype in _HALF) else torch.float32


def _tensor(t: Optional[torch.Tensor]) -> _lib.PeTensor:
    d = _lib.PeTensor()
    if t is None:
        return d
    if t.dim() != 4:
        raise ValueError(f"pe_attention expects (B, H, S, D) tensors, got shape {tuple(t.shape)}")
    d.data = t.data_ptr()
    d.dtype = _dtype_code(t.dtype)
    for i, s in enumerate(t.stride()):
        d.stride[i] = s
    if t.shape[3] == 1:
        d.stride[3] = 1
    return d


def _prep_in(t: Optional[torch.Tensor]) -> Optional[torch.Tensor]:
    if t is None:
        return None
    if t.dtype not in (torch.bfloat16, torch.float32, torch.float16):
        t = t.to(torch.float32)
    if t.stride(-1) != 1 and t.shape[-1] != 1:
        t = t.contiguous()
    return t


def _params(cfg, qr, kr, v, qc, delta) -> _lib.PeParams:
    p = _lib.PeParams()
    B, Hq, Sq = qr.shape[0], qr.shape[1], qr.shape[2]
    Hkv, Sk = kr.shape[1], kr.shape[2]
    p.B, p.Hq, p.Hkv, p.Sq, p.Sk = B, Hq, Hkv, Sq, Sk
    p.Dc = 0 if qc is None else qc.shape[3]
    p.Dr = qr.shape[3]
    p.Dv = v.shape[3]
    p.mode = cfg["mode"]
    p.dtype = cfg["dtype"]
    p.causal = cfg["causal"]
    p.start_pos_q, p.start_pos_k = cfg["start_pos_q"], cfg["start_pos_k"]
    p.qk_l2norm = int(cfg["qk_norm"])
    p.scale = cfg["scale"]
    p.rope_mscale = cfg["mscale"]
    p.delta_head_stride = 0 if (delta is None or delta.dim() == 1) else delta.shape[-1]
    p.position_rounding = cfg["pos_round"]
    return p


def position_rounding(position_dtype, mode: int) -> int:
    """PE_POS_* for a ``position_dtype``: None / torch.float32 keep positions exact; torch.bfloat16
    / torch.float16 round them to that type before the phase product, as the reference FoPE's
    torch.arange(..., dtype=x.dtype) does for a bf16 / fp16 x (src/model/fpope.py:285,322).
    Rounding applies to PoPE / FoPE only."""
    if position_dtype is None or position_dtype == torch.float32:
        return _lib.PE_POS_EXACT
    if mode != _lib.PE_MODE_POPE:
        raise ValueError("position_dtype applies to PoPE / FoPE only")
    if position_dtype == torch.bfloat16:
        return _lib.PE_POS_BF16
    if position_dtype == torch.float16:
        return _lib.PE_POS_FP16
    raise ValueError(f"position_dtype must be None, torch.float32, torch.bfloat16 or torch.float16, "
                     f"got {position_dtype}")


def _shape_error(msg: str) -> ValueError:
    return ValueError(f"pe_attention: {msg}")


def check_operands(q, k, v, q_c=None, k_c=None, freqs=None, delta=None, *, mode: int,
                   q_norm_weight=None, k_norm_weight=None) -> None:
    """Shape and device agreement of every operand, checked before anything is enqueued.

    The C ABI sees pointers and strides only, so a short freqs, a CPU delta or a v with fewer rows
    than k would otherwise reach the kernels as an out-of-bounds read or write.  The reference's
    torch ops raise on the same mismatches (src/model/fpope_attention.py:145-177 concatenates and
    multiplies these tensors), so this raises ValueError instead.  q (B,Hq,Sq,Dr), k (B,Hkv,Sk,Dr),
    v (B,Hkv,Sk,Dv), q_c (B,Hq,Sq,Dc) and k_c (B,Hkv,Sk,Dc) together or not at all; freqs (Dr,)
    for PoPE / FoPE, (Dr/2,) for RoPE; delta (Dr,) or (Hkv,Dr); norm weights (Hq*Dr,) / (Hkv*Dr,).
    Every tensor must sit on q's device."""
    for name, t in (("q", q), ("k", k), ("v", v), ("q_c", q_c), ("k_c", k_c)):
        if t is not None and t.dim() != 4:
            raise _shape_error(f"{name} must be (B, H, S, D), got shape {tuple(t.shape)}")
    B, Hq, Sq, Dr = q.shape
    if k.shape[0] != B or k.shape[3] != Dr:
        raise _shape_error(f"k {tuple(k.shape)} must match q {tuple(q.shape)} in batch and width")
    Hkv, Sk = k.shape[1], k.shape[2]
    if Hkv == 0 or Hq % Hkv != 0:
        raise _shape_error(f"query heads {Hq} must be a multiple of key heads {Hkv}")
    if tuple(v.shape[:3]) != (B, Hkv, Sk):
        raise _shape_error(f"v {tuple(v.shape)} must be (B, Hkv, Sk, Dv) = ({B}, {Hkv}, {Sk}, Dv)")
    if (q_c is None) != (k_c is None):
        raise _shape_error("pass q_c and k_c together (content dims on both sides) or neither")
    if q_c is not None:
        if tuple(q_c.shape[:3]) != (B, Hq, Sq) or tuple(k_c.shape[:3]) != (B, Hkv, Sk):
            raise _shape_error(f"q_c {tuple(q_c.shape)} / k_c {tuple(k_c.shape)} must share the rows of q / k")
        if q_c.shape[3] != k_c.shape[3]:
            raise _shape_error(f"q_c and k_c widths differ ({q_c.shape[3]} vs {k_c.shape[3]})")
    if mode == _lib.PE_MODE_POPE or mode == _lib.PE_MODE_ROPE:
        want = Dr if mode == _lib.PE_MODE_POPE else Dr // 2
        if freqs is None or freqs.dim() != 1 or freqs.shape[0] != want:
            got = None if freqs is None else tuple(freqs.shape)
            raise _shape_error(f"freqs must have shape ({want},) for this mode, got {got}")
    if delta is not None:
        if mode != _lib.PE_MODE_POPE:
            raise _shape_error("delta (phase bias) only applies to PoPE/FoPE")
        if not (tuple(delta.shape) == (Dr,) or tuple(delta.shape) == (Hkv, Dr)):
            raise _shape_error(f"delta must be ({Dr},) or ({Hkv}, {Dr}), got {tuple(delta.shape)}")
    if q_norm_weight is not None and tuple(q_norm_weight.shape) != (Hq * Dr,):
        raise _shape_error(f"qr_norm_weight must be ({Hq * Dr},), got {tuple(q_norm_weight.shape)}")
    if k_norm_weight is not None and tuple(k_norm_weight.shape) != (Hkv * Dr,):
        raise _shape_error(f"kr_norm_weight must be ({Hkv * Dr},), got {tuple(k_norm_weight.shape)}")
    dev = q.device
    for name, t in (("k", k), ("v", v), ("q_c", q_c), ("k_c", k_c), ("freqs", freqs), ("delta", delta),
                    ("qr_norm_weight", q_norm_weight), ("kr_norm_weight", k_norm_weight)):
        if t is not None and t.device != dev:
            raise _shape_error(f"{name} is on {t.device}, q on {dev}: every operand must be on one device")


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(dev: torch.device):
    """The current stream of dev as a raw hipStream_t (torch's raw-stream query when it has one)."""
    if _raw_stream is not None:
        return _raw_stream(dev.index)
    return torch.cuda.current_stream(dev).cuda_stream


def _on(dev: torch.device):
    """Make dev current for the library call (a no-op context when it already is)."""
    if dev.index == torch.cuda.current_device():
        return contextlib.nullcontext()
    return torch.cuda.device(dev)


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else t.data_ptr()


def _sig(t: Optional[torch.Tensor]):
    return None if t is None else (tuple(t.shape), t.stride(), t.dtype, t.device)


class _Desc:
    """A PeTensor descriptor whose shape, strides and dtype are fixed by a launch plan's key; only
    the data pointer changes from call to call."""
    __slots__ = ("t", "ref")

    def __init__(self, t: Optional[torch.Tensor]):
        self.t = _tensor(t)
        self.ref = ctypes.byref(self.t)

    def bind(self, x: Optional[torch.Tensor]):
        if x is not None:
            self.t.data = x.data_ptr()
        return self.ref


class _FwdPlan:
    """Per-signature launch state of PEAttentionFn: the parameter block (checked once), the
    workspace sizes and the tensor descriptors.  Backward plans hang off it, keyed by dout's
    signature and the gradients needed."""
    __slots__ = ("p", "pref", "ws", "cdt", "out_shape", "d", "bwd")

    def __init__(self, cfg, qr, kr, v, qc, kc, delta):
        L = _lib.lib()
        self.p = _params(cfg, qr, kr, v, qc, delta)
        self.pref = ctypes.byref(self.p)
        _lib.check(L.pe_attn_check(self.pref))
        self.ws = L.pe_attn_fwd_workspace_bytes(self.pref)
        self.cdt = _TORCH_DTYPE[cfg["dtype"]]
        B, Hq, Sq, Dv = qr.shape[0], qr.shape[1], qr.shape[2], v.shape[3]
        self.out_shape = (B, Sq, Hq, Dv)
        out = torch.empty(self.out_shape, dtype=self.cdt, device=qr.device).transpose(1, 2)
        self.d = [_Desc(t) for t in (qc, qr, kc, kr, v, out)]
        self.bwd = {}


class _BwdPlan:
    __slots__ = ("bws", "d")

    def __init__(self, fp: _FwdPlan, tensors, masked: bool = False):
        L = _lib.lib()
        self.bws = (L.pe_attn_bwd_masked_workspace_bytes if masked else L.pe_attn_bwd_workspace_bytes)(fp.pref)
        self.d = [_Desc(t) for t in tensors]


def _mask_view(mask, B, Hq, Sq, Sk, dev, dt) -> torch.Tensor:
    """SDPA's attn_mask (src/model/attention.py:91-96) as the (B, Hq, Sq, Sk) view the library reads:
    bool (True = the key takes part) or a float added to the scaled score, broadcast by stride 0
    (torch's expand, no copy).  Under autocast a float mask is rounded to the autocast dtype, as
    autocast rounds SDPA's floating-point inputs."""
    if not isinstance(mask, torch.Tensor):
        raise TypeError(f"mask must be a tensor, got {type(mask).__name__}")
    if mask.device != dev:
        raise ValueError(f"mask is on {mask.device}, the operands on {dev}")
    if mask.requires_grad and torch.is_grad_enabled():
        raise NotImplementedError("pe_attention: no gradient flows to an explicit mask; pass mask.detach()")
    if mask.dtype != torch.bool:
        if not mask.is_floating_point():
            raise TypeError(f"mask must be bool or floating point (SDPA's attn_mask), got {mask.dtype}")
        if torch.is_autocast_enabled() and dt != _lib.PE_DTYPE_FP32:
            mask = mask.to(_TORCH_DTYPE[dt])
        elif mask.dtype not in (torch.bfloat16, torch.float16, torch.float32):
            mask = mask.float()
    try:
        return mask.expand(B, Hq, Sq, Sk)
    except RuntimeError as e:
        raise ValueError(f"mask of shape {tuple(mask.shape)} does not broadcast to {(B, Hq, Sq, Sk)}") from e


def _mask_desc(m: torch.Tensor) -> _lib.PeTensor:
    d = _lib.PeTensor()
    d.data = m.data_ptr()
    d.dtype = _lib.PE_DTYPE_BOOL if m.dtype == torch.bool else _dtype_code(m.dtype)
    for i, st in enumerate(m.stride()):
        d.stride[i] = st
    return d


# Launch plans per thread (torch runs backward passes on its own device thread), keyed by the
# operands' shapes, strides, dtypes and devices and the call's options; rebuilt from scratch when
# the table grows past _PLAN_LIMIT (e.g. many distinct KV-cache start positions).
_tls = threading.local()
_PLAN_LIMIT = 256


def _plans() -> dict:
    d = getattr(_tls, "plans", None)
    if d is None or len(d) > _PLAN_LIMIT:
        d = _tls.plans = {}
    return d


class PEAttentionFn(torch.autograd.Function):
    """forward(qr, kr, v, qc, kc, freqs, delta, cfg) -> out (B, Hq, Sq, Dv).

    Saves the raw inputs, out, lse and the forward workspace (transformed operands); the backward
    recomputes P from lse.  Gradients: qr, kr, v, qc, kc, freqs (PoPE/FoPE), delta."""

    @staticmethod
    def forward(ctx, qr, kr, v, qc, kc, freqs, delta, cfg):
        return _attn_forward(ctx, qr, kr, v, qc, kc, freqs, delta, cfg)

    @staticmethod
    def backward(ctx, dout, _dlse):
        qr, kr, v, qc, kc, freqs, delta, out, lse, fws = ctx.saved_tensors
        grads = _attn_backward(ctx.key, ctx.cfg, qr, kr, v, qc, kc, freqs, delta, out, lse, fws, dout,
                               freqs is not None and ctx.needs_input_grad[5],
                               delta is not None and ctx.needs_input_grad[6])
        return grads + (None,)


class PEMaskedAttentionFn(torch.autograd.Function):
    """PEAttentionFn with an explicit mask: forward(qr, kr, v, qc, kc, freqs, delta, mask, cfg), mask
    the (B, Hq, Sq, Sk) view of _mask_view, through pe_attn_fwd_masked / pe_attn_bwd_masked.  The
    mask gets no gradient."""

    @staticmethod
    def forward(ctx, qr, kr, v, qc, kc, freqs, delta, mask, cfg):
        return _attn_forward(ctx, qr, kr, v, qc, kc, freqs, delta, cfg, mask)

    @staticmethod
    def backward(ctx, dout, _dlse):
        qr, kr, v, qc, kc, freqs, delta, out, lse, fws, mask = ctx.saved_tensors
        grads = _attn_backward(ctx.key, ctx.cfg, qr, kr, v, qc, kc, freqs, delta, out, lse, fws, dout,
                               freqs is not None and ctx.needs_input_grad[5],
                               delta is not None and ctx.needs_input_grad[6], mask=mask)
        return grads + (None, None)


def _attn_forward(ctx, qr, kr, v, qc, kc, freqs, delta, cfg, mask=None):
    """pe_attn_fwd (pe_attn_fwd_masked with a mask) for the autograd functions above; saves what
    _attn_backward needs and returns (out, lse)."""
    L = _lib.lib()
    dev = qr.device
    key = (cfg["key"], _sig(qr), _sig(kr), _sig(v), _sig(qc), _sig(kc),
           None if delta is None else delta.dim())
    plans = _plans()
    fp = plans.get(key)
    if fp is None:
        fp = plans[key] = _FwdPlan(cfg, qr, kr, v, qc, kc, delta)
    fws = torch.empty(fp.ws, dtype=torch.uint8, device=dev)
    out = torch.empty(fp.out_shape, dtype=fp.cdt, device=dev).transpose(1, 2)
    lse = torch.empty((fp.out_shape[0], fp.out_shape[2], fp.out_shape[1]), dtype=torch.float32, device=dev)
    d = fp.d
    with _on(dev):
        if mask is None:
            rc = L.pe_attn_fwd(fp.pref, d[0].bind(qc), d[1].bind(qr), d[2].bind(kc), d[3].bind(kr), d[4].bind(v),
                               _ptr(freqs), _ptr(delta), d[5].bind(out), lse.data_ptr(), fws.data_ptr(), fp.ws,
                               _stream(dev))
        else:
            md = _mask_desc(mask)
            rc = L.pe_attn_fwd_masked(fp.pref, d[0].bind(qc), d[1].bind(qr), d[2].bind(kc), d[3].bind(kr),
                                      d[4].bind(v), _ptr(freqs), _ptr(delta), ctypes.byref(md), d[5].bind(out),
                                      lse.data_ptr(), fws.data_ptr(), fp.ws, _stream(dev))
    _lib.check(rc)
    ctx.cfg = cfg
    ctx.key = key
    saved = (qr, kr, v, qc, kc, freqs, delta, out, lse, fws)
    ctx.save_for_backward(*(saved if mask is None else saved + (mask,)))
    ctx.mark_non_differentiable(lse)
    # lse carries no gradient: without this, autograd fills a zero (B, Hq, Sq) tensor for it in
    # every backward
    ctx.set_materialize_grads(False)
    return out, lse


def _attn_backward(key, cfg, qr, kr, v, qc, kc, freqs, delta, out, lse, fws, dout, need_f, need_d, mask=None):
    """pe_attn_bwd (pe_attn_bwd_masked with a mask) for a forward saved as (qr, kr, v, qc, kc, freqs,
    delta, out, lse, workspace): returns (dqr, dkr, dv, dqc, dkc, dfreqs, ddelta), each gradient in
    its input's dtype."""
    L = _lib.lib()
    dev = qr.device
    plans = _plans()
    fp = plans.get(key)
    if fp is None:
        fp = plans[key] = _FwdPlan(cfg, qr, kr, v, qc, kc, delta)
    if dout is None:  # out was not used by the loss either
        dout = torch.zeros_like(out)
    if dout.stride(-1) != 1:
        dout = dout.contiguous()
    if dout.dtype not in (torch.bfloat16, torch.float32, torch.float16):
        dout = dout.float()
    dqr, dkr = torch.empty_like(qr), torch.empty_like(kr)
    dqc = None if qc is None else torch.empty_like(qc)
    dkc = None if kc is None else torch.empty_like(kc)
    cdt = fp.cdt
    dv = torch.empty_like(v, dtype=cdt) if v.dtype != cdt else torch.empty_like(v)
    dfreqs = torch.empty(freqs.shape, dtype=torch.float32, device=dev) if need_f else None
    ddelta = torch.empty(delta.shape, dtype=torch.float32, device=dev) if need_d else None
    bkey = (_sig(dout), _sig(dqr), _sig(dkr), _sig(dqc), _sig(dkc), _sig(dv), mask is not None)
    bp = fp.bwd.get(bkey)
    if bp is None:
        bp = fp.bwd[bkey] = _BwdPlan(fp, (qc, qr, kc, kr, v, out, dout, dqc, dqr, dkc, dkr, dv), mask is not None)
    bws = torch.empty(bp.bws, dtype=torch.uint8, device=dev)
    d = bp.d
    with _on(dev):
        if mask is None:
            rc = L.pe_attn_bwd(fp.pref, d[0].bind(qc), d[1].bind(qr), d[2].bind(kc), d[3].bind(kr), d[4].bind(v),
                               _ptr(freqs), _ptr(delta), d[5].bind(out), lse.data_ptr(), d[6].bind(dout),
                               d[7].bind(dqc), d[8].bind(dqr), d[9].bind(dkc), d[10].bind(dkr), d[11].bind(dv),
                               _ptr(dfreqs), _ptr(ddelta), fws.data_ptr(), fp.ws, bws.data_ptr(), bp.bws,
                               _stream(dev))
        else:
            md = _mask_desc(mask)
            rc = L.pe_attn_bwd_masked(fp.pref, d[0].bind(qc), d[1].bind(qr), d[2].bind(kc), d[3].bind(kr),
                                      d[4].bind(v), _ptr(freqs), _ptr(delta), ctypes.byref(md), d[5].bind(out),
                                      lse.data_ptr(), d[6].bind(dout), d[7].bind(dqc), d[8].bind(dqr),
                                      d[9].bind(dkc), d[10].bind(dkr), d[11].bind(dv), _ptr(dfreqs),
                                      _ptr(ddelta), fws.data_ptr(), fp.ws, bws.data_ptr(), bp.bws, _stream(dev))
    _lib.check(rc)
    if dv.dtype != v.dtype:
        dv = dv.to(v.dtype)
    return dqr, dkr, dv, dqc, dkc, dfreqs, ddelta


def ref(x):
    import ctypes
    return ctypes.byref(x)


ctypes_ref = ref


def _compute_dtype(tensors) -> int:
    """The dtype SDPA would compute in: autocast's (fp16 or bf16) when autocast is on, else the
    inputs' 16-bit type (bf16 when both occur), else fp32."""
    if torch.is_autocast_enabled():
        return _lib.PE_DTYPE_FP16 if torch.get_autocast_dtype("cuda") == torch.float16 else _lib.PE_DTYPE_BF16
    dts = {t.dtype for t in tensors if t is not None}
    if torch.bfloat16 in dts:
        return _lib.PE_DTYPE_BF16
    if torch.float16 in dts:
        return _lib.PE_DTYPE_FP16
    return _lib.PE_DTYPE_FP32


def pe_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, mode: str = "pope",
                 q_c: Optional[torch.Tensor] = None, k_c: Optional[torch.Tensor] = None,
                 freqs: Optional[torch.Tensor] = None, delta: Optional[torch.Tensor] = None,
                 scale: Optional[float] = None, causal=True, start_pos_q: int = 0,
                 start_pos_k: int = 0, rope_mscale: float = 1.0, qk_norm: bool = False,
                 return_lse: bool = False, compute_dtype: Optional[torch.dtype] = None,
                 qr_norm_weight: Optional[torch.Tensor] = None, kr_norm_weight: Optional[torch.Tensor] = None,
                 norm_eps: float = 1e-6, position_dtype: Optional[torch.dtype] = None,
                 mask: Optional[torch.Tensor] = None):
    """Fused PE attention on one GPU.

    q (B,Hq,Sq,Dr), k (B,Hkv,Sk,Dr): positional parts, transformed inside the kernel library;
    q_c/k_c optional content parts (Dc) placed ahead of them; v (B,Hkv,Sk,Dv).
    mode "pope"/"fope": freqs (Dr,) per-dim frequency, delta key phase bias ((Dr,) shared or
    (Hkv, Dr) per head) used as given (clamping is the caller's autograd op).
    mode "rope": freqs (Dr/2,) inverse frequencies, rope_mscale (YaRN), qk_norm (QKNorm).
    scale defaults to (Dc + Dqk)^-1/2 with Dqk = 2 Dr (PoPE) or Dr.
    causal: True / "top_left" (SDPA is_causal), "bottom_right" (KV-cache mask) or False.
    qr_norm_weight / kr_norm_weight (PoPE only): q / k are the raw position projections and the
    library applies the modules' RMSNorm over each token's H*Dr features in the transform kernel
    (pe_attn_fwd_normed); with a gradient needed the backward also runs the norm's backward
    (PENormedAttentionFn), giving the gradients of the raw projections and of the norm weights.
    position_dtype (PoPE / FoPE): None or torch.float32 keeps positions exact; torch.bfloat16 /
    torch.float16 rounds each position to that type before the phase product (and in the phase
    gradient), reproducing FoPE's positions in x.dtype (src/model/fpope.py:285,322).
    mask: SDPA's attn_mask (src/model/attention.py:91-96), broadcastable to (B, Hq, Sq, Sk): bool
    (True = the key takes part) or a float added to the scaled score; applied together with
    ``causal`` (the reference module passes is_causal=False with a mask, so pass causal=False to
    match).  A row with every key masked gives zeros, as torch's SDPA does.  The mask gets no
    gradient; it does not combine with the fused norm.
    Returns out (B,Hq,Sq,Dv) [and lse (B,Hq,Sq) fp32]."""
    if mode not in _MODES:
        raise ValueError(f"unknown PE mode {mode!r}")
    if not q.is_cuda:
        raise RuntimeError("pe_attention runs on the GPU only (got a CPU tensor); "
                           "the HIP kernels have no CPU path")
    m = _MODES[mode]
    check_operands(q, k, v, q_c, k_c, freqs if m != _lib.PE_MODE_NONE else None, delta, mode=m,
                   q_norm_weight=qr_norm_weight, k_norm_weight=kr_norm_weight)
    q, k, v, q_c, k_c = (_prep_in(t) for t in (q, k, v, q_c, k_c))
    if m != _lib.PE_MODE_NONE:
        if freqs is None:
            raise ValueError(f"mode {mode!r} needs freqs")
        freqs = freqs.float().contiguous()
    else:
        freqs = None
    if delta is not None:
        if m != _lib.PE_MODE_POPE:
            raise ValueError("delta (phase bias) only applies to PoPE/FoPE")
        delta = delta.float().contiguous()
    Dc = 0 if q_c is None else q_c.shape[-1]
    dqk = Dc + (2 * q.shape[-1] if m == _lib.PE_MODE_POPE else q.shape[-1])
    if scale is None:
        scale = dqk ** -0.5
    if compute_dtype is None:
        dt = _compute_dtype((q, k, v, q_c, k_c))
    else:
        dt = _dtype_code(compute_dtype)
    if dt != _lib.PE_DTYPE_FP32:
        # the other 16-bit type goes in as fp32 (exact); the kernels round it to the compute's
        q, k, v, q_c, k_c = (t.float() if t is not None and t.dtype in _HALF and t.dtype != _TORCH_DTYPE[dt]
                             else t for t in (q, k, v, q_c, k_c))
    cfg = dict(mode=m, dtype=dt, causal=_CAUSAL[causal], start_pos_q=int(start_pos_q),
               start_pos_k=int(start_pos_k), qk_norm=bool(qk_norm), scale=float(scale),
               mscale=float(rope_mscale), pos_round=position_rounding(position_dtype, m))
    cfg["key"] = tuple(cfg.values())
    if mask is not None:
        if qr_norm_weight is not None or kr_norm_weight is not None:
            raise ValueError("pe_attention: an explicit mask does not combine with the fused norm")
        mview = _mask_view(mask, q.shape[0], q.shape[1], q.shape[2], k.shape[2], q.device, dt)
        out, lse = PEMaskedAttentionFn.apply(q, k, v, q_c, k_c, freqs, delta, mview, cfg)
    elif qr_norm_weight is not None or kr_norm_weight is not None:
        out, lse = _fwd_normed(q, k, v, q_c, k_c, freqs, delta, cfg, qr_norm_weight, kr_norm_weight, norm_eps)
    else:
        out, lse = PEAttentionFn.apply(q, k, v, q_c, k_c, freqs, delta, cfg)
    return (out, lse) if return_lse else out


def default_pope_scale(d: int) -> float:
    """1/sqrt(D), D the pre-transform head dim (legacy fused API, tests/test_fpope.py:1537)."""
    return 1.0 / math.sqrt(d)


def _fwd_normed(qr, kr, v, qc, kc, freqs, delta, cfg, wq, wk, eps):
    """Forward through pe_attn_fwd_normed: RMSNorm of the raw position projections fused into the
    PoPE prologue.  With a gradient needed it runs as PENormedAttentionFn, whose backward applies
    the attention backward to the normalised projections and then the norm's backward
    (pe_rmsnorm_bwd); otherwise no graph is recorded."""
    if cfg["mode"] != _lib.PE_MODE_POPE:
        raise ValueError("the fused position-projection RMSNorm applies to PoPE / FoPE only")
    if wq is None or wk is None:
        raise ValueError("pass both qr_norm_weight and kr_norm_weight")
    if wq.dtype != wk.dtype or wq.dtype not in (torch.bfloat16, torch.float32, torch.float16):
        raise TypeError("qr/kr norm weights must share one dtype, bf16, fp16 or fp32")
    if torch.is_grad_enabled() and any(t is not None and t.requires_grad
                                       for t in (qr, kr, v, qc, kc, freqs, delta, wq, wk)):
        return PENormedAttentionFn.apply(qr, kr, v, qc, kc, freqs, delta, wq, wk, cfg, float(eps))
    out, lse, _ = _launch_normed(qr, kr, v, qc, kc, freqs, delta, cfg, wq, wk, eps)
    return out, lse


def _launch_normed(qr, kr, v, qc, kc, freqs, delta, cfg, wq, wk, eps):
    L = _lib.lib()
    dev = qr.device
    wq, wk = wq.contiguous(), wk.contiguous()
    p = _params(cfg, qr, kr, v, qc, delta)
    _lib.check(L.pe_attn_check(ctypes_ref(p)))
    n = _lib.PeNormParams()
    n.q_weight, n.k_weight = wq.data_ptr(), wk.data_ptr()
    n.weight_dtype, n.eps = _dtype_code(wq.dtype), float(eps)
    cdt = _TORCH_DTYPE[cfg["dtype"]]
    B, Hq, Sq, Dv = qr.shape[0], qr.shape[1], qr.shape[2], v.shape[3]
    ws_bytes = L.pe_attn_fwd_workspace_bytes(ctypes_ref(p))
    fws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    out = torch.empty((B, Sq, Hq, Dv), dtype=cdt, device=dev).transpose(1, 2)
    lse = torch.empty((B, Hq, Sq), dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        rc = L.pe_attn_fwd_normed(ctypes_ref(p), ctypes_ref(n), ref(_tensor(qc)), ref(_tensor(qr)),
                                  ref(_tensor(kc)), ref(_tensor(kr)), ref(_tensor(v)), _ptr(freqs), _ptr(delta),
                                  ref(_tensor(out)), lse.data_ptr(), fws.data_ptr(), ws_bytes, _stream(dev))
    _lib.check(rc)
    return out, lse, fws


def _token_rows(x: torch.Tensor) -> torch.Tensor:
    """(B, H, S, D) view of a projection -> its (B * S, H * D) token rows (a view when x is the
    (B, S, H, D) transpose the modules pass, else a copy)."""
    B, H, S, D = x.shape
    return x.transpose(1, 2).reshape(B * S, H * D)


class PENormedAttentionFn(torch.autograd.Function):
    """forward(qr, kr, v, qc, kc, freqs, delta, wq, wk, cfg, eps) -> (out, lse): the modules'
    RMSNorm of the raw position projections qr / kr over each token's H*Dr features
    (src/model/fpope_attention.py:132-137, src/model/normalization.py:22-27) fused into the PoPE
    prologue (pe_attn_fwd_normed).  The backward recomputes the normalised projections y with
    pe_rmsnorm_fwd (the prologue's arithmetic and summation order, so bitwise the y it used), runs
    pe_attn_bwd on y, and turns the gradient of y into those of the raw projections and the norm
    weights with pe_rmsnorm_bwd.  Gradients: qr, kr, v, qc, kc, freqs, delta, wq, wk."""

    @staticmethod
    def forward(ctx, qr, kr, v, qc, kc, freqs, delta, wq, wk, cfg, eps):
        out, lse, fws = _launch_normed(qr, kr, v, qc, kc, freqs, delta, cfg, wq, wk, eps)
        ctx.cfg, ctx.eps = cfg, eps
        ctx.save_for_backward(qr, kr, v, qc, kc, freqs, delta, wq, wk, out, lse, fws)
        ctx.mark_non_differentiable(lse)
        ctx.set_materialize_grads(False)
        return out, lse

    @staticmethod
    def backward(ctx, dout, _dlse):
        qr, kr, v, qc, kc, freqs, delta, wq, wk, out, lse, fws = ctx.saved_tensors
        B, Hq, Sq, Dr = qr.shape
        Hkv, Sk = kr.shape[1], kr.shape[2]
        xq, xk = _token_rows(qr), _token_rows(kr)
        yq = rms_norm(xq, wq, ctx.eps).view(B, Sq, Hq, Dr).transpose(1, 2)
        yk = rms_norm(xk, wk, ctx.eps).view(B, Sk, Hkv, Dr).transpose(1, 2)
        key = ("normed-bwd", ctx.cfg["key"], _sig(yq), _sig(yk), _sig(v), _sig(qc), _sig(kc),
               None if delta is None else delta.dim())
        dyq, dyk, dv, dqc, dkc, dfreqs, ddelta = _attn_backward(
            key, ctx.cfg, yq, yk, v, qc, kc, freqs, delta, out, lse, fws, dout,
            freqs is not None and ctx.needs_input_grad[5], delta is not None and ctx.needs_input_grad[6])
        dxq, dwq = rms_norm_backward(xq, wq, _token_rows(dyq), ctx.eps)
        dxk, dwk = rms_norm_backward(xk, wk, _token_rows(dyk), ctx.eps)
        dqr = dxq.view(B, Sq, Hq, Dr).transpose(1, 2)
        dkr = dxk.view(B, Sk, Hkv, Dr).transpose(1, 2)
        return dqr, dkr, dv, dqc, dkc, dfreqs, ddelta, dwq, dwk, None, None


def rms_norm_backward(x: torch.Tensor, weight: torch.Tensor, dy: torch.Tensor, eps: float = 1e-6):
    """Gradients (dx, dweight) of rms_norm(x, weight, eps) for the output gradient dy, as autograd
    computes them through the reference module (src/model/normalization.py:22-27), through
    pe_rmsnorm_bwd: (rows, n) views with unit element stride; dy in rms_norm's output dtype; dx in
    x's dtype, dweight in weight's dtype (summed over the rows in a fixed order)."""
    if not x.is_cuda:
        raise RuntimeError("rms_norm_backward runs on the GPU only (got a CPU tensor)")
    n = x.shape[-1]
    ydt = norm_out_dtype(x.dtype, weight.dtype)
    x2 = x.reshape(-1, n)
    dy2 = dy.reshape(-1, n).to(ydt)
    if x2.stride(-1) != 1 or x2.data_ptr() % 16 or x2.stride(0) % (8 if x.dtype in _HALF else 4):
        x2 = x2.contiguous()
    if dy2.stride(-1) != 1 or dy2.data_ptr() % 16 or dy2.stride(0) % (8 if ydt in _HALF else 4):
        dy2 = dy2.contiguous()
    w = weight.contiguous()
    dx = torch.empty((x2.shape[0], n), dtype=x.dtype, device=x.device)
    dw = torch.empty(n, dtype=weight.dtype, device=x.device)
    if x2.shape[0] == 0:
        return dx.view(x.shape), dw.zero_()
    L = _lib.lib()
    ws = L.pe_rmsnorm_bwd_workspace_bytes(x2.shape[0], n)
    part = torch.empty(ws, dtype=torch.uint8, device=x.device)
    with _on(x.device):
        rc = L.pe_rmsnorm_bwd(x2.data_ptr(), _dtype_code(x2.dtype), x2.stride(0), x2.shape[0], n, w.data_ptr(),
                              _dtype_code(w.dtype), float(eps), dy2.data_ptr(), dy2.stride(0), dx.data_ptr(),
                              dx.stride(0), dw.data_ptr(), part.data_ptr(), ws, _stream(x.device))
    _lib.check(rc)
    return dx.view(x.shape), dw


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """RMSNorm forward over the last dim through pe_rmsnorm_fwd (src/model/normalization.py:22-27):
    (x * rsqrt(mean(x^2) + eps)).type_as(x) * weight, result dtype bf16 when x and weight are both
    bf16, else fp32.  No autograd: the module uses it when no gradient is needed."""
    if not x.is_cuda:
        raise RuntimeError("rms_norm runs on the GPU only (got a CPU tensor)")
    if x.dtype not in (torch.bfloat16, torch.float32, torch.float16) or \
            weight.dtype not in (torch.bfloat16, torch.float32, torch.float16):
        raise TypeError("rms_norm supports bf16 / fp16 / fp32 tensors")
    n = x.shape[-1]
    x2 = x.reshape(-1, n)
    if x2.stride(-1) != 1 or x2.data_ptr() % 16 or x2.stride(0) % (8 if x.dtype in _HALF else 4):
        x2 = x2.contiguous()
    w = weight.contiguous()
    ydt = norm_out_dtype(x.dtype, w.dtype)
    y = torch.empty((x2.shape[0], n), dtype=ydt, device=x.device)
    if x2.shape[0] == 0:
        return y.view(*x.shape[:-1], n)
    L = _lib.lib()
    with torch.cuda.device(x.device):
        rc = L.pe_rmsnorm_fwd(x2.data_ptr(), _dtype_code(x2.dtype), x2.stride(0), x2.shape[0], n,
                              w.data_ptr(), _dtype_code(w.dtype), float(eps), y.data_ptr(), _dtype_code(ydt),
                              y.stride(0), _stream(x.device))
    _lib.check(rc)
    return y.view(*x.shape[:-1], n)


def swiglu(x: torch.Tensor, gate: torch.Tensor) -> torch.Tensor:
    """F.silu(gate) * x over bf16 through pe_swiglu_fwd (src/model/ffn.py:17-27), bitwise torch's
    result for the two bf16 ops, in one pass.  Both tensors bf16, same shape, on the GPU.  No
    autograd: the module uses it when no gradient is needed."""
    if not (x.is_cuda and gate.is_cuda):
        raise RuntimeError("swiglu runs on the GPU only")
    if x.dtype != torch.bfloat16 or gate.dtype != torch.bfloat16 or x.shape != gate.shape:
        raise TypeError("swiglu takes two bf16 tensors of one shape")
    if x.device != gate.device:
        raise ValueError("swiglu: x and gate are on different devices")
    xc, gc = x.contiguous(), gate.contiguous()
    out = torch.empty_like(xc)
    n = xc.numel()
    if n % 8 or xc.data_ptr() % 16 or gc.data_ptr() % 16:
        return torch.nn.functional.silu(gate) * x
    if n:
        with torch.cuda.device(x.device):
            _lib.check(_lib.lib().pe_swiglu_fwd(xc.data_ptr(), gc.data_ptr(), out.data_ptr(), n, _stream(x.device)))
    return out


# ------------------------------------------------------------------------------------------------
# KV cache (src/model/fpope_attention.py:226-327): caches of transformed keys and values, and the
# split-key decode attention over them, without gradients (the modules' cache path under autograd is
# fpope_attention._cached_attention_autograd).

def _cache_params(*, B, Hq, Hkv, Sq, Sk, Dc, Dr, Dv, mode, dtype, causal, start_q, start_k, scale,
                  mscale, qk_norm, delta, pos_round=0) -> _lib.PeParams:
    p = _lib.PeParams()
    p.B, p.Hq, p.Hkv, p.Sq, p.Sk = B, Hq, Hkv, Sq, Sk
    p.Dc, p.Dr, p.Dv = Dc, Dr, Dv
    p.mode, p.dtype, p.causal = mode, dtype, causal
    p.start_pos_q, p.start_pos_k = int(start_q), int(start_k)
    p.qk_l2norm = int(qk_norm)
    p.scale, p.rope_mscale = float(scale), float(mscale)
    p.delta_head_stride = 0 if (delta is None or delta.dim() == 1) else delta.shape[-1]
    p.position_rounding = pos_round
    return p


def cache_widths(*, mode: str = "pope", d_content: int = 0, d_pe: int, d_v: int) -> tuple[int, int]:
    """(key width, value width) of the cache rows pe_cache_append writes: the library's transformed
    operand rows [content | transform | zero pad] and the zero-padded value rows."""
    m = _MODES[mode]
    p = _cache_params(B=1, Hq=1, Hkv=1, Sq=1, Sk=1, Dc=d_content, Dr=d_pe, Dv=d_v, mode=m,
                      dtype=_lib.PE_DTYPE_BF16, causal=_lib.PE_CAUSAL_NONE, start_q=0, start_k=0, scale=1.0,
                      mscale=1.0, qk_norm=False, delta=None)
    L = _lib.lib()
    _lib.check(L.pe_attn_check(ref(p)))
    return L.pe_attn_operand_width(ref(p)), L.pe_attn_value_width(ref(p))


def _check_cache(k_cache, v_cache, B, Hkv, wk, wv, cdt, dev):
    for name, c, wdt in (("k_cache", k_cache, wk), ("v_cache", v_cache, wv)):
        if c.dim() != 4 or tuple(c.shape[:2]) != (B, Hkv) or c.shape[3] != wdt:
            raise ValueError(f"{name} must be (B, Hkv, capacity, {wdt}) = ({B}, {Hkv}, C, {wdt}), got {tuple(c.shape)}")
        if not c.is_contiguous() or c.dtype != cdt or c.device != dev or c.data_ptr() % 16:
            raise ValueError(f"{name} must be a contiguous, 16-byte aligned {cdt} tensor on {dev}")
    if k_cache.shape[2] != v_cache.shape[2]:
        raise ValueError("k_cache and v_cache capacities differ")


class _AppendPlan:
    """Per-signature launch state of pe_cache_append: the parameter block (checked once against the
    caches) and the tensor descriptors; a call sets the start position and swaps the pointers."""
    __slots__ = ("p", "pref", "dk", "dv", "dkc", "S", "cap")

    def __init__(self, p, k, v, k_c, S, cap):
        self.p = p
        self.pref = ref(p)
        self.dk, self.dv, self.dkc = _Desc(k), _Desc(v), _Desc(k_c)
        self.S, self.cap = S, cap


def pe_cache_append(k: torch.Tensor, v: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, *,
                    start_pos: int, mode: str = "pope", k_c: Optional[torch.Tensor] = None,
                    freqs: Optional[torch.Tensor] = None, delta: Optional[torch.Tensor] = None,
                    rope_mscale: float = 1.0, qk_norm: bool = False,
                    position_dtype: Optional[torch.dtype] = None) -> None:
    """Write the transformed key rows of k (B, Hkv, S, Dr) [with content k_c (B, Hkv, S, Dc)] and
    the value rows v (B, Hkv, S, Dv) to cache rows start_pos .. start_pos + S - 1, phases at those
    positions (the reference's k_cache[:, :, start_pos:start_pos+S] = [k_c | PoPE(k_r)],
    src/model/fpope_attention.py:294-296).  The caches are (B, Hkv, capacity, width) in the compute
    dtype with the widths of ``cache_widths``.  Shapes, strides, dtypes and devices are checked
    once per operand signature (one token per step keeps the same signature), the rows to write
    on every call."""
    if torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in (k, v, k_c, freqs, delta)):
        raise RuntimeError("the KV-cache path is inference only (run it under torch.no_grad())")
    if not k.is_cuda:
        raise RuntimeError("pe_cache_append runs on the GPU only (got a CPU tensor)")
    m = _MODES[mode]
    k, v, k_c = (_prep_in(t) for t in (k, v, k_c))
    freqs = freqs.float().contiguous() if m != _lib.PE_MODE_NONE and freqs is not None else None
    delta = None if delta is None else delta.float().contiguous()
    pos_round = position_rounding(position_dtype, m)
    key = ("append", m, _sig(k), _sig(v), _sig(k_c), _sig(freqs), _sig(delta), _sig(k_cache), _sig(v_cache),
           float(rope_mscale), bool(qk_norm), pos_round)
    plans = _plans()
    ap = plans.get(key)
    L = _lib.lib()
    if ap is None:
        check_operands(k, k, v, k_c, k_c, freqs if m != _lib.PE_MODE_NONE else None, delta, mode=m)
        if m != _lib.PE_MODE_NONE and freqs is None:
            raise ValueError("freqs is required for a positional mode")
        B, Hkv, S, Dr = k.shape
        Dc = 0 if k_c is None else k_c.shape[-1]
        cdt = k_cache.dtype
        p = _cache_params(B=B, Hq=Hkv, Hkv=Hkv, Sq=S, Sk=S, Dc=Dc, Dr=Dr, Dv=v.shape[-1], mode=m,
                          dtype=_dtype_code(cdt), causal=_lib.PE_CAUSAL_NONE, start_q=0, start_k=0, scale=1.0,
                          mscale=rope_mscale, qk_norm=qk_norm, delta=delta, pos_round=pos_round)
        _lib.check(L.pe_attn_check(ref(p)))
        _check_cache(k_cache, v_cache, B, Hkv, L.pe_attn_operand_width(ref(p)), L.pe_attn_value_width(ref(p)), cdt,
                     k.device)
        ap = plans[key] = _AppendPlan(p, k, v, k_c, S, k_cache.shape[2])
    if start_pos < 0 or start_pos + ap.S > ap.cap:
        raise ValueError(f"rows {start_pos}..{start_pos + ap.S - 1} do not fit a cache of capacity {ap.cap}")
    ap.p.start_pos_q = ap.p.start_pos_k = int(start_pos)
    with _on(k.device):
        rc = L.pe_attn_cache_append(ap.pref, ap.dkc.bind(k_c), ap.dk.bind(k), ap.dv.bind(v), _ptr(freqs),
                                    _ptr(delta), k_cache.data_ptr(), v_cache.data_ptr(), ap.cap, _stream(k.device))
    _lib.check(rc)


class _DecodePlan:
    """Per-signature launch state of pe_attention_decode: the parameter block, the descriptors and a
    workspace sized for the whole cache (the largest any cache length needs), reused by every call
    on the same stream; a call sets the cache length and the query position and swaps pointers."""
    __slots__ = ("p", "pref", "dq", "dqc", "dout", "lse", "ws", "nb", "cap", "out_shape", "cdt")

    def __init__(self, p, q, q_c, out, cap, out_shape, cdt, L):
        self.p = p
        self.pref = ref(p)
        self.dq, self.dqc, self.dout = _Desc(q), _Desc(q_c), _Desc(out)
        self.cap, self.out_shape, self.cdt = cap, out_shape, cdt
        p.Sk = cap
        self.nb = L.pe_attn_decode_workspace_bytes(self.pref)
        self.ws = torch.empty(self.nb, dtype=torch.uint8, device=q.device)
        self.lse = torch.empty((out_shape[0], out_shape[2], out_shape[1]), dtype=torch.float32, device=q.device)


def pe_attention_decode(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, cache_len: int, *,
                        d_v: int, mode: str = "pope", q_c: Optional[torch.Tensor] = None,
                        freqs: Optional[torch.Tensor] = None, scale: Optional[float] = None,
                        causal="bottom_right", start_pos_q: Optional[int] = None, rope_mscale: float = 1.0,
                        qk_norm: bool = False, return_lse: bool = False,
                        position_dtype: Optional[torch.dtype] = None):
    """Attention of the new queries q (B, Hq, Sq, Dr) [content q_c] against the first ``cache_len``
    rows of caches filled by pe_cache_append (src/model/fpope_attention.py:301-324): bottom-right
    causal mask by default, query phases at start_pos_q (default cache_len - Sq), GQA by index.
    position_dtype as for pe_attention (the cached keys must have been appended with the same).
    Returns out (B, Hq, Sq, d_v) in the cache dtype [and lse (B, Hq, Sq)].  Shapes, strides, dtypes
    and devices are checked once per operand signature and stream, whose workspace is then reused;
    cache_len and the query position on every call."""
    if torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in (q, q_c, freqs)):
        raise RuntimeError("the KV-cache path is inference only (run it under torch.no_grad())")
    if not q.is_cuda:
        raise RuntimeError("pe_attention_decode runs on the GPU only (got a CPU tensor)")
    m = _MODES[mode]
    q, q_c = _prep_in(q), _prep_in(q_c)
    freqs = freqs.float().contiguous() if m != _lib.PE_MODE_NONE and freqs is not None else None
    pos_round = position_rounding(position_dtype, m)
    dev = q.device
    stream = _stream(dev)
    key = ("decode", m, _sig(q), _sig(q_c), _sig(freqs), _sig(k_cache), _sig(v_cache), int(d_v),
           None if scale is None else float(scale), causal, float(rope_mscale), bool(qk_norm), pos_round, stream)
    plans = _plans()
    dp = plans.get(key)
    L = _lib.lib()
    if dp is None:
        if q.dim() != 4:
            raise ValueError(f"q must be (B, Hq, Sq, D), got shape {tuple(q.shape)}")
        if m != _lib.PE_MODE_NONE:
            want = q.shape[-1] if m == _lib.PE_MODE_POPE else q.shape[-1] // 2
            if freqs is None or freqs.dim() != 1 or freqs.shape[0] != want or freqs.device != dev:
                raise ValueError(f"freqs must be a ({want},) tensor on {dev}")
        if q_c is not None and (q_c.dim() != 4 or tuple(q_c.shape[:3]) != tuple(q.shape[:3]) or q_c.device != dev):
            raise ValueError(f"q_c {tuple(q_c.shape)} must share the rows of q {tuple(q.shape)}")
        B, Hq, Sq, Dr = q.shape
        Hkv = k_cache.shape[1]
        Dc = 0 if q_c is None else q_c.shape[-1]
        dqk = Dc + (2 * Dr if m == _lib.PE_MODE_POPE else Dr)
        sc = dqk ** -0.5 if scale is None else scale
        cdt = k_cache.dtype
        p = _cache_params(B=B, Hq=Hq, Hkv=Hkv, Sq=Sq, Sk=max(Sq, 1), Dc=Dc, Dr=Dr, Dv=d_v, mode=m,
                          dtype=_dtype_code(cdt), causal=_CAUSAL[causal], start_q=0, start_k=0, scale=sc,
                          mscale=rope_mscale, qk_norm=qk_norm, delta=None, pos_round=pos_round)
        _lib.check(L.pe_attn_check(ref(p)))
        _check_cache(k_cache, v_cache, B, Hkv, L.pe_attn_operand_width(ref(p)), L.pe_attn_value_width(ref(p)), cdt,
                     dev)
        out_shape = (B, Sq, Hq, d_v)
        probe = torch.empty(out_shape, dtype=cdt, device=dev).transpose(1, 2)
        dp = plans[key] = _DecodePlan(p, q, q_c, probe, k_cache.shape[2], out_shape, cdt, L)
    Sq = dp.out_shape[1]
    if cache_len > dp.cap:
        raise ValueError(f"cache_len {cache_len} exceeds the cache capacity {dp.cap}")
    dp.p.Sk = int(cache_len)
    dp.p.start_pos_q = int(cache_len - Sq if start_pos_q is None else start_pos_q)
    out = torch.empty(dp.out_shape, dtype=dp.cdt, device=dev).transpose(1, 2)
    lse = torch.empty_like(dp.lse) if return_lse else dp.lse
    with _on(dev):
        rc = L.pe_attn_decode(dp.pref, dp.dqc.bind(q_c), dp.dq.bind(q), k_cache.data_ptr(), v_cache.data_ptr(),
                              dp.cap, _ptr(freqs), dp.dout.bind(out), lse.data_ptr(), dp.ws.data_ptr(), dp.nb,
                              stream)
    _lib.check(rc)
    return (out, lse) if return_lse else out
