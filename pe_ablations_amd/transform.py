"""Standalone positional transform (PoPE/FoPE polar map or RoPE rotation) on the HIP library.

``pe_transform`` is what the drop-in embeddings' ``forward_query`` / ``forward_key`` / RoPE
``forward`` run (src/model/pope.py:124-183, src/model/fpope.py:266-338, src/model/rope.py:35-57):
pe_attn_transform forward, pe_attn_transform_bwd backward.  The fused attention never calls it;
it exists for callers that use the embeddings on their own.  Inputs are in the reference's
(B, S, H, D) layout; the output is a (B, S, H, W) view (W = 2D for PoPE, D for RoPE) of the
library's padded (B, H, S, width) buffer.
"""

from __future__ import annotations

import ctypes
from typing import Optional

import torch

from . import _lib
from .functional import position_rounding


def _params(B, H, S, D, mode, dtype, start_pos, delta, mscale, pos_round) -> _lib.PeParams:
    p = _lib.PeParams()
    p.B, p.Hq, p.Hkv, p.Sq, p.Sk = B, H, H, S, S
    p.Dc, p.Dr, p.Dv = 0, D, 64
    p.mode, p.dtype, p.causal = mode, dtype, _lib.PE_CAUSAL_NONE
    p.start_pos_q = p.start_pos_k = int(start_pos)
    p.qk_l2norm = 0
    p.scale, p.rope_mscale = 1.0, float(mscale)
    p.delta_head_stride = 0 if (delta is None or delta.dim() == 1) else D
    p.position_rounding = pos_round
    return p


_CODE = {torch.bfloat16: _lib.PE_DTYPE_BF16, torch.float16: _lib.PE_DTYPE_FP16, torch.float32: _lib.PE_DTYPE_FP32}


def _view(t: Optional[torch.Tensor]) -> _lib.PeTensor:
    d = _lib.PeTensor()
    if t is None:
        return d
    d.data = t.data_ptr()
    d.dtype = _CODE.get(t.dtype, _lib.PE_DTYPE_FP32)
    for i, s in enumerate(t.stride()):
        d.stride[i] = s
    if t.shape[3] == 1:
        d.stride[3] = 1
    return d


class PETransformFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, freqs, delta, mode, start_pos, is_key, mscale, pos_round):
        L = _lib.lib()
        if x.dtype not in _CODE:
            x = x.float()
        xv = x.transpose(1, 2)                       # (B, H, S, D) view
        if xv.stride(-1) != 1:
            xv = xv.contiguous()
        B, H, S, D = xv.shape
        cdt = _CODE[x.dtype]
        p = _params(B, H, S, D, mode, cdt, start_pos, delta if is_key else None, mscale, pos_round)
        _lib.check(L.pe_attn_check(ctypes.byref(p)))
        width = L.pe_attn_operand_width(ctypes.byref(p))
        out_w = 2 * D if mode == _lib.PE_MODE_POPE else D
        dst = torch.empty((B, H, S, width), dtype=x.dtype, device=x.device)
        fptr = None if freqs is None else freqs.data_ptr()
        dptr = None if (delta is None or not is_key) else delta.data_ptr()
        with torch.cuda.device(x.device):
            rc = L.pe_attn_transform(ctypes.byref(p), int(is_key), None, ctypes.byref(_view(xv)), fptr, dptr,
                                     dst.data_ptr(), torch.cuda.current_stream(x.device).cuda_stream)
        _lib.check(rc)
        ctx.save_for_backward(xv, freqs, delta)
        ctx.cfg = (mode, start_pos, is_key, mscale, cdt, width, x.dtype, pos_round)
        return dst[..., :out_w].transpose(1, 2)

    @staticmethod
    def backward(ctx, grad):
        L = _lib.lib()
        xv, freqs, delta = ctx.saved_tensors
        mode, start_pos, is_key, mscale, cdt, width, xdtype, pos_round = ctx.cfg
        B, H, S, D = xv.shape
        out_w = 2 * D if mode == _lib.PE_MODE_POPE else D
        g = torch.zeros((B, H, S, width), dtype=torch.float32, device=xv.device)
        g[..., :out_w] = grad.transpose(1, 2)
        dx = torch.empty((B, S, H, D), dtype=xv.dtype, device=xv.device)
        dxv = dx.transpose(1, 2)
        p = _params(B, H, S, D, mode, cdt, start_pos, delta if is_key else None, mscale, pos_round)
        need_f = freqs is not None and ctx.needs_input_grad[1] and mode == _lib.PE_MODE_POPE
        need_d = delta is not None and is_key and ctx.needs_input_grad[2]
        dfreqs = torch.empty(freqs.shape, dtype=torch.float32, device=xv.device) if need_f else None
        ddelta = torch.empty(delta.shape, dtype=torch.float32, device=xv.device) if need_d else None
        ws_bytes = L.pe_attn_transform_bwd_workspace_bytes(ctypes.byref(p), int(is_key))
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=xv.device)
        with torch.cuda.device(xv.device):
            rc = L.pe_attn_transform_bwd(ctypes.byref(p), int(is_key), g.data_ptr(), ctypes.byref(_view(xv)),
                                         None if freqs is None else freqs.data_ptr(),
                                         None if (delta is None or not is_key) else delta.data_ptr(),
                                         None, ctypes.byref(_view(dxv)),
                                         None if dfreqs is None else dfreqs.data_ptr(),
                                         None if ddelta is None else ddelta.data_ptr(),
                                         ws.data_ptr(), ws_bytes, torch.cuda.current_stream(xv.device).cuda_stream)
        _lib.check(rc)
        return dx.to(xdtype), dfreqs, ddelta, None, None, None, None, None


def check_transform_operands(x, freqs, delta, *, mode: str, is_key: bool) -> None:
    """x (B, S, H, D); freqs (D,) for PoPE or (D/2,) for RoPE; delta (D,) or (H, D) for PoPE keys;
    all on x's device.  Raises ValueError before anything is enqueued (the library only sees
    pointers, so a short freqs or delta would be read out of bounds)."""
    if x.dim() != 4:
        raise ValueError(f"pe_transform: x must be (B, S, H, D), got shape {tuple(x.shape)}")
    H, D = x.shape[2], x.shape[3]
    want = D if mode == "pope" else D // 2
    if mode == "rope" and D % 2:
        raise ValueError(f"pe_transform: RoPE needs an even width, got {D}")
    if freqs is None or freqs.dim() != 1 or freqs.shape[0] != want:
        got = None if freqs is None else tuple(freqs.shape)
        raise ValueError(f"pe_transform: freqs must have shape ({want},), got {got}")
    if delta is not None and is_key:
        if mode != "pope":
            raise ValueError("pe_transform: delta (phase bias) only applies to PoPE keys")
        if not (tuple(delta.shape) == (D,) or tuple(delta.shape) == (H, D)):
            raise ValueError(f"pe_transform: delta must be ({D},) or ({H}, {D}), got {tuple(delta.shape)}")
    for name, t in (("freqs", freqs), ("delta", delta)):
        if t is not None and t.device != x.device:
            raise ValueError(f"pe_transform: {name} is on {t.device}, x on {x.device}")


def pe_transform(x: torch.Tensor, freqs: torch.Tensor, delta: Optional[torch.Tensor], *, start_pos: int = 0,
                 is_key: bool = False, mode: str = "pope", mscale: float = 1.0,
                 position_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """x (B, S, H, D) -> PoPE [mu cos, mu sin] (B, S, H, 2D) or RoPE-rotated (B, S, H, D) on the GPU.

    fp32 inputs are transformed in fp32; bf16 and fp16 inputs produce their own type (the reference
    returns fp32 there, which SDPA under autocast rounds to the autocast type).  position_dtype (PoPE):
    None / torch.float32 exact positions, torch.bfloat16 / torch.float16 positions rounded to that
    type (FoPE's torch.arange(..., dtype=x.dtype), src/model/fpope.py:285,322)."""
    if not x.is_cuda:
        raise RuntimeError("the positional transform runs on the GPU only (got a CPU tensor); "
                           "the HIP library has no CPU path")
    if mode not in ("pope", "rope"):
        raise ValueError(f"pe_transform: unknown mode {mode!r}")
    check_transform_operands(x, freqs, delta, mode=mode, is_key=is_key)
    m = {"pope": _lib.PE_MODE_POPE, "rope": _lib.PE_MODE_ROPE}[mode]
    freqs = freqs.float().contiguous()
    if delta is not None:
        delta = delta.float().contiguous()
    pr = position_rounding(position_dtype, m)
    return PETransformFn.apply(x, freqs, delta, m, int(start_pos), bool(is_key), float(mscale), pr)
