"""BASELINE.json configurations at their full sizes, checked slice by slice.

The kernel runs the whole configuration; the oracle (the row-chunked closed form,
oracle.pe_attention_chunked: fp32 transforms in the reference order, bf16 operand rounding in
bf16 mode, fp32 or fp64 GEMMs) recomputes complete (batch, head) slices, which the attention of
one head depends on alone.  A per-head phase-bias gradient sums its head over the batch, so the
slices cover every batch entry of the heads they check.  Tolerances: raw max-abs 2e-2 in bf16
mode, 1e-5 in fp32 mode (north star), bf16 results included with their own rounding to bf16
(tests/_cmp.py); phase-bias gradients relative to their largest entry.  Each check prints its raw
and net-of-rounding errors.
"""

import math

import pytest
import torch

from oracle import pe_oracle as O
from tests._cmp import err, err_both
from pe_ablations_amd.functional import pe_attention

pytestmark = pytest.mark.gpu


def md(a, b):
    return err(a, b)


def make(B, H, S, D, seed, dtype=torch.bfloat16, dev="cpu"):
    g = torch.Generator().manual_seed(seed)
    q, k, v, do = (torch.randn(B, H, S, D, generator=g).to(dtype) for _ in range(4))
    delta = torch.rand(H, D, generator=g) * (-2 * math.pi)
    return q, k, v, do, delta


def run_kernel(cuda, q, k, v, do, freqs, delta, scale, backward=True):
    qg, kg, vg = (t.to(cuda).requires_grad_(backward) for t in (q, k, v))
    dg = delta.to(cuda).requires_grad_(backward)
    out, lse = pe_attention(qg, kg, vg, mode="pope", freqs=freqs.to(cuda), delta=dg, scale=scale, return_lse=True)
    if backward:
        out.backward(do.to(cuda))
    torch.cuda.synchronize()
    res = {"out": out.detach().cpu(), "lse": lse.cpu()}
    if backward:
        res.update(dq=qg.grad.cpu(), dk=kg.grad.cpu(), dv=vg.grad.cpu(), ddelta=dg.grad.cpu())
    return res


def check_slices(res, q, k, v, do, freqs, delta, scale, heads, batches, tol, backward=True,
                 core=torch.float32, bf16=True):
    od = torch.bfloat16 if bf16 else None
    for h in heads:
        dd = torch.zeros(q.shape[-1], dtype=torch.float64)
        for b in batches:
            ref = O.pope_attention_chunked(q[b, h].float(), k[b, h].float(), v[b, h].float(), freqs, delta[h],
                                           dout=do[b, h].float() if backward else None, scale=scale,
                                           core_dtype=core, operand_dtype=od, chunk=2048)
            names = ["out", "lse"] + (["dq", "dk", "dv"] if backward else [])
            both = {n: err_both(res[n][b, h], ref[n]) for n in names}
            errs = {n: r for n, (r, _) in both.items()}
            print(f"parity h={h} b={b} " + " ".join(f"{n}: raw {r:.2e} net {nt:.2e}" for n, (r, nt) in both.items()),
                  flush=True)
            if backward:
                dd += ref["ddelta"]
            for name, e in errs.items():
                assert e < tol, (h, b, name, errs)
        if backward and len(batches) == q.shape[0]:
            rel = md(res["ddelta"][h], dd) / max(1.0, dd.abs().max().item())
            assert rel < tol, (h, "ddelta", rel)


def test_config2_gpt125m_fwd_bwd_bf16(cuda):
    """C2: B=8, H=12, S=2048, D=64, bf16 fwd+bwd, grads q, k, v, delta."""
    B, H, S, D = 8, 12, 2048, 64
    q, k, v, do, delta = make(B, H, S, D, seed=2)
    freqs = O.pope_freqs(D)
    res = run_kernel(cuda, q, k, v, do, freqs, delta, 1 / math.sqrt(D))
    check_slices(res, q, k, v, do, freqs, delta, 1 / math.sqrt(D), heads=[0, 11], batches=range(B), tol=2e-2)


def test_one_launch_prologue_projection_views_ragged_heads_start_pos(cuda):
    """A shape that takes the one-launch PoPE prologue (more than 1024 blocks; queries in groups of
    eight heads): six heads (a single, ragged group), three batch entries, the projections'
    (B, S, H, D) layout seen as (B, H, S, D) views, and positions starting at 37 on both sides.
    Every (b, h) slice of two heads is checked against the oracle at the north-star bar."""
    B, H, S, D, start = 3, 6, 2000, 64, 37
    assert B * H * S * (D // 8) // 256 > 1024          # the launch the small path does not take
    g = torch.Generator().manual_seed(7)
    q, k, v, do = (torch.randn(B, S, H, D, generator=g).to(torch.bfloat16).transpose(1, 2) for _ in range(4))
    delta = torch.rand(H, D, generator=g) * (-2 * math.pi)
    freqs = O.pope_freqs(D)
    scale = 1 / math.sqrt(D)
    qg, kg, vg = (t.to(cuda).requires_grad_(True) for t in (q, k, v))
    assert qg.stride(1) == D and qg.stride(2) == H * D   # still the projection layout on the GPU
    dg = delta.to(cuda).requires_grad_(True)
    out, lse = pe_attention(qg, kg, vg, mode="pope", freqs=freqs.to(cuda), delta=dg, scale=scale,
                            start_pos_q=start, start_pos_k=start, return_lse=True)
    out.backward(do.to(cuda))
    torch.cuda.synchronize()
    res = {"out": out.detach().cpu(), "lse": lse.cpu(), "dq": qg.grad.cpu(), "dk": kg.grad.cpu(),
           "dv": vg.grad.cpu(), "ddelta": dg.grad.cpu()}
    for h in (0, 5):
        dd = torch.zeros(D, dtype=torch.float64)
        for b in range(B):
            ref = O.pope_attention_chunked(q[b, h].float(), k[b, h].float(), v[b, h].float(), freqs, delta[h],
                                           dout=do[b, h].float(), scale=scale, start_q=start, start_k=start,
                                           operand_dtype=torch.bfloat16, chunk=1024)
            both = {n: err_both(res[n][b, h], ref[n]) for n in ("out", "lse", "dq", "dk", "dv")}
            print(f"prologue case h={h} b={b} " + " ".join(f"{n}: raw {r:.2e} net {nt:.2e}"
                                                           for n, (r, nt) in both.items()), flush=True)
            for n, (r, _) in both.items():
                assert r < 2e-2, (h, b, n, r)
            dd += ref["ddelta"]
        assert md(res["ddelta"][h], dd) / max(1.0, dd.abs().max().item()) < 2e-2


def test_config3_fope_fwd_bwd_bf16(cuda):
    """C3: FoPE, B=4, H=16, S=4096, D=128, 4 frequencies per dim (base + 3 ~ U(0, theta_0)),
    coefficients ~ N(0, 0.1^2), floor 2pi/2048, bf16 fwd+bwd."""
    B, H, S, D, M = 4, 16, 4096, 128, 4
    q, k, v, do, delta = make(B, H, S, D, seed=3)
    base = O.pope_freqs(D)
    g = torch.Generator().manual_seed(33)
    table = torch.cat([base.unsqueeze(1), torch.rand(D, M - 1, generator=g) * float(base[0])], 1)
    coeffs = torch.randn(D, M, generator=g) * 0.1
    omega = O.fope_effective_freqs(base, coeffs, freq_table=table, training_length=2048)
    res = run_kernel(cuda, q, k, v, do, omega, delta, 1 / math.sqrt(D))
    check_slices(res, q, k, v, do, omega, delta, 1 / math.sqrt(D), heads=[5], batches=range(B), tol=2e-2)


def test_config4_long_context_forward_bf16(cuda):
    """C4: B=1, H=16, S=16384, D=128, bf16 forward (the 16k perplexity sweep's shape)."""
    B, H, S, D = 1, 16, 16384, 128
    q, k, v, do, delta = make(B, H, S, D, seed=4)
    freqs = O.pope_freqs(D)
    res = run_kernel(cuda, q, k, v, do, freqs, delta, 1 / math.sqrt(D), backward=False)
    check_slices(res, q, k, v, do, freqs, delta, 1 / math.sqrt(D), heads=[0, 15], batches=[0], tol=2e-2,
                 backward=False)


def test_config4_long_context_forward_fp32(cuda):
    """The reference's long-context evaluation runs in fp32 (scripts/evaluate_long_context.py:
    109-112): S=16384, D=128 fp32 forward against an fp64 oracle at 1e-5."""
    B, H, S, D = 1, 2, 16384, 128
    q, k, v, do, delta = make(B, H, S, D, seed=5, dtype=torch.float32)
    freqs = O.pope_freqs(D)
    res = run_kernel(cuda, q, k, v, do, freqs, delta, 1 / math.sqrt(D), backward=False)
    check_slices(res, q, k, v, do, freqs, delta, 1 / math.sqrt(D), heads=[1], batches=[0], tol=1e-5,
                 backward=False, core=torch.float64, bf16=False)


def test_headline_fwd_bwd_bf16_full_head(cuda):
    """Headline: PoPE fwd+bwd, B=1, H=16, S=16384, D=128 bf16; head 3 checked end to end."""
    B, H, S, D = 1, 16, 16384, 128
    q, k, v, do, delta = make(B, H, S, D, seed=6)
    freqs = O.pope_freqs(D)
    res = run_kernel(cuda, q, k, v, do, freqs, delta, 1 / math.sqrt(D))
    check_slices(res, q, k, v, do, freqs, delta, 1 / math.sqrt(D), heads=[3], batches=[0], tol=2e-2)


def test_long_fwd_bwd_runs_over_capped_head_groups(cuda):
    """S = 32768, H = 16, D = 128 bf16 fwd+bwd.  The whole dS would be 17.2 GB; the backward holds
    at most PE_BWD_DS_CAP_BYTES (4.5 GiB) of it and runs its gradient kernels over 4 groups of 4
    heads.  Heads 0 and 13 (first and last group) are checked end to end against the chunked
    oracle, and the workspace the call asks for is measured."""
    from pe_ablations_amd import _lib
    import ctypes
    B, H, S, D = 1, 16, 32768, 128
    q, k, v, do, delta = make(B, H, S, D, seed=7)
    freqs = O.pope_freqs(D)
    p = _lib.PeParams()
    for name, val in dict(B=B, Hq=H, Hkv=H, Sq=S, Sk=S, Dc=0, Dr=D, Dv=D, mode=_lib.PE_MODE_POPE,
                          dtype=_lib.PE_DTYPE_BF16, causal=_lib.PE_CAUSAL_TOP_LEFT, scale=1 / math.sqrt(D),
                          rope_mscale=1.0, delta_head_stride=D).items():
        setattr(p, name, val)
    fn = _lib.lib().pe_attn_bwd_workspace_bytes
    fn.restype = ctypes.c_size_t
    ws = fn(ctypes.byref(p))
    cap = 4608 << 20
    assert cap - 2 ** 30 < ws < cap + 2 ** 28, ws   # 4 heads of dS (4.29 GB) plus the small buffers
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    base = torch.cuda.memory_allocated()
    res = run_kernel(cuda, q, k, v, do, freqs, delta, 1 / math.sqrt(D))
    peak = torch.cuda.max_memory_allocated() - base
    print(f"bwd workspace {ws / 2**30:.2f} GiB, peak allocated {peak / 2**30:.2f} GiB", flush=True)
    assert peak < 6 * 2 ** 30, peak
    check_slices(res, q, k, v, do, freqs, delta, 1 / math.sqrt(D), heads=[0, 13], batches=[0], tol=2e-2)
