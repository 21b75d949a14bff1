"""The fwd+bwd step captured in a HIP graph (torch.cuda.CUDAGraph) and replayed: every replay must
equal the eager step bit for bit (the kernels are deterministic), with eager work and
synchronisations between the replays, and after the static inputs are refilled in place.  The
library's calls record only kernel launches (no memset, allocation or synchronisation), so the
launch-bound small shapes, such as the reference's training shape, can be replayed without host
overhead."""

import math

import pytest
import torch

from pe_ablations_amd.fpope_attention import FPoPEGroupedQueryAttention
from pe_ablations_amd.functional import pe_attention
from pe_ablations_amd.pope import PoPEEmbedding

pytestmark = pytest.mark.gpu

SHAPES = [
    dict(B=2, Hq=8, Hkv=4, S=256, Dc=64, Dr=32, Dv=64),   # split form, GQA (query-head split in dK/dV)
    dict(B=1, Hq=2, Hkv=2, S=640, Dc=0, Dr=128, Dv=128),  # fused form at the headline's widths
]


def capture(step):
    """torch's recipe: warm up on a side stream, then capture one step."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = step()
    return g, outs


@pytest.mark.parametrize("cfg", SHAPES)
def test_graph_replay_matches_eager(cuda, cfg):
    B, Hq, Hkv, S, Dc, Dr, Dv = (cfg[k] for k in ("B", "Hq", "Hkv", "S", "Dc", "Dr", "Dv"))
    gen = torch.Generator(device=cuda).manual_seed(S)
    mk = lambda h, d: torch.randn(B, h, S, d, generator=gen, device=cuda).to(torch.bfloat16).requires_grad_(True)
    q, k, v = mk(Hq, Dr), mk(Hkv, Dr), mk(Hkv, Dv)
    qc, kc = (mk(Hq, Dc), mk(Hkv, Dc)) if Dc else (None, None)
    dO = torch.randn(B, Hq, S, Dv, generator=gen, device=cuda).to(torch.bfloat16)
    delta = (-2 * math.pi * torch.rand(Dr, generator=gen, device=cuda)).requires_grad_(True)
    freqs = (10000.0 ** (-(torch.arange(0, Dr, dtype=torch.float32) / Dr))).to(cuda)
    leaves = [t for t in (q, k, v, qc, kc, delta) if t is not None]

    def step():
        out = pe_attention(q, k, v, mode="pope", q_c=qc, k_c=kc, freqs=freqs, delta=delta)
        return (out.detach(),) + torch.autograd.grad(out, leaves, dO)

    print(f"graph replay {cfg}", flush=True)
    g, outs = capture(step)
    for rep in range(4):
        if rep == 2:  # new contents in the same buffers
            with torch.no_grad():
                for t in leaves[:-1]:
                    t.copy_(torch.randn(t.shape, generator=gen, device=cuda).to(t.dtype))
                dO.copy_(torch.randn(dO.shape, generator=gen, device=cuda).to(dO.dtype))
        eager = [t.clone() for t in step()]
        torch.randn(1 << 16, device=cuda).sum().item()  # unrelated eager work and a synchronisation
        g.replay()
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(outs, eager)):
            assert torch.equal(a, b), (rep, i, (a.float() - b.float()).abs().max().item())


def test_graph_replay_module_training_step(cuda):
    """The split-form module with the fused norm under bf16 autocast (the reference trainer's step
    at its attention shape, B=8 S=512 hidden 512, 8 -> 4 heads): replays equal the eager step."""
    torch.manual_seed(3)
    pe = PoPEEmbedding(32, 512, delta_init="uniform")
    m = FPoPEGroupedQueryAttention(512, 8, 4, 64, 32, fpope=pe).to(cuda)
    x = torch.randn(8, 512, 512, device=cuda, requires_grad=True)
    dout = torch.randn(8, 512, 512, device=cuda)
    params = [x] + list(m.parameters())

    def step():
        with torch.autocast("cuda", dtype=torch.bfloat16):
            out = m(x)
        return (out.detach(),) + torch.autograd.grad(out, params, dout)

    g, outs = capture(step)
    for rep in range(3):
        eager = [t.clone() for t in step()]
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(outs, eager)):
            assert torch.equal(a, b), (rep, i, (a.float() - b.float()).abs().max().item())


def test_graph_replay_masked_step(cuda):
    """The explicit-mask path (pe_attn_fwd_masked / pe_attn_bwd_masked, generic kernels) captured and
    replayed: a broadcast key-padding bool mask and a float mask with -inf, replays equal to the eager
    step bit for bit, also after the mask's contents change in place."""
    B, Hq, Hkv, S, D = 2, 4, 2, 200, 64
    gen = torch.Generator(device=cuda).manual_seed(5)
    mk = lambda h: torch.randn(B, h, S, D, generator=gen, device=cuda).to(torch.bfloat16).requires_grad_(True)
    q, k, v = mk(Hq), mk(Hkv), mk(Hkv)
    dO = torch.randn(B, Hq, S, D, generator=gen, device=cuda).to(torch.bfloat16)
    masks = [(torch.arange(S, device=cuda).view(1, S) < torch.tensor([S, 77], device=cuda).view(B, 1)).view(B, 1, 1, S),
             torch.randn(B, 1, S, S, generator=gen, device=cuda).masked_fill(
                 torch.rand(B, 1, S, S, generator=gen, device=cuda) > 0.8, float("-inf"))]
    for mask in masks:
        def step():
            out = pe_attention(q, k, v, mode="none", causal=False, mask=mask)
            return (out.detach(),) + torch.autograd.grad(out, (q, k, v), dO)

        print(f"graph replay masked {mask.dtype}", flush=True)
        g, outs = capture(step)
        for rep in range(3):
            if rep == 2:
                with torch.no_grad():
                    if mask.dtype == torch.bool:
                        mask.copy_(torch.rand(mask.shape, generator=gen, device=cuda) > 0.3)
                    else:
                        mask.copy_(torch.randn(mask.shape, generator=gen, device=cuda))
            eager = [t.clone() for t in step()]
            torch.randn(1 << 16, device=cuda).sum().item()
            g.replay()
            torch.cuda.synchronize()
            for i, (a, b) in enumerate(zip(outs, eager)):
                assert torch.equal(a, b), (str(mask.dtype), rep, i, (a.float() - b.float()).abs().max().item())
