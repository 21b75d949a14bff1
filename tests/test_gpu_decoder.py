"""The decoder drop-in and the long-context harness on the GPU against the oracle's whole-decoder
restatement (oracle.decoder_forward, CPU, attention core in fp64) with the same weights.

The attention projections are re-drawn with a larger spread than the N(0, 0.02^2) init so that
the scores are far from uniform and the positional transform shows in the logits.  fp32 model
logits are held to 1e-4 absolute (max |logit| is O(1) here); bf16 autocast losses to 2e-2.
"""

import math

import pytest
import torch

from oracle import pe_oracle as O
from pe_ablations_amd import evaluation as E
from pe_ablations_amd.fpope_attention import FPoPEGroupedQueryAttention, FPoPEGroupedQueryAttentionWithCache
from pe_ablations_amd.pope import PoPEEmbedding
from pe_ablations_amd.transformer import Transformer, TransformerConfig

pytestmark = pytest.mark.gpu

BASE = dict(vocab_size=211, hidden_dim=128, num_layers=2, num_heads=4, num_kv_heads=2, head_dim=32,
            pope_d_rope=16, fpope_d_rope=16, fpope_num_fourier_terms=4, max_seq_len=256,
            pope_delta_init="uniform", fpope_delta_init="uniform")

CASES = {
    "pope_split": dict(pe_mode="pope"),
    "pope_fused": dict(pe_mode="pope", pope_fused=True, num_kv_heads=4),
    "pope_floor": dict(pe_mode="pope_floor", pope_training_length=64),
    "fpope": dict(pe_mode="fpope"),
    "rope_yarn": dict(pe_mode="rope", rope_type="yarn", rope_scale=4.0, head_dim=64),
    "nope": dict(pe_mode="nope"),
}


def md(a, b):
    return (a.detach().double().cpu() - b.detach().double().cpu()).abs().max().item()


def make(case, seed=0):
    torch.manual_seed(seed)
    cfg = TransformerConfig(**dict(BASE, **CASES[case]))
    m = Transformer(cfg)
    g = torch.Generator().manual_seed(seed + 100)
    with torch.no_grad():
        for name, p in m.named_parameters():
            if ".attention.w" in name:
                p.copy_(torch.randn(p.shape, generator=g) * 0.25)
            elif name.endswith("norm.weight"):
                p.copy_(0.5 + torch.rand(p.shape, generator=g))
    return cfg, m


def ids_for(cfg, B, S, seed=1):
    return torch.randint(0, cfg.vocab_size, (B, S), generator=torch.Generator().manual_seed(seed))


@pytest.mark.parametrize("case", list(CASES))
def test_decoder_fp32_matches_oracle(cuda, case):
    cfg, m = make(case)
    ids = ids_for(cfg, 2, 97)
    print(f"decoder fp32 {case} B=2 S=97", flush=True)
    ref = O.decoder_forward(m.state_dict(), cfg, ids, labels=ids)
    g = m.to(cuda).eval()
    with torch.no_grad():
        out = g(ids.to(cuda), labels=ids.to(cuda))
    torch.cuda.synchronize()
    assert md(out["logits"], ref["logits"]) < 1e-4
    assert abs(out["loss"].item() - ref["loss"].item()) < 1e-5


@pytest.mark.parametrize("case", ["pope_split", "pope_fused", "rope_yarn"])
def test_decoder_start_pos(cuda, case):
    cfg, m = make(case, seed=3)
    ids = ids_for(cfg, 1, 50, seed=4)
    ref = O.decoder_forward(m.state_dict(), cfg, ids, start=37)
    with torch.no_grad():
        out = m.to(cuda).eval()(ids.to(cuda), start_pos=37)
    assert md(out["logits"], ref["logits"]) < 1e-4


@pytest.mark.parametrize("case", ["pope_split", "pope_fused"])
def test_decoder_bf16_autocast_loss(cuda, case):
    cfg, m = make(case, seed=5)
    ids = ids_for(cfg, 1, 300, seed=6)
    m.extend_context_length(300)
    ref = O.decoder_forward(m.state_dict(), cfg, ids, labels=ids)["loss"].item()
    g = m.to(cuda).eval()
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        loss = g(ids.to(cuda), labels=ids.to(cuda))["loss"].item()
    assert abs(loss - ref) < 2e-2


def test_decoder_loss_at_init(cuda):
    """Plain N(0, 0.02^2) init, bf16 weights, one 2048-token sequence.  The tied head sees a
    unit-RMS input, so each logit is ~ N(0, 0.02^2 * d) and E[CE] ~ ln(vocab) + 0.02^2 * d / 2."""
    torch.manual_seed(7)
    cfg = TransformerConfig(vocab_size=4096, hidden_dim=256, num_layers=2, num_heads=2, num_kv_heads=2,
                            head_dim=128, pe_mode="pope", pope_fused=True, max_seq_len=2048,
                            pope_delta_init="uniform")
    m = Transformer(cfg).to(cuda).to(torch.bfloat16).eval()
    ids = torch.randint(0, 4096, (1, 2048), device=cuda)
    with torch.no_grad():
        loss = m(ids, labels=ids)["loss"].float().item()
    assert abs(loss - (math.log(4096) + 0.02 ** 2 * 256 / 2)) < 0.03


def test_checkpoint_load_to_gpu_same_logits(cuda, tmp_path):
    cfg, m = make("fpope", seed=8)
    p = tmp_path / "checkpoint_step_1.pt"
    E.save_checkpoint(m, str(p))
    ids = ids_for(cfg, 1, 64, seed=9).to(cuda)
    a = m.to(cuda).eval()
    m2, _, _ = E.load_model(str(p), cuda)
    with torch.no_grad():
        assert torch.equal(a(ids)["logits"], m2(ids)["logits"])


@pytest.mark.parametrize("case", ["pope_split", "pope_fused"])
def test_sliding_window_ppl_matches_oracle(cuda, case):
    """Context 64, default stride 32, 300 tokens: windows at 0, 32, 64, 96 (4*64 = 256-token cap,
    stop at 128 counted tokens); PPL = exp(mean window loss) with the oracle's losses."""
    cfg, m = make(case, seed=10)
    toks = ids_for(cfg, 1, 300, seed=11)[0].tolist()
    sd = {k: v.clone() for k, v in m.state_dict().items()}
    ppl, oom = E.compute_ppl_sliding_window(m.to(cuda).eval(), toks, 64, cuda)
    assert not oom
    losses = []
    for s in (0, 32, 64, 96):
        ids = torch.tensor([toks[s:s + 64]])
        losses.append(O.decoder_forward(sd, cfg, ids, labels=ids)["loss"].item())
    assert ppl == pytest.approx(math.exp(sum(losses) / 4), rel=1e-5)


@pytest.mark.parametrize("case", list(CASES))
def test_generate_greedy_follows_oracle_argmax(cuda, case):
    """Greedy generation through the KV caches (prefill, then one token per step through the
    split-key decode kernel) picks, at every step, a token whose oracle logit (full re-run of the
    sequence, as the reference's generate does) is the maximum within 1e-4."""
    cfg, m = make(case, seed=12)
    prompt = ids_for(cfg, 2, 9, seed=13)
    out = m.to(cuda).eval().generate(prompt.to(cuda), max_new_tokens=6, temperature=0.0).cpu()
    assert out.shape == (2, 15) and torch.equal(out[:, :9], prompt)
    assert all(layer.attention.cache.k is None for layer in m.layers)   # caches freed
    sd = {k: v.cpu() for k, v in m.state_dict().items()}
    for t in range(9, 15):
        logits = O.decoder_forward(sd, cfg, out[:, :t])["logits"][:, -1]
        for b in range(2):
            assert logits[b, out[b, t]].item() >= logits[b].max().item() - 1e-4, (case, t, b)


def test_fused_form_module_matches_oracle(cuda):
    """d_content = 0: the legacy fused form, q = PoPE(RMSNorm(wq_r x)) with scale 1/sqrt(head_dim)."""
    torch.manual_seed(14)
    pe = PoPEEmbedding(64, 512, delta_init="uniform")
    m = FPoPEGroupedQueryAttention(128, 4, 2, 64, 64, fpope=pe, d_content=0)
    x = torch.randn(2, 70, 128)
    B, S = 2, 70
    qr = O.rms_norm(x @ m.wq_r.weight.T, m.qr_norm.weight).view(B, S, 4, 64).transpose(1, 2)
    kr = O.rms_norm(x @ m.wk_r.weight.T, m.kr_norm.weight).view(B, S, 2, 64).transpose(1, 2)
    v = (x @ m.wv.weight.T).view(B, S, 2, 64).transpose(1, 2)
    ref, _ = O.pope_attention(qr, kr, v, pe.effective_freqs, pe.phase_bias, scale=64 ** -0.5, start_q=3,
                              start_k=3)
    ref = ref.float().transpose(1, 2).reshape(B, S, -1) @ m.wo.weight.T
    out = m.to(cuda)(x.to(cuda), start_pos=3)
    assert md(out, ref) < 1e-4


def test_fused_form_kv_cache_decode(cuda):
    torch.manual_seed(15)
    pe = PoPEEmbedding(64, 512, delta_init="uniform")
    m = FPoPEGroupedQueryAttentionWithCache(128, 4, 2, 64, 64, fpope=pe, max_cache_len=96, d_content=0).to(cuda)
    x = torch.randn(1, 35, 128, device=cuda)
    with torch.no_grad():
        full = m(x)
        outs = [m(x[:, :32], use_cache=True)] + [m(x[:, t:t + 1], start_pos=t, use_cache=True)
                                                 for t in range(32, 35)]
    assert tuple(m.k_cache.shape) == (1, 2, 96, 128) and m.cache_len == 35
    assert md(torch.cat(outs, 1), full) < 1e-5
