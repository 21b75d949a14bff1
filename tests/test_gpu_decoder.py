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


def test_generate_yarn_crossing_max_seq_len_follows_oracle(cuda, monkeypatch):
    """YaRN generation that runs past max_seq_len.  The reference extends the tables when the
    running length passes max_seq_len (src/model/transformer.py:412-414), and YaRN's extension
    rebuilds the plain RoPE table with mscale kept (src/model/rope.py:103-119), under which the
    whole sequence is re-run.  With a 100-token prompt and max_seq_len 103, the logits behind tokens
    100..103 follow the YaRN table and those behind 104 and 105 the plain one: every step's logits
    (captured on their way to the sampler) equal the oracle's under the right table, and differ
    from the oracle's under the other table after the crossing."""
    from pe_ablations_amd import transformer as TR
    seen = []
    real = TR._next_token
    monkeypatch.setattr(TR, "_next_token", lambda lg, *a: (seen.append(lg.detach().cpu()), real(lg, *a))[1])
    cfg, m = make("rope_yarn", seed=16)
    for c in (cfg, m.config):
        c.max_seq_len = 103
    m.rope.max_seq_len = 103
    prompt = ids_for(cfg, 2, 100, seed=17)
    out = m.to(cuda).eval().generate(prompt.to(cuda), max_new_tokens=6, temperature=0.0).cpu()
    assert out.shape == (2, 106) and m.config.max_seq_len == 105 and len(seen) == 6
    sd = {k: v.cpu() for k, v in m.state_dict().items()}
    for i, t in enumerate(range(100, 106)):
        right = O.decoder_forward(sd, cfg, out[:, :t], yarn_extended=t > 103)["logits"][:, -1]
        assert md(seen[i], right) < 1e-4, (t, md(seen[i], right))
        assert torch.equal(out[:, t], seen[i].argmax(-1))
        if t > 103:
            wrong = O.decoder_forward(sd, cfg, out[:, :t])["logits"][:, -1]
            assert md(seen[i], wrong) > 3e-4, (t, md(seen[i], wrong))


def test_kv_cache_rewind_growth_and_gap(cuda):
    """The cache path accepts any start_pos up to the cached length, as the reference's does
    (src/model/fpope_attention.py:296-302): a chunk at an earlier start_pos overwrites the rows from
    there and the length becomes start_pos + S.  Growing max_cache_len mid-sequence keeps the rows
    cached so far; a start_pos past the cached length (rows never written) raises."""
    torch.manual_seed(18)
    pe = PoPEEmbedding(32, 512, delta_init="uniform")
    m = FPoPEGroupedQueryAttentionWithCache(128, 4, 2, 32, 32, fpope=pe, max_cache_len=48).to(cuda)
    x = torch.randn(1, 40, 128, device=cuda)
    other = torch.randn(1, 6, 128, device=cuda)
    with torch.no_grad():
        full = m(x)
        m(x[:, :30], use_cache=True)
        m(other, start_pos=30, use_cache=True)          # rows 30..35 hold other tokens
        assert m.cache_len == 36
        outs = [m(x[:, 30:33], start_pos=30, use_cache=True)]   # rewind: overwrite from 30
        assert m.cache_len == 33
        m.max_cache_len = 64                               # larger buffers, rows 0..32 carried over
        outs += [m(x[:, t:t + 1], start_pos=t, use_cache=True) for t in range(33, 40)]
        assert tuple(m.k_cache.shape[:3]) == (1, 2, 64) and m.cache_len == 40
        with pytest.raises(ValueError, match="gap"):
            m(x[:, :1], start_pos=41, use_cache=True)
    assert md(torch.cat(outs, 1), full[:, 30:40]) < 1e-5


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
