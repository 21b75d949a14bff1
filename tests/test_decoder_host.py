"""CPU tests of the decoder drop-in and the long-context harness: module tree / state-dict names
(what a reference checkpoint must match), checkpoint round trip, the sliding-window accounting of
scripts/evaluate_long_context.py:80-137 (with a stub model, no kernel calls), and the pins of the
oracle's whole-decoder restatement."""

import math

import pytest
import torch
import torch.nn as nn

from oracle import pe_oracle as O
from pe_ablations_amd import evaluation as E
from pe_ablations_amd.transformer import Transformer, TransformerConfig

TINY = dict(vocab_size=97, hidden_dim=64, num_layers=2, num_heads=4, num_kv_heads=2, head_dim=16,
            pope_d_rope=8, fpope_d_rope=8, fpope_num_fourier_terms=4, max_seq_len=64)

# per-layer names of the reference module tree (src/model/transformer.py:127-184,
# src/model/fpope_attention.py:79-104, src/model/attention.py:33-48, src/model/ffn.py:53-58)
_BLOCK = ["attention_norm.weight", "ffn_norm.weight", "feed_forward.w1.weight", "feed_forward.w2.weight",
          "feed_forward.w3.weight"]
_GQA = ["attention.wq.weight", "attention.wk.weight", "attention.wv.weight", "attention.wo.weight"]
_SPLIT = ["attention.wq_c.weight", "attention.wk_c.weight", "attention.wq_r.weight", "attention.wk_r.weight",
          "attention.qr_norm.weight", "attention.kr_norm.weight", "attention.wv.weight", "attention.wo.weight"]
# persistent PE state (src/model/pope.py:72-97, src/model/fpope.py:82-105); rope tables are not persistent
_POPE = ["freqs", "effective_freqs", "base_angles", "phase_bias"]
_FOPE = ["base_freqs", "fourier_coeffs", "fourier_indices", "phase_bias", "positions"]
_TOP = ["token_embedding.embedding.weight", "norm.weight", "output.weight"]


def expected_keys(mode: str, layers: int) -> set:
    keys = set(_TOP)
    attn = _GQA if mode in ("rope", "nope") else _SPLIT
    pe = {"pope": ("pope", _POPE), "pope_floor": ("pope", _POPE), "fpope": ("fpope", _FOPE)}.get(mode)
    if pe:
        keys |= {f"{pe[0]}.{n}" for n in pe[1]}
    for i in range(layers):
        keys |= {f"layers.{i}.{n}" for n in _BLOCK + attn}
        if pe:
            keys |= {f"layers.{i}.attention.fpope.{n}" for n in pe[1]}
    return keys


@pytest.mark.parametrize("mode", ["rope", "nope", "pope", "pope_floor", "fpope"])
def test_state_dict_names_match_reference_tree(mode):
    m = Transformer(TransformerConfig(pe_mode=mode, **TINY))
    assert set(m.state_dict()) == expected_keys(mode, TINY["num_layers"])
    # one PE module shared by every layer, as the reference (src/model/transformer.py:291-294)
    pe = m.pope if mode.startswith("pope") else m.fpope
    if pe is not None:
        assert all(layer.attention.fpope is pe for layer in m.layers)
    # tied head (src/model/transformer.py:298-300)
    assert m.output.weight is m.token_embedding.embedding.weight


def test_state_dict_shapes_split_and_fused():
    c = TransformerConfig(pe_mode="pope", **TINY)
    sd = Transformer(c).state_dict()
    H, Hkv, D, Dr, hid = 4, 2, 16, 8, 64
    assert sd["layers.0.attention.wq_c.weight"].shape == (H * D, hid)
    assert sd["layers.0.attention.wk_r.weight"].shape == (Hkv * Dr, hid)
    assert sd["layers.0.attention.qr_norm.weight"].shape == (H * Dr,)
    assert sd["pope.base_angles"].shape == (TINY["max_seq_len"], Dr)
    assert sd["layers.0.feed_forward.w1.weight"].shape == (256, hid)  # 4*64*2/3 = 170 -> 256
    f = Transformer(TransformerConfig(pe_mode="pope", pope_fused=True, **TINY))
    sdf = f.state_dict()
    assert "layers.0.attention.wq_c.weight" not in sdf
    assert sdf["layers.0.attention.wq_r.weight"].shape == (H * D, hid)
    assert sdf["pope.freqs"].shape == (D,)
    assert f.layers[0].attention.scale == pytest.approx(D ** -0.5)
    assert Transformer(c).layers[0].attention.scale == pytest.approx((D + 2 * Dr) ** -0.5)


def test_alibi_is_rejected_with_a_reason():
    with pytest.raises(NotImplementedError, match="alibi"):
        Transformer(TransformerConfig(pe_mode="alibi", **TINY))


def test_init_distribution():
    torch.manual_seed(0)
    m = Transformer(TransformerConfig(pe_mode="pope", **dict(TINY, vocab_size=4096, hidden_dim=256)))
    w = m.layers[0].feed_forward.w1.weight
    assert abs(w.std().item() - 0.02) < 1e-3 and abs(w.mean().item()) < 1e-3
    assert torch.all(m.layers[0].attention.qr_norm.weight == 1)


def test_num_params_matches_reference_formula_at_1b_shape():
    """The reference's estimate counts plain GQA projections (src/model/transformer.py:79-106):
    vocab*d + L*(d*H*D + 2*d*Hkv*D + H*D*d + 3*d*ffn) + (2L+1)*d."""
    c = TransformerConfig(vocab_size=32000, hidden_dim=2048, num_layers=24, num_heads=16, num_kv_heads=16,
                          head_dim=128, ffn_dim=5632)
    d, L = 2048, 24
    assert c.num_params == 32000 * d + L * (4 * d * 2048 + 3 * d * 5632) + (2 * L + 1) * d


def test_checkpoint_round_trip(tmp_path):
    torch.manual_seed(1)
    m = Transformer(TransformerConfig(pe_mode="pope", pope_delta_init="uniform", **TINY))
    p = tmp_path / "checkpoint_step_5.pt"
    E.save_checkpoint(m, str(p), step=5)
    m2, cfg, mode = E.load_model(str(p), torch.device("cpu"))
    assert mode == "pope" and cfg.pope_d_rope == 8 and not m2.training
    for k, v in m.state_dict().items():
        assert torch.equal(v, m2.state_dict()[k]), k


def test_checkpoint_reference_layout_and_compile_prefix(tmp_path):
    """A trainer checkpoint (src/training/trainer.py:203-214) whose model_config holds only the
    keys the reference script reads, and whose state dict carries torch.compile's prefix."""
    torch.manual_seed(2)
    m = Transformer(TransformerConfig(pe_mode="fpope", **TINY))
    cfg = {k: getattr(m.config, k) for k in E._CONFIG_KEYS}
    ck = {"model_state_dict": {"_orig_mod." + k: v for k, v in m.state_dict().items()},
          "optimizer_state_dict": {"state": {}, "param_groups": [{"lr": 3e-4}]},
          "scheduler_state_dict": {"last_epoch": 3}, "step": 3, "tokens_seen": 10, "epoch": 0,
          "config": {"learning_rate": 3e-4, "checkpoint_dir": "checkpoints"}, "model_config": cfg}
    p = tmp_path / "c.pt"
    torch.save(ck, p)
    m2, c2, mode = E.load_model(str(p), torch.device("cpu"))
    assert mode == "fpope" and c2.fpope_num_fourier_terms == 4
    assert torch.equal(m2.fpope.fourier_coeffs, m.fpope.fourier_coeffs)


def test_config_defaults_when_model_config_missing():
    c = E.config_from_checkpoint({"model_state_dict": {}})
    assert (c.vocab_size, c.hidden_dim, c.num_layers, c.pe_mode, c.pope_fused) == (50257, 512, 24, "rope", False)
    c = E.config_from_checkpoint({"config": {"model": {"pe_mode": "pope", "hidden_dim": 128}}, "model_config": {}})
    assert c.pe_mode == "pope" and c.hidden_dim == 128


class StubModel(nn.Module):
    """Records each window; its loss is a fixed function of the window's first token."""

    def __init__(self, oom_at=None):
        super().__init__()
        self.windows, self.ext, self.oom_at = [], [], oom_at

    def extend_context_length(self, n):
        self.ext.append(n)

    def forward(self, input_ids, labels=None):
        assert labels is input_ids
        ids = input_ids[0].tolist()
        if self.oom_at is not None and len(self.windows) == self.oom_at:
            raise RuntimeError("HIP out of memory. Tried to allocate")
        self.windows.append(ids)
        return {"loss": torch.tensor(0.01 * (ids[0] % 7) + 1.0)}


def test_sliding_window_accounting():
    """Windows every ctx/2 over the first 4*ctx tokens, each weighted ctx//2, stop at 2*ctx counted
    tokens: four windows at starts 0, ctx/2, ctx, 3ctx/2."""
    toks = list(range(1000))
    m = StubModel()
    ppl, oom = E.compute_ppl_sliding_window(m, toks, 64, torch.device("cpu"))
    assert not oom and m.ext == [64]
    assert [w[0] for w in m.windows] == [0, 32, 64, 96] and all(len(w) == 64 for w in m.windows)
    losses = [0.01 * (s % 7) + 1.0 for s in (0, 32, 64, 96)]
    assert ppl == pytest.approx(math.exp(sum(losses) / 4), rel=1e-6)


def test_sliding_window_short_stream_and_stride():
    m = StubModel()
    # 4*ctx cap: only 100 tokens; range(0, 100 - 64, 16) = 0, 16, 32 -> 3 windows (< 2*ctx tokens)
    ppl, oom = E.compute_ppl_sliding_window(m, list(range(100)), 64, torch.device("cpu"), stride=16)
    assert [w[0] for w in m.windows] == [0, 16, 32] and not oom and math.isfinite(ppl)
    m = StubModel()
    ppl, oom = E.compute_ppl_sliding_window(m, list(range(64)), 64, torch.device("cpu"))
    assert m.windows == [] and ppl == float("inf") and not oom


def test_sliding_window_oom():
    m = StubModel(oom_at=0)
    assert E.compute_ppl_sliding_window(m, list(range(500)), 32, torch.device("cpu")) == (float("inf"), True)
    m = StubModel(oom_at=2)
    ppl, oom = E.compute_ppl_sliding_window(m, list(range(500)), 32, torch.device("cpu"))
    assert oom and len(m.windows) == 2 and math.isfinite(ppl)


def test_load_tokens(tmp_path):
    import numpy as np
    np.save(tmp_path / "t.npy", np.arange(10, dtype=np.int32))
    (tmp_path / "t.txt").write_text("3 4\n5  6\n")
    assert E.load_tokens(str(tmp_path / "t.npy")) == list(range(10))
    assert E.load_tokens(str(tmp_path / "t.txt")) == [3, 4, 5, 6]


# ---------------------------------------------------------------------------------------------
# pins of oracle.decoder_forward
# ---------------------------------------------------------------------------------------------

def _tiny(mode, **kw):
    torch.manual_seed(3)
    c = TransformerConfig(pe_mode=mode, **dict(TINY, **kw))
    return c, Transformer(c).state_dict()


@pytest.mark.parametrize("mode,extra", [("pope", {}), ("pope", {"pope_fused": True}), ("fpope", {}),
                                        ("rope", {"rope_type": "yarn", "rope_scale": 4.0, "head_dim": 64}),
                                        ("nope", {})])
def test_oracle_decoder_single_token(mode, extra):
    """S = 1: softmax over one key is 1, so each attention is wo(wv(h)) whatever the PE: the
    decoder reduces to embedding -> (x + wo wv norm(x), x + ffn) -> head."""
    c, sd = _tiny(mode, **extra)
    ids = torch.tensor([[5], [42]])
    got = O.decoder_forward(sd, c, ids)["logits"]
    w = {k: v.float() for k, v in sd.items()}
    x = w["token_embedding.embedding.weight"][ids]
    for i in range(c.num_layers):
        p = f"layers.{i}."
        h = O.rms_norm(x, w[p + "attention_norm.weight"])
        x = x + _gqa_v(h, w, p, c)
        h = O.rms_norm(x, w[p + "ffn_norm.weight"])
        f = p + "feed_forward."
        x = x + (torch.nn.functional.silu(h @ w[f + "w3.weight"].T) * (h @ w[f + "w1.weight"].T)) @ w[f + "w2.weight"].T
    ref = O.rms_norm(x, w["norm.weight"]) @ w["output.weight"].T
    assert (got - ref).abs().max().item() < 1e-5


def _gqa_v(h, w, p, c):
    """wo applied to the per-query-head copy of the kv head's value (head h reads kv head h // g)."""
    D, g = c.head_dim, c.num_heads // c.num_kv_heads
    v = (h @ w[p + "attention.wv.weight"].T).view(*h.shape[:-1], c.num_kv_heads, D)
    v = v.repeat_interleave(g, dim=-2).reshape(*h.shape[:-1], c.num_heads * D)
    return v @ w[p + "attention.wo.weight"].T


def test_oracle_decoder_zero_layers_and_loss_at_init():
    c, sd = _tiny("pope", num_layers=0)
    ids = torch.randint(0, 97, (1, 12), generator=torch.Generator().manual_seed(0))
    r = O.decoder_forward(sd, c, ids, labels=ids)
    emb = sd["token_embedding.embedding.weight"]
    ref = O.rms_norm(emb[ids], sd["norm.weight"]) @ emb.T
    assert (r["logits"] - ref).abs().max().item() < 1e-6
    # N(0, 0.02^2) weights: logits are ~0, so the loss is ln(vocab) to within a few hundredths
    c, sd = _tiny("pope", vocab_size=512)
    ids = torch.randint(0, 512, (1, 40), generator=torch.Generator().manual_seed(1))
    assert abs(O.decoder_forward(sd, c, ids, labels=ids)["loss"].item() - math.log(512)) < 0.05


def test_oracle_decoder_causal_prefix():
    """Causality: logits of a prefix do not depend on the tokens after it."""
    c, sd = _tiny("pope", pope_delta_init="uniform")
    a = torch.randint(0, 97, (1, 20), generator=torch.Generator().manual_seed(2))
    b = a.clone()
    b[0, 12:] = (b[0, 12:] + 1) % 97
    la, lb = O.decoder_forward(sd, c, a)["logits"], O.decoder_forward(sd, c, b)["logits"]
    assert torch.allclose(la[:, :12], lb[:, :12], atol=1e-6)
    assert not torch.allclose(la[:, 12:], lb[:, 12:], atol=1e-3)


def test_next_token_sampling_rules():
    """The sampling rules of generate (src/model/transformer.py:389-446): temperature 0 is argmax;
    top-k keeps the k largest logits; nucleus filtering drops a token once the probability mass
    ranked above it exceeds top_p, so the most likely token always survives."""
    from pe_ablations_amd.transformer import _next_token
    torch.manual_seed(0)
    logits = torch.tensor([[0.0, 3.0, 1.0, 2.9, -1.0], [5.0, 0.0, 0.0, 0.0, 4.0]])
    assert _next_token(logits, 0.0, None, None).tolist() == [[1], [0]]
    for _ in range(20):
        assert _next_token(logits, 1.0, 1, None).tolist() == [[1], [0]]
        assert _next_token(logits, 1.0, None, 1e-6).tolist() == [[1], [0]]
        assert _next_token(logits, 0.7, 2, None)[0].item() in (1, 3)
    # top_p = 0.6: row 0 mass is (0.45, 0.41, ...) -> tokens 1 and 3 survive, nothing else
    picks = {int(_next_token(logits[:1], 1.0, None, 0.6).item()) for _ in range(200)}
    assert picks <= {1, 3} and len(picks) == 2
    counts = torch.bincount(torch.cat([_next_token(logits[1:], 1.0, None, None) for _ in range(400)]).flatten(),
                            minlength=5)
    assert counts[0] > counts[4] > 0 and counts[1:4].sum() < 40


def test_oracle_decoder_gate_order_and_prenorm_by_numbers():
    """The decoder oracle's SwiGLU gate order and pre-norm residuals pinned by numbers, not by a
    restated formula.  One layer, one token with embedding 2 * ones (RMS 2); with one key the
    attention output is wo wv h.  Every weight is zero except the final norm, the sub-layer norms
    (ones) and, in two separate runs:
      attention run: wv row 0 = ones / d (v0 = mean of h), wo[1, 0] = 1  -> adds v0 to dim 1;
      FFN run: w1 row 0 = 2 ones / d, w3 row 0 = 3 ones / d, w2[0, 0] = 0.5 -> adds 0.5 g to dim 0;
    output rows 0, 1, 2 = unit vectors 0, 1, 2 (the final RMSNorm keeps ratios).  The reference
    (src/model/transformer.py:205-206, src/model/ffn.py:27,68) normalises before each sub-layer and
    adds to the raw residual, so h = ones: v0 = 1, logit1 / logit2 = 3 / 2; g = silu(3) * 2 (silu on
    the w3 branch), logit0 / logit2 = (2 + silu(3)) / 2 with silu(3) = 3 / (1 + e^-3) =
    2.857722380...  A swapped gate gives (2 + 1.5 silu(2)) / 2; a sub-layer that reads the raw
    stream (no pre-norm, or a post-norm block) sees h = 2 ones and gives logit1 / logit2 = 2 and
    (2 + 2 silu(6)) / 2."""
    c, sd = _tiny("pope", num_layers=1, pope_fused=True)
    d = c.hidden_dim
    p, f = "layers.0.", "layers.0.feed_forward."

    def run(attn: bool):
        w = {k: torch.zeros_like(v) for k, v in sd.items()}
        for k in w:
            if k.endswith("norm.weight"):
                w[k] = torch.ones_like(w[k])
        w["token_embedding.embedding.weight"][7] = 2.0
        if attn:
            w[p + "attention.wv.weight"][0] = 1.0 / d
            w[p + "attention.wo.weight"][1, 0] = 1.0
        else:
            w[f + "w1.weight"][0] = 2.0 / d
            w[f + "w3.weight"][0] = 3.0 / d
            w[f + "w2.weight"][0, 0] = 0.5
        for i in range(3):
            w["output.weight"][i, i] = 1.0
        return O.decoder_forward(w, c, torch.tensor([[7]]))["logits"][0, 0].double()

    silu = lambda t: t / (1.0 + math.exp(-t))
    assert abs(silu(3.0) - 2.8577223804673) < 1e-12
    la, lf = run(True), run(False)
    # h = 2 / sqrt(4 + eps) per dim: the RMSNorm eps moves the ratios by < 1e-6
    assert abs(la[1] / la[2] - 1.5) < 1e-5
    assert abs(lf[0] / lf[2] - (2.0 + 0.5 * 2.0 * silu(3.0)) / 2.0) < 1e-5
    for wrong in ((2.0 + 0.5 * 3.0 * silu(2.0)) / 2.0, (2.0 + 0.5 * 4.0 * silu(6.0)) / 2.0):
        assert abs(lf[0] / lf[2] - wrong) > 0.1
