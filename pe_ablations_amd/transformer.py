"""Drop-in for src/model/transformer.py: TransformerConfig, TransformerBlock, Transformer.

Same config fields, module tree and state-dict names as the reference (token_embedding.embedding,
layers.N.{attention_norm, attention, ffn_norm, feed_forward}, norm, output, and the one shared PE
module registered as ``rope`` / ``fpope`` / ``pope`` and again under every layer's attention), so a
checkpoint written by the reference's trainer loads with ``load_state_dict`` unchanged
(src/model/transformer.py:109-301).  The attention of every layer is the library's fused HIP
kernel; the projections, norms, SwiGLU and the LM head are torch ops (hipBLASLt GEMMs).

One addition: ``pope_fused`` (default False).  When True, pe_mode "pope" / "pope_floor" layers use
the fused form of the legacy API, all ``head_dim`` dims PoPE-encoded with no content half (the
shape of the 1B long-context configuration), instead of the reference's content + ``pope_d_rope``
split.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Literal, Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from .attention import GroupedQueryAttention
from .embeddings import TokenEmbedding
from .ffn import FeedForward
from .fpope import FoPEPoPEEmbedding
from .fpope_attention import FPoPEGroupedQueryAttentionWithCache
from .normalization import RMSNorm
from .pope import PoPEEmbedding
from .rope import NTKAwareRotaryEmbedding, RotaryEmbedding, YaRNRotaryEmbedding


@dataclass
class TransformerConfig:
    """Fields and defaults of src/model/transformer.py:21-106, plus ``pope_fused``."""

    vocab_size: int = 50257
    hidden_dim: int = 512
    num_layers: int = 24
    num_heads: int = 8
    num_kv_heads: int = 4
    head_dim: int = 64
    ffn_dim: Optional[int] = None
    ffn_multiple_of: int = 256

    pe_mode: Literal["rope", "fpope", "pope", "pope_floor", "alibi", "nope"] = "rope"
    max_seq_len: int = 512

    rope_theta: float = 10000.0
    rope_type: Literal["standard", "ntk", "yarn"] = "standard"
    rope_scale: float = 1.0

    fpope_theta: float = 10000.0
    fpope_num_fourier_terms: int = 64
    fpope_sigma: float = 0.4
    fpope_training_length: int = 512
    fpope_delta_init: str = "zero"
    fpope_d_rope: int = 32
    fpope_freeze_coeffs: bool = False
    fpope_use_ceiling: bool = False
    fpope_normalize_coeffs: bool = True

    pope_theta: float = 10000.0
    pope_training_length: int = 512
    pope_delta_init: str = "zero"
    pope_d_rope: int = 32
    pope_fused: bool = False

    norm_eps: float = 1e-6
    use_qk_norm: bool = True
    dropout: float = 0.0
    tie_embeddings: bool = True
    gradient_checkpointing: bool = False

    def __post_init__(self) -> None:
        if self.head_dim is None:
            self.head_dim = self.hidden_dim // self.num_heads

    @property
    def num_params(self) -> int:
        """The reference's estimate (src/model/transformer.py:79-106): it counts plain GQA
        projections for every pe_mode."""
        embed = self.vocab_size * self.hidden_dim
        attn = (self.hidden_dim * self.num_heads * self.head_dim
                + 2 * self.hidden_dim * self.num_kv_heads * self.head_dim
                + self.num_heads * self.head_dim * self.hidden_dim)
        ffn_dim = self.ffn_dim or int(4 * self.hidden_dim * 2 / 3)
        ffn_dim = self.ffn_multiple_of * ((ffn_dim + self.ffn_multiple_of - 1) // self.ffn_multiple_of)
        ffn = 3 * self.hidden_dim * ffn_dim
        norms = (2 * self.num_layers + 1) * self.hidden_dim
        total = embed + self.num_layers * (attn + ffn) + norms
        if not self.tie_embeddings:
            total += self.vocab_size * self.hidden_dim
        return total


def _pope_dims(config: TransformerConfig) -> tuple[int, Optional[int]]:
    """(d_rope, d_content) of pe_mode "pope" / "pope_floor" layers."""
    if config.pope_fused:
        return config.head_dim, 0
    return config.pope_d_rope, None


class TransformerBlock(nn.Module):
    """Pre-RMSNorm block: x + attn(norm(x)), then x + ffn(norm(x)) (src/model/transformer.py:109-205)."""

    def __init__(self, config: TransformerConfig, rope: Optional[nn.Module] = None,
                 fpope: Optional[nn.Module] = None, pope: Optional[nn.Module] = None):
        super().__init__()
        self.attention_norm = RMSNorm(config.hidden_dim, eps=config.norm_eps)
        mode = config.pe_mode
        if mode == "fpope":
            self.attention = FPoPEGroupedQueryAttentionWithCache(
                hidden_dim=config.hidden_dim, num_heads=config.num_heads, num_kv_heads=config.num_kv_heads,
                head_dim=config.head_dim, d_rope=config.fpope_d_rope, use_qk_norm=config.use_qk_norm,
                fpope=fpope)
        elif mode in ("pope", "pope_floor"):
            d_rope, d_content = _pope_dims(config)
            self.attention = FPoPEGroupedQueryAttentionWithCache(
                hidden_dim=config.hidden_dim, num_heads=config.num_heads, num_kv_heads=config.num_kv_heads,
                head_dim=config.head_dim, d_rope=d_rope, use_qk_norm=config.use_qk_norm, fpope=pope,
                d_content=d_content)
        elif mode == "alibi":
            raise NotImplementedError(
                "pe_mode 'alibi' (src/model/alibi.py) is not part of this library: it adds a bias to "
                "the scores instead of transforming q/k, and has no fused kernel here")
        elif mode == "nope":
            self.attention = GroupedQueryAttention(
                hidden_dim=config.hidden_dim, num_heads=config.num_heads, num_kv_heads=config.num_kv_heads,
                head_dim=config.head_dim, use_qk_norm=config.use_qk_norm, rope=None)
        else:
            self.attention = GroupedQueryAttention(
                hidden_dim=config.hidden_dim, num_heads=config.num_heads, num_kv_heads=config.num_kv_heads,
                head_dim=config.head_dim, use_qk_norm=config.use_qk_norm, rope=rope)
        self.ffn_norm = RMSNorm(config.hidden_dim, eps=config.norm_eps)
        self.feed_forward = FeedForward(hidden_dim=config.hidden_dim, ffn_dim=config.ffn_dim,
                                        multiple_of=config.ffn_multiple_of)

    def forward(self, x: torch.Tensor, mask: Optional[torch.Tensor] = None, start_pos: int = 0,
                use_cache: bool = False) -> torch.Tensor:
        """``use_cache`` routes the attention through its KV cache."""
        h = self.attention_norm(x)
        a = self.attention(h, mask, start_pos, use_cache=True) if use_cache else self.attention(h, mask, start_pos)
        x = x + a
        x = x + self.feed_forward(self.ffn_norm(x))
        return x


class Transformer(nn.Module):
    """Decoder-only LM (src/model/transformer.py:208-446): token embedding, ``num_layers`` blocks
    sharing one PE module, final RMSNorm, LM head (tied to the embedding by default)."""

    def __init__(self, config: TransformerConfig):
        super().__init__()
        self.config = config
        self.token_embedding = TokenEmbedding(config.vocab_size, config.hidden_dim)
        self.rope = None
        self.fpope = None
        self.pope = None
        mode = config.pe_mode
        if mode == "rope":
            if config.rope_type == "standard":
                self.rope = RotaryEmbedding(config.head_dim, config.max_seq_len, config.rope_theta)
            elif config.rope_type == "ntk":
                self.rope = NTKAwareRotaryEmbedding(config.head_dim, config.max_seq_len, config.rope_theta,
                                                    config.rope_scale)
            elif config.rope_type == "yarn":
                # the reference hard-codes the original length 512 (src/model/transformer.py:250-256)
                self.rope = YaRNRotaryEmbedding(config.head_dim, config.max_seq_len, config.rope_theta,
                                                config.rope_scale, original_max_seq_len=512)
            else:
                raise ValueError(f"Unknown rope_type: {config.rope_type}")
        elif mode == "fpope":
            self.fpope = FoPEPoPEEmbedding(
                dim=config.fpope_d_rope, max_seq_len=config.max_seq_len, theta=config.fpope_theta,
                num_fourier_terms=config.fpope_num_fourier_terms, fourier_sigma=config.fpope_sigma,
                training_length=config.fpope_training_length, delta_init=config.fpope_delta_init,
                freeze_coeffs=config.fpope_freeze_coeffs, use_ceiling=config.fpope_use_ceiling,
                normalize_coeffs=config.fpope_normalize_coeffs)
        elif mode in ("pope", "pope_floor"):
            d_rope, _ = _pope_dims(config)
            self.pope = PoPEEmbedding(dim=d_rope, max_seq_len=config.max_seq_len, theta=config.pope_theta,
                                      training_length=config.pope_training_length,
                                      use_floor=(mode == "pope_floor"), delta_init=config.pope_delta_init)
        elif mode in ("alibi", "nope"):
            pass
        else:
            raise ValueError(f"Unknown pe_mode: {mode}")
        self.layers = nn.ModuleList([TransformerBlock(config, rope=self.rope, fpope=self.fpope, pope=self.pope)
                                     for _ in range(config.num_layers)])
        self.norm = RMSNorm(config.hidden_dim, eps=config.norm_eps)
        self.output = nn.Linear(config.hidden_dim, config.vocab_size, bias=False)
        if config.tie_embeddings:
            self.output.weight = self.token_embedding.weight
        self.gradient_checkpointing = config.gradient_checkpointing
        self._init_weights()

    def _init_weights(self) -> None:
        """N(0, 0.02^2) for every Linear and Embedding weight, zero biases (src/model/transformer.py:303-311)."""
        for module in self.modules():
            if isinstance(module, nn.Linear):
                torch.nn.init.normal_(module.weight, mean=0.0, std=0.02)
                if module.bias is not None:
                    torch.nn.init.zeros_(module.bias)
            elif isinstance(module, nn.Embedding):
                torch.nn.init.normal_(module.weight, mean=0.0, std=0.02)

    def forward(self, input_ids: torch.Tensor, labels: Optional[torch.Tensor] = None,
                start_pos: int = 0, use_cache: bool = False) -> dict:
        """{'logits'} and, with ``labels``, {'loss'}: next-token cross entropy over the shifted
        sequence with ignore_index -100 (src/model/transformer.py:313-364).  ``use_cache``
        (an addition) feeds the tokens at absolute positions start_pos.. through
        every layer's KV cache, which must hold exactly start_pos earlier rows."""
        x = self.token_embedding(input_ids)
        for layer in self.layers:
            if self.gradient_checkpointing and self.training:
                x = torch.utils.checkpoint.checkpoint(layer, x, None, start_pos, use_reentrant=False)
            else:
                x = layer(x, mask=None, start_pos=start_pos, use_cache=use_cache)
        x = self.norm(x)
        logits = self.output(x)
        out = {"logits": logits}
        if labels is not None:
            shift_logits = logits[..., :-1, :].contiguous()
            shift_labels = labels[..., 1:].contiguous()
            out["loss"] = F.cross_entropy(shift_logits.view(-1, self.config.vocab_size), shift_labels.view(-1),
                                          ignore_index=-100)
        return out

    def extend_context_length(self, new_max_seq_len: int) -> None:
        """Extend the shared PE module's tables (src/model/transformer.py:366-378)."""
        for pe in (self.rope, self.fpope, self.pope):
            if pe is not None:
                pe.extend_seq_len(new_max_seq_len)
        self.config.max_seq_len = new_max_seq_len

    def reset_caches(self) -> None:
        for layer in self.layers:
            layer.attention.reset_cache()

    @torch.no_grad()
    def generate(self, input_ids: torch.Tensor, max_new_tokens: int = 100, temperature: float = 1.0,
                 top_k: Optional[int] = None, top_p: Optional[float] = None) -> torch.Tensor:
        """Autoregressive continuation of ``input_ids`` (B, P) by ``max_new_tokens`` tokens, with the
        reference's sampling semantics (src/model/transformer.py:389-446): greedy at temperature 0;
        otherwise logits / temperature, optional top-k, optional nucleus (top-p) filtering that
        always keeps the most likely token, then one multinomial draw.

        Unlike the reference, which re-runs the whole sequence for every new token, the prompt is
        run once (prefill) and every layer keeps a cache of transformed keys and values sized for
        P + max_new_tokens; each further step feeds one token through the caches (the split-key
        decode kernel).  As in the reference, the PE tables are extended only when the running
        length passes max_seq_len, to that length.  An extension that changes the kernel
        frequencies (YaRN reverts to the plain RoPE table) invalidates the cached rows, so the
        whole sequence is then run again through fresh caches, which is what the reference's
        full re-run computes.  The caches are freed on return."""
        self.eval()
        B, P = input_ids.shape
        total = P + max_new_tokens
        for layer in self.layers:
            layer.attention.max_cache_len = max(layer.attention.max_cache_len, total)

        def prefill(ids):
            self.reset_caches()
            return self.forward(ids, start_pos=0, use_cache=True)["logits"][:, -1, :]

        seq = input_ids
        try:
            if P > self.config.max_seq_len:
                self.extend_context_length(P)
            logits = prefill(seq)
            for step in range(max_new_tokens):
                nxt = _next_token(logits, temperature, top_k, top_p)
                seq = torch.cat([seq, nxt], dim=1)
                if step + 1 == max_new_tokens:
                    break
                n = seq.shape[1]
                if n > self.config.max_seq_len:
                    before = self._kernel_tables()
                    self.extend_context_length(n)
                    after = self._kernel_tables()
                    if any(not torch.equal(a, b) for a, b in zip(before, after)):
                        logits = prefill(seq)
                        continue
                logits = self.forward(nxt, start_pos=n - 1, use_cache=True)["logits"][:, -1, :]
        finally:
            self.reset_caches()
        return seq

    def _kernel_tables(self) -> list:
        """Copies of what the kernels read from the RoPE module (frequencies, mscale): rows cached
        under one set are invalid under another.  The PoPE / FoPE extensions only lengthen their
        position tables (src/model/pope.py:106-122, src/model/fpope.py:246-264); their frequencies
        and phase bias stay, so cached rows stay valid."""
        if self.rope is None:
            return []
        return [self.rope.kernel_inv_freq().detach().clone(), torch.tensor(self.rope.kernel_mscale())]


def _next_token(logits: torch.Tensor, temperature: float, top_k: Optional[int], top_p: Optional[float]) -> torch.Tensor:
    """(B, V) logits of the last position -> (B, 1) next token ids."""
    if temperature == 0.0:
        return logits.argmax(dim=-1, keepdim=True)
    z = logits / temperature
    if top_k is not None:
        kth = torch.topk(z, min(top_k, z.shape[-1]), dim=-1).values[:, -1:]
        z = z.masked_fill(z < kth, float("-inf"))
    if top_p is not None:
        # a token is dropped when the probability mass of the tokens ranked above it already
        # exceeds top_p, so the most likely token always survives
        probs, order = torch.sort(F.softmax(z, dim=-1), dim=-1, descending=True)
        mass_before = torch.cumsum(probs, dim=-1) - probs
        drop = torch.zeros_like(mass_before, dtype=torch.bool).scatter(-1, order, mass_before > top_p)
        z = z.masked_fill(drop, float("-inf"))
    return torch.multinomial(F.softmax(z, dim=-1), num_samples=1)
