"""Drop-in for src/model/embeddings.py: TokenEmbedding (parameter ``embedding.weight``), whose
weight the Transformer ties to its output projection (src/model/embeddings.py:7-34)."""

import torch
import torch.nn as nn


class TokenEmbedding(nn.Module):
    def __init__(self, vocab_size: int, embed_dim: int):
        super().__init__()
        self.vocab_size = vocab_size
        self.embed_dim = embed_dim
        self.embedding = nn.Embedding(vocab_size, embed_dim)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.embedding(x)

    @property
    def weight(self) -> torch.Tensor:
        return self.embedding.weight
