"""Vocab-parallel embedding and LM head at tp_size == 1 (minitp/parallel/embedding.py).

The embedding gathers rows with a HIP kernel; the LM head is a HIP linear;
``distributed_argmax`` at tp_size == 1 is the first-maximum argmax
(embedding.py:146-147) as a HIP reduction. A context with tp_size > 1 is
refused at construction: the multi-rank exchange encodings (bitpack / fp32 /
fp64 / split, embedding.py:149-213) have no counterpart here.
"""

from __future__ import annotations

import torch
import torch.nn as nn

from minitp import kernels as K
from minitp.distributed.context import ParallelContext
from minitp.parallel.linear import require_tp1, shard_range

ARGMAX_ENCODING = "bitpack"


class VocabParallelEmbedding(nn.Module):
    def __init__(self, vocab_size: int, hidden_size: int, ctx: ParallelContext, init_weights: bool = True) -> None:
        super().__init__()
        self.vocab_size = vocab_size
        self.hidden_size = hidden_size
        self.ctx = ctx
        require_tp1(ctx, "VocabParallelEmbedding")
        self.vocab_start, self.vocab_end = shard_range(vocab_size, ctx.tp_rank, ctx.tp_size)
        n = self.vocab_end - self.vocab_start
        self.weight = nn.Parameter(torch.zeros(n, hidden_size) if init_weights else torch.empty(n, hidden_size))
        # Ablation toggle of the reference. At tp_size == 1 its masked path
        # keeps every in-range row, so both settings gather the same rows.
        self.tp1_fast = True

    def forward(self, ids: torch.Tensor) -> torch.Tensor:
        return K.embedding(ids, self.weight)


class VocabParallelLMHead(nn.Module):
    def __init__(self, hidden_size: int, vocab_size: int, ctx: ParallelContext, gather_logits: bool = False,
                 init_weights: bool = True) -> None:
        super().__init__()
        self.vocab_size = vocab_size
        self.hidden_size = hidden_size
        self.ctx = ctx
        self.gather_logits = gather_logits
        require_tp1(ctx, "VocabParallelLMHead")
        self.vocab_start, self.vocab_end = shard_range(vocab_size, ctx.tp_rank, ctx.tp_size)
        n = self.vocab_end - self.vocab_start
        self.weight = nn.Parameter(torch.zeros(n, hidden_size) if init_weights else torch.empty(n, hidden_size))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        # one rank holds the whole vocabulary: gathered logits are the local ones
        return K.linear(x, self.weight)

    @torch.no_grad()
    def distributed_argmax(self, local_logits: torch.Tensor, encoding: str | None = None) -> torch.Tensor:
        """Greedy id [..., 1] (long): first maximum, NaN wins, like torch.argmax."""
        # one rank holds the whole vocabulary: the reference returns the local
        # argmax before any encoding is looked at (embedding.py:146-147)
        return K.argmax(local_logits).unsqueeze(-1)
