"""Vocab-parallel embedding and LM head at tp_size == 1 (minitp/parallel/embedding.py).

The embedding gathers rows with a HIP kernel; the LM head is a HIP linear;
``distributed_argmax`` at tp_size == 1 is the first-maximum argmax
(embedding.py:146-147) as a HIP reduction. The multi-rank exchange encodings
(bitpack / fp32 / fp64 / split, embedding.py:149-213) need collectives and
are not built; their host-side guard still raises as the reference does.
"""

from __future__ import annotations

import torch
import torch.nn as nn

from minitp import kernels as K
from minitp.distributed import all_gather
from minitp.distributed.context import ParallelContext
from minitp.parallel.linear import shard_range

ARGMAX_ENCODING = "bitpack"


class VocabParallelEmbedding(nn.Module):
    def __init__(self, vocab_size: int, hidden_size: int, ctx: ParallelContext, init_weights: bool = True) -> None:
        super().__init__()
        self.vocab_size = vocab_size
        self.hidden_size = hidden_size
        self.ctx = ctx
        self.vocab_start, self.vocab_end = shard_range(vocab_size, ctx.tp_rank, ctx.tp_size)
        n = self.vocab_end - self.vocab_start
        self.weight = nn.Parameter(torch.zeros(n, hidden_size) if init_weights else torch.empty(n, hidden_size))
        # Ablation toggle of the reference. At tp_size == 1 its masked path
        # keeps every in-range row, so both settings gather the same rows.
        self.tp1_fast = True

    def forward(self, ids: torch.Tensor) -> torch.Tensor:
        if self.ctx.tp_size != 1:
            raise NotImplementedError("vocab-sharded embedding needs an all-reduce: tp_size > 1 is not built")
        return K.embedding(ids, self.weight)


class VocabParallelLMHead(nn.Module):
    def __init__(self, hidden_size: int, vocab_size: int, ctx: ParallelContext, gather_logits: bool = False,
                 init_weights: bool = True) -> None:
        super().__init__()
        self.vocab_size = vocab_size
        self.hidden_size = hidden_size
        self.ctx = ctx
        self.gather_logits = gather_logits
        self.vocab_start, self.vocab_end = shard_range(vocab_size, ctx.tp_rank, ctx.tp_size)
        n = self.vocab_end - self.vocab_start
        self.weight = nn.Parameter(torch.zeros(n, hidden_size) if init_weights else torch.empty(n, hidden_size))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        local = K.linear(x, self.weight)
        if not self.gather_logits or self.ctx.tp_size == 1:
            return local
        out = torch.empty(*local.shape[:-1], self.vocab_size, dtype=local.dtype, device=local.device)
        return all_gather(out, local, self.ctx.process_group)

    @torch.no_grad()
    def distributed_argmax(self, local_logits: torch.Tensor, encoding: str | None = None) -> torch.Tensor:
        """Greedy id [..., 1] (long): first maximum, NaN wins, like torch.argmax."""
        if self.ctx.tp_size == 1:
            return K.argmax(local_logits).unsqueeze(-1)
        enc = encoding or ARGMAX_ENCODING
        if enc == "fp32" and self.vocab_size > 2 ** 24:
            raise ValueError(f"fp32 argmax encoding cannot represent ids >= 2**24 exactly "
                             f"(vocab_size={self.vocab_size}); use the bitpack encoding")
        if enc not in ("bitpack", "fp32", "fp64", "split"):
            raise ValueError(f"unknown argmax encoding {enc!r}")
        raise NotImplementedError("distributed argmax over tp_size > 1 needs an all-gather: not built on MI355X")
