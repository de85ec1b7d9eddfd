"""Tensor-parallel layers at tp_size == 1, backed by the minitp HIP kernels."""

from minitp.parallel.embedding import VocabParallelEmbedding, VocabParallelLMHead
from minitp.parallel.linear import ColumnParallelLinear, RowParallelLinear

__all__ = ["ColumnParallelLinear", "RowParallelLinear", "VocabParallelEmbedding", "VocabParallelLMHead"]
