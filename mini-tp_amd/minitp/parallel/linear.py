"""Column- and Row-parallel linear layers (minitp/parallel/linear.py:13-122).

Same constructor signatures, parameter names, layouts ([out, in] weights)
and divisibility errors as the reference. Forward runs the minitp GEMV (few
rows) or MFMA GEMM (many rows) kernel. This build runs tensor parallelism 1
only: a context with tp_size > 1 is refused at construction, so no layer
ever shards, splits its input or calls a collective.
"""

from __future__ import annotations

import torch
import torch.nn as nn

from minitp import kernels as K
from minitp.distributed.context import ParallelContext


def require_tp1(ctx: ParallelContext, what: str) -> None:
    if ctx.tp_size != 1:
        raise NotImplementedError(f"{what} at tp_size={ctx.tp_size}: this MI355X build runs tensor parallelism 1 only")


def shard_range(size: int, tp_rank: int, tp_size: int) -> tuple[int, int]:
    """Contiguous [start, end) slice for a rank; uneven sizes allowed (linear.py:13-17)."""
    base, rem = divmod(size, tp_size)
    start = tp_rank * base + min(tp_rank, rem)
    return start, start + base + (1 if tp_rank < rem else 0)


class ColumnParallelLinear(nn.Module):
    """Y = X W^T (+ b) with W's output dimension sharded (linear.py:20-70)."""

    def __init__(self, input_size: int, output_size: int, ctx: ParallelContext, bias: bool = True,
                 gather_output: bool = False, init_weights: bool = True) -> None:
        super().__init__()
        if output_size % ctx.tp_size != 0:
            raise ValueError(f"output_size={output_size} not divisible by tp_size={ctx.tp_size}")
        require_tp1(ctx, "ColumnParallelLinear")
        self.input_size = input_size
        self.output_size = output_size
        self.ctx = ctx
        self.gather_output = gather_output
        self.output_size_local = output_size // ctx.tp_size
        self.output_start, _ = shard_range(output_size, ctx.tp_rank, ctx.tp_size)
        self.weight = nn.Parameter(torch.empty(self.output_size_local, input_size))
        if bias:
            self.bias = nn.Parameter(torch.empty(self.output_size_local))
        else:
            self.register_parameter("bias", None)
        if init_weights:
            nn.init.kaiming_uniform_(self.weight, a=5 ** 0.5)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        # one rank holds every output column: gathering is the identity
        return K.linear(x, self.weight, self.bias)


class RowParallelLinear(nn.Module):
    """Y = X W^T with W's input dimension sharded; bias added once, after the
    (tp_size == 1: skipped) reduction, as its own rounding step (linear.py:73-122)."""

    def __init__(self, input_size: int, output_size: int, ctx: ParallelContext, bias: bool = True,
                 input_is_parallel: bool = True, reduce_output: bool = True, init_weights: bool = True) -> None:
        super().__init__()
        if input_size % ctx.tp_size != 0:
            raise ValueError(f"input_size={input_size} not divisible by tp_size={ctx.tp_size}")
        require_tp1(ctx, "RowParallelLinear")
        self.input_size = input_size
        self.output_size = output_size
        self.ctx = ctx
        self.input_is_parallel = input_is_parallel
        self.reduce_output = reduce_output
        self.input_size_local = input_size // ctx.tp_size
        self.weight = nn.Parameter(torch.empty(output_size, self.input_size_local))
        if bias:
            self.bias = nn.Parameter(torch.empty(output_size))
        else:
            self.register_parameter("bias", None)
        if init_weights:
            nn.init.kaiming_uniform_(self.weight, a=5 ** 0.5)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        # one rank holds every input column, so the product is the whole sum
        # (the reduction is the identity); the bias is still added after it,
        # as its own rounding step
        y = K.linear(x, self.weight)
        return K.add_bias(y, self.bias) if self.bias is not None else y
