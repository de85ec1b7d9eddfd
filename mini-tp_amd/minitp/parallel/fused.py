"""Packed projections: one GEMV/GEMM over [q; k; v] or [gate; up] rows
(minitp/parallel/fused.py:26-113). The split afterwards is a zero-copy view.

The unfused ablation forms run one kernel per row block, written into
column slices of one output buffer, so the values are identical and only
the kernel count differs (fused.py:63-74, 106-113).
"""

from __future__ import annotations

import torch
import torch.nn as nn

from minitp import kernels as K
from minitp.distributed.context import ParallelContext


class FusedQKVColumnParallelLinear(nn.Module):
    def __init__(self, hidden_size: int, q_out_local: int, kv_out_local: int, ctx: ParallelContext, bias: bool = True,
                 init_weights: bool = True) -> None:
        super().__init__()
        if hidden_size % ctx.tp_size != 0:
            raise ValueError(f"hidden_size={hidden_size} not divisible by tp_size={ctx.tp_size}")
        self.hidden_size = hidden_size
        self.q_out_local = q_out_local
        self.kv_out_local = kv_out_local
        self.ctx = ctx
        out_rows = q_out_local + 2 * kv_out_local
        self.weight = nn.Parameter(torch.empty(out_rows, hidden_size))
        if bias:
            self.bias = nn.Parameter(torch.empty(out_rows))
        else:
            self.register_parameter("bias", None)
        if init_weights:
            nn.init.kaiming_uniform_(self.weight, a=5 ** 0.5)

    def out_features(self) -> int:
        return self.weight.shape[0]

    def _split(self, y: torch.Tensor):
        return torch.split(y, [self.q_out_local, self.kv_out_local, self.kv_out_local], dim=-1)

    def project(self, x: torch.Tensor, fused: bool = True) -> torch.Tensor:
        """The packed output y [..., q + 2 kv] (fused: one kernel; else three)."""
        if fused:
            return K.linear(x, self.weight, self.bias)
        y = torch.empty(*x.shape[:-1], self.weight.shape[0], dtype=x.dtype, device=x.device)
        q, kv = self.q_out_local, self.kv_out_local
        b = self.bias
        for lo, hi in ((0, q), (q, q + kv), (q + kv, q + 2 * kv)):
            K.linear(x, self.weight[lo:hi], b[lo:hi] if b is not None else None, out=y[..., lo:hi])
        return y

    def forward(self, x: torch.Tensor):
        return self._split(self.project(x, fused=True))

    def forward_unfused(self, x: torch.Tensor):
        return self._split(self.project(x, fused=False))


class FusedGateUpColumnParallelLinear(nn.Module):
    def __init__(self, hidden_size: int, intermediate_local: int, ctx: ParallelContext, bias: bool = False,
                 init_weights: bool = True) -> None:
        super().__init__()
        if intermediate_local * ctx.tp_size == 0 or hidden_size % ctx.tp_size != 0:
            raise ValueError(f"hidden_size={hidden_size} not divisible by tp_size={ctx.tp_size}")
        self.hidden_size = hidden_size
        self.intermediate_local = intermediate_local
        self.ctx = ctx
        self.weight = nn.Parameter(torch.empty(2 * intermediate_local, hidden_size))
        if bias:
            self.bias = nn.Parameter(torch.empty(2 * intermediate_local))
        else:
            self.register_parameter("bias", None)
        if init_weights:
            nn.init.kaiming_uniform_(self.weight, a=5 ** 0.5)

    def project(self, x: torch.Tensor, fused: bool = True) -> torch.Tensor:
        if fused:
            return K.linear(x, self.weight, self.bias)
        n = self.intermediate_local
        y = torch.empty(*x.shape[:-1], 2 * n, dtype=x.dtype, device=x.device)
        b = self.bias
        for lo, hi in ((0, n), (n, 2 * n)):
            K.linear(x, self.weight[lo:hi], b[lo:hi] if b is not None else None, out=y[..., lo:hi])
        return y

    def forward(self, x: torch.Tensor):
        return torch.chunk(self.project(x, fused=True), 2, dim=-1)

    def forward_unfused(self, x: torch.Tensor):
        return torch.chunk(self.project(x, fused=False), 2, dim=-1)
