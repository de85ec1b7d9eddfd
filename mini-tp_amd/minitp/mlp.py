"""Qwen2 SwiGLU MLP (minitp/mlp.py:18-38): packed gate/up, silu(gate)*up, down."""

from __future__ import annotations

import torch.nn as nn

from minitp import kernels as K
from minitp.config import ModelConfig
from minitp.distributed.context import ParallelContext
from minitp.parallel.fused import FusedGateUpColumnParallelLinear
from minitp.parallel.linear import RowParallelLinear


class TPQwen2MLP(nn.Module):
    def __init__(self, cfg: ModelConfig, ctx: ParallelContext, init_weights: bool = True) -> None:
        super().__init__()
        self.intermediate_local = cfg.intermediate_size // ctx.tp_size
        self.gate_up_proj = FusedGateUpColumnParallelLinear(cfg.hidden_size, self.intermediate_local, ctx, bias=False,
                                                            init_weights=init_weights)
        self.down_proj = RowParallelLinear(cfg.intermediate_size, cfg.hidden_size, ctx, bias=False,
                                           init_weights=init_weights)
        self.use_fused_gateup = True  # ablation toggle (mlp.py:32)

    def forward(self, x):
        y = self.gate_up_proj.project(x, fused=self.use_fused_gateup)
        n = self.intermediate_local
        return self.down_proj(K.silu_mul(y[..., :n], y[..., n:]))
