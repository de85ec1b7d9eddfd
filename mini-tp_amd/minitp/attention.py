"""Qwen2 GQA attention (minitp/attention.py:22-106) on the minitp kernels.

Module-level path: packed QKV projection, one kernel that splits q/k/v,
applies RoPE and writes k/v into the cache, GQA attention reading KV head
h // (Hq/Hkv) directly (no repeat_interleave copy), then o_proj.
"""

from __future__ import annotations

import torch
import torch.nn as nn

from minitp import kernels as K
from minitp.config import ModelConfig
from minitp.distributed.context import ParallelContext
from minitp.kv_cache import KVCache
from minitp.parallel.fused import FusedQKVColumnParallelLinear
from minitp.parallel.linear import RowParallelLinear
from minitp.rope import RotaryEmbedding, host_tables


class TPQwen2Attention(nn.Module):
    def __init__(self, cfg: ModelConfig, ctx: ParallelContext, init_weights: bool = True) -> None:
        super().__init__()
        self.cfg = cfg
        self.ctx = ctx
        tp = ctx.tp_size
        self.q_heads_local = cfg.num_attention_heads // tp
        self.kv_replication = cfg.kv_replication(tp)
        self.kv_heads_local = max(1, cfg.num_key_value_heads // tp)
        self.head_dim = cfg.head_dim
        self.q_local = self.q_heads_local * self.head_dim
        self.kv_local = self.kv_heads_local * self.head_dim
        self.qkv_proj = FusedQKVColumnParallelLinear(cfg.hidden_size, self.q_local, self.kv_local, ctx, bias=True,
                                                     init_weights=init_weights)
        self.o_proj = RowParallelLinear(cfg.hidden_size, cfg.hidden_size, ctx, bias=False,
                                        init_weights=init_weights)
        self.use_fused_qkv = True  # ablation toggle (attention.py:47)

    def forward(self, x: torch.Tensor, positions: torch.Tensor, kv_cache: KVCache | None, layer_idx: int,
                rotary: RotaryEmbedding | None = None) -> torch.Tensor:
        b, t, _ = x.shape
        hq, hkv, d = self.q_heads_local, self.kv_heads_local, self.head_dim
        if hq % hkv != 0:
            raise ValueError(f"local q heads {hq} not divisible by local kv heads {hkv}")
        y = self.qkv_proj.project(x, fused=self.use_fused_qkv)
        if kv_cache is not None:
            kv_cache.check_room(t)
            cache_len = kv_cache.seq_len
            kc, vc = kv_cache.k[layer_idx], kv_cache.v[layer_idx]
        else:
            cache_len = 0
            kc = torch.empty(b, hkv, t, d, dtype=x.dtype, device=x.device)
            vc = torch.empty_like(kc)
        if rotary is not None:
            cos, sin, pos = rotary.cos_cache, rotary.sin_cache, positions
        else:  # uncached RoPE: tables for exactly these positions (rope.py:67-88)
            cos, sin = host_tables(d, self.cfg.rope_theta, positions.cpu())
            cos, sin = cos.to(x.device), sin.to(x.device)
            pos = torch.arange(t, device=x.device)
        q = torch.empty(b, t, hq, d, dtype=x.dtype, device=x.device)
        K.rope_kv_write(y, q, kc, vc, cos, sin, pos, hq, hkv, cache_len)
        out = K.attention(q, kc, vc, cache_len)
        return self.o_proj(out)
