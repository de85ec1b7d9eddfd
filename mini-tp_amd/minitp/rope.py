"""Rotary position embedding, rotate_half convention (minitp/rope.py).

The fp32 cos/sin tables are built on the host with the reference's own op
sequence (rope.py:27-35), so their bits equal the reference CPU tables, and
are then copied to the device. Rotation runs in the minitp RoPE kernels.
"""

from __future__ import annotations

import torch

from minitp import _native as N
from minitp import kernels as K


def host_tables(head_dim: int, theta: float, positions: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """fp32 [len(positions), head_dim] cos / sin, computed on the CPU."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
    freqs = positions.float()[:, None] * inv_freq[None, :]
    emb = torch.cat([freqs, freqs], dim=-1)
    return emb.cos(), emb.sin()


def _check_positions(positions: torch.Tensor, limit: int) -> None:
    """Out-of-table positions must fail loudly (rope.py:37-45). Host check
    (it synchronises; the hot path checks positions on the host instead)."""
    if positions.numel() == 0:
        return
    lo, hi = int(positions.min()), int(positions.max())
    if lo < -limit or hi >= limit:
        raise IndexError(f"position {hi if hi >= limit else lo} out of range for RoPE table of {limit} rows")


class RotaryEmbedding:
    """Precomputed rotary tables for absolute positions [0, max_seq_len)."""

    def __init__(self, head_dim: int, theta: float, max_seq_len: int, device: torch.device | None = None) -> None:
        pos = torch.arange(max_seq_len, dtype=torch.float32)
        cos, sin = host_tables(head_dim, theta, pos)
        self.cos_cache = cos.to(device) if device is not None else cos
        self.sin_cache = sin.to(device) if device is not None else sin
        self.max_seq_len = max_seq_len
        self.head_dim = head_dim
        self.theta = theta

    def cos_sin(self, positions: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        return self.cos_cache[positions], self.sin_cache[positions]

    def apply(self, q: torch.Tensor, k: torch.Tensor, positions: torch.Tensor):
        """q [B, Hq, T, D], k [B, Hkv, T, D] -> rotated copies (dtype kept)."""
        _check_positions(positions, self.max_seq_len)
        N.require_gpu(q, k, what="RotaryEmbedding.apply")
        pos = positions.to(q.device).long()
        pos = torch.where(pos < 0, pos + self.max_seq_len, pos)
        return K.rope(q, k, self.cos_cache, self.sin_cache, pos)


def apply_rope(q: torch.Tensor, k: torch.Tensor, positions: torch.Tensor, theta: float):
    """Uncached RoPE (rope.py:67-88): tables for exactly these positions."""
    N.require_gpu(q, k, what="apply_rope")
    cos, sin = host_tables(q.shape[-1], theta, positions.cpu())
    idx = torch.arange(positions.numel(), device=q.device)
    return K.rope(q, k, cos.to(q.device), sin.to(q.device), idx)
