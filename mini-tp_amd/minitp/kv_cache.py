"""Contiguous KV cache (minitp/kv_cache.py:8-63).

One buffer each for K and V, laid out [layer, batch, kv_head, seq, head_dim]
so a whole forward's cache is one allocation the kernels index directly.
``k[i]`` / ``v[i]`` are the per-layer [B, Hkv, S, D] views of the reference
API. ``seq_len`` is the host-side fill cursor; only rows [0, seq_len) are
ever read (write-before-read, so ``init="empty"`` is safe).

The buffers hold ``capacity`` >= max_seq_len rows per (batch row, KV head):
max_seq_len rounded up to a power of two (a multiple of 8192 past 8192).
The kernels index the cache with that row stride, so the native program
records one decode graph per capacity rather than one per generation length
(a 128-token prompt with 200 or with 256 new tokens replays the same graph).
The views keep the reference's [B, Hkv, max_seq_len, D] shape, and every
bound (``update``, ``check_room``) is max_seq_len.
"""

from __future__ import annotations

import torch

from minitp import kernels as K


def cache_capacity(max_seq_len: int) -> int:
    """Rows the buffers hold for a cache of max_seq_len positions."""
    if max_seq_len <= 8192:
        return 1 << max(0, (max_seq_len - 1).bit_length())
    return -(-max_seq_len // 8192) * 8192


class KVCache:
    def __init__(self, num_layers: int, batch_size: int, kv_heads_local: int, head_dim: int, max_seq_len: int,
                 dtype: torch.dtype, device: torch.device, init: str = "empty") -> None:
        if init not in ("empty", "zeros"):
            raise ValueError(f"init must be 'empty' or 'zeros', got {init!r}")
        self.max_seq_len = max_seq_len
        self.capacity = cache_capacity(max_seq_len)
        self.seq_len = 0
        self.num_layers = num_layers
        shape = (num_layers, batch_size, kv_heads_local, self.capacity, head_dim)
        self.k_buf = torch.empty(shape, dtype=dtype, device=device)
        self.v_buf = torch.empty(shape, dtype=dtype, device=device)
        if init == "zeros":
            self._fill(0.0)
        self.k = [t[:, :, :max_seq_len] for t in self.k_buf.unbind(0)]
        self.v = [t[:, :, :max_seq_len] for t in self.v_buf.unbind(0)]

    def _fill(self, value: float) -> None:
        for buf in (self.k_buf, self.v_buf):
            if buf.is_cuda:
                K.fill_(buf, value)
            else:
                buf.fill_(value)

    def update(self, layer_idx: int, k_new: torch.Tensor, v_new: torch.Tensor):
        """Write [B, H, T, D] at the cursor; return the valid [:, :, :end] views."""
        t = k_new.shape[2]
        end = self.seq_len + t
        if end > self.max_seq_len:
            raise ValueError(f"KV cache overflow: seq {self.seq_len}+{t} > max_seq_len={self.max_seq_len}")
        K.kv_write(k_new, v_new, self.k[layer_idx], self.v[layer_idx], self.seq_len)
        return self.k[layer_idx][:, :, :end], self.v[layer_idx][:, :, :end]

    def check_room(self, t: int) -> None:
        if self.seq_len + t > self.max_seq_len:
            raise ValueError(f"KV cache overflow: seq {self.seq_len}+{t} > max_seq_len={self.max_seq_len}")

    def advance(self, tokens: int) -> None:
        self.seq_len += tokens

    def poison(self, value: float = float("nan")) -> None:
        """Test helper: fill every slot (written or not) with a sentinel."""
        self._fill(value)
