"""Qwen2 model configuration (the ``ModelConfig`` interface of minitp/config.py:17-112).

Field names, defaults, the frozen dataclass and the validation messages are
the reference's interface (callers match on "divisible" / "incompatible").
Reading a Hugging Face ``config.json`` goes through one table of
(field, source key, fallback) entries, so the same reader serves a
``transformers`` config object and a plain dict.
"""

from __future__ import annotations

from collections.abc import Mapping
from dataclasses import dataclass, fields
from typing import Any

from minitp.distributed.context import ParallelContext

# field -> (key in config.json, fallback when the key is absent or null)
_MISSING = object()


def _head_dim_fallback(src: dict) -> int:
    return src["hidden_size"] // src["num_attention_heads"]


def _theta_fallback(src: dict) -> float:
    # transformers >= 5 moved rope_theta into the rope_parameters dict
    params = src.get("rope_parameters") or {}
    return params["rope_theta"]


_HF_KEYS: dict[str, tuple[str, Any]] = {
    "hidden_size": ("hidden_size", _MISSING),
    "intermediate_size": ("intermediate_size", _MISSING),
    "num_hidden_layers": ("num_hidden_layers", _MISSING),
    "num_attention_heads": ("num_attention_heads", _MISSING),
    "num_key_value_heads": ("num_key_value_heads", _MISSING),
    "head_dim": ("head_dim", _head_dim_fallback),
    "vocab_size": ("vocab_size", _MISSING),
    "rms_norm_eps": ("rms_norm_eps", _MISSING),
    "rope_theta": ("rope_theta", _theta_fallback),
    "max_position_embeddings": ("max_position_embeddings", _MISSING),
    "tie_word_embeddings": ("tie_word_embeddings", True),
}


def _as_dict(hf_config) -> dict:
    if isinstance(hf_config, Mapping):
        return dict(hf_config)
    if hasattr(hf_config, "to_dict"):
        return dict(hf_config.to_dict())
    return dict(vars(hf_config))


@dataclass(frozen=True)
class ModelConfig:
    hidden_size: int
    intermediate_size: int
    num_hidden_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    head_dim: int
    vocab_size: int
    rms_norm_eps: float
    rope_theta: float
    max_position_embeddings: int
    tie_word_embeddings: bool = True

    @classmethod
    def from_hf(cls, hf_config, tp_size: int = 1) -> ModelConfig:
        """From a transformers ``Qwen2Config`` (or the dict of a config.json),
        validated for ``tp_size``."""
        src = _as_dict(hf_config)
        values = {}
        for f in fields(cls):
            key, fallback = _HF_KEYS[f.name]
            v = src.get(key)
            if v is None:
                if fallback is _MISSING:
                    raise KeyError(f"config has no {key!r}")
                v = fallback(src) if callable(fallback) else fallback
            values[f.name] = v
        values["rope_theta"] = float(values["rope_theta"])
        cfg = cls(**values)
        cfg.validate(tp_size)
        return cfg

    def _tp_split_sizes(self) -> tuple[tuple[str, int], ...]:
        return (("hidden_size", self.hidden_size), ("num_attention_heads", self.num_attention_heads),
                ("intermediate_size", self.intermediate_size))

    def validate(self, tp_size: int) -> None:
        """Raise ValueError when tensor parallelism of ``tp_size`` cannot
        split this model evenly."""
        uneven = [(n, v) for n, v in self._tp_split_sizes() if v % tp_size]
        if uneven:
            name, value = uneven[0]
            raise ValueError(f"{name}={value} not divisible by tp_size={tp_size}; "
                             "tensor-parallel sharding would be incorrect")
        kv = self.num_key_value_heads
        shards, replicates = kv % tp_size == 0, tp_size % kv == 0
        if not (shards or replicates):
            raise ValueError(f"num_key_value_heads={kv} incompatible with tp_size={tp_size}: "
                             "need kv%tp==0 (shard) or tp%kv==0 (replicate)")

    def local_heads(self, tp_size: int) -> tuple[int, int]:
        """(query heads, KV heads) held by one rank; KV heads never drop below one."""
        kv_local = self.num_key_value_heads // tp_size
        return self.num_attention_heads // tp_size, kv_local if kv_local else 1

    def kv_replication(self, tp_size: int) -> int:
        """Number of ranks holding a copy of each KV head (1 when they shard)."""
        return max(1, tp_size // self.num_key_value_heads)


def tiny_config(tp_size: int = 1) -> ModelConfig:
    """The reference's tiny layer-test model (config.py:81-97): hidden 64,
    2 layers, 4 query / 2 KV heads of 16, vocab 128, untied head."""
    cfg = ModelConfig(64, 128, 2, 4, 2, 16, 128, 1e-6, 10000.0, 256, False)
    cfg.validate(tp_size)
    return cfg


def context_for(tp_size: int, device: str = "cpu") -> ParallelContext:
    """A single-process context (config.py:100-112): rank 0 of one, no
    process group, whatever tp_size is asked for."""
    import torch

    del tp_size  # one process: always tp_size 1
    return ParallelContext(0, 0, 1, 0, 1, torch.device(device), None)
