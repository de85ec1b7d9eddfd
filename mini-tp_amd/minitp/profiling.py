"""Trace labels (minitp/profiling.py:21-42). Off by default; when enabled the
labels become torch.profiler ranges, which rocprofv3/roctracer also record."""

from __future__ import annotations

import contextlib

_ENABLED = False


def set_enabled(flag: bool) -> None:
    global _ENABLED
    _ENABLED = bool(flag)


def is_enabled() -> bool:
    return _ENABLED


def scope(name: str):
    if not _ENABLED:
        return contextlib.nullcontext()
    import torch

    return torch.profiler.record_function(name)
