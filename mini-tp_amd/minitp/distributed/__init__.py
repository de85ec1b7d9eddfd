"""Collective wrappers (minitp/distributed/collectives.py:144-245) at tp_size == 1.

With no process group the reference wrappers return without communicating
(all_reduce / broadcast return the input, the gathers copy it into ``out``;
collectives.py:148-150, 165-167, 195-197, 224-226); that is all a single GPU
needs. A process group means tensor parallelism > 1, which is not built here.
"""

from __future__ import annotations

import torch

from minitp.distributed.context import ParallelContext, init_context

__all__ = ["ParallelContext", "init_context", "all_reduce", "all_gather", "all_gather_dim0", "reduce_scatter",
           "broadcast"]


def _no_group(pg, name: str) -> None:
    if pg is not None:
        raise NotImplementedError(f"{name} with a process group: tensor parallelism > 1 is not built on MI355X")


def all_reduce(t: torch.Tensor, pg=None, op=None) -> torch.Tensor:
    _no_group(pg, "all_reduce")
    return t


def all_gather(out: torch.Tensor, t: torch.Tensor, pg=None) -> torch.Tensor:
    _no_group(pg, "all_gather")
    out.copy_(t)
    return out


def all_gather_dim0(out: torch.Tensor, t: torch.Tensor, pg=None) -> torch.Tensor:
    _no_group(pg, "all_gather_dim0")
    out.copy_(t.unsqueeze(0))
    return out


def reduce_scatter(out: torch.Tensor, t: torch.Tensor, pg=None) -> torch.Tensor:
    _no_group(pg, "reduce_scatter")
    out.copy_(t)
    return out


def broadcast(t: torch.Tensor, src: int = 0, pg=None) -> torch.Tensor:
    _no_group(pg, "broadcast")
    return t
