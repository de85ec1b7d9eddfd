"""ParallelContext (minitp/distributed/context.py:18-78), tp_size == 1 only.

This build serves one GPU: a context with tp_size > 1 can be constructed (the
reference's tests build such contexts to reach pre-collective validation),
but any layer that would need a collective refuses it.
"""

from __future__ import annotations

import os
from dataclasses import dataclass

import torch


@dataclass
class ParallelContext:
    global_rank: int
    local_rank: int
    world_size: int
    tp_rank: int
    tp_size: int
    device: torch.device
    process_group: object | None  # None => TP=1, no collectives

    @property
    def is_rank_zero(self) -> bool:
        return self.global_rank == 0

    @property
    def has_tp(self) -> bool:
        return self.tp_size > 1

    def barrier(self) -> None:
        if self.process_group is not None:
            import torch.distributed as dist

            dist.barrier(self.process_group)

    def destroy(self) -> None:
        import torch.distributed as dist

        if dist.is_initialized():
            dist.destroy_process_group()


def init_context(backend: str | None = None) -> ParallelContext:
    """Standalone TP=1 context on the ROCm device (context.py:45-78). A
    multi-rank launch (WORLD_SIZE > 1) is refused: TP > 1 is not built."""
    world = int(os.environ.get("WORLD_SIZE", "1"))
    rank = int(os.environ.get("RANK", "0"))
    local_rank = int(os.environ.get("LOCAL_RANK", "0"))
    if world != 1:
        raise NotImplementedError(f"WORLD_SIZE={world}: this MI355X build runs tensor parallelism 1 only")
    force_cpu = os.environ.get("MINITP_BACKEND", "").lower() == "gloo"
    device = torch.device("cpu" if force_cpu or not torch.cuda.is_available() else "cuda")
    return ParallelContext(rank, local_rank, 1, 0, 1, device, None)
