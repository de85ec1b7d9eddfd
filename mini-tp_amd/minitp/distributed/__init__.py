"""The process context of minitp/distributed (context.py:18-42) at tp_size == 1.

A single GPU needs no collectives: with no process group the reference's
wrappers return without communicating (collectives.py:148-150), so the
layers here call none, and a tensor-parallel context is refused where a
layer is built.
"""

from minitp.distributed.context import ParallelContext, init_context

__all__ = ["ParallelContext", "init_context"]
