"""Phase timing of one generation through ``GenerationState``.

The windows are mini-tp's (minitp/bench/benchmark.py:97-158):

* TTFT: from just before ``prefill()`` to just after the first
  ``select_next()``; nothing synchronises inside it;
* prefill: ``prefill()`` alone, nested inside TTFT;
* TPOT: one sample per later token, each covering ``append`` +
  ``decode_step`` + ``select_next``.

Percentiles use the reference's nearest-rank rule (benchmark.py:58-74).

Here every mark is a point on one timeline: a HIP event recorded on the
current stream when the prompt lives on a ROCm device, or a host
``perf_counter`` reading otherwise. GPU marks are resolved by one
synchronisation after the last token, so the decode steps are queued back to
back exactly as ``generate_greedy`` queues them. Loading checkpoints from the
Hugging Face hub (the rest of the reference module) is outside this build;
the workloads use seeded synthetic models (``minitp.synthetic``).
"""

from __future__ import annotations

import time
from dataclasses import dataclass, field

import torch

from minitp.generation import GenerationState


def _rank_index(q: float, n: int) -> int:
    """0-based index of the q-quantile among n sorted samples: the
    reference's ``round(q * n) - 1`` (Python rounding), clamped to the
    samples; q == 0 is the minimum."""
    if q <= 0:
        return 0
    return min(n - 1, max(0, round(q * n) - 1))


def percentiles(samples: list[float]) -> dict | None:
    """mean / p50 / p90 / p99 / min / max of the samples, rounded to 3 places."""
    if not samples:
        return None
    xs = sorted(samples)
    n = len(xs)
    out = {"mean": round(sum(xs) / n, 3)}
    for name, q in (("p50", 0.50), ("p90", 0.90), ("p99", 0.99)):
        out[name] = round(xs[_rank_index(q, n)], 3)
    out["min"] = round(xs[0], 3)
    out["max"] = round(xs[-1], 3)
    return out


class _Timeline:
    """Marks on one clock: HIP events (device) or perf_counter (host)."""

    def __init__(self, device_clock: bool) -> None:
        self.device_clock = device_clock
        self._marks: list = []

    def mark(self) -> int:
        if self.device_clock:
            ev = torch.cuda.Event(enable_timing=True)
            ev.record()
            self._marks.append(ev)
        else:
            self._marks.append(time.perf_counter())
        return len(self._marks) - 1

    def settle(self) -> None:
        if self.device_clock:
            torch.cuda.synchronize()

    def ms(self, a: int, b: int) -> float:
        """Milliseconds from mark a to mark b (after settle())."""
        x, y = self._marks[a], self._marks[b]
        return x.elapsed_time(y) if self.device_clock else (y - x) * 1e3


@dataclass
class IterTiming:
    prefill_s: float
    ttft_s: float
    first_selection_ms: float
    step_ms: list[float] = field(default_factory=list)

    def astuple(self) -> tuple[float, float, float, list[float]]:
        return self.prefill_s, self.ttft_s, self.first_selection_ms, self.step_ms


def time_generation(model, input_ids: torch.Tensor, max_new_tokens: int, distributed_argmax: bool = True,
                    kv_init: str = "empty", prefill_logits: str = "all") -> IterTiming:
    """One fixed-length generation of ``max_new_tokens`` tokens with the
    windows above. ``prefill_logits="all"`` is the reference's prefill
    (logits of every prompt position) and every decode step returns a new
    logits tensor; ``"last"`` runs the loop as generate_greedy does (last
    position's logits, one reused decode logits buffer)."""
    state = GenerationState(model, input_ids, max_new_tokens, distributed_argmax=distributed_argmax,
                            kv_init=kv_init, prefill_logits=prefill_logits,
                            reuse_decode_logits=prefill_logits == "last")
    clock = _Timeline(input_ids.device.type == "cuda")
    begin = clock.mark()
    logits = state.prefill()
    after_prefill = clock.mark()
    tok = state.select_next(logits)
    first = clock.mark()
    spans = []
    for _ in range(max_new_tokens - 1):
        s = clock.mark()
        pos = state.append(tok)
        logits = state.decode_step(tok, pos)
        tok = state.select_next(logits)
        spans.append((s, clock.mark()))
    clock.settle()
    return IterTiming(prefill_s=clock.ms(begin, after_prefill) / 1e3, ttft_s=clock.ms(begin, first) / 1e3,
                      first_selection_ms=clock.ms(after_prefill, first),
                      step_ms=[clock.ms(a, b) for a, b in spans])


def bench_one_iter(model, input_ids, max_new_tokens, distributed_argmax=True, kv_init="empty"):
    """The reference's entry point (benchmark.py:97-158): returns
    (prefill_s, ttft_s, first_selection_ms, step_ms list)."""
    return time_generation(model, input_ids, max_new_tokens, distributed_argmax, kv_init).astuple()
