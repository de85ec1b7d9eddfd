"""Phase-separated timing of the token loop (minitp/bench/benchmark.py:58-194).

``bench_one_iter`` keeps the reference's windows: TTFT is one event pair
from before ``prefill()`` to after the first ``select_next()`` with no sync
inside; each TPOT sample brackets ``append + decode_step + select_next``.
Percentiles are nearest-rank. Model loading from the HF hub (the rest of the
reference module) is not part of this build: workloads use seeded synthetic
models (minitp.synthetic).
"""

from __future__ import annotations

import time

import torch

from minitp.distributed.context import ParallelContext
from minitp.generation import GenerationState


def _percentiles(samples: list[float]) -> dict | None:
    """benchmark.py:58-74 (nearest rank)."""
    if not samples:
        return None
    xs = sorted(samples)

    def pct(q: float) -> float:
        idx = max(0, min(len(xs) - 1, round(q * len(xs)) - 1 if q > 0 else 0))
        return round(xs[idx], 3)

    return {"mean": round(sum(xs) / len(xs), 3), "p50": pct(0.50), "p90": pct(0.90), "p99": pct(0.99),
            "min": round(xs[0], 3), "max": round(xs[-1], 3)}


def bench_one_iter(model, input_ids, max_new_tokens, distributed_argmax=True, kv_init="empty"):
    """One fixed-length generation through GenerationState (benchmark.py:97-158).

    Returns (prefill_s, ttft_s, first_selection_ms, step_ms list)."""
    use_cuda = input_ids.device.type == "cuda"
    state = GenerationState(model, input_ids, max_new_tokens, distributed_argmax=distributed_argmax,
                            kv_init=kv_init)
    if use_cuda:
        ttft0 = torch.cuda.Event(True)
        prefill0, prefill1 = torch.cuda.Event(True), torch.cuda.Event(True)
        sel1 = torch.cuda.Event(True)
        ttft0.record()
        prefill0.record()
    else:
        t0 = time.perf_counter()
    logits = state.prefill()
    if use_cuda:
        prefill1.record()
    else:
        prefill_s = time.perf_counter() - t0
        t0 = time.perf_counter()
    tok = state.select_next(logits)
    if use_cuda:
        sel1.record()
        torch.cuda.synchronize()
        ttft_s = ttft0.elapsed_time(sel1) / 1e3
        prefill_s = prefill0.elapsed_time(prefill1) / 1e3
        first_selection_ms = prefill1.elapsed_time(sel1)
    else:
        first_selection_ms = (time.perf_counter() - t0) * 1e3
        ttft_s = prefill_s + first_selection_ms / 1e3
    events = []
    for _ in range(max_new_tokens - 1):
        if use_cuda:
            s, e = torch.cuda.Event(True), torch.cuda.Event(True)
            s.record()
        else:
            t0 = time.perf_counter()
        pos = state.append(tok)
        logits = state.decode_step(tok, pos)
        tok = state.select_next(logits)
        if use_cuda:
            e.record()
            events.append((s, e))
        else:
            events.append(time.perf_counter() - t0)
    if use_cuda:
        torch.cuda.synchronize()
        step_ms = [s.elapsed_time(e) for s, e in events]
    else:
        step_ms = [x * 1e3 for x in events]
    return prefill_s, ttft_s, first_selection_ms, step_ms


def _aggregate_max(ctx: ParallelContext, samples: list[float]) -> list[float]:
    """Element-wise MAX across ranks (benchmark.py:161-172); one rank here."""
    if ctx.tp_size == 1 or ctx.process_group is None:
        return samples
    raise NotImplementedError("multi-rank aggregation: tensor parallelism > 1 is not built on MI355X")


def _feature_flags(model, ctx: ParallelContext, loader: str, argmax_encoding: str) -> dict:
    """Flags read from the live objects (benchmark.py:175-194)."""
    impls = sorted({layer.input_layernorm.implementation for layer in model.model.layers})
    return {
        "fused_qkv": bool(model.model.layers[0].self_attn.use_fused_qkv),
        "fused_gate_up": bool(model.model.layers[0].mlp.use_fused_gateup),
        "rope_cache": bool(model.use_rotary_cache),
        "rmsnorm_backend": impls[0] if len(impls) == 1 else impls,
        "argmax_encoding": argmax_encoding,
        "loader": loader,
        "inference_mode": True,
        "kv_init": "empty",
        "comm_backend": "none",
        "nccl_available": False,
        "cuda_graph": bool(model.native_path()),
        "compile": False,
        "native_program": bool(model.native_path()),
    }
