"""Decode benchmark: Qwen2.5-0.5B-shape bf16, batch 1, 128-token prompt + 256 greedy tokens.

The workload is one generation of 256 greedy tokens after a 128-token
prompt, KV cache of 384 positions: the prefill picks token 1, then 255
decode steps (contexts 128 .. 382) pick tokens 2 .. 256. A *step* is one
decode token: append + decode_step + select_next, the reference's TPOT window
(minitp/bench/benchmark.py:138-157), replayed from the decode hipGraph.

Generations of this workload run back to back. The first W decode steps are
warm-up (the first of them captures the decode graph); the next K steps are
timed. When a generation's 255 steps run out, the next generation's prefill
runs with the clock stopped, so the timed region holds exactly K decode
steps, each at the context it has in the workload, bracketed by
torch.cuda.synchronize() on both sides of every timed stretch.

Reported beside the headline tok/s:
  * the HBM roofline of the timed steps (algorithmic bytes per token:
    weights once, LM head once, norms, QKV bias, KV read of ctx + 1
    positions) and of the dominant kernel (the fused RMSNorm + gate/up GEMV
    + SwiGLU, timed with HIP events on its stream; its HBM traffic from the
    committed rocprofv3 counter summary);
  * one whole generation timed with the reference's windows: TTFT, prefill
    tok/s, TPOT percentiles, peak device memory;
  * the other workloads (7B decode, 0.5B batch-32 decode, 7B 4 x 4096
    prefill), each with its roofline fraction;
  * the CPU baseline: the oracle restatement of the reference TP=1 loop on
    the host cores, per workload and dtype, over bounded samples.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (os.path.join(ROOT, "mini-tp_amd"), ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)

METRIC = "decode tok/s & % HBM roofline, Qwen2.5-0.5B-shape bf16 bs=1; p50 TTFT"
HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
PROMPT_LEN = 128
NEW_TOKENS = 256
DECODE_STEPS = NEW_TOKENS - 1  # token 1 comes from the prefill

# name -> (shape, batch, prompt tokens, new tokens); new tokens 1 = prefill only
WORKLOADS = {
    "q7b": ("QWEN7B", 1, 512, 256),
    "q05b-b32": ("QWEN05B", 32, 2048, 512),
    "q7b-prefill": ("QWEN7B", 4, 4096, 1),
}


def step_bytes(cfg, ctx: int, batch: int = 1, esize: int = 2) -> int:
    """Algorithmic HBM bytes of one decode step that reads `ctx` cached positions."""
    L, H, hq, hkv, d, inter, v = (cfg.num_hidden_layers, cfg.hidden_size, cfg.num_attention_heads,
                                  cfg.num_key_value_heads, cfg.head_dim, cfg.intermediate_size, cfg.vocab_size)
    p_stream = L * (H * (hq + 2 * hkv) * d + hq * d * H + 3 * inter * H) + v * H + H * (2 * L + 1) + L * (hq + 2 * hkv) * d
    kv = batch * esize * L * 2 * hkv * d * (ctx + 1)
    return esize * p_stream + kv


def prefill_flops(cfg, batch: int, t: int, all_logits: bool = False) -> float:
    """Dense FLOPs of a prefill of `t` tokens per row: the linear layers,
    causal attention (QK^T and PV over the visible keys) and the LM head of
    the last position only (what generate_greedy's prefill computes), or of
    every position with `all_logits` (the reference's prefill, layer.py:117-124)."""
    L, H, hq, hkv, d, inter, v = (cfg.num_hidden_layers, cfg.hidden_size, cfg.num_attention_heads,
                                  cfg.num_key_value_heads, cfg.head_dim, cfg.intermediate_size, cfg.vocab_size)
    m = batch * t
    linear = 2.0 * m * L * (H * (hq + 2 * hkv) * d + hq * d * H + 3 * inter * H)
    attn = 2.0 * 2.0 * batch * L * hq * d * (t * (t + 1) / 2)
    return linear + attn + 2.0 * batch * (t if all_logits else 1) * v * H


def parse(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=DECODE_STEPS, help="timed decode steps K")
    ap.add_argument("--warmup", type=int, default=DECODE_STEPS,
                    help="untimed decode steps W before them (at least 1: the first captures the decode graph)")
    ap.add_argument("--ttft-iters", type=int, default=10)
    ap.add_argument("--no-workloads", action="store_true", help="skip the 7B and batch-32 workloads")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget-s", type=float, default=10.0,
                    help="host seconds of decode steps per CPU-baseline sample (the prefill comes on top)")
    ap.add_argument("--cpu-configs", default="tiny-fp32,q05b-bf16,q05b-fp32,q7b-bf16,q7b-fp32",
                    help="comma-separated CPU-baseline samples")
    ap.add_argument("--workload", default="q05b", choices=["q05b", *sorted(WORKLOADS)],
                    help="q05b (default): the headline line; another name prints only that workload's line")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain copy of MIB MiB (the --pmc byte-counter calibration) and exit")
    ap.add_argument("--prefill-attention", type=int, default=0, metavar="ITERS",
                    help="only time the causal prefill attention of the 7B 4 x 4096 prefill (q [4, 4096, 28, 128], "
                         "4 KV heads, bf16) ITERS times after 3 warm-up calls, print one JSON line and exit")
    ap.add_argument("--dominant-only", action="store_true",
                    help="only launch the dominant kernel, eagerly (no graphs), once per layer 4 times over, and "
                         "exit: the workload of the --pmc byte-counter passes")
    ap.add_argument("--dominant-graph", type=int, default=0, metavar="REPS",
                    help="only run the roofline's timing of the dominant kernel (one captured graph of a launch per "
                         "layer, replayed REPS times), print its JSON and exit: the workload of the kernel-trace "
                         "summary that the roofline's us_per_launch is checked against")
    ap.add_argument("--gemm", default="", metavar="M,N,K[,swiglu]",
                    help="only time one bf16 product y = x W^T (minitp_linear; swiglu: W is [2N, K] and y = "
                         "silu(gate) * up) 10 times after 3 warm-up calls, print one JSON line and exit")
    ap.add_argument("--decode-only", type=int, default=0, metavar="TOKENS",
                    help="only run one generation of the headline workload with TOKENS new tokens after a warm-up "
                         "one and exit: the workload of the decode kernel profiles")
    ap.add_argument("--eager-decode", type=int, default=0, metavar="STEPS",
                    help="prefill the --workload's prompt, then run STEPS decode steps as eager launches (no graph) "
                         "and exit: the workload of the per-kernel counter passes")
    return ap.parse_args(argv)


def note(msg: str) -> None:
    """One progress line on stderr as a phase of the run finishes."""
    print(f"[bench {time.strftime('%H:%M:%S')}] {msg}", file=sys.stderr, flush=True)


# ---------------------------------------------------------------------------
# decode steps of back-to-back generations


class StepSource:
    """Decode steps of back-to-back generations of one workload. run(k)
    performs the next k steps and returns the seconds they took; prefills
    between generations run with the clock stopped."""

    def __init__(self, model, prompt, new_tokens: int) -> None:
        self.model, self.prompt, self.new_tokens = model, prompt, new_tokens
        self.state = None
        self.tok = None
        self.left = 0
        self.generations = 0
        self.contexts: list[int] = []  # cached positions before each step run so far

    def _next_generation(self) -> None:
        import torch

        from minitp.generation import GenerationState

        torch.cuda.synchronize()
        self.state = GenerationState(self.model, self.prompt, self.new_tokens, prefill_logits="last",
                                     reuse_decode_logits=True)  # as generate_greedy runs it
        self.tok = self.state.select_next(self.state.prefill())
        self.left = self.new_tokens - 1
        self.generations += 1
        torch.cuda.synchronize()

    def run(self, k: int) -> float:
        import torch

        seconds = 0.0
        while k > 0:
            if self.left == 0:
                self._next_generation()
            m = min(k, self.left)
            st, tok = self.state, self.tok
            start = st.cursor  # positions cached before the next step
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(m):
                pos = st.append(tok)
                tok = st.select_next(st.decode_step(tok, pos))
            torch.cuda.synchronize()
            seconds += time.perf_counter() - t0
            self.tok = tok
            self.contexts += range(start, start + m)
            self.left -= m
            k -= m
        return seconds


def one_generation(model, prompt, new_tokens: int, prefill_logits: str = "last") -> dict:
    """One generation with the reference's windows (TTFT, prefill, TPOT) and
    the peak device memory it reached."""
    import torch

    from minitp.bench.benchmark import percentiles, time_generation

    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    it = time_generation(model, prompt, new_tokens, prefill_logits=prefill_logits)
    b, t = prompt.shape
    tp = percentiles(it.step_ms)
    out = {"ttft_ms": round(it.ttft_s * 1e3, 3), "prefill_ms": round(it.prefill_s * 1e3, 3),
           "prefill_tok_s": round(b * t / it.prefill_s, 1), "tpot_ms": tp,
           "peak_memory_gib": round(torch.cuda.max_memory_allocated() / 2 ** 30, 3)}
    if tp:
        out["decode_tok_s"] = round(b * 1e3 / tp["mean"], 1)  # reference: B * 1e3 / TPOT mean
    return out


def ttft_samples(model, prompt, iters: int, prefill_logits: str) -> list[float]:
    """TTFT (prefill start -> first token selected) of `iters` prefills, ms."""
    import torch

    from minitp.generation import GenerationState

    out = []
    for _ in range(iters):
        st = GenerationState(model, prompt, 1, prefill_logits=prefill_logits)
        a, b = torch.cuda.Event(True), torch.cuda.Event(True)
        a.record()
        st.select_next(st.prefill())
        b.record()
        torch.cuda.synchronize()
        out.append(a.elapsed_time(b))
        del st
    return out


def p50(xs: list[float]) -> float:
    from minitp.bench.benchmark import percentiles

    return percentiles(xs)["p50"]


# ---------------------------------------------------------------------------
# the other workloads


def eager_decode(name: str, steps: int) -> dict:
    """Prefill one workload's prompt (last-position logits), then `steps`
    T = 1 forwards through the native program launched eagerly, each
    feeding back its greedy pick: the same kernels as the decode graph, one
    dispatch at a time, so counter profilers see every launch."""
    import torch

    from minitp import kernels as K
    from minitp import synthetic
    from minitp.generation import make_kv_cache

    shape, batch, plen, _ = ("QWEN05B", 1, PROMPT_LEN, NEW_TOKENS) if name == "q05b" else WORKLOADS[name]
    cfg = getattr(synthetic, shape)
    model = synthetic.build_synthetic_model(cfg, dtype=torch.bfloat16, device="cuda", seed=0)
    prompt = synthetic.synthetic_prompt(cfg.vocab_size, batch, plen, seed=0, device="cuda")
    kv = make_kv_cache(model, batch, plen + steps)
    logits = model._native(prompt, torch.arange(plen, device="cuda"), kv, last_only=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        tok = K.argmax(logits[:, -1]).view(batch, 1)
        logits = model(tok, kv_cache=kv)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    return {"workload": name, "eager_steps": steps, "contexts": [plen + 1, plen + steps],
            "ms_per_step": round(dt * 1e3 / max(steps, 1), 4)}


def measure_workload(name: str, model=None) -> dict:
    """Decode tok/s and step roofline (decode workloads) or TTFT and the
    dense-FLOP MFMA fraction (the prefill workload) of one workload, after
    one untimed run of it."""
    import torch

    from minitp import synthetic

    shape, batch, plen, new = WORKLOADS[name]
    cfg = getattr(synthetic, shape)
    out = {"shape": shape, "batch": batch, "prompt": plen, "new_tokens": new, "dtype": "bf16"}
    if model is None:
        model = synthetic.build_synthetic_model(cfg, dtype=torch.bfloat16, device="cuda", seed=0)
    prompt = synthetic.synthetic_prompt(cfg.vocab_size, batch, plen, seed=0, device="cuda")
    torch.cuda.synchronize()
    if new > 1:
        src = StepSource(model, prompt, new)
        src.run(new - 1)  # warm-up generation (graph capture for this batch / cache size)
        src.contexts.clear()
        dt = src.run(new - 1)
        total = sum(step_bytes(cfg, c, batch=batch) for c in src.contexts)
        steps = len(src.contexts)
        out.update({"decode_tok_s": round(batch * steps / dt, 1), "ms_per_step": round(dt * 1e3 / steps, 4),
                    "steps": steps, "step_roofline_frac": round(total / dt / 1e9 / HBM_PEAK_GBS, 4),
                    "roofline_tok_s": round(batch * HBM_PEAK_GBS * 1e9 / (total / steps), 1)})
        gen = one_generation(model, prompt, new)
        out.update({k: gen[k] for k in ("ttft_ms", "prefill_tok_s", "peak_memory_gib")})
        out["tpot_ms"] = gen["tpot_ms"]
    else:
        # a prompt shape runs its launches directly on its first call and
        # records its graph on the second; the timed samples are replays
        first = ttft_samples(model, prompt, 1, "last")
        ttft_samples(model, prompt, 1, "last")
        torch.cuda.reset_peak_memory_stats()
        xs = ttft_samples(model, prompt, 3, "last")
        fl = prefill_flops(cfg, batch, plen)
        ms = p50(xs)
        # the reference's semantics: every position's logits (never a graph: an
        # LM head this large stores to the pointer it is given)
        full = ttft_samples(model, prompt, 2, "all")
        fl_all = prefill_flops(cfg, batch, plen, all_logits=True)
        ms_all = p50(full)
        out.update({"ttft_ms": ms, "ttft_ms_all": [round(x, 3) for x in xs],
                    "ttft_samples": "graph replays (the shape's third and later calls)",
                    "ttft_first_call_ms": round(first[0], 3), "prefill_tflop": round(fl / 1e12, 2),
                    "prefill_tok_s": round(batch * plen / ms * 1e3, 1),
                    "mfma_frac": round(fl / (ms * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
                    "ttft_full_logits_ms": ms_all, "prefill_tflop_full_logits": round(fl_all / 1e12, 2),
                    "mfma_frac_full_logits": round(fl_all / (ms_all * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
                    "peak_memory_gib": round(torch.cuda.max_memory_allocated() / 2 ** 30, 3)})
    note(f"workload {name} done")
    return out


# ---------------------------------------------------------------------------
# the dominant kernel


DOMINANT = "gemv_reg_kernel<minitp::bf16, 1, 1, 2, 2, 2, 2>"  # PRO_PART_NORM, EPI_SWIGLU, 2 pairs a tuple: rocprofv3's name
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "gate_up_gemv_q05b_decode_traffic.json")


def _dominant_launcher(model):
    """Launches the dominant kernel once per layer on the current stream,
    with that layer's weights: the residual add of the o_proj partial rows
    (one per query head, as the fused attention leaves them), the RMSNorm,
    gate/up and SwiGLU (minitp_add_rmsnorm_linear_parts)."""
    import torch

    from minitp import _native as N

    cfg = model.cfg
    layers = list(model.model.layers)
    h, hq = cfg.hidden_size, cfg.num_attention_heads
    x = torch.randn(h, device="cuda").to(torch.bfloat16)
    parts = torch.randn(hq, h, device="cuda") * 0.05
    x_out = torch.empty_like(x)
    out = torch.empty(cfg.intermediate_size, dtype=torch.bfloat16, device="cuda")
    lib = N.lib()

    def launch_all():
        for layer in layers:
            N.check(lib.minitp_add_rmsnorm_linear_parts(
                N.stream(), N.BF16, x.data_ptr(), parts.data_ptr(), hq, x_out.data_ptr(),
                layer.post_attention_layernorm.weight.data_ptr(), cfg.rms_norm_eps,
                layer.mlp.gate_up_proj.weight.data_ptr(), out.data_ptr(), cfg.intermediate_size, h, N.EPI_SWIGLU),
                "add_rmsnorm_linear_parts")

    return launch_all


def dominant_kernel(model, reps: int = 20) -> dict:
    """The kernel with the largest share of a decode step: the residual add
    of the o_proj partials + RMSNorm + gate/up GEMV + SwiGLU, with the
    decode graph's per-layer weights, once per layer in a captured graph (no
    launch re-reads a cache-resident matrix, no host launch cost), timed with
    HIP events on the stream the graph replays on. The kernel alone, not
    between its neighbours in the step: the step's own per-kernel durations
    are in the rocprofv3 kernel-trace summary of the decode, and
    `--dominant-graph` runs this timing alone for a kernel-trace summary of
    it."""
    import torch

    launch_all = _dominant_launcher(model)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        launch_all()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        launch_all()
    graph.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(True), torch.cuda.Event(True)
    a.record()
    for _ in range(reps):
        graph.replay()
    b.record()
    torch.cuda.synchronize()
    n = reps * model.cfg.num_hidden_layers
    us = a.elapsed_time(b) * 1e3 / n
    h, i, hq = model.cfg.hidden_size, model.cfg.intermediate_size, model.cfg.num_attention_heads
    # W_gate_up, x, norm weight, x_out, SwiGLU output (bf16) and the fp32 partial rows
    nbytes = 2 * (2 * i * h + 3 * h + i) + 4 * hq * h
    return {"name": DOMINANT + f" (x + {hq} o_proj partial rows -> RMSNorm -> gate/up [{2 * i}, {h}] -> SwiGLU)",
            "bytes_per_launch": nbytes, "us_per_launch": us, "launches": n,
            "timing": f"isolated: {model.cfg.num_hidden_layers} launches of the kernel alone per captured graph, "
                      "each with its layer's weights, HIP events around the replays"}


def measured_traffic():
    """HBM bytes per launch of the dominant kernel from the committed
    rocprofv3 --pmc summary, or None when that summary is absent."""
    try:
        with open(TRAFFIC_FILE) as f:
            d = json.load(f)
        # only a summary of the kernel the step runs now counts
        return int(d["traffic_bytes_per_launch"]) if d["kernel"].startswith(DOMINANT) else None
    except (OSError, KeyError, ValueError):
        return None


# ---------------------------------------------------------------------------
# single-purpose runs (profiling workloads)


def prefill_attention(iters: int) -> None:
    """The 7B 4 x 4096 prefill's attention alone (one layer's call), timed with
    HIP events on the launch stream: the workload of the attention counter runs."""
    import torch

    from minitp import kernels as K

    b, t, hq, hkv, d = 4, 4096, 28, 4, 128
    g = torch.Generator(device="cuda").manual_seed(0)
    q = torch.randn(b, t, hq, d, device="cuda", dtype=torch.bfloat16, generator=g)
    kc = torch.randn(b, hkv, t, d, device="cuda", dtype=torch.bfloat16, generator=g)
    vc = torch.randn(b, hkv, t, d, device="cuda", dtype=torch.bfloat16, generator=g)
    for _ in range(3):
        K.attention(q, kc, vc, 0)
    e0, e1 = torch.cuda.Event(True), torch.cuda.Event(True)
    e0.record()
    for _ in range(iters):
        K.attention(q, kc, vc, 0)
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / iters
    flop = 4.0 * b * hq * d * t * (t + 1) / 2
    print(json.dumps({"kernel": "prefill_attn_fa_kernel<128>", "us_per_call": round(us, 1),
                      "tflop_s": round(flop / us / 1e6, 1), "calls": iters + 3}), flush=True)


def gemm_alone(spec: str, iters: int = 10) -> None:
    """One bf16 product of a prompt (the kernel minitp_linear picks for the
    shape), timed with HIP events on the launch stream."""
    import torch

    from minitp import _native as N
    from minitp import kernels as K

    parts = spec.split(",")
    m, n, k = (int(v) for v in parts[:3])
    swiglu = len(parts) > 3 and parts[3] == "swiglu"
    g = torch.Generator(device="cuda").manual_seed(0)
    x = torch.randn(m, k, device="cuda", generator=g).to(torch.bfloat16)
    w = (torch.randn(2 * n if swiglu else n, k, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    epi = N.EPI_SWIGLU if swiglu else N.EPI_NONE
    out = K.linear(x, w, epilogue=epi)
    for _ in range(2):
        K.linear(x, w, out=out, epilogue=epi)
    e0, e1 = torch.cuda.Event(True), torch.cuda.Event(True)
    e0.record()
    for _ in range(iters):
        K.linear(x, w, out=out, epilogue=epi)
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / iters
    flop = 2.0 * m * (2 * n if swiglu else n) * k
    print(json.dumps({"gemm": spec, "us_per_call": round(us, 1), "tflop_s": round(flop / us / 1e6, 1),
                      "mfma_frac": round(flop / us / 1e6 / MFMA_BF16_PEAK_TFLOPS, 4), "calls": iters + 3}),
          flush=True)


def copy_calibration(mib: int) -> None:
    """A plain device copy of `mib` MiB (bf16 tensor copy_), three times: the
    known-size kernel that --pmc FETCH_SIZE / WRITE_SIZE are scaled by."""
    import torch

    n = mib * (1 << 20) // 2
    src = torch.ones(n, dtype=torch.bfloat16, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_read": n * 2, "copy_bytes_written": n * 2, "launches": 3}), flush=True)


# ---------------------------------------------------------------------------
# CPU baseline


CPU_SAMPLES = {
    # name -> (shape, dtype, batch, prompt tokens, new tokens)
    "tiny-fp32": ("TINY", "fp32", 1, 8, 16),
    "q05b-bf16": ("QWEN05B", "bf16", 1, 128, 256),
    "q05b-fp32": ("QWEN05B", "fp32", 1, 128, 256),
    "q7b-bf16": ("QWEN7B", "bf16", 1, 512, 256),
    "q7b-fp32": ("QWEN7B", "fp32", 1, 512, 256),
}


def cpu_threads() -> tuple[int, int]:
    """(threads used, affinity cores): the cores this process may run on,
    capped by OMP_NUM_THREADS when the environment sets it (the host's CPU
    share for this GPU)."""
    affinity = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    cap = os.environ.get("OMP_NUM_THREADS", "")
    threads = min(affinity, int(cap)) if cap.isdigit() and int(cap) > 0 else affinity
    return threads, affinity


def cpu_model_name() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            return next(line.split(":", 1)[1].strip() for line in f if line.startswith("model name"))
    except (OSError, StopIteration):
        return ""


def cpu_sample(name: str, budget_s: float, gpu_models: dict) -> dict:
    """The oracle (the CPU restatement of the reference TP=1 loop) on the
    host cores: the workload's prefill, then greedy decode steps until the
    workload ends or `budget_s` seconds of decode are spent. Weights are the
    workload's seeded synthetic ones (generated on the GPU, bit-identical to
    the oracle's generator, copied to host memory)."""
    import torch

    from minitp import synthetic
    from oracle import qwen2_ref as R

    shape, dt, batch, plen, new = CPU_SAMPLES[name]
    dtype = {"fp32": torch.float32, "bf16": torch.bfloat16}[dt]
    cfg = getattr(synthetic, shape)
    gm = gpu_models.get((shape, dtype))
    built = gm is None
    if built:
        gm = synthetic.build_synthetic_model(cfg, dtype=dtype, device="cuda", seed=0)
    sd = {k: v.detach().to("cpu") for k, v in gm.state_dict().items()}
    if built:
        del gm
        torch.cuda.empty_cache()
    if cfg.tie_word_embeddings:
        sd["lm_head.weight"] = sd["model.embed_tokens.weight"]
    oshape = R.Qwen2Shape(cfg.hidden_size, cfg.intermediate_size, cfg.num_hidden_layers, cfg.num_attention_heads,
                          cfg.num_key_value_heads, cfg.head_dim, cfg.vocab_size, cfg.rms_norm_eps, cfg.rope_theta,
                          cfg.max_position_embeddings, cfg.tie_word_embeddings)
    oracle = R.OracleQwen2(oshape, sd)
    ids = R.synthetic_prompt(cfg.vocab_size, batch, plen, seed=0)
    with torch.inference_mode():
        st = R.OracleGenerationState(oracle, ids, new)
        t0 = time.perf_counter()
        tok = st.select_next(st.prefill())
        ttft = time.perf_counter() - t0
        steps, t0 = 0, time.perf_counter()
        while steps < new - 1 and (steps < 2 or time.perf_counter() - t0 < budget_s):
            pos = st.append(tok)
            tok = st.select_next(st.decode_step(tok, pos))
            steps += 1
        dt_s = time.perf_counter() - t0
    del oracle, sd, st
    bounded = steps < new - 1
    note(f"CPU sample {name}: {batch * steps / dt_s:.3f} tok/s")
    return {"workload": name, "value": round(batch * steps / dt_s, 3), "unit": "tok/s", "ttft_s": round(ttft, 3),
            "decode_steps": steps,
            "sample": f"{shape} {dt}: prefill {batch} x {plen} tokens, then {steps} of the workload's {new - 1} "
                      f"decode steps in {dt_s:.1f} s" + (" (bounded by the time budget)" if bounded else "")}


def cpu_baseline(names: list[str], budget_s: float, gpu_models: dict) -> tuple[dict, list[dict]]:
    import torch

    threads, affinity = cpu_threads()
    torch.set_num_threads(threads)
    rows = [cpu_sample(n, budget_s, gpu_models) for n in names]
    head = next((r for r in rows if r["workload"] == "q05b-bf16"), rows[0] if rows else None)
    common = {"cores": threads, "affinity_cores": affinity, "kind": "port", "cpu": cpu_model_name()}
    main = None
    if head is not None:
        main = {"value": head["value"], "unit": "tok/s", **common,
                "sample": "oracle restatement of the reference TP=1 loop, " + head["sample"]}
    return main, [dict(r, **common) for r in rows]


# ---------------------------------------------------------------------------


def headline(args) -> dict:
    import torch

    from minitp.synthetic import QWEN05B, build_synthetic_model, synthetic_prompt

    cfg = QWEN05B
    warm = max(1, args.warmup)
    with torch.inference_mode():
        model = build_synthetic_model(cfg, dtype=torch.bfloat16, device="cuda", seed=0)
        prompt = synthetic_prompt(cfg.vocab_size, 1, PROMPT_LEN, seed=0, device="cuda")
        src = StepSource(model, prompt, NEW_TOKENS)
        src.run(warm)
        first_ctx = len(src.contexts)
        dt = src.run(args.steps)
        ctxs = src.contexts[first_ctx:]
        gens = src.generations
        model.program().check_decode()
        note(f"headline: {len(ctxs)} timed decode steps, {len(ctxs) / dt:.1f} tok/s")

        # after the timed region: the reference's windows on whole generations
        gen = one_generation(model, prompt, NEW_TOKENS)
        # TTFT samples are graph replays: a prompt shape runs directly on its
        # first call and records on its second (the last-position shape has
        # had both in the generations above)
        ttft_samples(model, prompt, 2, "all")
        full = ttft_samples(model, prompt, 3, "all")
        ttfts = ttft_samples(model, prompt, args.ttft_iters, "last")
        kern = dominant_kernel(model)
        note("headline: generation windows, TTFT samples and the dominant kernel done")

    tok_s = len(ctxs) / dt
    total = sum(step_bytes(cfg, c) for c in ctxs)
    achieved = total / dt / 1e9
    k_gbs = kern["bytes_per_launch"] / (kern["us_per_launch"] * 1e-6) / 1e9
    from minitp.bench.benchmark import percentiles

    tt = percentiles(ttfts)
    result = {
        "metric": METRIC,
        "value": round(tok_s, 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": len(ctxs),
        "warmup": warm,
        "ms_per_step": round(dt * 1e3 / len(ctxs), 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,0.02) random-init weights, uniform prompt ids)",
        "config": {"workload": f"Qwen2.5-0.5B-shape bf16 decode, batch 1, {PROMPT_LEN}-token prompt + {NEW_TOKENS} "
                               f"greedy tokens (KV cache {PROMPT_LEN + NEW_TOKENS} positions); timed: decode steps "
                               f"{warm + 1}-{warm + len(ctxs)} of back-to-back generations",
                   "global_batch": 1, "seq_len": PROMPT_LEN + NEW_TOKENS, "parallelism": "tp1"},
        "timed_contexts": {"min": min(ctxs), "max": max(ctxs), "mean": round(sum(ctxs) / len(ctxs), 1),
                           "generations_started": gens},
        "roofline": {"bound": "hbm", "achieved": round(k_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(k_gbs / HBM_PEAK_GBS, 4), "traffic": measured_traffic(), "kernel": kern["name"],
                     "bytes_per_launch": kern["bytes_per_launch"], "us_per_launch": round(kern["us_per_launch"], 3),
                     "timing": kern["timing"]},
        "step_roofline": {"achieved_gbs": round(achieved, 1), "frac": round(achieved / HBM_PEAK_GBS, 4),
                          "bytes_per_token_avg": int(total / len(ctxs)),
                          "roofline_tok_s": round(HBM_PEAK_GBS * 1e9 / (total / len(ctxs)), 1)},
        "ttft_ms": {"p50": tt["p50"], "mean": tt["mean"], "samples": len(ttfts),
                    "prefill": "generate_greedy's (LM head on the last position), graph replays"},
        "ttft_full_logits_ms": {"p50": p50(full), "samples": len(full),
                                "prefill": "the reference's GenerationState.prefill (logits of all 128 positions), "
                                           "graph replays"},
        "generation": gen,
        "tpot_ms": gen["tpot_ms"],
        "prefill_tok_s": gen["prefill_tok_s"],
        "peak_memory_gib": gen["peak_memory_gib"],
        "decode_path": model.program().decode_path_name(),
    }
    return result, model


def main(argv=None):
    args = parse(argv)
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": f"--gpus {args.gpus} (WORLD_SIZE {world}): this build runs the token loop on one "
                                   "GPU; the path's sharding is a design note, no figure at several GPUs is measured"}))
        sys.exit(2)
    import torch

    torch.cuda.set_device(0)
    if args.copy_calibration:
        copy_calibration(args.copy_calibration)
        return
    if args.prefill_attention:
        prefill_attention(args.prefill_attention)
        return
    if args.gemm:
        gemm_alone(args.gemm)
        return
    if args.eager_decode:
        if args.workload == "q7b-prefill":
            raise SystemExit("--eager-decode needs a decode workload (q05b, q7b, q05b-b32)")
        with torch.inference_mode():
            print(json.dumps(eager_decode(args.workload, args.eager_decode)), flush=True)
        return
    if args.workload != "q05b":
        with torch.inference_mode():
            print(json.dumps({"workload": args.workload, **measure_workload(args.workload)}), flush=True)
        return
    if args.dominant_only or args.decode_only or args.dominant_graph:
        from minitp.synthetic import QWEN05B, build_synthetic_model, synthetic_prompt

        with torch.inference_mode():
            model = build_synthetic_model(QWEN05B, dtype=torch.bfloat16, device="cuda", seed=0)
            if args.dominant_graph:
                print(json.dumps(dominant_kernel(model, args.dominant_graph)), flush=True)
                return
            if args.dominant_only:
                launch_all = _dominant_launcher(model)
                for _ in range(4):
                    launch_all()
                torch.cuda.synchronize()
                print(json.dumps({"kernel": DOMINANT, "launches": 4 * QWEN05B.num_hidden_layers}), flush=True)
                return
            prompt = synthetic_prompt(QWEN05B.vocab_size, 1, PROMPT_LEN, seed=0, device="cuda")
            src = StepSource(model, prompt, args.decode_only)
            src.run(args.decode_only - 1)
            dt = src.run(args.decode_only - 1)
            model.program().check_decode()
            print(json.dumps({"decode_path": model.program().decode_path_name(),
                              "ms_per_step": round(dt * 1e3 / (args.decode_only - 1), 4)}), flush=True)
            return

    result, model = headline(args)
    gpu_models = {("QWEN05B", torch.bfloat16): model}
    if not args.no_workloads:
        from minitp import synthetic

        with torch.inference_mode():
            q7b = synthetic.build_synthetic_model(synthetic.QWEN7B, dtype=torch.bfloat16, device="cuda", seed=0)
            gpu_models[("QWEN7B", torch.bfloat16)] = q7b
            result["workloads"] = {
                "q7b": measure_workload("q7b", q7b),
                "q05b-b32": measure_workload("q05b-b32", model),
                "q7b-prefill": measure_workload("q7b-prefill", q7b),
            }
    if not args.no_cpu_baseline:
        names = [n for n in args.cpu_configs.split(",") if n]
        main_cpu, rows = cpu_baseline(names, args.cpu_budget_s, gpu_models)
        if main_cpu is not None:
            result["cpu_baseline"] = main_cpu
        result["cpu_baselines"] = rows
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
