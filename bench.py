"""Decode benchmark: Qwen2.5-0.5B-shape bf16, batch 1, 128-token prompt, greedy decode.

A step is one decode token (append + decode_step + select_next, the
reference's TPOT window, minitp/bench/benchmark.py:138-157), replayed from the
decode hipGraph. W untimed warmup steps, then exactly K timed steps in one
region bracketed by torch.cuda.synchronize(). The default K = 255 is the
workload's 256 greedy tokens (the first comes from the prefill).

Reported beside the headline tok/s:
  * HBM roofline of the whole step: algorithmic bytes per token (weights once,
    LM head once, norms, QKV bias, KV read of ctx + 1 positions) / time,
    against MI355X's 8 TB/s;
  * the dominant kernel (the fused RMSNorm + gate/up GEMV + SwiGLU) timed
    with HIP events on its stream: algorithmic bytes per launch / mean
    launch time, and its measured HBM traffic per launch when the committed
    rocprofv3 counter summary is present;
  * TTFT (prefill start -> first token selected) p50 / mean, TPOT percentiles;
    the prefill is generate_greedy's: the LM head on the last position only;
  * the CPU baseline: the oracle restatement of the reference's TP=1 path on
    the host cores, bf16, over a bounded sample of the same workload.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (os.path.join(ROOT, "mini-tp_amd"), ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)

METRIC = "decode tok/s & % HBM roofline, Qwen2.5-0.5B-shape bf16 bs=1; p50 TTFT"
HBM_PEAK_GBS = 8000.0
PROMPT_LEN = 128


def step_bytes(cfg, ctx: int, batch: int = 1, esize: int = 2) -> int:
    """Algorithmic HBM bytes of one decode step reading ctx cached positions."""
    L, H, hq, hkv, d, inter, v = (cfg.num_hidden_layers, cfg.hidden_size, cfg.num_attention_heads,
                                  cfg.num_key_value_heads, cfg.head_dim, cfg.intermediate_size, cfg.vocab_size)
    p_stream = L * (H * (hq + 2 * hkv) * d + hq * d * H + 3 * inter * H) + v * H + H * (2 * L + 1) + L * (hq + 2 * hkv) * d
    kv = batch * esize * L * 2 * hkv * d * (ctx + 1)
    return esize * p_stream + kv


def parse(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=255)
    ap.add_argument("--warmup", type=int, default=510)
    ap.add_argument("--prompt-len", type=int, default=PROMPT_LEN)
    ap.add_argument("--ttft-iters", type=int, default=10)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget-s", type=float, default=15.0)
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain copy of MIB MiB (the --pmc byte-counter calibration) and exit")
    ap.add_argument("--workload", default="q05b", choices=sorted(WORKLOADS),
                    help="q05b (default): the headline line; the others measure the remaining workloads "
                         "(one JSON line each, not the headline metric)")
    ap.add_argument("--prefill-attention", type=int, default=0, metavar="ITERS",
                    help="only time the causal prefill attention of the 7B 4 x 4096 prefill (q [4, 4096, 28, 128], "
                         "4 KV heads, bf16) ITERS times after 3 warm-up calls, print one JSON line and exit")
    ap.add_argument("--dominant-only", action="store_true",
                    help="only launch the dominant kernel, eagerly (no graphs), once per layer 4 times over, and "
                         "exit: the workload of the --pmc byte-counter passes")
    return ap.parse_args(argv)


# Other workloads: (shape, batch, prompt length, decode steps after the first token)
WORKLOADS = {
    "q05b": None,  # the headline line below
    "q05b-b32": ("QWEN05B", 32, 2048, 511),
    "q7b": ("QWEN7B", 1, 512, 255),
    "q7b-prefill": ("QWEN7B", 4, 4096, 0),
}
MFMA_BF16_PEAK_TFLOPS = 2500.0


def prefill_flops(cfg, batch: int, t: int) -> float:
    """Dense FLOPs of a prefill of `t` tokens per row: the linear layers, causal
    attention (QK^T and PV over the visible keys) and the LM head of the last
    position only (what the prefill computes when no full logits are asked)."""
    L, H, hq, hkv, d, inter, v = (cfg.num_hidden_layers, cfg.hidden_size, cfg.num_attention_heads,
                                  cfg.num_key_value_heads, cfg.head_dim, cfg.intermediate_size, cfg.vocab_size)
    m = batch * t
    linear = 2.0 * m * L * (H * (hq + 2 * hkv) * d + hq * d * H + 3 * inter * H)
    attn = 2.0 * 2.0 * batch * L * hq * d * (t * (t + 1) / 2)
    return linear + attn + 2.0 * batch * v * H


def secondary(args):
    """One JSON line for a non-headline workload: decode tok/s with the step
    roofline, or (prefill-only) TTFT with the dense-FLOP MFMA fraction."""
    import torch

    from minitp import synthetic
    from minitp.generation import GenerationState

    shape, batch, plen, steps = WORKLOADS[args.workload]
    cfg = getattr(synthetic, shape)
    torch.cuda.set_device(0)
    out = {"workload": args.workload, "shape": shape, "batch": batch, "prompt": plen, "dtype": "bf16"}
    with torch.inference_mode():
        model = synthetic.build_synthetic_model(cfg, dtype=torch.bfloat16, device="cuda", seed=0)
        prompt = synthetic.synthetic_prompt(cfg.vocab_size, batch, plen, seed=0, device="cuda")
        torch.cuda.synchronize()
        if steps:
            decode_run(model, prompt, steps)  # warmup (graph capture for this batch / length)
            dt, ttft, _, _ = decode_run(model, prompt, steps)
            total = sum(step_bytes(cfg, plen + s, batch=batch) for s in range(steps))
            out.update({"decode_tok_s": round(batch * steps / dt, 1), "ms_per_step": round(dt * 1e3 / steps, 4),
                        "step_roofline_frac": round(total / dt / 1e9 / HBM_PEAK_GBS, 4),
                        "roofline_tok_s": round(batch * HBM_PEAK_GBS * 1e9 / (total / steps), 1),
                        "ttft_ms": round(ttft * 1e3, 3)})
        else:
            ttfts = []
            for _ in range(4):
                st = GenerationState(model, prompt, 1, prefill_logits="last")
                a, b = torch.cuda.Event(True), torch.cuda.Event(True)
                a.record()
                st.select_next(st.prefill())
                b.record()
                torch.cuda.synchronize()
                ttfts.append(a.elapsed_time(b) / 1e3)
                del st
            ttft = sorted(ttfts)[1]  # p50 of the last three (the first includes one-time setup)
            fl = prefill_flops(cfg, batch, plen)
            out.update({"ttft_ms": round(ttft * 1e3, 3), "prefill_tflop": round(fl / 1e12, 2),
                        "mfma_frac": round(fl / ttft / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
                        "ttft_ms_all": [round(t * 1e3, 3) for t in ttfts]})
    print(json.dumps(out), flush=True)


def decode_run(model, prompt, n_steps, record_steps=False):
    """Prefill + first pick, then n_steps decode steps. Returns
    (decode_seconds, ttft_s, step_ms list, out_ids)."""
    import torch

    from minitp.generation import GenerationState

    st = GenerationState(model, prompt, n_steps + 1, prefill_logits="last")
    e_t0, e_t1 = torch.cuda.Event(True), torch.cuda.Event(True)
    e_t0.record()
    logits = st.prefill()
    tok = st.select_next(logits)
    e_t1.record()
    torch.cuda.synchronize()
    ttft = e_t0.elapsed_time(e_t1) / 1e3
    evs = []
    t0 = time.perf_counter()
    for _ in range(n_steps):
        if record_steps:
            a, b = torch.cuda.Event(True), torch.cuda.Event(True)
            a.record()
        pos = st.append(tok)
        logits = st.decode_step(tok, pos)
        tok = st.select_next(logits)
        if record_steps:
            b.record()
            evs.append((a, b))
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    return dt, ttft, [a.elapsed_time(b) for a, b in evs], st.out_ids


DOMINANT = "gemv_reg_kernel<minitp::bf16, 1, 1, 2, 1, 2>"  # PRO_NORM, EPI_SWIGLU: rocprofv3's name for it
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "gate_up_gemv_q05b_decode_traffic.json")


def _dominant_launcher(model):
    """A function launching the dominant kernel once per layer on the current
    stream, with that layer's weights."""
    import torch

    from minitp import _native as N
    from minitp import kernels as K

    cfg = model.cfg
    layers = list(model.model.layers)
    x = torch.randn(1, cfg.hidden_size, device="cuda").to(torch.bfloat16)
    out = torch.empty(1, cfg.intermediate_size, dtype=torch.bfloat16, device="cuda")

    def launch_all():
        for layer in layers:
            K.rmsnorm_linear(x, layer.post_attention_layernorm.weight, cfg.rms_norm_eps, layer.mlp.gate_up_proj.weight,
                             out=out, epilogue=N.EPI_SWIGLU)

    return launch_all


def dominant_kernel(model, reps: int = 20):
    """The kernel with the largest share of a decode step: the fused
    post-attention RMSNorm + gate/up GEMV + SwiGLU that the decode graph runs
    once per layer. The same entry point and the same per-layer weights,
    launched once per layer in a captured graph (so no launch re-reads a
    cache-resident matrix and no host launch cost is counted), timed with
    HIP events on the stream the graph replays on."""
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
    h, i = model.cfg.hidden_size, model.cfg.intermediate_size
    nbytes = 2 * (2 * i * h + 2 * h + i)  # W_gate_up, x, norm weight, SwiGLU output (bf16)
    return {"name": DOMINANT + " (RMSNorm + gate/up [9728, 896] + SwiGLU)", "bytes_per_launch": nbytes,
            "us_per_launch": us, "launches": n}


def measured_traffic():
    """HBM bytes per launch of the dominant kernel from the committed
    rocprofv3 --pmc summary (FETCH_SIZE, WRITE_SIZE scaled by a plain copy of
    known size), or None when that summary is absent."""
    try:
        with open(TRAFFIC_FILE) as f:
            return int(json.load(f)["traffic_bytes_per_launch"])
    except (OSError, KeyError, ValueError):
        return None


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


def cpu_baseline(model, prompt, budget_s: float):
    """The oracle (CPU restatement of the reference TP=1 path) in bf16 on the
    host cores: prefill of the same prompt, then decode steps until the time
    budget is spent. Reports decode tok/s."""
    import torch

    from oracle import qwen2_ref as R

    threads = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    threads = min(threads, 16)
    torch.set_num_threads(threads)
    c = model.cfg
    shape = R.Qwen2Shape(c.hidden_size, c.intermediate_size, c.num_hidden_layers, c.num_attention_heads,
                         c.num_key_value_heads, c.head_dim, c.vocab_size, c.rms_norm_eps, c.rope_theta,
                         c.max_position_embeddings, c.tie_word_embeddings)
    sd = {k: v.detach().cpu() for k, v in model.state_dict().items()}
    if c.tie_word_embeddings:
        sd["lm_head.weight"] = sd["model.embed_tokens.weight"]
    oracle = R.OracleQwen2(shape, sd)
    ids = prompt.cpu()
    with torch.inference_mode():
        st = R.OracleGenerationState(oracle, ids, 1024)
        t0 = time.perf_counter()
        logits = st.prefill()
        tok = st.select_next(logits)
        ttft = time.perf_counter() - t0
        steps, t0 = 0, time.perf_counter()
        while steps < 3 or (time.perf_counter() - t0 < budget_s and steps < 255):
            pos = st.append(tok)
            logits = st.decode_step(tok, pos)
            tok = st.select_next(logits)
            steps += 1
        dt = time.perf_counter() - t0
    model_name = ""
    try:
        with open("/proc/cpuinfo") as f:
            model_name = next(line.split(":", 1)[1].strip() for line in f if line.startswith("model name"))
    except (OSError, StopIteration):
        pass
    return {"value": round(steps / dt, 3), "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"oracle bf16 restatement of the reference TP=1 loop: prefill {ids.shape[1]} tokens "
                      f"(TTFT {ttft:.2f} s) then {steps} greedy decode steps in {dt:.1f} s",
            "cpu": model_name}


def main(argv=None):
    args = parse(argv)
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": f"--gpus {args.gpus} (WORLD_SIZE {world}): this build runs the token loop on one "
                                   "GPU only; multi-GPU sharding is a design note, not a measured path"}))
        sys.exit(2)
    import torch

    if args.copy_calibration:
        torch.cuda.set_device(0)
        copy_calibration(args.copy_calibration)
        return
    if args.prefill_attention:
        torch.cuda.set_device(0)
        prefill_attention(args.prefill_attention)
        return
    if WORKLOADS[args.workload] is not None:
        secondary(args)
        return
    from minitp.bench.benchmark import _percentiles
    from minitp.synthetic import QWEN05B, build_synthetic_model, synthetic_prompt

    torch.cuda.set_device(0)
    cfg = QWEN05B
    with torch.inference_mode():
        model = build_synthetic_model(cfg, dtype=torch.bfloat16, device="cuda", seed=0)
        if args.dominant_only:
            launch_all = _dominant_launcher(model)
            for _ in range(4):
                launch_all()
            torch.cuda.synchronize()
            print(json.dumps({"kernel": DOMINANT, "launches": 4 * cfg.num_hidden_layers}), flush=True)
            return
        prompt = synthetic_prompt(cfg.vocab_size, 1, args.prompt_len, seed=0, device="cuda")
        torch.cuda.synchronize()

        # warmup: whole generations of 255 steps (graph capture happens here);
        # the last one records per-step events for the TPOT percentiles
        step_ms, ttfts = [], []
        n_warm = max(1, math.ceil(args.warmup / 255))
        for i in range(n_warm):
            _, ttft, ms, _ = decode_run(model, prompt, 255, record_steps=(i == n_warm - 1))
            if i > 0:  # the first prefill holds one-time setup (GEMM algorithm timing, first launches)
                ttfts.append(ttft)
            step_ms = ms or step_ms
        for _ in range(args.ttft_iters):
            from minitp.generation import GenerationState

            st = GenerationState(model, prompt, 1, prefill_logits="last")
            a, b = torch.cuda.Event(True), torch.cuda.Event(True)
            a.record()
            st.select_next(st.prefill())
            b.record()
            torch.cuda.synchronize()
            ttfts.append(a.elapsed_time(b) / 1e3)

        # timed region: exactly K decode steps
        torch.cuda.synchronize()
        dt, _, _, out_ids = decode_run(model, prompt, args.steps)
        kern = dominant_kernel(model)

    tok_s = args.steps / dt
    total_bytes = sum(step_bytes(cfg, args.prompt_len + s) for s in range(args.steps))
    achieved = total_bytes / dt / 1e9
    k_gbs = kern["bytes_per_launch"] / (kern["us_per_launch"] * 1e-6) / 1e9
    ttft_ms = sorted(t * 1e3 for t in ttfts)
    result = {
        "metric": METRIC,
        "value": round(tok_s, 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": n_warm * 255,
        "ms_per_step": round(dt * 1e3 / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,0.02) random-init weights, uniform prompt ids)",
        "config": {"workload": f"Qwen2.5-0.5B-shape bf16 decode, batch 1, prompt {args.prompt_len}, "
                               f"{args.steps + 1} greedy tokens",
                   "global_batch": 1, "seq_len": args.prompt_len + args.steps + 1, "parallelism": "tp1"},
        "roofline": {"bound": "hbm", "achieved": round(k_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(k_gbs / HBM_PEAK_GBS, 4), "traffic": measured_traffic(), "kernel": kern["name"],
                     "bytes_per_launch": kern["bytes_per_launch"], "us_per_launch": round(kern["us_per_launch"], 3)},
        "step_roofline": {"achieved_gbs": round(achieved, 1), "frac": round(achieved / HBM_PEAK_GBS, 4),
                          "bytes_per_token_avg": int(total_bytes / args.steps),
                          "roofline_tok_s": round(HBM_PEAK_GBS * 1e9 / (total_bytes / args.steps), 1)},
        "ttft_ms": {"p50": round(ttft_ms[(len(ttft_ms) + 1) // 2 - 1], 3),
                    "mean": round(sum(ttft_ms) / len(ttft_ms), 3), "samples": len(ttft_ms)},
        "tpot_ms": _percentiles(step_ms),
        "decode_path": "one hipGraph replay per token: embedding; per layer norm+QKV+RoPE+KV write, attention, "
                       "o_proj+residual, norm+gate/up+SwiGLU, down+residual; norm+LM head+argmax partials, merge",
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(model, prompt, args.cpu_budget_s)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
