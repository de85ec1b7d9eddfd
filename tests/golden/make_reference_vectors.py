"""Write golden vectors for the Qwen2 token loop from the mini-tp reference.

Run in the build container only (the reference is not present on GPU hosts):

    python tests/golden/make_reference_vectors.py tiny_fp32 tiny_bf16 q05b_fp32 q05b_bf16
    python tests/golden/make_reference_vectors.py q7b2_fp32 q7b2_bf16 q05b2_b32_fp32 q05b2_b32_bf16 q7b1_b2_p256_bf16

It imports the reference package from /root/reference, builds
``TPQwen2ForCausalLM`` at tp_size=1, copies the seeded synthetic weights in
through ``load_state_dict`` (the pattern of the reference's
tests/test_qwen_tiny.py:53-82), and drives the reference's own
``GenerationState`` exactly as ``generate_greedy`` does (generation.py:133-171,
fixed-length mode), recording the logits row each selection reads. The
oracle restatement is run on the same inputs and must match bit for bit
before anything is written. Output: ``tests/golden/<case>.npz`` holding only
numbers (inputs, ids, logit summaries).
"""

from __future__ import annotations

import os
import sys
import time

import numpy as np
import torch

REPO = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
REFERENCE = "/root/reference"

CASES = {
    # name: (shape, dtype, batch, prompt_len, new_tokens)
    "tiny_fp32": ("TINY", torch.float32, 1, 8, 16),
    "tiny_bf16": ("TINY", torch.bfloat16, 1, 8, 16),
    "tiny_b3_fp32": ("TINY", torch.float32, 3, 5, 12),
    "q05b_fp32": ("QWEN05B", torch.float32, 1, 128, 256),
    "q05b_bf16": ("QWEN05B", torch.bfloat16, 1, 128, 256),
}
# Cases at the other workloads' layer shapes with fewer layers (every layer
# runs the same code), written from the oracle alone: the oracle reproduces
# the reference bit for bit on the cases above, and these add sizes, batch
# and the untied 7B head, not new operations.
#   name: (shape, layers, dtype, batch, prompt_len, new_tokens)
ORACLE_CASES = {
    "q7b2_fp32": ("QWEN7B", 2, torch.float32, 1, 16, 8),  # 7B decode shape (GEMV rows of 3584 / 18944)
    "q7b2_bf16": ("QWEN7B", 2, torch.bfloat16, 1, 16, 8),
    "q05b2_b32_fp32": ("QWEN05B", 2, torch.float32, 32, 24, 8),  # batch-32 decode (GEMM + batched attention)
    "q05b2_b32_bf16": ("QWEN05B", 2, torch.bfloat16, 32, 24, 8),
    "q05b2_b3_bf16": ("QWEN05B", 2, torch.bfloat16, 3, 40, 24),  # small-batch decode GEMV path, batch 3
    "q7b1_b2_p256_bf16": ("QWEN7B", 1, torch.bfloat16, 2, 256, 2),  # 7B prefill shape (MFMA GEMM + attention)
}
TOPK = 16
N_SAMPLE = 64
SAMPLE_STREAM = 9  # generator stream for the sampled vocab columns


def sample_columns(vocab: int) -> np.ndarray:
    from oracle import synth

    return np.unique(synth.uniform_ids(0, SAMPLE_STREAM, N_SAMPLE, vocab))


def summarize(rows: torch.Tensor, cols: np.ndarray):
    """rows: [S, B, V] float -> top-k ids/values, sampled values, top-2 margin."""
    r = rows.float()
    vals, idx = torch.topk(r, TOPK, dim=-1)  # sorted, descending
    return {
        "topk_ids": idx.numpy().astype(np.int64),
        "topk_vals": vals.numpy().astype(np.float32),
        "sample_vals": r[..., torch.from_numpy(cols)].numpy().astype(np.float32),
        "margin": (vals[..., 0] - vals[..., 1]).numpy().astype(np.float32),
    }


def run_reference(shape, state, dtype, prompt, new_tokens):
    sys.path.insert(0, REFERENCE)
    try:
        from minitp.config import ModelConfig
        from minitp.distributed.context import ParallelContext
        from minitp.generation import GenerationState
        from minitp.layer import TPQwen2ForCausalLM
    finally:
        sys.path.remove(REFERENCE)
    cfg = ModelConfig(**shape.__dict__)
    ctx = ParallelContext(0, 0, 1, 0, 1, torch.device("cpu"), None)
    model = TPQwen2ForCausalLM(cfg, ctx)
    sd = model.state_dict()
    for k in sd:
        sd[k] = state[k].float()
    model.load_state_dict(sd)
    model = model.to(dtype).eval()
    assert sys.modules["minitp"].__file__.startswith(REFERENCE), "imported the wrong minitp"
    rows, prefill_logits = [], None
    with torch.inference_mode():
        st = GenerationState(model, prompt, new_tokens)
        logits = st.prefill()
        prefill_logits = logits.clone()
        for step in range(new_tokens):
            rows.append(logits[:, -1].clone())
            tok = st.select_next(logits)
            pos = st.append(tok)
            if step + 1 < new_tokens:
                logits = st.decode_step(tok, pos)
    return st.out_ids.clone(), torch.stack(rows), prefill_logits


def run_oracle(shape, state, dtype, prompt, new_tokens):
    from oracle.qwen2_ref import OracleQwen2, generate_greedy

    sd = {k: v.to(dtype) for k, v in state.items()}
    if shape.tie_word_embeddings:
        sd["lm_head.weight"] = sd["model.embed_tokens.weight"]
    m = OracleQwen2(shape, sd)
    rows = []
    ids = generate_greedy(m, prompt, new_tokens, early_stop=False, on_logits=lambda s, lg: rows.append(lg[:, -1].clone()))
    return ids, torch.stack(rows)


def write_fixture(name, shape, dtype, prompt, ids, rows, prefill):
    prompt_len = prompt.shape[1]
    cols = sample_columns(shape.vocab_size)
    out = {
        "prompt": prompt.numpy(),
        "ids": ids.numpy(),
        "sample_cols": cols,
        "dtype": np.array(str(dtype)),
    }
    out.update({f"step_{k}": v for k, v in summarize(rows, cols).items()})
    # prefill logits at first / middle / last prompt position
    pick = sorted({0, prompt_len // 2, prompt_len - 1})
    out["prefill_positions"] = np.array(pick, dtype=np.int64)
    out.update({f"prefill_{k}": v for k, v in summarize(prefill[:, pick].transpose(0, 1), cols).items()})
    if shape.vocab_size <= 4096:
        out["step_logits"] = rows.float().numpy()
        out["prefill_logits"] = prefill.float().numpy()
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), f"{name}.npz")
    np.savez_compressed(path, **out)
    print(f"  wrote {path} ({os.path.getsize(path)} B); min top-2 margin {out['step_margin'].min():.3e}")


def run_oracle_case(name):
    """A fixture from the oracle alone (ORACLE_CASES)."""
    import dataclasses

    from oracle import qwen2_ref
    from oracle.qwen2_ref import OracleQwen2, generate_greedy, synthetic_prompt, synthetic_state

    shape_name, layers, dtype, batch, prompt_len, new_tokens = ORACLE_CASES[name]
    shape = dataclasses.replace(getattr(qwen2_ref, shape_name), num_hidden_layers=layers)
    t0 = time.time()
    state = synthetic_state(shape, seed=0, dtype=dtype)
    prompt = synthetic_prompt(shape.vocab_size, batch, prompt_len, seed=0)
    m = OracleQwen2(shape, state)
    rows, prefill = [], []

    def keep(step, lg):
        if step == 0:
            prefill.append(lg.clone())
        rows.append(lg[:, -1].clone())

    with torch.inference_mode():
        ids = generate_greedy(m, prompt, new_tokens, early_stop=False, on_logits=keep)
    print(f"{name}: oracle {time.time() - t0:.1f}s")
    write_fixture(name, shape, dtype, prompt, ids, torch.stack(rows), prefill[0])


def main(names):
    sys.path.insert(0, REPO)
    from oracle import qwen2_ref
    from oracle.qwen2_ref import synthetic_prompt, synthetic_state

    torch.set_num_threads(os.cpu_count() or 1)
    for name in names:
        if name in ORACLE_CASES:
            run_oracle_case(name)
            continue
        shape_name, dtype, batch, prompt_len, new_tokens = CASES[name]
        shape = getattr(qwen2_ref, shape_name)
        t0 = time.time()
        state = synthetic_state(shape, seed=0, dtype=torch.float32)
        prompt = synthetic_prompt(shape.vocab_size, batch, prompt_len, seed=0)
        ref_ids, ref_rows, ref_prefill = run_reference(shape, state, dtype, prompt, new_tokens)
        t1 = time.time()
        orc_ids, orc_rows = run_oracle(shape, state, dtype, prompt, new_tokens)
        t2 = time.time()
        same_ids = torch.equal(ref_ids, orc_ids)
        same_logits = torch.equal(ref_rows.view(torch.int16) if dtype == torch.bfloat16 else ref_rows.view(torch.int32),
                                  orc_rows.view(torch.int16) if dtype == torch.bfloat16 else orc_rows.view(torch.int32))
        print(f"{name}: reference {t1 - t0:.1f}s oracle {t2 - t1:.1f}s ids_equal={same_ids} logits_bitwise_equal={same_logits}")
        if not (same_ids and same_logits):
            raise SystemExit(f"{name}: oracle does not reproduce the reference bit for bit")
        write_fixture(name, shape, dtype, prompt, ref_ids, ref_rows, ref_prefill)


if __name__ == "__main__":
    main(sys.argv[1:] or list(CASES) + list(ORACLE_CASES))
