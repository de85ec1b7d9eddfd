"""Write golden vectors for the Qwen2 token loop from the mini-tp reference.

Run in the build container only (the reference is not present on GPU hosts):

    python tests/golden/make_reference_vectors.py tiny_fp32 tiny_bf16 q05b_fp32 q05b_bf16
    python tests/golden/make_reference_vectors.py q7b2_fp32 q7b2_bf16 q05b2_b32_fp32 q05b2_b32_bf16 q7b1_b2_p256_bf16
    python tests/golden/make_reference_vectors.py q05b_b32_fp32 q05b_b32_bf16 q7b_fp32 q7b_bf16 q7b_b4_p640_bf16
    python tests/golden/make_reference_vectors.py q05b2_b20_bf16
    python tests/golden/make_reference_vectors.py tiny_chunked_fp32 tiny_eos_fp32

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
    "q05b2_b20_bf16": ("QWEN05B", 2, torch.bfloat16, 20, 24, 8),  # 17-31 rows: the second 16-row half part-filled
    "q05b2_b48_bf16": ("QWEN05B", 2, torch.bfloat16, 48, 24, 8),  # past 32 rows: decode products on the GEMM
    "q7b1_b2_p256_bf16": ("QWEN7B", 1, torch.bfloat16, 2, 256, 2),  # 7B prefill shape (MFMA GEMM + attention)
    # every layer, shorter prompts: batch-32 decode at the 0.5B shape, 7B
    # batch-1 decode, 7B 4-row prefill long enough for the long-prompt
    # attention kernel (4 x 28 heads x 5 query tiles of 128)
    "q05b_b32_fp32": ("QWEN05B", 24, torch.float32, 32, 24, 8),
    "q05b_b32_bf16": ("QWEN05B", 24, torch.bfloat16, 32, 24, 8),
    "q7b_fp32": ("QWEN7B", 28, torch.float32, 1, 16, 8),
    "q7b_bf16": ("QWEN7B", 28, torch.bfloat16, 1, 16, 8),
    "q7b_b4_p640_bf16": ("QWEN7B", 28, torch.bfloat16, 4, 640, 2),
}
# Branches of the loop the cases above never take, driven through the
# reference's own calls (written by run_branch_case):
#   tiny_chunked_fp32: a 22-token prompt fed as chunks of 7, 9, 1 and 5 tokens
#     through model(ids, positions=, kv_cache=) (cache_len > 0 takes the
#     tril(diagonal=cache_len) mask, attention.py:96-103; one chunk is a single
#     token), then a GenerationState resumed on that filled cache
#     (generation.py:93,103) with a 4-token prompt and 6 new tokens;
#   tiny_eos_fp32: generate_greedy(..., eos_token_id=e, early_stop=True)
#     (generation.py:150-168) on the tiny shape with weights of std 0.3 (at
#     0.02 each greedy row repeats one token), for EOS ids taken from the
#     fixed-length runs: batch 2, an id both rows produce first at different
#     steps (every row stops, the loop ends early); batch 3, an id only one
#     row produces (it is padded with EOS after it, the loop runs to the end)
#     and a row's first pick; batch 1, an id produced part-way and one never
#     produced.
BRANCH_CASES = ("tiny_chunked_fp32", "tiny_eos_fp32")
CHUNKS = (7, 9, 1, 5)
RESUME_PROMPT, RESUME_NEW = 4, 6
EOS_NEW = 12
EOS_STD = 0.3
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


def reference_modules():
    """The reference's config / context / generation / layer modules."""
    sys.path.insert(0, REFERENCE)
    try:
        from minitp import generation
        from minitp.config import ModelConfig
        from minitp.distributed.context import ParallelContext
        from minitp.layer import TPQwen2ForCausalLM
    finally:
        sys.path.remove(REFERENCE)
    assert sys.modules["minitp"].__file__.startswith(REFERENCE), "imported the wrong minitp"
    return ModelConfig, ParallelContext, generation, TPQwen2ForCausalLM


def reference_model(shape, state, dtype):
    ModelConfig, ParallelContext, _, TPQwen2ForCausalLM = reference_modules()
    cfg = ModelConfig(**shape.__dict__)
    ctx = ParallelContext(0, 0, 1, 0, 1, torch.device("cpu"), None)
    model = TPQwen2ForCausalLM(cfg, ctx)
    sd = model.state_dict()
    for k in sd:
        sd[k] = state[k].float()
    model.load_state_dict(sd)
    return model.to(dtype).eval()


def drive_state(st, new_tokens):
    """generate_greedy's fixed-length loop on a state; the logits row each
    selection reads, and the prefill logits."""
    rows = []
    logits = st.prefill()
    prefill_logits = logits.clone()
    for step in range(new_tokens):
        rows.append(logits[:, -1].clone())
        tok = st.select_next(logits)
        pos = st.append(tok)
        if step + 1 < new_tokens:
            logits = st.decode_step(tok, pos)
    return torch.stack(rows), prefill_logits


def run_reference(shape, state, dtype, prompt, new_tokens):
    _, _, generation, _ = reference_modules()
    model = reference_model(shape, state, dtype)
    with torch.inference_mode():
        st = generation.GenerationState(model, prompt, new_tokens)
        rows, prefill_logits = drive_state(st, new_tokens)
    return st.out_ids.clone(), rows, prefill_logits


def chunked_run(model, make_kv, state_cls, prompt, resume_prompt):
    """Chunks of `prompt` through model(..., kv_cache=), then a state resumed
    on the filled cache. Works on the reference and on the oracle."""
    b = prompt.shape[0]
    kv = make_kv(b, prompt.shape[1] + RESUME_PROMPT + RESUME_NEW)
    chunks, start = [], 0
    with torch.inference_mode():
        for c in CHUNKS:
            chunks.append(model(prompt[:, start:start + c], positions=torch.arange(start, start + c),
                                kv_cache=kv).clone())
            start += c
        st = state_cls(model, resume_prompt, RESUME_NEW, kv=kv)
        rows, prefill = drive_state(st, RESUME_NEW)
    return torch.cat(chunks, dim=1), st.out_ids.clone(), rows, prefill, kv.seq_len


def eos_cases(generate, model, prompt_fn) -> list[tuple[torch.Tensor, int]]:
    """(prompt, eos) pairs for the early-stop fixture, chosen from the
    fixed-length runs of the model (see tiny_eos_fp32 above)."""
    def fixed(prompt):
        with torch.inference_mode():
            return generate(model, prompt, EOS_NEW, early_stop=False)[:, prompt.shape[1]:].tolist()

    cases = []
    for seed in range(20, 400):  # batch 2: a shared id first produced at different steps
        prompt = prompt_fn(2, seed)
        a, b = fixed(prompt)
        shared = [t for t in a if t in b and a.index(t) != b.index(t) and max(a.index(t), b.index(t)) < EOS_NEW - 2]
        if shared:
            cases.append((prompt, shared[0]))
            break
    prompt = prompt_fn(3, 8)
    rows = fixed(prompt)
    only_one = next(t for t in rows[1][2:] if t not in rows[0] and t not in rows[2])
    cases += [(prompt, only_one), (prompt, rows[2][0])]
    prompt = prompt_fn(1, 8)
    (row,) = fixed(prompt)
    never = next(v for v in range(1000) if v not in row)
    cases += [(prompt, row[EOS_NEW // 2]), (prompt, never)]
    return cases


def eos_run(generate, model, make_kv, prompt, eos):
    kv = make_kv(prompt.shape[0], prompt.shape[1] + EOS_NEW)
    with torch.inference_mode():
        ids = generate(model, prompt, EOS_NEW, eos_token_id=eos, early_stop=True, kv=kv)
    return ids.clone(), kv.seq_len


def run_branch_case(name):
    """Reference-driven fixture of a branch (BRANCH_CASES); the oracle must
    reproduce it bit for bit first."""
    from oracle import qwen2_ref as R

    shape, dtype = R.TINY, torch.float32
    state = R.synthetic_state(shape, seed=0, dtype=torch.float32)
    _, _, generation, _ = reference_modules()
    ref = reference_model(shape, state, dtype)
    sd = {k: v.to(dtype) for k, v in state.items()}
    orc = R.OracleQwen2(shape, sd)

    def ref_kv(b, n):
        return generation.make_kv_cache(ref, b, n)

    def orc_kv(b, n):
        return orc.make_kv_cache(b, n)

    out = {"dtype": np.array(str(dtype))}
    if name == "tiny_chunked_fp32":
        prompt = R.synthetic_prompt(shape.vocab_size, 2, sum(CHUNKS), seed=5)
        resume = R.synthetic_prompt(shape.vocab_size, 2, RESUME_PROMPT, seed=6)
        got_r = chunked_run(ref, ref_kv, generation.GenerationState, prompt, resume)
        got_o = chunked_run(orc, orc_kv, R.OracleGenerationState, prompt, resume)
        for a, b in zip(got_r[:4], got_o[:4]):
            if not torch.equal(a, b):
                raise SystemExit(f"{name}: oracle does not reproduce the reference bit for bit")
        if got_r[4] != got_o[4]:
            raise SystemExit(f"{name}: cache cursors differ")
        chunk_logits, ids, rows, prefill, seq_len = got_r
        out.update({"prompt": prompt.numpy(), "chunks": np.array(CHUNKS, dtype=np.int64),
                    "chunk_logits": chunk_logits.float().numpy(), "resume_prompt": resume.numpy(),
                    "resume_ids": ids.numpy(), "resume_step_logits": rows.float().numpy(),
                    "resume_prefill_logits": prefill.float().numpy(), "seq_len": np.array(seq_len)})
    else:
        state = R.synthetic_state(shape, seed=0, dtype=torch.float32, std=EOS_STD)
        ref = reference_model(shape, state, dtype)
        orc = R.OracleQwen2(shape, {k: v.to(dtype) for k, v in state.items()})
        cases = []
        for prompt, eos in eos_cases(generation.generate_greedy, ref,
                                     lambda b, seed: R.synthetic_prompt(shape.vocab_size, b, 5, seed=seed)):
            ids_r, len_r = eos_run(generation.generate_greedy, ref, ref_kv, prompt, eos)
            ids_o, len_o = eos_run(R.generate_greedy, orc, orc_kv, prompt, eos)
            if not torch.equal(ids_r, ids_o) or len_r != len_o:
                raise SystemExit(f"{name}: oracle early stop differs (batch {prompt.shape[0]}, eos {eos})")
            cases.append((prompt, eos, ids_r, len_r))
        out["weight_std"] = np.array(EOS_STD)
        width = 5 + EOS_NEW
        out["prompts"] = np.stack([np.pad(p.numpy(), ((0, 3 - p.shape[0]), (0, 0)), constant_values=-1)
                                   for p, _, _, _ in cases])
        out["batch"] = np.array([p.shape[0] for p, _, _, _ in cases], dtype=np.int64)
        out["eos"] = np.array([e for _, e, _, _ in cases], dtype=np.int64)
        out["ids"] = np.stack([np.pad(i.numpy(), ((0, 3 - i.shape[0]), (0, width - i.shape[1])), constant_values=-1)
                               for _, _, i, _ in cases])
        out["length"] = np.array([i.shape[1] for _, _, i, _ in cases], dtype=np.int64)
        out["seq_len"] = np.array([n for _, _, _, n in cases], dtype=np.int64)
        print(f"  eos cases (batch, eos, length): "
              f"{[(int(b), int(e), int(n)) for b, e, n in zip(out['batch'], out['eos'], out['length'])]}")
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), f"{name}.npz")
    np.savez_compressed(path, **out)
    print(f"  wrote {path} ({os.path.getsize(path)} B)")


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
        if name in BRANCH_CASES:
            run_branch_case(name)
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
    main(sys.argv[1:] or list(CASES) + list(ORACLE_CASES) + list(BRANCH_CASES))
