"""Parity at the other workloads' layer shapes, with fewer layers (every
layer runs the same kernels): the 7B decode shape with its untied LM head,
batch-32 decode at the 0.5B shape (GEMM + batched attention paths) and the 7B
prefill shape (MFMA GEMMs and prefill attention at 2 x 256 tokens),
batch-3 decode at the 0.5B shape (the MFMA GEMV forms at their fewest rows),
batch 20 (the one-tuple MFMA GEMVs' second 16-row half part-filled) and batch
48 (past the GEMV forms' 32 rows: the decode products on the GEMM).
More cases run every layer of the model with shorter prompts than the
workloads: batch-32 decode at the 0.5B shape (24 layers, fp32 and bf16), 7B
batch-1 decode (28 layers, fp32 and bf16) and the 7B 4-row prefill at 640
tokens (bf16; the long-prompt attention kernel serves it).

Fixtures: tests/golden/{q7b2,q05b2_b32,q05b2_b3,q05b2_b20,q05b2_b48,q7b1_b2_p256,q05b_b32,q7b,q7b_b4_p640}_*.npz,
written by tests/golden/make_reference_vectors.py from the oracle (which reproduces the
reference bit for bit on the tiny and 0.5B cases). Bars as for the 0.5B
model: fp32 greedy ids exact and logits within 1e-3; bf16 logits within 0.5,
teacher-forced, and the greedy pick where the oracle's top-2 margin is clear.
"""

import dataclasses
import os

import numpy as np
import pytest
import torch

from tests.conftest import GOLDEN
from tests.test_gpu_model import BF16_LOGIT_ATOL, FP32_LOGIT_ATOL, _check_summaries, _teacher_forced_rows

pytestmark = pytest.mark.gpu
DEV = "cuda"

CASES = {  # fixture: (shape key, layers, dtype)
    "q7b2_fp32": ("qwen2.5-7b", 2, torch.float32),
    "q7b2_bf16": ("qwen2.5-7b", 2, torch.bfloat16),
    "q05b2_b32_fp32": ("qwen2.5-0.5b", 2, torch.float32),
    "q05b2_b32_bf16": ("qwen2.5-0.5b", 2, torch.bfloat16),
    "q05b2_b3_bf16": ("qwen2.5-0.5b", 2, torch.bfloat16),
    "q05b2_b20_bf16": ("qwen2.5-0.5b", 2, torch.bfloat16),
    "q05b2_b48_bf16": ("qwen2.5-0.5b", 2, torch.bfloat16),
    "q7b1_b2_p256_bf16": ("qwen2.5-7b", 1, torch.bfloat16),
    # every layer of the model (shorter prompts than the workloads)
    "q05b_b32_fp32": ("qwen2.5-0.5b", 24, torch.float32),
    "q05b_b32_bf16": ("qwen2.5-0.5b", 24, torch.bfloat16),
    "q7b_fp32": ("qwen2.5-7b", 28, torch.float32),
    "q7b_bf16": ("qwen2.5-7b", 28, torch.bfloat16),
    "q7b_b4_p640_bf16": ("qwen2.5-7b", 28, torch.bfloat16),
}


def _model(name):
    from minitp import synthetic

    key, layers, dtype = CASES[name]
    cfg = dataclasses.replace(synthetic.SHAPES[key], num_hidden_layers=layers)
    return synthetic.build_synthetic_model(cfg, dtype=dtype, device=DEV, seed=0)


@pytest.mark.parametrize("name", ["q7b2_fp32", "q05b2_b32_fp32", "q05b_b32_fp32", "q7b_fp32"])
def test_fp32_greedy_ids_exact_and_logits(name):
    from minitp.generation import generate_greedy

    fx = np.load(os.path.join(GOLDEN, f"{name}.npz"))
    model = _model(name)
    prompt = torch.from_numpy(fx["prompt"]).to(DEV)
    n = fx["ids"].shape[1] - prompt.shape[1]
    ids = generate_greedy(model, prompt, n, early_stop=False).cpu().numpy()
    assert np.array_equal(ids, fx["ids"]), np.argwhere(ids != fx["ids"])[:4]
    rows, prefill = _teacher_forced_rows(model, prompt, torch.from_numpy(fx["ids"]), n)
    err = _check_summaries(rows, fx, "step", FP32_LOGIT_ATOL)
    pre = prefill[:, torch.from_numpy(fx["prefill_positions"])].transpose(0, 1)
    err_p = _check_summaries(pre, fx, "prefill", FP32_LOGIT_ATOL)
    print(f"{name}: ids exact; max logit err decode {err:.2e} prefill {err_p:.2e}")


@pytest.mark.parametrize("name", ["q7b2_bf16", "q05b2_b32_bf16", "q05b2_b3_bf16", "q05b2_b20_bf16", "q05b2_b48_bf16",
                                  "q7b1_b2_p256_bf16",
                                  "q05b_b32_bf16",
                                  "q7b_bf16", "q7b_b4_p640_bf16"])
def test_bf16_logits_teacher_forced(name):
    fx = np.load(os.path.join(GOLDEN, f"{name}.npz"))
    model = _model(name)
    prompt = torch.from_numpy(fx["prompt"]).to(DEV)
    n = fx["ids"].shape[1] - prompt.shape[1]
    rows, prefill = _teacher_forced_rows(model, prompt, torch.from_numpy(fx["ids"]), n)
    err = _check_summaries(rows, fx, "step", BF16_LOGIT_ATOL)
    pre = prefill[:, torch.from_numpy(fx["prefill_positions"])].transpose(0, 1)
    err_p = _check_summaries(pre, fx, "prefill", BF16_LOGIT_ATOL)
    picks = rows.argmax(-1).numpy()  # [S, B]
    ref = fx["ids"][:, prompt.shape[1]:].T
    clear = fx["step_margin"] > 0.1
    assert np.array_equal(picks[clear], ref[clear])
    print(f"{name}: max logit err decode {err:.3f} prefill {err_p:.3f}")
