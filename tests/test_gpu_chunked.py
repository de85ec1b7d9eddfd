"""Prefill into a non-empty cache and generation resumed on a filled cache.

The reference serves both through the same forward: a T > 1 forward on a cache
holding ``cache_len`` tokens attends with the mask ``tril(diagonal=cache_len)``
(attention.py:96-103), and ``GenerationState(kv=...)`` prefills its prompt on
top of whatever the cache already holds, positions restarting at 0
(generation.py:93,103,112-116). Here the oracle runs the same chunk sequence
live on the CPU from the same weights. Bars as for the other model tests: fp32
logits within 1e-3 and greedy ids exact; bf16 logits within 0.5.
"""

import dataclasses

import pytest
import torch

from tests.test_gpu_model import BF16_LOGIT_ATOL, FP32_LOGIT_ATOL, _model_from_state

pytestmark = pytest.mark.gpu
DEV = "cuda"

ATOL = {torch.float32: FP32_LOGIT_ATOL, torch.bfloat16: BF16_LOGIT_ATOL}


def _pair(shape, dtype):
    """The build's model and the oracle, from one seeded reference state."""
    from oracle import qwen2_ref

    state = qwen2_ref.synthetic_state(shape, seed=0, dtype=torch.float32)
    model = _model_from_state(shape, state, dtype)
    oracle = qwen2_ref.OracleQwen2(shape, {k: v.to(dtype) for k, v in state.items()})
    return model, oracle


def _run_chunks(model, oracle, prompt, chunks, max_seq, dtype):
    from minitp.generation import make_kv_cache

    b = prompt.shape[0]
    kv = make_kv_cache(model, b, max_seq)
    kv.poison(float("nan"))  # nothing beyond the cursor may be read
    okv = oracle.make_kv_cache(b, max_seq)
    s, worst = 0, 0.0
    for n in chunks:
        pos = torch.arange(s, s + n)
        got = model(prompt[:, s : s + n].to(DEV), positions=pos.to(DEV), kv_cache=kv).float().cpu()
        ref = oracle(prompt[:, s : s + n], positions=pos, kv_cache=okv).float()
        err = (got - ref).abs().max().item()
        print(f"chunk at {s} of {n}: max logit err {err:.2e}", flush=True)
        assert err <= ATOL[dtype], (s, n, err)
        if dtype == torch.float32:
            assert torch.equal(got.argmax(-1), ref.argmax(-1)), (s, n)
        worst = max(worst, err)
        s += n
    assert kv.seq_len == okv.seq_len == s
    return worst


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_chunked_prefill_tiny(dtype):
    from oracle import qwen2_ref

    model, oracle = _pair(qwen2_ref.TINY, dtype)
    prompt = qwen2_ref.synthetic_prompt(qwen2_ref.TINY.vocab_size, 2, 30, seed=5)
    # a one-token chunk in the middle runs the decode path on the same cache
    _run_chunks(model, oracle, prompt, [7, 9, 1, 5, 8], 40, dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_chunked_prefill_q05b_shape(dtype):
    """0.5B layer shape, two layers: the MFMA GEMM and prefill-attention paths
    with a key offset, chunks crossing the 64-query and 64-key tiles."""
    from oracle import qwen2_ref

    shape = dataclasses.replace(qwen2_ref.QWEN05B, num_hidden_layers=2)
    model, oracle = _pair(shape, dtype)
    prompt = qwen2_ref.synthetic_prompt(shape.vocab_size, 1, 150, seed=6)
    _run_chunks(model, oracle, prompt, [40, 70, 1, 39], 160, dtype)


def test_chunked_equals_one_prefill_fp32():
    """Chunked and whole-prompt prefills give the same last-chunk logits."""
    from oracle import qwen2_ref

    from minitp.generation import make_kv_cache

    model, _ = _pair(qwen2_ref.TINY, torch.float32)
    prompt = qwen2_ref.synthetic_prompt(qwen2_ref.TINY.vocab_size, 2, 24, seed=7).to(DEV)
    kv_a = make_kv_cache(model, 2, 24)
    whole = model(prompt, kv_cache=kv_a)
    kv_b = make_kv_cache(model, 2, 24)
    model(prompt[:, :16], kv_cache=kv_b)
    last = model(prompt[:, 16:], positions=torch.arange(16, 24, device=DEV), kv_cache=kv_b)
    assert (last - whole[:, 16:]).abs().max().item() <= FP32_LOGIT_ATOL
    for a, b in zip(kv_a.k + kv_a.v, kv_b.k + kv_b.v):
        assert (a - b).abs().max().item() <= 1e-5


def _filled(model, oracle, first):
    from minitp.generation import make_kv_cache

    kv = make_kv_cache(model, first.shape[0], 32)
    okv = oracle.make_kv_cache(first.shape[0], 32)
    model(first.to(DEV), kv_cache=kv)
    oracle(first, kv_cache=okv)
    return kv, okv


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_generation_resumes_on_filled_cache(dtype):
    """GenerationState(kv=...) on a cache already holding a first prompt:
    logits of every selection, teacher-forced with the oracle's tokens, and
    for fp32 the greedy ids of a free-running generation."""
    from oracle import qwen2_ref

    from minitp.generation import GenerationState, generate_greedy

    model, oracle = _pair(qwen2_ref.TINY, dtype)
    first = qwen2_ref.synthetic_prompt(qwen2_ref.TINY.vocab_size, 2, 9, seed=8)
    second = qwen2_ref.synthetic_prompt(qwen2_ref.TINY.vocab_size, 2, 6, seed=9)
    n = 10
    kv, okv = _filled(model, oracle, first)
    ref_rows = []
    ref = qwen2_ref.generate_greedy(oracle, second, n, early_stop=False, kv=okv,
                                    on_logits=lambda step, lg: ref_rows.append(lg[:, -1].float().clone()))
    assert okv.seq_len == 9 + 6 + n - 1

    st = GenerationState(model, second.to(DEV), n, kv=kv)
    logits = st.prefill()
    worst = 0.0
    for step in range(n):
        worst = max(worst, (logits[:, -1].float().cpu() - ref_rows[step]).abs().max().item())
        pos = st.append(ref[:, 6 + step].to(DEV))
        if step + 1 < n:
            logits = st.decode_step(ref[:, 6 + step].to(DEV), pos)
    print(f"resume: max logit err {worst:.2e}")
    assert worst <= ATOL[dtype]
    assert kv.seq_len == okv.seq_len

    if dtype == torch.float32:
        kv2, _ = _filled(model, oracle, first)
        out = generate_greedy(model, second.to(DEV), n, early_stop=False, kv=kv2).cpu()
        assert torch.equal(out, ref)


def test_chunks_and_resume_match_the_reference_fixture():
    """The reference's own chunked prefill (7, 9, 1, 5 tokens) and the
    generation it resumed on that cache (tests/golden/tiny_chunked_fp32.npz):
    chunk logits within the fp32 bar with the same argmax, resumed ids exact,
    the same cache cursor."""
    import os

    import numpy as np

    from oracle import qwen2_ref
    from tests.conftest import GOLDEN

    from minitp.generation import generate_greedy, make_kv_cache

    fx = np.load(os.path.join(GOLDEN, "tiny_chunked_fp32.npz"))
    shape = qwen2_ref.TINY
    model = _model_from_state(shape, qwen2_ref.synthetic_state(shape, seed=0, dtype=torch.float32), torch.float32)
    prompt = torch.from_numpy(fx["prompt"]).to(DEV)
    resume = torch.from_numpy(fx["resume_prompt"]).to(DEV)
    new = fx["resume_ids"].shape[1] - resume.shape[1]
    kv = make_kv_cache(model, prompt.shape[0], prompt.shape[1] + fx["resume_ids"].shape[1])
    kv.poison(float("nan"))
    outs, s = [], 0
    with torch.inference_mode():
        for n in fx["chunks"].tolist():
            pos = torch.arange(s, s + n, device=DEV)
            outs.append(model(prompt[:, s:s + n], positions=pos, kv_cache=kv).float().cpu())
            s += n
        got = torch.cat(outs, dim=1)
        ref = torch.from_numpy(fx["chunk_logits"])
        assert (got - ref).abs().max().item() <= FP32_LOGIT_ATOL
        assert torch.equal(got.argmax(-1), ref.argmax(-1))
        ids = generate_greedy(model, resume, new, early_stop=False, kv=kv).cpu()
    assert np.array_equal(ids.numpy(), fx["resume_ids"])
    assert kv.seq_len == int(fx["seq_len"])
