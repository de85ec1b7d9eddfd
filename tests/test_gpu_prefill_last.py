"""Prefill that computes only the last position's logits.

``GenerationState(prefill_logits="last")`` (what ``generate_greedy`` uses)
runs the LM head on one row per sequence instead of T. Its logits must be the
reference's last row (the oracle's full forward, run live on the CPU) within
the model tests' bars, and its fused greedy pick must be the first maximum of
the row it returned. Batches 1-4 take the fused norm + GEMV + argmax head,
larger ones the GEMM head over the strided last rows.
"""

import pytest
import torch

from tests.test_gpu_model import BF16_LOGIT_ATOL, FP32_LOGIT_ATOL, _model_from_state, _synthetic

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(scope="module")
def tiny_state():
    from oracle import qwen2_ref

    return qwen2_ref.TINY, qwen2_ref.synthetic_state(qwen2_ref.TINY, seed=0, dtype=torch.float32)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("batch,t", [(1, 9), (3, 17), (4, 2), (6, 33)])
def test_last_row_logits_and_pick_match_oracle(tiny_state, dtype, batch, t):
    from oracle import qwen2_ref

    from minitp.generation import GenerationState

    shape, state = tiny_state
    model = _model_from_state(shape, state, dtype)
    oracle = qwen2_ref.OracleQwen2(shape, state)
    prompt = qwen2_ref.synthetic_prompt(shape.vocab_size, batch, t, seed=batch * 100 + t)
    ref = oracle(prompt, kv_cache=oracle.make_kv_cache(batch, t + 1))[:, -1].float()

    st = GenerationState(model, prompt.to(DEV), 1, prefill_logits="last")
    logits = st.prefill()
    tok = st.select_next(logits).cpu()
    assert logits.shape == (batch, 1, shape.vocab_size)
    got = logits[:, 0].float().cpu()
    atol = FP32_LOGIT_ATOL if dtype == torch.float32 else BF16_LOGIT_ATOL
    err = (got - ref).abs().max().item()
    assert err <= atol, f"max |logit - oracle| {err} > {atol}"
    assert torch.equal(tok, got.argmax(-1)), (tok, got.argmax(-1))
    if dtype == torch.float32:
        assert torch.equal(tok, ref.argmax(-1)), (tok, ref.argmax(-1))
    assert st.kv.seq_len == t


@pytest.mark.parametrize("batch", [2, 5])
def test_last_form_equals_full_form_q05b_bf16(batch):
    """0.5B shape: the last-only prefill against the full prefill's last row,
    and the same cache contents after both."""
    from minitp import synthetic
    from minitp.generation import GenerationState

    model = _synthetic("QWEN05B", torch.bfloat16)
    prompt = synthetic.synthetic_prompt(model.cfg.vocab_size, batch, 64, seed=7, device=DEV)
    full = GenerationState(model, prompt, 4)
    last = GenerationState(model, prompt, 4, prefill_logits="last")
    lf = full.prefill()
    ll = last.prefill()
    assert lf.shape[1] == 64 and ll.shape[1] == 1
    err = (lf[:, -1].float() - ll[:, 0].float()).abs().max().item()
    assert err <= BF16_LOGIT_ATOL, err
    tok = last.select_next(ll)
    assert torch.equal(tok, ll[:, 0].float().argmax(-1))
    for a, b in zip(full.kv.k + full.kv.v, last.kv.k + last.kv.v):
        assert torch.equal(a[:, :, :64], b[:, :, :64])


def test_bad_prefill_logits_value_raises():
    from minitp.generation import GenerationState

    model = _synthetic("TINY", torch.float32)
    with pytest.raises(ValueError, match="prefill_logits"):
        GenerationState(model, torch.zeros(1, 3, dtype=torch.long, device=DEV), 2, prefill_logits="none")
