"""Early stop on an EOS token with the finished mask on the device.

generate_greedy(early_stop=True, eos_token_id=e) (generation.py:133-171)
against the oracle's loop, run live on the CPU: the same trimmed ids, the
same KV fill cursor, and no KV row written past it (the cache is poisoned
with NaN first, so a row written by a step queued past the stop shows up).
Batches 1-3 run the fused GEMV program, batch 5 the GEMM one. On the bf16
0.5B layer shape (batches 1, 4 and 40) the reference is the same model's
fixed-length run cut at the stop.
"""

import pytest
import torch

from tests.test_gpu_model import _model_from_state

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(scope="module")
def pair():
    from oracle import qwen2_ref

    shape = qwen2_ref.TINY
    state = qwen2_ref.synthetic_state(shape, seed=0, dtype=torch.float32)
    return _model_from_state(shape, state, torch.float32), qwen2_ref.OracleQwen2(shape, state)


def _both(pair, prompt, n, eos, max_seq=None):
    from oracle import qwen2_ref

    from minitp.generation import generate_greedy, make_kv_cache

    model, oracle = pair
    b, t = prompt.shape
    max_seq = max_seq or t + n
    kv = make_kv_cache(model, b, max_seq)
    kv.poison(float("nan"))
    okv = oracle.make_kv_cache(b, max_seq)
    got = generate_greedy(model, prompt.to(DEV), n, eos_token_id=eos, early_stop=True, kv=kv).cpu()
    ref = qwen2_ref.generate_greedy(oracle, prompt, n, eos_token_id=eos, early_stop=True, kv=okv)
    assert got.shape == ref.shape and torch.equal(got, ref), (got, ref)
    assert kv.seq_len == okv.seq_len, (kv.seq_len, okv.seq_len)
    for buf in kv.k + kv.v:
        assert torch.isfinite(buf[:, :, : kv.seq_len]).all()
        assert torch.isnan(buf[:, :, kv.seq_len :]).all(), "a KV row was written past the stop"
    return got


def _free_run(pair, prompt, n):
    from oracle import qwen2_ref

    return qwen2_ref.generate_greedy(pair[1], prompt, n, early_stop=False)


@pytest.mark.parametrize("batch", [1, 3, 5])
def test_rows_finishing_at_different_steps(pair, batch):
    prompt, eos, firsts = _rows_sharing_a_token(pair, batch, 32)
    out = _both(pair, prompt, 32, eos)
    print(f"batch {batch}: eos {eos}, first reached per row {firsts}, stopped at {out.shape[1]} of {6 + 32}")
    assert out.shape[1] == 6 + max(firsts) + 1


def _rows_sharing_a_token(pair, batch, n):
    """Prompts of `batch` rows that all generate one token, each row reaching
    it at a different step, picked from 256 candidate rows (rows of a batch
    do not interact, so the subset's runs are the candidates' runs). The
    tiny model mostly repeats one token per row, so few tokens qualify."""
    from oracle import qwen2_ref

    cand = qwen2_ref.synthetic_prompt(qwen2_ref.TINY.vocab_size, 256, 6, seed=11)
    gen = _free_run(pair, cand, n)[:, 6:]
    best = None
    for v in torch.unique(gen).tolist():
        hit = gen == v
        by_step = {}
        for r in hit.any(1).nonzero().flatten().tolist():
            by_step.setdefault(int(hit[r].int().argmax()), r)
        if len(by_step) < batch:
            continue
        steps = sorted(by_step)
        pick = [steps[round(i * (len(steps) - 1) / max(batch - 1, 1))] for i in range(batch)]
        if best is None or pick[-1] - pick[0] > best[0]:
            best = (pick[-1] - pick[0], v, [by_step[k] for k in pick], pick)
    assert best is not None, "no token reached by enough rows at different steps"
    return cand[best[2]], best[1], best[3]


def test_eos_never_produced_runs_full_length(pair):
    from oracle import qwen2_ref

    prompt = qwen2_ref.synthetic_prompt(qwen2_ref.TINY.vocab_size, 2, 5, seed=12)
    free = _free_run(pair, prompt, 10)
    unused = next(v for v in range(qwen2_ref.TINY.vocab_size) if not (free[:, 5:] == v).any())
    out = _both(pair, prompt, 10, unused)
    assert out.shape[1] == 15


def test_stop_on_the_prefill_token(pair):
    """Every row's first pick is EOS: no decode step may leave a trace."""
    from oracle import qwen2_ref

    prompt = qwen2_ref.synthetic_prompt(qwen2_ref.TINY.vocab_size, 1, 7, seed=13)
    free = _free_run(pair, prompt, 4)
    out = _both(pair, prompt, 12, int(free[0, 7]))
    assert out.shape[1] == 8


def test_stop_on_the_last_step_and_single_token(pair):
    from oracle import qwen2_ref

    prompt = qwen2_ref.synthetic_prompt(qwen2_ref.TINY.vocab_size, 1, 5, seed=14)
    free = _free_run(pair, prompt, 6)
    last = int(free[0, -1])
    if not (free[0, 5:-1] == last).any():
        assert _both(pair, prompt, 6, last).shape[1] == 11
    _both(pair, prompt, 1, int(free[0, 5]))


def test_resume_with_eos_on_a_filled_cache(pair):
    """kv= holding an earlier prompt: the stop cursor counts from it."""
    from oracle import qwen2_ref

    from minitp.generation import generate_greedy, make_kv_cache

    model, oracle = pair
    first = qwen2_ref.synthetic_prompt(qwen2_ref.TINY.vocab_size, 2, 4, seed=15)
    second = qwen2_ref.synthetic_prompt(qwen2_ref.TINY.vocab_size, 2, 5, seed=16)
    kv = make_kv_cache(model, 2, 30)
    okv = oracle.make_kv_cache(2, 30)
    model(first.to(DEV), kv_cache=kv)
    oracle(first, kv_cache=okv)
    free = qwen2_ref.generate_greedy(oracle, second, 12, early_stop=False,
                                     kv=_copy_cache(oracle, okv))
    eos = int(free[1, 5 + 2])
    got = generate_greedy(model, second.to(DEV), 12, eos_token_id=eos, kv=kv).cpu()
    ref = qwen2_ref.generate_greedy(oracle, second, 12, eos_token_id=eos, kv=okv)
    assert torch.equal(got, ref) and kv.seq_len == okv.seq_len


def _copy_cache(oracle, okv):
    c = oracle.make_kv_cache(okv.k[0].shape[0], okv.max_seq_len)
    for dst, src in zip(c.k + c.v, okv.k + okv.v):
        dst.copy_(src)
    c.seq_len = okv.seq_len
    return c


def test_early_stop_matches_the_reference_fixture():
    """generate_greedy(eos_token_id=e) against the reference's own outputs
    (tests/golden/tiny_eos_fp32.npz, tiny shape with std-0.3 weights): every
    row stopping at a different step, partial finishes padded with EOS, a
    first pick and an EOS never produced; ids, length and cache cursor
    exact, nothing written past the cursor."""
    import os

    import numpy as np

    from oracle import qwen2_ref
    from tests.conftest import GOLDEN

    from minitp.generation import generate_greedy, make_kv_cache

    fx = np.load(os.path.join(GOLDEN, "tiny_eos_fp32.npz"))
    shape = qwen2_ref.TINY
    state = qwen2_ref.synthetic_state(shape, seed=0, dtype=torch.float32, std=float(fx["weight_std"]))
    model = _model_from_state(shape, state, torch.float32)
    for i, eos in enumerate(fx["eos"].tolist()):
        b, n = int(fx["batch"][i]), int(fx["length"][i])
        prompt = torch.from_numpy(fx["prompts"][i, :b]).to(DEV)
        kv = make_kv_cache(model, b, prompt.shape[1] + 12)
        kv.poison(float("nan"))
        got = generate_greedy(model, prompt, 12, eos_token_id=eos, early_stop=True, kv=kv).cpu()
        assert np.array_equal(got.numpy(), fx["ids"][i, :b, :n]), (i, eos, got)
        assert kv.seq_len == int(fx["seq_len"][i])
        for buf in kv.k + kv.v:
            assert torch.isnan(buf[:, :, kv.seq_len:]).all()


@pytest.mark.parametrize("batch", [1, 4, 40])
def test_bf16_q05b_early_stop_equals_the_fixed_length_run_cut_at_the_stop(batch):
    """The device early stop on the bf16 0.5B layer shape (2 layers): batch 1
    (the argmax GEMV epilogue), 4 (the MFMA LM head and the argmax kernels)
    and 40 (the GEMM programs). Rows do not interact, so against the same
    model's fixed-length run, with EOS = the token row 0 produces at step 5:
    every row is its fixed-length row up to its first EOS and EOS after it,
    the loop ends after the step at which the last row finished (or runs to
    the end when a row never produces it), and the cache holds exactly the
    rows of the steps run."""
    import dataclasses

    from minitp import synthetic
    from minitp.generation import generate_greedy, make_kv_cache

    cfg = dataclasses.replace(synthetic.QWEN05B, num_hidden_layers=2)
    model = synthetic.build_synthetic_model(cfg, dtype=torch.bfloat16, device=DEV, seed=5)
    t, n = 8, 24
    half = synthetic.synthetic_prompt(cfg.vocab_size, 2, t, seed=13, device=DEV)
    rows = [half[0]] * ((batch + 1) // 2) + [half[1]] * (batch // 2)  # two distinct prompts
    prompt = torch.stack(rows) if batch > 1 else half[:1]
    fixed = generate_greedy(model, prompt, n, early_stop=False).cpu()
    eos = int(fixed[0, t + 5])
    kv = make_kv_cache(model, batch, t + n)
    kv.poison(float("nan"))
    got = generate_greedy(model, prompt, n, eos_token_id=eos, early_stop=True, kv=kv).cpu()
    gen = fixed[:, t:]
    hit = gen == eos
    first = [int(hit[r].int().argmax()) if hit[r].any() else None for r in range(batch)]
    steps = n if any(f is None for f in first) else max(first) + 1
    want = fixed[:, : t + steps].clone()
    for r, f in enumerate(first):
        if f is not None:
            want[r, t + f + 1:] = eos
    assert torch.equal(got, want), (got, want)
    assert kv.seq_len == t + steps - 1
    for buf in kv.k + kv.v:
        assert torch.isfinite(buf[:, :, : kv.seq_len]).all()
        assert torch.isnan(buf[:, :, kv.seq_len:]).all()
