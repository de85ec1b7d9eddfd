"""Whole-model parity on the GPU against golden vectors written from the reference.

Bars: fp32 greedy ids bit-exact with the reference's fp32 TP=1 path and
logits within 1e-3 abs; bf16 logits within 0.5 abs, compared teacher-forced
(the reference's own token sequence is fed back) so one near-tie cannot
cascade. Golden fixtures: tests/golden/*.npz (see make_reference_vectors.py).
"""

import os

import numpy as np
import pytest
import torch

from tests.conftest import GOLDEN

pytestmark = pytest.mark.gpu
DEV = "cuda"

FP32_LOGIT_ATOL = 1e-3
BF16_LOGIT_ATOL = 0.5


def _fixture(name):
    return np.load(os.path.join(GOLDEN, f"{name}.npz"))


def _oracle_state(shape_name, dtype):
    from oracle import qwen2_ref

    shape = getattr(qwen2_ref, shape_name)
    return shape, qwen2_ref.synthetic_state(shape, seed=0, dtype=torch.float32)


def _model_from_state(shape, state, dtype):
    """Reference pattern: build the model, copy weights through state_dict."""
    from minitp.config import ModelConfig
    from minitp.distributed.context import ParallelContext
    from minitp.layer import TPQwen2ForCausalLM

    cfg = ModelConfig(**shape.__dict__)
    model = TPQwen2ForCausalLM(cfg, ParallelContext(0, 0, 1, 0, 1, torch.device(DEV), None))
    sd = model.state_dict()
    for k in sd:
        sd[k] = state[k]
    model.load_state_dict(sd)
    return model.to(DEV, dtype).eval()


def _synthetic(shape_name, dtype):
    from minitp import synthetic

    cfg = {"TINY": synthetic.TINY, "QWEN05B": synthetic.QWEN05B}[shape_name]
    return synthetic.build_synthetic_model(cfg, dtype=dtype, device=DEV, seed=0)


def _teacher_forced_rows(model, prompt, ref_ids, n_steps):
    """Logits row each selection reads, feeding the reference's tokens."""
    from minitp.generation import GenerationState

    st = GenerationState(model, prompt, n_steps)
    logits = st.prefill()
    prefill = logits.clone()
    rows = [logits[:, -1].float().clone()]
    t = prompt.shape[1]
    for s in range(n_steps - 1):
        tok = ref_ids[:, t + s].to(DEV)
        pos = st.append(tok)
        logits = st.decode_step(tok, pos)
        rows.append(logits[:, -1].float().clone())
    return torch.stack(rows).cpu(), prefill.float().cpu()


def _check_summaries(rows, fx, prefix, atol):
    """rows [S, B, V] vs the fixture's top-k / sampled-column values."""
    topk_ids = torch.from_numpy(fx[f"{prefix}_topk_ids"])
    topk_vals = torch.from_numpy(fx[f"{prefix}_topk_vals"])
    got_topk = torch.gather(rows, -1, topk_ids)
    err_topk = (got_topk - topk_vals).abs().max().item()
    cols = torch.from_numpy(fx["sample_cols"])
    err_cols = (rows[..., cols] - torch.from_numpy(fx[f"{prefix}_sample_vals"])).abs().max().item()
    assert err_topk <= atol and err_cols <= atol, (prefix, err_topk, err_cols)
    return max(err_topk, err_cols)


# ---------------------------------------------------------------------------


@pytest.mark.parametrize("name", ["tiny_fp32", "tiny_b3_fp32"])
def test_tiny_fp32_greedy_ids_bitexact_and_logits(name):
    from minitp.generation import generate_greedy

    fx = _fixture(name)
    shape, state = _oracle_state("TINY", torch.float32)
    model = _model_from_state(shape, state, torch.float32)
    prompt = torch.from_numpy(fx["prompt"]).to(DEV)
    n = fx["ids"].shape[1] - prompt.shape[1]
    ids = generate_greedy(model, prompt, n, early_stop=False)
    assert np.array_equal(ids.cpu().numpy(), fx["ids"])
    rows, prefill = _teacher_forced_rows(model, prompt, torch.from_numpy(fx["ids"]), n)
    assert (rows - torch.from_numpy(fx["step_logits"])).abs().max().item() <= FP32_LOGIT_ATOL
    assert (prefill - torch.from_numpy(fx["prefill_logits"])).abs().max().item() <= FP32_LOGIT_ATOL


def test_generation_lengths_sharing_a_cache_capacity_replay_one_graph():
    """Caches of 28 and 32 positions both hold 32 rows (the capacity the
    kernels index by), so the second generation replays the decode graph the
    first recorded: its 16 + 8 ids are the fixture's, and the shorter run's ids
    are the longer's prefix (fixed-length greedy)."""
    from minitp.generation import generate_greedy

    fx = _fixture("tiny_fp32")
    shape, state = _oracle_state("TINY", torch.float32)
    model = _model_from_state(shape, state, torch.float32)
    prompt = torch.from_numpy(fx["prompt"]).to(DEV)
    n = fx["ids"].shape[1] - prompt.shape[1]  # 16 new tokens: a 24-row cache of capacity 32
    full = generate_greedy(model, prompt, n, early_stop=False)
    short = generate_greedy(model, prompt, n - 4, early_stop=False)  # 20 rows, capacity 32
    longer = generate_greedy(model, prompt, n + 8, early_stop=False)  # 32 rows, capacity 32
    assert np.array_equal(full.cpu().numpy(), fx["ids"])
    assert torch.equal(short, full[:, : prompt.shape[1] + n - 4])
    assert torch.equal(longer[:, : full.shape[1]], full)
    model.program().check_decode()


def test_tiny_bf16_logits_teacher_forced():
    fx = _fixture("tiny_bf16")
    shape, state = _oracle_state("TINY", torch.float32)
    model = _model_from_state(shape, state, torch.bfloat16)
    prompt = torch.from_numpy(fx["prompt"]).to(DEV)
    n = fx["ids"].shape[1] - prompt.shape[1]
    rows, prefill = _teacher_forced_rows(model, prompt, torch.from_numpy(fx["ids"]), n)
    assert (rows - torch.from_numpy(fx["step_logits"])).abs().max().item() <= BF16_LOGIT_ATOL
    assert (prefill - torch.from_numpy(fx["prefill_logits"])).abs().max().item() <= BF16_LOGIT_ATOL


def test_synthetic_tiny_equals_state_dict_copy():
    """The GPU generator builds the same model the oracle state describes."""
    shape, state = _oracle_state("TINY", torch.float32)
    a = _model_from_state(shape, state, torch.float32)
    b = _synthetic("TINY", torch.float32)
    for (ka, va), (kb, vb) in zip(a.state_dict().items(), b.state_dict().items(), strict=True):
        assert ka == kb and torch.equal(va, vb), ka


def test_q05b_fp32_256_greedy_ids_bitexact():
    from minitp.generation import generate_greedy

    fx = _fixture("q05b_fp32")
    model = _synthetic("QWEN05B", torch.float32)
    prompt = torch.from_numpy(fx["prompt"]).to(DEV)
    n = fx["ids"].shape[1] - prompt.shape[1]
    ids = generate_greedy(model, prompt, n, early_stop=False).cpu().numpy()
    model.program().check_decode()
    mism = np.nonzero(ids[0] != fx["ids"][0])[0]
    assert mism.size == 0, f"first mismatch at column {mism[0]} (prompt {prompt.shape[1]})"
    rows, prefill = _teacher_forced_rows(model, prompt, torch.from_numpy(fx["ids"]), n)
    err = _check_summaries(rows, fx, "step", FP32_LOGIT_ATOL)
    pre = prefill[:, torch.from_numpy(fx["prefill_positions"])].transpose(0, 1)
    err_p = _check_summaries(pre, fx, "prefill", FP32_LOGIT_ATOL)
    model.program().check_decode()
    print(f"q05b fp32: 256/256 ids exact; max logit err decode {err:.2e} prefill {err_p:.2e}")


def test_q05b_bf16_logits_teacher_forced():
    fx = _fixture("q05b_bf16")
    model = _synthetic("QWEN05B", torch.bfloat16)
    prompt = torch.from_numpy(fx["prompt"]).to(DEV)
    n = fx["ids"].shape[1] - prompt.shape[1]
    rows, prefill = _teacher_forced_rows(model, prompt, torch.from_numpy(fx["ids"]), n)
    err = _check_summaries(rows, fx, "step", BF16_LOGIT_ATOL)
    pre = prefill[:, torch.from_numpy(fx["prefill_positions"])].transpose(0, 1)
    err_p = _check_summaries(pre, fx, "prefill", BF16_LOGIT_ATOL)
    # agreement of the greedy pick where the reference margin is clear
    picks = rows.argmax(-1)[:, 0].numpy()
    ref = fx["ids"][0, prompt.shape[1]:]
    clear = fx["step_margin"][:, 0] > 0.1
    assert np.array_equal(picks[clear], ref[clear])
    model.program().check_decode()
    print(f"q05b bf16: max logit err decode {err:.3f} prefill {err_p:.3f}")


# ---------------------------------------------------------------------------
# execution paths agree


def _program_with_env(model, name, value):
    """(Re)create the model's native program with an environment switch set
    (the library reads it when the program is created)."""
    import os

    old = os.environ.get(name)
    os.environ[name] = value
    try:
        model._prog = None
        model.program()
    finally:
        if old is None:
            del os.environ[name]
        else:
            os.environ[name] = old


@pytest.mark.parametrize("shape_name", ["TINY", "QWEN05B"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_fused_attention_oproj_matches_separate_oproj(shape_name, dtype):
    """Batch-1 decode folds o_proj into the attention kernel (per-head fp32
    partials, summed with the residual by the gate/up prologue). Against the
    separate o_proj GEMV (MINITP_FUSE_OPROJ=0) only o_proj's summation order
    differs: teacher-forced logits agree to fp32 rounding (fp32) or within
    the bf16 logit bar, the greedy picks wherever the top-2 margin is clear,
    and the fused run's ids are the greedy ids of its own logits."""
    from minitp.generation import generate_greedy

    fused = _synthetic(shape_name, dtype)
    split = _synthetic(shape_name, dtype)
    _program_with_env(split, "MINITP_FUSE_OPROJ", "0")
    v = fused.cfg.vocab_size
    prompt = torch.randint(0, v, (1, 12), generator=torch.Generator().manual_seed(11)).to(DEV)
    ids = generate_greedy(fused, prompt, 48, early_stop=False)
    rf, _ = _teacher_forced_rows(fused, prompt, ids.cpu(), 48)
    rs, _ = _teacher_forced_rows(split, prompt, ids.cpu(), 48)
    fused.program().check_decode()
    split.program().check_decode()
    atol = 2e-4 if dtype == torch.float32 else BF16_LOGIT_ATOL
    err = (rf - rs).abs().max().item()
    assert torch.isfinite(rf).all() and err <= atol, err
    top2 = rs.topk(2, dim=-1).values
    clear = (top2[..., 0] - top2[..., 1]) > 2 * atol
    assert torch.equal(rf.argmax(-1)[clear], rs.argmax(-1)[clear])
    # decode rows (the prefill row comes from the every-position prompt form)
    assert torch.equal(rf.argmax(-1)[1:, 0], ids[0, 13:].cpu())
    print(f"{shape_name} {dtype}: fused vs separate o_proj max logit diff {err:.3e}")


def _tiny(dtype=torch.float32):
    shape, state = _oracle_state("TINY", torch.float32)
    return _model_from_state(shape, state, dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_graph_decode_equals_direct_forward(dtype):
    from minitp.generation import GenerationState, make_kv_cache

    model = _tiny(dtype)  # the decode graph replays the direct launch sequence
    prompt = torch.tensor([[3, 17, 256, 999, 41]], device=DEV)
    st = GenerationState(model, prompt, 6)
    kv = make_kv_cache(model, 1, 11)
    direct = model(prompt, positions=torch.arange(5, device=DEV), kv_cache=kv)
    logits = st.prefill()
    assert torch.equal(logits, direct)
    for _ in range(5):
        tok = st.select_next(logits)
        pos = st.append(tok)
        logits = st.decode_step(tok, pos)
        d = model(tok.unsqueeze(-1), positions=pos.reshape(1), kv_cache=kv)
        assert torch.equal(logits, d)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_module_path_matches_native_program(dtype):
    from minitp.generation import generate_greedy, make_kv_cache

    model = _tiny(dtype)
    prompt = torch.tensor([[3, 17, 256, 999, 41, 7, 8, 9]], device=DEV)
    kv_a = make_kv_cache(model, 1, 9)
    native = model(prompt, positions=torch.arange(8, device=DEV), kv_cache=kv_a)
    nat_dec = model(prompt[:, :1], positions=torch.tensor([8], device=DEV), kv_cache=kv_a)
    for layer in model.model.layers:  # ablation toggles force the module path
        layer.self_attn.use_fused_qkv = False
        layer.mlp.use_fused_gateup = False
    assert not model.native_path()
    kv_b = make_kv_cache(model, 1, 9)
    modules = model(prompt, positions=torch.arange(8, device=DEV), kv_cache=kv_b)
    mod_dec = model(prompt[:, :1], positions=torch.tensor([8], device=DEV), kv_cache=kv_b)
    # same kernels except the RMSNorm before each projection: fused into the
    # GEMV prologue natively, a separate kernel on the module path (its sum of
    # squares runs in a different order), so agreement is to rounding
    tol = dict(atol=1e-5, rtol=1e-5) if dtype == torch.float32 else dict(atol=0.05, rtol=0.02)
    torch.testing.assert_close(native, modules, **tol)
    torch.testing.assert_close(nat_dec, mod_dec, **tol)
    ids_mod = generate_greedy(model, prompt, 6, early_stop=False)
    for layer in model.model.layers:
        layer.self_attn.use_fused_qkv = True
        layer.mlp.use_fused_gateup = True
    assert torch.equal(ids_mod, generate_greedy(model, prompt, 6, early_stop=False))


def test_uncached_rope_toggle_matches_cached_values():
    model = _tiny()
    prompt = torch.tensor([[3, 17, 256, 999]], device=DEV)
    a = model(prompt)
    model.use_rotary_cache = False
    b = model(prompt)
    # identical tables (uncached rows equal cached rows); the toggle also moves
    # the forward onto the module path, which normalises in its own kernel
    torch.testing.assert_close(a, b, atol=1e-5, rtol=1e-5)


# ---------------------------------------------------------------------------
# token loop and KV-cache contracts (test_qwen_tiny.py, test_kv_cache.py)


def test_kv_decode_matches_full_prefill():
    from minitp.generation import generate_greedy

    model = _tiny()
    ids = torch.tensor([[5, 60, 7, 99, 120, 33]], device=DEV)
    ref_tokens = generate_greedy(model, ids, max_new_tokens=5, distributed_argmax=False)
    logits = model(ref_tokens)
    assert torch.equal(logits[:, 5:-1].argmax(-1), ref_tokens[:, 6:])


def test_fixed_length_matches_early_stop_prefix():
    from minitp.generation import generate_greedy

    model = _tiny()
    ids = torch.tensor([[5, 60, 7, 99, 120], [1, 2, 3, 4, 5]], device=DEV)
    eager = generate_greedy(model, ids, max_new_tokens=8, eos_token_id=None, early_stop=True)
    fixed = generate_greedy(model, ids, max_new_tokens=8, eos_token_id=None, early_stop=False)
    assert eager.shape == (2, 13) and torch.equal(eager, fixed)


def test_early_stop_on_eos_trims_and_pads():
    from minitp.generation import generate_greedy

    model = _tiny()
    ids = torch.tensor([[5, 60, 7, 99, 120]], device=DEV)
    fixed = generate_greedy(model, ids, max_new_tokens=8, early_stop=False)
    eos = int(fixed[0, 6])  # the second generated token
    out = generate_greedy(model, ids, max_new_tokens=8, eos_token_id=eos, early_stop=True)
    assert torch.equal(out, fixed[:, : out.shape[1]]) and int(out[0, -1]) == eos


def test_poisoned_cache_k_and_v_separately():
    from minitp.generation import generate_greedy, make_kv_cache

    model = _tiny()
    ids = torch.tensor([[5, 60, 7, 99, 120, 33]], device=DEV)
    ref = generate_greedy(model, ids, max_new_tokens=8, early_stop=False)
    for which in ("k", "v"):
        kv = make_kv_cache(model, 1, 24)
        for buf in kv.k if which == "k" else kv.v:
            buf.fill_(float("nan"))
        out = generate_greedy(model, ids, max_new_tokens=8, early_stop=False, kv=kv)
        assert torch.equal(out, ref), which


def test_cursor_bounds_after_each_advance():
    from minitp.generation import GenerationState, make_kv_cache

    model = _tiny()
    ids = torch.tensor([[5, 60, 7, 99]], device=DEV)
    kv = make_kv_cache(model, 1, 16)
    kv.poison(float("nan"))
    st = GenerationState(model, ids, max_new_tokens=4, kv=kv)
    logits = st.prefill()
    tok = st.select_next(logits)
    for _ in range(4):
        pos = st.append(tok)
        logits = st.decode_step(tok, pos)
        tok = st.select_next(logits)
    assert kv.seq_len == 8
    for buf in (*kv.k, *kv.v):
        assert torch.isfinite(buf[:, :, :8]).all() and torch.isnan(buf[:, :, 8:]).all()


def test_overflow_raises_before_launch():
    from minitp.generation import make_kv_cache

    model = _tiny()
    kv = make_kv_cache(model, 1, 6)
    with pytest.raises(ValueError, match="overflow"):
        model(torch.randint(3, 100, (1, 8), device=DEV), kv_cache=kv)
    assert kv.seq_len == 0


def test_zeros_init_matches_empty_init():
    from minitp.generation import generate_greedy

    model = _tiny()
    ids = torch.tensor([[5, 60, 7, 99, 120, 33]], device=DEV)
    a = generate_greedy(model, ids, max_new_tokens=8, early_stop=False, kv_init="zeros")
    b = generate_greedy(model, ids, max_new_tokens=8, early_stop=False, kv_init="empty")
    assert torch.equal(a, b)


def test_exactly_one_arange_per_generation():
    from minitp.bench.benchmark import bench_one_iter
    from minitp.generation import generate_greedy

    model = _tiny()
    ids = torch.tensor([[5, 60, 7, 99, 120, 33]], device=DEV)
    with torch.inference_mode():
        bench_one_iter(model, ids, 8)
        generate_greedy(model, ids, max_new_tokens=8, early_stop=False)
    real = torch.arange
    calls = {"n": 0}

    def counting(*a, **kw):
        calls["n"] += 1
        return real(*a, **kw)

    torch.arange = counting
    try:
        bench_one_iter(model, ids, 8)
        bench_n, calls["n"] = calls["n"], 0
        generate_greedy(model, ids, max_new_tokens=8, early_stop=False)
        gen_n = calls["n"]
    finally:
        torch.arange = real
    assert bench_n == gen_n == 1


def test_bench_windows_ttft_covers_prefill_and_selection():
    from minitp.bench.benchmark import bench_one_iter

    model = _tiny()
    ids = torch.tensor([[5, 60, 7, 99, 120, 33]], device=DEV)
    prefill_s, ttft_s, sel_ms, steps = bench_one_iter(model, ids, 4)
    assert len(steps) == 3 and ttft_s + 1e-3 >= prefill_s + sel_ms / 1e3 - 2e-3


@pytest.mark.parametrize("batch", [1, 3])
def test_bench_timed_loop_produces_generate_greedy_ids(batch):
    """The decode loop bench.py times (StepSource: a GenerationState with
    last-position prompt logits and reused decode logits, append +
    decode_step + select_next per step) computes the real generation: after
    one generation its ids are generate_greedy's for the same prompt, and a
    second back-to-back generation repeats them."""
    import bench
    from minitp.generation import generate_greedy

    model = _synthetic("QWEN05B", torch.bfloat16)
    g = torch.Generator().manual_seed(batch)
    prompt = torch.randint(0, model.cfg.vocab_size, (batch, 16), generator=g).to(DEV)
    new = 24
    src = bench.StepSource(model, prompt, new)
    src.run(new - 1)
    first = src.state.out_ids.clone()
    src.run(new - 1)
    assert src.generations == 2
    ref = generate_greedy(model, prompt, new, early_stop=False)
    model.program().check_decode()
    assert torch.equal(first, ref)
    assert torch.equal(src.state.out_ids, ref)


@pytest.mark.parametrize("batch,plen", [(1, 1), (2, 1), (1, 2), (40, 6), (64, 3)])
def test_shortest_prompts_and_wide_batches_match_the_oracle(batch, plen):
    """One- and two-token prompts (a one-token prompt's forward takes the
    single-token launch sequence the decode steps use, with no cached rows)
    and batches past the GEMV forms' 32 rows (40 and 64: decode products on
    the GEMM), tiny fp32: greedy ids equal the oracle's generate_greedy on the
    same weights, bit for bit."""
    from oracle import qwen2_ref as R

    from minitp.generation import generate_greedy

    shape, state = _oracle_state("TINY", torch.float32)
    model = _model_from_state(shape, state, torch.float32)
    g = torch.Generator().manual_seed(100 * batch + plen)
    prompt = torch.randint(0, shape.vocab_size, (batch, plen), generator=g)
    ref = R.generate_greedy(R.OracleQwen2(shape, state), prompt, 12, early_stop=False)
    got = generate_greedy(model, prompt.to(DEV), 12, early_stop=False)
    model.program().check_decode()
    assert torch.equal(got.cpu(), ref)
