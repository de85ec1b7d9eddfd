"""Drop-in API behaviour on the GPU: what reference callers see.

* ``decode_step`` returns a new logits tensor each step (generation.py:129-130);
* inputs that do not fit the model raise instead of reaching a kernel;
* explicit positions index the RoPE table like ``cos_cache[positions]``
  (rope.py:37-45): past the table raises IndexError, negative ones wrap;
* a decode shape first run without a token pick still picks tokens later;
* zero new tokens return the prompt after its forward (generation.py:150-171);
* ColumnParallelLinear / RowParallelLinear / the fused projections equal
  ``F.linear`` (test_column_row_parallel.py:116-135,
  test_fused_projections.py:27-54), RowParallel's bias added after the
  (skipped) reduce (linear.py:120-121).
"""

import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _tiny(dtype=torch.float32):
    from minitp import synthetic

    return synthetic.build_synthetic_model(synthetic.TINY, dtype=dtype, device=DEV, seed=0)


def _ctx():
    from minitp.distributed.context import ParallelContext

    return ParallelContext(0, 0, 1, 0, 1, torch.device(DEV), None)


@torch.inference_mode()
def test_decode_step_returns_new_logits_each_step():
    from minitp.generation import GenerationState

    model = _tiny()
    ids = torch.tensor([[5, 60, 7, 99, 120, 33]], device=DEV)
    st = GenerationState(model, ids, 4)
    tok = st.select_next(st.prefill())
    pos = st.append(tok)
    first = st.decode_step(tok, pos)
    kept = first.clone()
    tok = st.select_next(first)
    pos = st.append(tok)
    second = st.decode_step(tok, pos)
    torch.cuda.synchronize()
    assert second.data_ptr() != first.data_ptr()
    assert torch.equal(first, kept)  # the earlier step's logits were not overwritten
    assert not torch.equal(first, second)


@torch.inference_mode()
def test_reused_decode_logits_is_an_opt_in():
    from minitp.generation import GenerationState

    model = _tiny()
    ids = torch.tensor([[5, 60, 7, 99, 120, 33]], device=DEV)
    st = GenerationState(model, ids, 4, reuse_decode_logits=True)
    tok = st.select_next(st.prefill())
    pos = st.append(tok)
    a = st.decode_step(tok, pos)
    tok = st.select_next(a)
    pos = st.append(tok)
    b = st.decode_step(tok, pos)
    assert a.data_ptr() == b.data_ptr()


@torch.inference_mode()
def test_cache_that_does_not_fit_the_model_raises():
    from minitp.generation import GenerationState, make_kv_cache
    from minitp.kv_cache import KVCache

    model = _tiny()
    ids = torch.tensor([[5, 60, 7, 99]], device=DEV)
    cfg = model.cfg
    bad = [
        KVCache(cfg.num_hidden_layers - 1, 1, 2, cfg.head_dim, 16, torch.float32, torch.device(DEV)),  # layers
        KVCache(cfg.num_hidden_layers, 2, 2, cfg.head_dim, 16, torch.float32, torch.device(DEV)),  # batch
        KVCache(cfg.num_hidden_layers, 1, 1, cfg.head_dim, 16, torch.float32, torch.device(DEV)),  # kv heads
        KVCache(cfg.num_hidden_layers, 1, 2, cfg.head_dim // 2, 16, torch.float32, torch.device(DEV)),  # head_dim
        KVCache(cfg.num_hidden_layers, 1, 2, cfg.head_dim, 16, torch.bfloat16, torch.device(DEV)),  # dtype
    ]
    for kv in bad:
        with pytest.raises(ValueError, match="does not fit"):
            model(ids, kv_cache=kv)
    kv = make_kv_cache(model, 1, 16)
    st = GenerationState(model, ids, 4, kv=kv)
    tok = st.select_next(st.prefill())
    pos = st.append(tok)
    with pytest.raises(RuntimeError, match="no CPU path"):
        st.decode_step(tok.cpu(), pos)
    with pytest.raises(ValueError, match="int64"):
        st.decode_step(tok, pos.to(torch.int32))
    # a cache for another batch size is refused at the decode step too
    with pytest.raises(ValueError, match="does not fit"):
        model.decode_native(tok.repeat(2), pos, kv, torch.empty(2, 1, cfg.vocab_size, device=DEV), None)


@torch.inference_mode()
def test_explicit_positions_past_the_rope_table_raise():
    model = _tiny()
    limit = model.cfg.max_position_embeddings
    ids = torch.tensor([[5, 60, 7]], device=DEV)
    with pytest.raises(IndexError):
        model(ids, positions=torch.tensor([0, 1, limit], device=DEV))
    # negative positions wrap, as indexing the reference's table does
    a = model(ids, positions=torch.tensor([limit - 3, limit - 2, limit - 1], device=DEV))
    b = model(ids, positions=torch.tensor([-3, -2, -1], device=DEV))
    assert torch.equal(a, b)


@torch.inference_mode()
def test_decode_shape_first_run_without_a_pick_still_picks_later():
    """Batch > 4 records the token pick as its own graph node; a decode
    graph captured for a step with no next column (cursor == total) must not
    serve a later step of the same shape that needs the pick."""
    from minitp.generation import GenerationState, generate_greedy, make_kv_cache
    from minitp.synthetic import synthetic_prompt

    model = _tiny()
    b, t = 6, 8
    prompt = synthetic_prompt(model.cfg.vocab_size, b, t, seed=3, device=DEV)
    expect = generate_greedy(_tiny(), prompt, 2, early_stop=False)  # another program: its own graphs

    st = GenerationState(model, prompt, 1, kv=make_kv_cache(model, b, t + 2))
    tok = st.select_next(st.prefill())
    pos = st.append(tok)
    assert st.cursor == st.total
    st.decode_step(tok, pos)  # no next column: captured without the pick
    got = generate_greedy(model, prompt, 2, early_stop=False, kv=make_kv_cache(model, b, t + 2))
    torch.cuda.synchronize()
    assert torch.equal(got, expect)


@pytest.mark.parametrize("dtype,atol", [(torch.float32, 1e-5), (torch.bfloat16, 3e-2)])
@pytest.mark.parametrize("rows", [1, 4, 64, 300])
@torch.inference_mode()
def test_column_and_row_parallel_equal_f_linear(dtype, atol, rows):
    from minitp.parallel.linear import ColumnParallelLinear, RowParallelLinear

    g = torch.Generator(device="cpu").manual_seed(rows)
    W = torch.randn(64, 96, generator=g)
    bias = torch.randn(64, generator=g)
    X = torch.randn(rows, 96, generator=g)
    col = ColumnParallelLinear(96, 64, _ctx(), bias=True, gather_output=True).to(DEV, dtype)
    row = RowParallelLinear(96, 64, _ctx(), bias=True, input_is_parallel=False).to(DEV, dtype)
    for layer in (col, row):
        layer.weight.copy_(W)
        layer.bias.copy_(bias)
    x = X.to(DEV, dtype)
    Wd, bd = W.to(dtype).double(), bias.to(dtype).double()
    ref = F.linear(x.double().cpu(), Wd, bd)
    got_col = col(x).double().cpu()
    got_row = row(x).double().cpu()
    torch.testing.assert_close(got_col, ref, atol=atol, rtol=atol)
    torch.testing.assert_close(got_row, ref, atol=atol, rtol=atol)
    if dtype == torch.bfloat16:
        # RowParallel rounds the product before the bias add: each is exactly
        # bf16(bf16(x W^T) + b)
        prod = F.linear(x.float().cpu(), W.to(dtype).float()).to(dtype)
        ref_row = (prod.float() + bias.to(dtype).float()).to(dtype)
        assert (row(x).float().cpu() - ref_row.float()).abs().max().item() <= \
            2 * ref_row.float().abs().max().item() * 2 ** -8


@pytest.mark.parametrize("rows", [1, 3, 40])
@torch.inference_mode()
def test_fused_projections_equal_separate_ones(rows):
    from minitp.parallel.fused import FusedGateUpColumnParallelLinear, FusedQKVColumnParallelLinear

    hidden, q_local, kv_local, inter = 32, 16, 8, 24
    g = torch.Generator(device="cpu").manual_seed(7)
    qkv = FusedQKVColumnParallelLinear(hidden, q_local, kv_local, _ctx(), bias=True).to(DEV)
    W = torch.randn(q_local + 2 * kv_local, hidden, generator=g)
    b = torch.randn(q_local + 2 * kv_local, generator=g)
    qkv.weight.copy_(W)
    qkv.bias.copy_(b)
    x = torch.randn(2, rows, hidden, generator=g)
    q, k, v = qkv(x.to(DEV))
    y = F.linear(x.double(), W.double(), b.double())
    q_ref, k_ref, v_ref = torch.split(y, [q_local, kv_local, kv_local], dim=-1)
    for got, ref in ((q, q_ref), (k, k_ref), (v, v_ref)):
        torch.testing.assert_close(got.double().cpu(), ref, atol=1e-5, rtol=1e-5)
    uq, uk, uv = qkv.forward_unfused(x.to(DEV))
    for a, c in ((q, uq), (k, uk), (v, uv)):
        torch.testing.assert_close(a, c, atol=1e-5, rtol=1e-5)

    gu = FusedGateUpColumnParallelLinear(hidden, inter, _ctx(), bias=False).to(DEV)
    W2 = torch.randn(2 * inter, hidden, generator=g)
    gu.weight.copy_(W2)
    gate, up = gu(x.to(DEV))
    y2 = F.linear(x.double(), W2.double())
    torch.testing.assert_close(gate.double().cpu(), y2[..., :inter], atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(up.double().cpu(), y2[..., inter:], atol=1e-5, rtol=1e-5)
    ug, uu = gu.forward_unfused(x.to(DEV))
    torch.testing.assert_close(gate, ug, atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(up, uu, atol=1e-5, rtol=1e-5)


@torch.inference_mode()
@pytest.mark.parametrize("hidden", [896, 3584])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_functional_rmsnorm_matches_f_rms_norm(hidden, dtype):
    """implementation="functional" runs F.rms_norm in the reference
    (layer.py:36-38); here the native kernel serves it. Same rounding (fp32
    math, one rounding after the weight); the sum of squares may add in
    another order, so a bf16 result may sit one unit in the last place away."""
    from minitp.layer import RMSNorm

    g = torch.Generator(device=DEV).manual_seed(hidden)
    x = (torch.randn(33, hidden, device=DEV, generator=g) * 3).to(dtype)
    norm = RMSNorm(hidden, 1e-6).to(DEV, dtype)
    norm.weight.copy_((torch.rand(hidden, device=DEV, generator=g) + 0.5).to(dtype))
    norm.implementation = "functional"
    got = norm(x)
    want = F.rms_norm(x, (hidden,), norm.weight, 1e-6)
    if dtype == torch.float32:
        torch.testing.assert_close(got, want, atol=1e-6, rtol=1e-5)
    else:
        ulp = torch.finfo(torch.bfloat16).eps * want.float().abs().clamp_min(2 ** -126)
        assert ((got.float() - want.float()).abs() <= ulp).all()
        assert (got == want).float().mean().item() > 0.99


@torch.inference_mode()
def test_functional_norms_keep_the_native_program_and_its_ids():
    from minitp.generation import generate_greedy

    model = _tiny()
    ids = torch.tensor([[5, 60, 7, 99, 120, 33]], device=DEV)
    want = generate_greedy(model, ids, 6)
    for layer in model.model.layers:
        layer.input_layernorm.implementation = "functional"
        layer.post_attention_layernorm.implementation = "functional"
    model.model.norm.implementation = "functional"
    assert model.native_path()
    assert torch.equal(generate_greedy(model, ids, 6), want)


@pytest.mark.parametrize("early_stop,eos", [(True, None), (False, None), (True, 5)])
def test_zero_new_tokens_returns_the_prompt_after_its_prefill(early_stop, eos):
    """generate_greedy(..., max_new_tokens=0) (generation.py:150-171): the
    prompt's forward still runs (its K/V land in a caller's cache, which
    advances by the prompt), no token is picked, and the prompt comes back."""
    from minitp.generation import generate_greedy, make_kv_cache

    model = _tiny()
    prompt = torch.tensor([[3, 17, 256, 999, 41], [8, 1, 0, 77, 500]], device=DEV)
    kv = make_kv_cache(model, 2, 5)
    out = generate_greedy(model, prompt, 0, eos_token_id=eos, early_stop=early_stop, kv=kv)
    assert torch.equal(out, prompt) and kv.seq_len == 5
    assert torch.isfinite(kv.k[0][:, :, :5]).all() and torch.isfinite(kv.v[1][:, :, :5]).all()
