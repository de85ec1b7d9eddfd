"""The 7B prefill workload at its full size (4 x 4096 tokens, bf16), checked
through properties that do not need the oracle to run at that size.

The model is the Qwen2.5-7B layer shape with 2 layers and the untied
152,064-row head (the oracle covers the same shapes at small sizes); the
batch-32 tests do the same for the batch-32 decode workload's shapes. At 4 x
4096 the prompt runs the long-prompt attention kernel, the 256 x 256 MFMA tile
GEMMs at M = 16,384 and the 16-byte elementwise kernels, so these properties
exercise exactly the full-size path:

* the whole-prompt prefill's last-position logits equal those of a prefill of
  the first 4,095 tokens followed by one decode step of the last token (the
  decode attention and GEMV path over the 4,095 cached rows);
* layer 0's K and V cache rows against float64 (embedding, the oracle's
  RMSNorm and RoPE, the QKV product in float64), on rows computed by split
  and by unsplit GEMM tiles;
* a prefill in two chunks of 2,048 (the second attending over the first
  through the cache offset, positions 2,048 .. 4,095 given explicitly) gives
  the same last-position logits and the same cache rows as the whole prompt;
* over a whole generation's contexts: every position of a 768-token 7B prompt
  (the 512 + 256 decode workload, contexts 513 .. 768) and checkpoints up to
  context 2,559 of the batch-32 workload (2,048 + 512) give the same logits
  from one whole-prompt prefill as from a prefill of the first part followed
  by one teacher-forced decode step per remaining token, on every decode
  form that serves the batch.

Bars: the bf16 logit bar of the model tests (0.5 abs); for layer 0's cache
rows a few bf16 steps (3e-2 + |value| / 32: the two prompts run the QKV GEMM
at different M, whose algorithms round differently in the last bit), for
layer 1's 0.125 abs (its inputs carry layer 0's rounding differences; values
reach about 6). Every logit and cache row must be finite.
"""

import dataclasses

import pytest
import torch

from tests.test_gpu_model import BF16_LOGIT_ATOL

pytestmark = pytest.mark.gpu
DEV = "cuda"
B, T = 4, 4096


@pytest.fixture(scope="module")
def model_prompt():
    from minitp import synthetic

    cfg = dataclasses.replace(synthetic.QWEN7B, num_hidden_layers=2)
    model = synthetic.build_synthetic_model(cfg, dtype=torch.bfloat16, device=DEV, seed=0)
    prompt = synthetic.synthetic_prompt(cfg.vocab_size, B, T, seed=3, device=DEV)
    yield model, prompt
    del model
    torch.cuda.empty_cache()


def _whole(model, prompt):
    from minitp.generation import GenerationState

    st = GenerationState(model, prompt, 1, prefill_logits="last")
    logits = st.prefill()[:, 0].float()
    return logits, st.kv


def test_full_prompt_last_row_equals_prefill_then_decode(model_prompt):
    from minitp.generation import GenerationState

    model, prompt = model_prompt
    whole, _ = _whole(model, prompt)
    st = GenerationState(model, prompt[:, :-1], 2, prefill_logits="last")
    st.prefill()
    tok = prompt[:, -1].contiguous()
    pos = st.append(tok)
    step = st.decode_step(tok, pos)[:, 0].float()
    assert torch.isfinite(whole).all() and torch.isfinite(step).all()
    err = (whole - step).abs().max().item()
    print(f"4 x 4096: whole-prompt vs prefill(4095) + decode: max |logit diff| {err:.4f}")
    assert err <= BF16_LOGIT_ATOL


@pytest.mark.parametrize("b,p0", [(3, 3968), (0, 0)])
def test_layer0_cache_rows_match_float64(model_prompt, b, p0):
    """Layer 0's K and V cache rows of 128 positions after the whole-prompt
    prefill, against embedding -> RMSNorm (the oracle's, bf16) -> the QKV
    product in float64 + bias, rounded to bf16 -> RoPE (the oracle's cached
    tables) for K. At M = 16,384 the QKV GEMM has 1,152 tiles: 4 full rounds
    of 256 and 128 tiles split over K in two parts. Batch row 3's last
    positions sit in split tiles, row 0's first in unsplit ones. Bar: a few
    bf16 steps (the GEMM's fp32 sums round to bf16 differently from float64's
    in the last bit, and RoPE multiplies that)."""
    from oracle.qwen2_ref import rms_norm, rope_apply, rope_tables

    model, prompt = model_prompt
    _, kv = _whole(model, prompt)
    sd = model.state_dict()
    hq, hkv, hd = 28, 4, 128
    emb = sd["model.embed_tokens.weight"]
    x = emb[prompt[b, p0:p0 + 128]]
    xn = rms_norm(x, sd["model.layers.0.input_layernorm.weight"], 1e-6)
    y = torch.nn.functional.linear(xn.double(), sd["model.layers.0.self_attn.qkv_proj.weight"].double(),
                                   sd["model.layers.0.self_attn.qkv_proj.bias"].double()).to(torch.bfloat16)
    k = y[:, hq * hd:(hq + hkv) * hd].view(128, hkv, hd).transpose(0, 1)[None]
    v = y[:, (hq + hkv) * hd:].view(128, hkv, hd).transpose(0, 1)[None]
    cos, sin = rope_tables(hd, 1e6, 4096)
    _, k = rope_apply(cos.to(DEV), sin.to(DEV), k, k, torch.arange(p0, p0 + 128, device=DEV))
    for name, got, ref in (("k", kv.k[0], k), ("v", kv.v[0], v)):
        g = got[b:b + 1, :, p0:p0 + 128].float()
        r = ref.float()
        d = (g - r).abs()
        print(f"row {b}, positions {p0}..{p0 + 127}, {name}: max |ref| {r.abs().max().item():.3f}, "
              f"max |diff| {d.max().item():.4f}")
        assert torch.isfinite(g).all() and (d <= 3e-2 + r.abs() / 32).all()


def test_two_chunk_prefill_equals_whole_prompt(model_prompt):
    """Chunks through the model's forward with explicit positions (a T > 1
    forward without them starts at position 0, as the reference's does)."""
    from minitp.generation import make_kv_cache

    model, prompt = model_prompt
    whole, kv_whole = _whole(model, prompt)
    kv = make_kv_cache(model, B, T + 1)
    h = T // 2
    with torch.inference_mode():
        model(prompt[:, :h], positions=torch.arange(0, h, device=DEV), kv_cache=kv)
        chunked = model(prompt[:, h:], positions=torch.arange(h, T, device=DEV), kv_cache=kv)[:, -1].float()
    assert kv.seq_len == T
    err = (whole - chunked).abs().max().item()
    print(f"4 x 4096: whole vs 2 x 2048 chunks: max |logit diff| {err:.4f}")
    assert torch.isfinite(chunked).all() and err <= BF16_LOGIT_ATOL
    for i, (a, b) in enumerate(zip(kv_whole.k + kv_whole.v, kv.k + kv.v)):
        ra, rb = a[:, :, :T].float(), b[:, :, :T].float()
        assert torch.isfinite(rb).all()
        d = (ra - rb).abs()
        print(f"cache buffer {i}: max |row| {ra.abs().max().item():.3f}, max |diff| {d.max().item():.4f}, "
              f"rows differing {(d > 0).float().mean().item():.5f}")
        if i % len(kv.k) == 0:  # layer 0: its inputs are the same; GEMM rounding only
            assert (d <= 3e-2 + ra.abs() / 32).all()
        else:  # later layers also carry the earlier layers' rounding differences
            assert d.max().item() <= 0.125


def test_batch32_long_prompt_last_row_equals_prefill_then_decode():
    """The batch-32 decode workload's shapes (0.5B layers, 2 of them, 32 x 2048
    bf16): the long-prompt attention at head dim 64 against the batched decode
    path (GEMM path, decode attention split over the 2,047 cached rows)."""
    from minitp import synthetic
    from minitp.generation import GenerationState

    cfg = dataclasses.replace(synthetic.QWEN05B, num_hidden_layers=2)
    model = synthetic.build_synthetic_model(cfg, dtype=torch.bfloat16, device=DEV, seed=1)
    prompt = synthetic.synthetic_prompt(cfg.vocab_size, 32, 2048, seed=5, device=DEV)
    whole = GenerationState(model, prompt, 1, prefill_logits="last").prefill()[:, 0].float()
    st = GenerationState(model, prompt[:, :-1], 2, prefill_logits="last")
    st.prefill()
    tok = prompt[:, -1].contiguous()
    step = st.decode_step(tok, st.append(tok))[:, 0].float()
    err = (whole - step).abs().max().item()
    print(f"32 x 2048: whole-prompt vs prefill(2047) + decode: max |logit diff| {err:.4f}")
    assert torch.isfinite(whole).all() and torch.isfinite(step).all() and err <= BF16_LOGIT_ATOL



def _teacher_forced(model, prompt, start, check):
    """Prefill prompt[:, :start], then decode prompt[:, start:] one token per
    step; ``check(pos, logits)`` gets each step's [B, V] logits, the prefill's
    last row included (pos = start - 1)."""
    from minitp.generation import GenerationState

    t = prompt.shape[1]
    st = GenerationState(model, prompt[:, :start], t - start, prefill_logits="last")
    check(start - 1, st.prefill()[:, -1])
    for i in range(start, t):
        tok = prompt[:, i].contiguous()
        pos = st.append(tok)
        check(i, st.decode_step(tok, pos)[:, 0])
    assert st.kv.seq_len == t


def test_7b_every_decode_context_equals_whole_prompt():
    """7B shapes (2 layers, batch 1): the whole 768-token prompt's logits at
    each position 511 .. 767 against prefill(512) plus 256 teacher-forced
    decode steps (contexts 513 .. 768: the generation's 255 steps plus one)."""
    from minitp import synthetic
    from minitp.generation import GenerationState

    cfg = dataclasses.replace(synthetic.QWEN7B, num_hidden_layers=2)
    model = synthetic.build_synthetic_model(cfg, dtype=torch.bfloat16, device=DEV, seed=2)
    prog = model.program()
    prompt = synthetic.synthetic_prompt(cfg.vocab_size, 1, 768, seed=7, device=DEV)
    whole = GenerationState(model, prompt, 1, prefill_logits="all").prefill()[0].float()
    assert whole.shape == (768, cfg.vocab_size) and torch.isfinite(whole).all()
    errs = {}

    def check(pos, logits):
        assert torch.isfinite(logits).all(), pos
        errs[pos] = (whole[pos] - logits[0].float()).abs().max().item()

    with torch.inference_mode():
        _teacher_forced(model, prompt, 512, check)
    prog.check_decode()
    worst = max(errs, key=errs.get)
    print(f"7B: {len(errs)} positions, max |logit diff| {errs[worst]:.4f} at position {worst}")
    assert len(errs) == 257 and errs[worst] <= BF16_LOGIT_ATOL


def test_batch32_decode_to_context_2559_equals_whole_prompts():
    """0.5B shapes (2 layers), batch 32: prefill(2048) plus 511 teacher-forced
    decode steps (contexts 2,049 .. 2,559) against whole-prompt prefills that
    end at the checkpoints 2,048, 2,049, 2,304 and 2,559 (last rows)."""
    from minitp import synthetic
    from minitp.generation import GenerationState

    cfg = dataclasses.replace(synthetic.QWEN05B, num_hidden_layers=2)
    model = synthetic.build_synthetic_model(cfg, dtype=torch.bfloat16, device=DEV, seed=4)
    prompt = synthetic.synthetic_prompt(cfg.vocab_size, 32, 2559, seed=9, device=DEV)
    checkpoints = (2048, 2049, 2304, 2559)
    whole = {}
    for n in checkpoints:
        whole[n - 1] = GenerationState(model, prompt[:, :n], 1, prefill_logits="last").prefill()[:, -1].float()
        assert torch.isfinite(whole[n - 1]).all(), n
    seen = []

    def check(pos, logits):
        if pos in whole:
            err = (whole[pos] - logits.float()).abs().max().item()
            print(f"batch 32, context {pos + 1}: max |logit diff| {err:.4f}")
            assert torch.isfinite(logits).all() and err <= BF16_LOGIT_ATOL, pos
            seen.append(pos)

    with torch.inference_mode():
        _teacher_forced(model, prompt, 2048, check)
    assert seen == [n - 1 for n in checkpoints]


def test_long_context_decode_equals_whole_prompts():
    """0.5B shapes (2 layers), batch 1, near the RoPE table's end: prefill(16,000)
    plus 384 teacher-forced decode steps (contexts 16,001 .. 16,384: the o_proj
    fold's attention walking 250+ chunks a block) against whole-prompt
    prefills that end at the checkpoints 16,000, 16,001, 16,192 and 16,384
    (the tile GEMM and the long-prompt attention; last rows)."""
    from minitp import synthetic
    from minitp.generation import GenerationState

    cfg = dataclasses.replace(synthetic.QWEN05B, num_hidden_layers=2)
    model = synthetic.build_synthetic_model(cfg, dtype=torch.bfloat16, device=DEV, seed=6)
    prompt = synthetic.synthetic_prompt(cfg.vocab_size, 1, 16384, seed=11, device=DEV)
    checkpoints = (16000, 16001, 16192, 16384)
    whole = {}
    for n in checkpoints:
        whole[n - 1] = GenerationState(model, prompt[:, :n], 1, prefill_logits="last").prefill()[:, -1].float()
        assert torch.isfinite(whole[n - 1]).all(), n
    seen = []

    def check(pos, logits):
        if pos in whole:
            err = (whole[pos] - logits.float()).abs().max().item()
            print(f"batch 1, context {pos + 1}: max |logit diff| {err:.4f}")
            assert torch.isfinite(logits).all() and err <= BF16_LOGIT_ATOL, pos
            seen.append(pos)

    with torch.inference_mode():
        _teacher_forced(model, prompt, 16000, check)
    model.program().check_decode()
    assert seen == [n - 1 for n in checkpoints]
