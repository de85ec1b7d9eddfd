"""The oracle (CPU restatement of the reference) pinned before it is trusted.

1. Against golden vectors written from the reference itself: bit-exact ids
   and logits (tiny configs, and the first steps of the 0.5B fixtures).
2. Against closed forms and invariants that fix each function, each chosen
   so that a plausible mistake (dropped term, sign, index, transpose) fails;
   a planted-mistake test shows that they do.
3. The generator spec: numpy statement == C statement, and its moments.
"""

import math
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import qwen2_ref as R
from oracle import synth
from tests.conftest import GOLDEN


def _fx(name):
    return np.load(os.path.join(GOLDEN, f"{name}.npz"))


def _run_oracle(shape, dtype, prompt, n):
    sd = {k: v.to(dtype) for k, v in R.synthetic_state(shape, seed=0, dtype=torch.float32).items()}
    if shape.tie_word_embeddings:
        sd["lm_head.weight"] = sd["model.embed_tokens.weight"]
    m = R.OracleQwen2(shape, sd)
    rows = []
    ids = R.generate_greedy(m, prompt, n, early_stop=False, on_logits=lambda s, lg: rows.append(lg[:, -1].clone()))
    return ids, torch.stack(rows)


@pytest.mark.parametrize("name,dtype", [("tiny_fp32", torch.float32), ("tiny_bf16", torch.bfloat16),
                                        ("tiny_b3_fp32", torch.float32)])
def test_oracle_reproduces_reference_vectors_bitwise(name, dtype):
    fx = _fx(name)
    prompt = torch.from_numpy(fx["prompt"])
    assert torch.equal(prompt, R.synthetic_prompt(R.TINY.vocab_size, *prompt.shape, seed=0))
    ids, rows = _run_oracle(R.TINY, dtype, prompt, fx["ids"].shape[1] - prompt.shape[1])
    assert np.array_equal(ids.numpy(), fx["ids"])
    assert torch.equal(rows.float(), torch.from_numpy(fx["step_logits"]))


@pytest.mark.parametrize("name,dtype", [("q05b_fp32", torch.float32), ("q05b_bf16", torch.bfloat16)])
def test_oracle_q05b_first_steps_bitwise(name, dtype):
    """Prefill + 3 decode steps of the 0.5B oracle against the reference's values."""
    fx = _fx(name)
    prompt = torch.from_numpy(fx["prompt"])
    assert torch.equal(prompt, R.synthetic_prompt(R.QWEN05B.vocab_size, 1, 128, seed=0))
    torch.set_num_threads(max(1, os.cpu_count() or 1))
    ids, rows = _run_oracle(R.QWEN05B, dtype, prompt, 4)
    assert np.array_equal(ids.numpy()[0], fx["ids"][0, :132])
    got = torch.gather(rows.float(), -1, torch.from_numpy(fx["step_topk_ids"][:4]))
    assert torch.equal(got, torch.from_numpy(fx["step_topk_vals"][:4]))


# ---------------------------------------------------------------------------
# closed forms / invariants


def test_rmsnorm_constant_row_and_scale_invariance():
    c, eps = 0.75, 1e-6
    x = torch.full((2, 896), c)
    w = torch.linspace(0.5, 1.5, 896)
    got = R.rms_norm(x, w, eps)
    torch.testing.assert_close(got, (c / math.sqrt(c * c + eps)) * w.expand(2, -1), atol=1e-6, rtol=1e-6)
    y = torch.randn(3, 64)
    torch.testing.assert_close(R.rms_norm(8.0 * y, torch.ones(64), 0.0), R.rms_norm(y, torch.ones(64), 0.0))


def test_rope_invariants():
    d = 64
    cos, sin = R.rope_tables(d, 1e6, 512)
    q = torch.randn(1, 2, 5, d, dtype=torch.float64).float()
    # position 0 is the identity
    q0, _ = R.rope_apply(cos, sin, q[:, :, :1], q[:, :, :1], torch.tensor([0]))
    assert torch.equal(q0, q[:, :, :1])
    # each (i, i + D/2) pair keeps its norm
    qr, _ = R.rope_apply(cos, sin, q, q, torch.arange(100, 105))
    pn = lambda t: t[..., : d // 2] ** 2 + t[..., d // 2:] ** 2  # noqa: E731
    torch.testing.assert_close(pn(qr), pn(q), atol=1e-5, rtol=1e-5)
    # <rot(q, m), rot(k, n)> depends only on m - n
    k = torch.randn(1, 1, 1, d)
    qq = torch.randn(1, 1, 1, d)
    dots = []
    for m, n in ((7, 3), (104, 100), (400, 396)):
        a, _ = R.rope_apply(cos, sin, qq, qq, torch.tensor([m]))
        b, _ = R.rope_apply(cos, sin, k, k, torch.tensor([n]))
        dots.append(float((a * b).sum()))
    assert max(dots) - min(dots) < 1e-4
    # table row p is [cos(p f), cos(p f)] with f_i = theta^(-2i/D) (closed form)
    p = 123
    f = 1e6 ** (-torch.arange(0, d, 2, dtype=torch.float64) / d)
    torch.testing.assert_close(cos[p].double(), torch.cos(p * f).repeat(2), atol=2e-4, rtol=0)
    # cached == uncached (test_rope_cache.py:17-29)
    rq, rk = R.rope_apply(cos, sin, q, q, torch.arange(95, 100))
    uq, uk = R.rope_apply_uncached(q, q, torch.arange(95, 100), 1e6)
    torch.testing.assert_close(rq, uq, atol=1e-6, rtol=1e-5)


def _attention_probe(q_bias=None, w_v_identity=False, seed=3):
    """Oracle attention of layer 0 with o_proj = I (hq * hd == hidden), so its
    output is the raw SDPA output [B, T, Hq * D]. The QKV projection is chosen
    per check: q from q_bias only (weight rows 0), k from random weights, v
    either the identity on the input's first Hkv * D dims or random."""
    hq, hkv, hd, hid = 4, 2, 8, 32
    shape = R.Qwen2Shape(hid, 64, 1, hq, hkv, hd, 50, 1e-6, 1e4, 64, True)
    sd = R.synthetic_state(shape, seed=1)
    g = torch.Generator().manual_seed(seed)
    w = torch.zeros((hq + 2 * hkv) * hd, hid)
    b = torch.zeros((hq + 2 * hkv) * hd)
    if q_bias is not None:
        b[: hq * hd] = q_bias
    w[hq * hd:(hq + hkv) * hd] = torch.randn(hkv * hd, hid, generator=g)  # k
    if w_v_identity:
        w[(hq + hkv) * hd:, : hkv * hd] = torch.eye(hkv * hd)  # v = x[:, :Hkv * D]
    else:
        w[(hq + hkv) * hd:] = torch.randn(hkv * hd, hid, generator=g)
    sd["model.layers.0.self_attn.qkv_proj.weight"] = w
    sd["model.layers.0.self_attn.qkv_proj.bias"] = b
    sd["model.layers.0.self_attn.o_proj.weight"] = torch.eye(hid)
    m = R.OracleQwen2(shape, sd)
    m.cos_cache, m.sin_cache = R.rope_tables(hd, 1e4, 64)
    return m, (hq, hkv, hd, hid)


def _check_attention_closed_forms(m, dims):
    """Closed forms of SDPA over a GQA cache (attention.py:77-103), checked
    on the oracle's attention output (o_proj = I):
    * one key: query head h returns V[0] of KV head h // (Hq / Hkv);
    * q = 0: uniform weights, so causal position t returns the mean of
      V[0..t] of its KV head."""
    hq, hkv, hd, hid = dims
    grp = hq // hkv
    g = torch.Generator().manual_seed(7)
    # (1) a single key: a one-token prompt on an empty cache
    x = torch.randn(1, 1, hid, generator=g)
    kv = m.make_kv_cache(1, 8)
    out = m.attention(0, x, torch.tensor([0]), kv, True)[0, 0].view(hq, hd)
    v0 = kv.v[0][0, :, 0]  # [Hkv, D], as the cache holds it
    for h in range(hq):
        torch.testing.assert_close(out[h], v0[h // grp], atol=1e-6, rtol=0)
    # (2) q = 0 over a 5-token causal prompt: prefix means of V
    x = torch.randn(1, 5, hid, generator=g)
    kv = m.make_kv_cache(1, 8)
    out = m.attention(0, x, torch.arange(5), kv, True)[0].view(5, hq, hd)
    vals = kv.v[0][0, :, :5]  # [Hkv, 5, D]
    for t in range(5):
        mean = vals[:, : t + 1].mean(dim=1)
        for h in range(hq):
            torch.testing.assert_close(out[t, h], mean[h // grp], atol=1e-5, rtol=0)


def test_attention_closed_forms_single_key_zero_query_and_gqa_mapping():
    m, dims = _attention_probe(q_bias=None, w_v_identity=True)
    hq, hkv, hd, hid = dims
    # the KV heads' values differ, so the head -> KV head map is observable
    _check_attention_closed_forms(m, dims)
    # a non-zero query with a single key still returns V[0] (softmax of one score)
    m2, _ = _attention_probe(q_bias=torch.randn(hq * hd, generator=torch.Generator().manual_seed(2)))
    x = torch.randn(1, 1, hid)
    kv = m2.make_kv_cache(1, 4)
    out = m2.attention(0, x, torch.tensor([0]), kv, True)[0, 0].view(hq, hd)
    for h in range(hq):
        torch.testing.assert_close(out[h], kv.v[0][0, h // (hq // hkv), 0], atol=1e-6, rtol=0)


def test_attention_closed_forms_catch_a_planted_gqa_mistake(monkeypatch):
    """Planted mistake: KV heads tiled (h % Hkv) instead of interleaved
    (h // G). The closed-form check must reject that oracle."""
    m, dims = _attention_probe(q_bias=None, w_v_identity=True)
    monkeypatch.setattr(torch.Tensor, "repeat_interleave", lambda self, n, dim: self.repeat(1, n, 1, 1))
    with pytest.raises(AssertionError):
        _check_attention_closed_forms(m, dims)


def test_attention_closed_forms_catch_a_planted_mask_mistake(monkeypatch):
    """Planted mistake: a causal mask shifted by one (the query sees one key
    fewer). The prefix-mean check must reject it."""
    m, dims = _attention_probe(q_bias=None, w_v_identity=True)
    real = F.scaled_dot_product_attention

    def shifted(q, k, v, attn_mask=None, is_causal=False, **kw):
        if is_causal:
            t, s = q.shape[-2], k.shape[-2]
            mask = torch.ones(t, s, dtype=torch.bool).tril(diagonal=-1)
            mask[0, 0] = True  # keep row 0 defined
            return real(q, k, v, attn_mask=mask)
        return real(q, k, v, attn_mask=attn_mask, is_causal=is_causal)

    monkeypatch.setattr(R.F, "scaled_dot_product_attention", shifted)
    with pytest.raises(AssertionError):
        _check_attention_closed_forms(m, dims)


def test_tril_offset_mask_is_causal_with_cache():
    t, cache_len = 3, 4
    mask = torch.ones(t, cache_len + t, dtype=torch.bool).tril(diagonal=cache_len)
    for i in range(t):
        assert mask[i].nonzero().max().item() == cache_len + i


def test_swiglu_closed_form():
    g = torch.tensor([-2.0, 0.0, 1.0, 3.0])
    u = torch.tensor([1.0, 5.0, 2.0, -1.0])
    want = g / (1 + torch.exp(-g)) * u
    torch.testing.assert_close(F.silu(g) * u, want)


def test_argmax_known_answers():
    x = torch.zeros(1, 8)
    x[0, 5] = x[0, 2] = 2.0
    assert R.select_token(x[:, None]).item() == 2
    x = torch.zeros(1, 200000)
    x[0, 150000] = x[0, 4242] = 1.0
    assert R.select_token(x[:, None]).item() == 4242
    x = torch.randn(1, 10)
    x[0, 6] = float("nan")
    assert R.select_token(x[:, None]).item() == 6


def test_kv_decode_equals_full_forward_oracle():
    """generation.py semantics: each greedy token is the argmax of a full
    no-cache forward at the previous position (test_qwen_tiny.py:122-138)."""
    m = R.OracleQwen2(R.TINY, R.synthetic_state(R.TINY, seed=0))
    ids = torch.tensor([[5, 60, 7, 99, 120, 33]])
    out = R.generate_greedy(m, ids, 5, early_stop=False)
    full = m(out)
    assert torch.equal(full[:, 5:-1].argmax(-1), out[:, 6:])


def test_planted_mistake_is_caught():
    """A plausible slip in the oracle (rotate_half without the minus sign)
    changes the greedy ids against the reference vectors."""
    fx = _fx("tiny_fp32")
    orig = R._rotate_half
    try:
        def wrong(x):
            x1, x2 = x.float().chunk(2, dim=-1)
            return torch.cat([x2, x1], dim=-1)

        R._rotate_half = wrong
        prompt = torch.from_numpy(fx["prompt"])
        _, rows = _run_oracle(R.TINY, torch.float32, prompt, fx["ids"].shape[1] - prompt.shape[1])
        assert not torch.equal(rows.float(), torch.from_numpy(fx["step_logits"]))
    finally:
        R._rotate_half = orig


# ---------------------------------------------------------------------------
# generator spec


def test_generator_numpy_and_c_statements_agree():
    for stream in (1, 2, 17, 999):
        a = synth.normal_f32(0, stream, 50_000)
        b = synth.normal_f32_c(0, stream, 50_000)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert np.array_equal(synth.uniform_ids(0, 3, 5000, 151936), synth.uniform_ids_c(0, 3, 5000, 151936))


def test_generator_is_normal():
    z = synth.normal_f32_c(0, 42, 2_000_000, std=1.0).astype(np.float64)
    assert abs(z.mean()) < 3e-3 and abs(z.std() - 1) < 3e-3
    kurt = ((z - z.mean()) ** 4).mean() / z.var() ** 2
    assert abs(kurt - 3) < 0.03
    from scipy import stats

    assert stats.kstest(z[:200_000], "norm").pvalue > 1e-3


def test_det_log_matches_libm():
    s = np.random.default_rng(0).random(100_000)
    s = s[s > 0]
    np.testing.assert_allclose(synth.det_log(s), np.log(s), rtol=1e-15, atol=0)


def test_uniform_ids_cover_vocab():
    ids = synth.uniform_ids_c(0, 3, 1_000_000, 1000)
    assert ids.min() == 0 and ids.max() == 999
    counts = np.bincount(ids, minlength=1000)
    assert counts.min() > 800 and counts.max() < 1200


def _tiny_oracle(std=0.02):
    sd = R.synthetic_state(R.TINY, seed=0, dtype=torch.float32, std=std)
    return R.OracleQwen2(R.TINY, sd)


def test_oracle_reproduces_reference_chunked_prefill_and_resume():
    """Chunks through forward(kv_cache=) (the tril(diagonal=cache_len) mask,
    attention.py:96-103) and a state resumed on the filled cache
    (generation.py:93,103): the reference's own values, bit for bit."""
    fx = _fx("tiny_chunked_fp32")
    m = _tiny_oracle()
    prompt = torch.from_numpy(fx["prompt"])
    kv = m.make_kv_cache(prompt.shape[0], prompt.shape[1] + int(fx["resume_ids"].shape[1]))
    start, outs = 0, []
    with torch.inference_mode():
        for c in fx["chunks"].tolist():
            outs.append(m(prompt[:, start:start + c], positions=torch.arange(start, start + c), kv_cache=kv))
            start += c
        assert torch.equal(torch.cat(outs, dim=1), torch.from_numpy(fx["chunk_logits"]))
        resume = torch.from_numpy(fx["resume_prompt"])
        new = fx["resume_ids"].shape[1] - resume.shape[1]
        rows = []
        ids = R.generate_greedy(m, resume, new, early_stop=False, kv=kv,
                                on_logits=lambda s, lg: rows.append(lg[:, -1].clone()))
    assert np.array_equal(ids.numpy(), fx["resume_ids"])
    assert torch.equal(torch.stack(rows), torch.from_numpy(fx["resume_step_logits"]))
    assert kv.seq_len == int(fx["seq_len"])


def test_oracle_reproduces_reference_early_stop():
    """generate_greedy's early stop (generation.py:150-168): trimmed ids,
    EOS padding of finished rows and the cache cursor, as the reference wrote
    them, over rows stopping at different steps, partial finishes, a first
    pick and an EOS never produced."""
    fx = _fx("tiny_eos_fp32")
    m = _tiny_oracle(float(fx["weight_std"]))
    stopped_early = 0
    for i, eos in enumerate(fx["eos"].tolist()):
        b, n = int(fx["batch"][i]), int(fx["length"][i])
        prompt = torch.from_numpy(fx["prompts"][i, :b])
        kv = m.make_kv_cache(b, prompt.shape[1] + 12)
        ids = R.generate_greedy(m, prompt, 12, eos_token_id=eos, early_stop=True, kv=kv)
        assert np.array_equal(ids.numpy(), fx["ids"][i, :b, :n]), (i, eos)
        assert kv.seq_len == int(fx["seq_len"][i])
        stopped_early += n < prompt.shape[1] + 12
    assert stopped_early >= 1  # the fixture holds a case where every row stops before the end
