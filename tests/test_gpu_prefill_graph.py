"""bf16 prompt forwards (last-position logits; every position's logits where
the LM head is the small-M GEMM) run through a graph per
shape (batch, tokens, max_seq, workspace, early stop, token pick, logits
form): the first call of a shape runs directly, the second runs directly and
is recorded, later calls patch the first kernel's per-call values and replay. Every later kernel reads the prompt ids,
positions, cache_len, the caches and the logits buffer from the step state, so
a replay with other prompts, other caches or a non-empty cache must give the
bits of a direct run (MINITP_PREFILL_GRAPH=0 when the program is created).
Shapes: the 0.5B layer shape with 2 layers at batch 1 and 3 (LM-head GEMV +
argmax) and 8 (the MFMA norm + LM-head GEMV of 5-32 rows, then argmax); the
fused GEMV path of a short prompt (batch 1, 8 tokens); the LM-head GEMM of 40
rows; and prompts whose products run on the 256 x 256 tile GEMM with its split
last round (0.5B, 3 x 256 tokens) and its every-tile split (the 7B layer
shape at 512 tokens), whose partials and arrival words live in the step
state."""

import dataclasses

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _models(monkeypatch, shape="qwen2.5-0.5b"):
    from minitp import synthetic

    cfg = dataclasses.replace(synthetic.SHAPES[shape], num_hidden_layers=2)
    graphed = synthetic.build_synthetic_model(cfg, dtype=torch.bfloat16, device=DEV, seed=0)
    direct = synthetic.build_synthetic_model(cfg, dtype=torch.bfloat16, device=DEV, seed=0)
    monkeypatch.setenv("MINITP_PREFILL_GRAPH", "0")
    direct_prog = direct.program()
    monkeypatch.delenv("MINITP_PREFILL_GRAPH")
    graphed_prog = graphed.program()
    return cfg, (graphed, graphed_prog), (direct, direct_prog)


def _run(model, prompts):
    """Last-position prefill logits and three greedy picks for each prompt in
    turn (the second of a shape records the graph, the third replays it)."""
    from minitp.generation import GenerationState

    out = []
    for p in prompts:
        st = GenerationState(model, p, 4, prefill_logits="last")
        logits = st.prefill()
        out.append(logits.float().clone())
        tok = st.select_next(logits)
        for _ in range(3):
            out.append(tok.clone())
            pos = st.append(tok)
            tok = st.select_next(st.decode_step(tok, pos))
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("batch", [1, 3, 8])
def test_prefill_graph_replays_match_direct_runs_bitwise(batch, monkeypatch):
    cfg, (graphed, gprog), (direct, dprog) = _models(monkeypatch)
    g = torch.Generator().manual_seed(11 + batch)
    prompts = [torch.randint(0, cfg.vocab_size, (batch, 40), generator=g).to(DEV) for _ in range(3)]
    resume = [torch.randint(0, cfg.vocab_size, (batch, 40), generator=g).to(DEV)]
    got = _run(graphed, prompts)
    ref = _run(direct, prompts)
    assert graphed.program() is gprog and direct.program() is dprog  # created once, as set above
    assert len(got) == len(ref)
    for i, (a, b) in enumerate(zip(got, ref)):
        assert torch.isfinite(a.float()).all(), i
        assert torch.equal(a, b), (i, (a.float() - b.float()).abs().max().item())
    # the prompts differ, so the replays were not returning the recorded call's values
    assert not torch.equal(got[0], got[4])
    # prefills of the same length on an empty cache, then on a filled one
    # (cache_len 40: recorded), then at cache_len 80 (a replay)
    from minitp.generation import GenerationState

    outs = []
    for model in (graphed, direct):
        first = GenerationState(model, prompts[0], 100, prefill_logits="last")
        first.prefill()
        second = GenerationState(model, prompts[1], 1, prefill_logits="last", kv=first.kv)
        a = second.prefill().float().clone()
        third = GenerationState(model, resume[0], 1, prefill_logits="last", kv=second.kv)
        outs.append((a, third.prefill().float().clone()))
    torch.cuda.synchronize()
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
    assert torch.isfinite(outs[0][1]).all()


@pytest.mark.parametrize("shape,batch,tokens", [("qwen2.5-0.5b", 1, 8), ("qwen2.5-0.5b", 40, 8),
                                                ("qwen2.5-0.5b", 3, 256), ("qwen2.5-7b", 1, 512)])
def test_prefill_graph_replays_other_launch_paths_bitwise(shape, batch, tokens, monkeypatch):
    """Three prompts of one shape (direct, recorded, replayed) against direct
    runs, bitwise: the fused short-prompt GEMVs (1 x 8), the LM-head GEMM
    that reads its logits pointer from the step state (40 rows), and the tile
    GEMM's split last round and every-tile split (3 x 256 at 0.5B; 512 tokens
    at 7B), which keep their arrival words and partials in the step state."""
    cfg, (graphed, _), (direct, _) = _models(monkeypatch, shape)
    g = torch.Generator().manual_seed(batch * 1000 + tokens)
    prompts = [torch.randint(0, cfg.vocab_size, (batch, tokens), generator=g).to(DEV) for _ in range(3)]
    got = _run(graphed, prompts)
    ref = _run(direct, prompts)
    for i, (a, b) in enumerate(zip(got, ref)):
        assert torch.isfinite(a.float()).all(), i
        assert torch.equal(a, b), (i, (a.float() - b.float()).abs().max().item())
    assert not torch.equal(got[0], got[4])


def test_prefill_graph_all_position_logits_bitwise(monkeypatch):
    """The reference's default prefill (every position's logits) replays a
    graph too when its LM head is the small-M GEMM, which stores through the
    step state's logits pointer: two prompts of 40 tokens, bitwise against a
    direct run, each into its own logits buffer."""
    from minitp.generation import GenerationState

    cfg, (graphed, _), (direct, _) = _models(monkeypatch)
    g = torch.Generator().manual_seed(3)
    prompts = [torch.randint(0, cfg.vocab_size, (1, 40), generator=g).to(DEV) for _ in range(3)]
    outs = []
    for model in (graphed, direct):
        outs.append([GenerationState(model, p, 2).prefill().float().clone() for p in prompts])
    torch.cuda.synchronize()
    for a, b in zip(*outs):
        assert a.shape == (1, 40, cfg.vocab_size) and torch.isfinite(a).all()
        assert torch.equal(a, b), (a - b).abs().max().item()
    assert not torch.equal(outs[0][0], outs[0][1])


def test_prefill_graphs_of_one_shape_keep_the_logits_form_apart(monkeypatch):
    """Every-position and last-position prefills of one shape run different
    LM heads into buffers of different sizes: each replays its own graph
    (alternating forms, bitwise against direct runs)."""
    from minitp.generation import GenerationState

    cfg, (graphed, _), (direct, _) = _models(monkeypatch)
    g = torch.Generator().manual_seed(9)
    prompts = [torch.randint(0, cfg.vocab_size, (2, 64), generator=g).to(DEV) for _ in range(2)]
    outs = []
    for model in (graphed, direct):
        got = []
        for p in prompts:
            for form in ("all", "last", "all"):
                got.append(GenerationState(model, p, 4, prefill_logits=form).prefill().float().clone())
        outs.append(got)
    torch.cuda.synchronize()
    for a, b in zip(*outs):
        assert torch.isfinite(a).all()
        assert torch.equal(a, b), (a - b).abs().max().item()
    assert outs[0][0].shape == (2, 64, cfg.vocab_size) and outs[0][1].shape == (2, 1, cfg.vocab_size)
