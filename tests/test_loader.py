"""Local safetensors loader (weight_loader.py): host-side tests on synthetic
checkpoints, mirroring tests/test_selective_loader.py and
tests/test_loader_coverage.py of the reference.

Each packed parameter is checked against ``torch.cat`` of the checkpoint's
own tensors (the packing rule of fused.py:57-61, 102-104), the loaders
against each other bit for bit, and the copy plan at tensor parallelism 1
(whole tensors; other layouts are refused).
"""

import json

import pytest
import torch
from safetensors.torch import save_file

from minitp.config import ModelConfig
from minitp.distributed.context import ParallelContext

CPU_CTX = ParallelContext(0, 0, 1, 0, 1, torch.device("cpu"), None)


def _cfg(kv_heads=2, tied=False, layers=2):
    return ModelConfig(hidden_size=32, intermediate_size=48, num_hidden_layers=layers, num_attention_heads=4,
                       num_key_value_heads=kv_heads, head_dim=8, vocab_size=24, rms_norm_eps=1e-6,
                       rope_theta=10000.0, max_position_embeddings=32, tie_word_embeddings=tied)


def _hf_state(cfg, seed=0, bias=True, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)

    def r(*shape):
        return torch.randn(*shape, generator=g).to(dtype)

    kv = cfg.num_key_value_heads * cfg.head_dim
    h, inter = cfg.hidden_size, cfg.intermediate_size
    s = {"model.embed_tokens.weight": r(cfg.vocab_size, h)}
    for i in range(cfg.num_hidden_layers):
        p = f"model.layers.{i}."
        s[p + "input_layernorm.weight"] = r(h) * 0.1 + 1
        s[p + "post_attention_layernorm.weight"] = r(h) * 0.1 + 1
        for name, rows in (("q_proj", cfg.num_attention_heads * cfg.head_dim), ("k_proj", kv), ("v_proj", kv)):
            s[f"{p}self_attn.{name}.weight"] = r(rows, h)
            if bias:
                s[f"{p}self_attn.{name}.bias"] = r(rows)
        s[p + "self_attn.o_proj.weight"] = r(h, h)
        s[p + "mlp.gate_proj.weight"] = r(inter, h)
        s[p + "mlp.up_proj.weight"] = r(inter, h)
        s[p + "mlp.down_proj.weight"] = r(h, inter)
    s["model.norm.weight"] = r(h) * 0.1 + 1
    if not cfg.tie_word_embeddings:
        s["lm_head.weight"] = r(cfg.vocab_size, h)
    return s


def _write(tmp_path, state, sharded, name="ckpt"):
    d = tmp_path / name
    d.mkdir()
    if sharded:  # three files, names spread across them
        files = {}
        for j, k in enumerate(sorted(state)):
            files.setdefault(f"model-{j % 3:05d}-of-00003.safetensors", {})[k] = state[k].contiguous()
        for f, ts in files.items():
            save_file(ts, str(d / f))
        (d / "model.safetensors.index.json").write_text(
            json.dumps({"metadata": {}, "weight_map": {k: f for f, ts in files.items() for k in ts}}))
    else:
        save_file({k: v.contiguous() for k, v in state.items()}, str(d / "model.safetensors"))
    return str(d)


def _expected(cfg, s):
    """The packed state dict by the packing rule itself."""
    e = {"model.embed_tokens.weight": s["model.embed_tokens.weight"], "model.norm.weight": s["model.norm.weight"]}
    for i in range(cfg.num_hidden_layers):
        p = f"model.layers.{i}."
        a, m = p + "self_attn.", p + "mlp."
        e[p + "input_layernorm.weight"] = s[p + "input_layernorm.weight"]
        e[p + "post_attention_layernorm.weight"] = s[p + "post_attention_layernorm.weight"]
        e[a + "qkv_proj.weight"] = torch.cat([s[a + "q_proj.weight"], s[a + "k_proj.weight"], s[a + "v_proj.weight"]])
        if a + "q_proj.bias" in s:
            e[a + "qkv_proj.bias"] = torch.cat([s[a + "q_proj.bias"], s[a + "k_proj.bias"], s[a + "v_proj.bias"]])
        else:
            e[a + "qkv_proj.bias"] = torch.zeros(e[a + "qkv_proj.weight"].shape[0])
        e[a + "o_proj.weight"] = s[a + "o_proj.weight"]
        e[m + "gate_up_proj.weight"] = torch.cat([s[m + "gate_proj.weight"], s[m + "up_proj.weight"]])
        e[m + "down_proj.weight"] = s[m + "down_proj.weight"]
    e["lm_head.weight"] = s["model.embed_tokens.weight"] if cfg.tie_word_embeddings else s["lm_head.weight"]
    return e


def _load(d, cfg, loader, dtype=torch.float32):
    from minitp.weight_loader import load_qwen2_tp

    return load_qwen2_tp(d, cfg, CPU_CTX, dtype=dtype, loader=loader)


@pytest.mark.parametrize("sharded", [False, True])
@pytest.mark.parametrize("tied", [False, True])
def test_packed_parameters_equal_the_packing_rule(tmp_path, sharded, tied):
    cfg = _cfg(tied=tied)
    s = _hf_state(cfg)
    d = _write(tmp_path, s, sharded)
    exp = _expected(cfg, s)
    models = {ld: _load(d, cfg, ld) for ld in ("legacy", "selective")}
    for ld, model in models.items():
        got = model.state_dict()
        assert set(got) == set(exp), ld
        for k in exp:
            assert torch.equal(got[k], exp[k]), (ld, k)
    if tied:
        m = models["selective"]
        assert m.lm_head.weight is m.model.embed_tokens.weight


def test_bf16_load_rounds_like_tensor_to(tmp_path):
    cfg = _cfg()
    s = _hf_state(cfg)
    d = _write(tmp_path, s, sharded=False)
    exp = _expected(cfg, s)
    got = _load(d, cfg, "selective", dtype=torch.bfloat16).state_dict()
    for k in exp:
        assert got[k].dtype == torch.bfloat16 and torch.equal(got[k], exp[k].to(torch.bfloat16)), k


def test_bf16_checkpoint_into_fp32_model(tmp_path):
    """Real Qwen checkpoints are bf16; an fp32 model widens them exactly."""
    cfg = _cfg()
    s = _hf_state(cfg, dtype=torch.bfloat16)
    d = _write(tmp_path, s, sharded=True)
    exp = _expected(cfg, s)
    for ld in ("legacy", "selective"):
        got = _load(d, cfg, ld).state_dict()
        for k in exp:
            assert torch.equal(got[k], exp[k].float()), (ld, k)


def test_checkpoint_without_qkv_bias_leaves_zero_bias(tmp_path):
    cfg = _cfg()
    s = _hf_state(cfg, bias=False)
    d = _write(tmp_path, s, sharded=False)
    got = _load(d, cfg, "selective").state_dict()
    for i in range(cfg.num_hidden_layers):
        assert torch.equal(got[f"model.layers.{i}.self_attn.qkv_proj.bias"], torch.zeros(64))


def test_missing_tensor_raises_with_its_name(tmp_path):
    cfg = _cfg()
    s = _hf_state(cfg)
    del s["model.layers.1.mlp.up_proj.weight"]
    for sharded in (False, True):
        d = _write(tmp_path, s, sharded, name=f"c{int(sharded)}")
        for ld in ("legacy", "selective"):
            with pytest.raises(KeyError, match="up_proj"):
                _load(d, cfg, ld)


def test_wrong_shape_raises(tmp_path):
    cfg = _cfg()
    s = _hf_state(cfg)
    s["model.layers.0.mlp.gate_proj.weight"] = s["model.layers.0.mlp.gate_proj.weight"][:, :16]
    d = _write(tmp_path, s, sharded=False)
    with pytest.raises(ValueError, match="gate_proj"):
        _load(d, cfg, "selective")


def test_selective_never_loads_the_full_state(tmp_path, monkeypatch):
    import minitp.weight_loader as wl

    called = []
    orig = wl._load_full_state
    monkeypatch.setattr(wl, "_load_full_state", lambda d: called.append(d) or orig(d))
    cfg = _cfg()
    d = _write(tmp_path, _hf_state(cfg), sharded=False)
    _load(d, cfg, "selective")
    assert called == []


def test_unknown_loader_and_missing_checkpoint(tmp_path):
    from minitp.weight_loader import load_qwen2_tp

    with pytest.raises(ValueError, match="unknown loader"):
        load_qwen2_tp(str(tmp_path), _cfg(), CPU_CTX, loader="mmap")
    with pytest.raises(FileNotFoundError):
        load_qwen2_tp(str(tmp_path), _cfg(), CPU_CTX)


def test_config_json_of_qwen25_05b(tmp_path):
    """The fields of Qwen2.5-0.5B's config.json, read without transformers."""
    from minitp.weight_loader import load_config

    (tmp_path / "config.json").write_text(json.dumps({
        "architectures": ["Qwen2ForCausalLM"], "hidden_size": 896, "intermediate_size": 4864,
        "num_hidden_layers": 24, "num_attention_heads": 14, "num_key_value_heads": 2, "vocab_size": 151936,
        "rms_norm_eps": 1e-06, "rope_theta": 1000000.0, "max_position_embeddings": 32768,
        "tie_word_embeddings": True, "torch_dtype": "bfloat16"}))
    cfg = load_config(str(tmp_path))
    assert (cfg.hidden_size, cfg.head_dim, cfg.num_key_value_heads, cfg.vocab_size) == (896, 64, 2, 151936)
    assert cfg.rope_theta == 1e6 and cfg.tie_word_embeddings


# ---------------------------------------------------------------------------
# the copy plan at tensor parallelism 1 (weight_loader.py:40-67 at tp_size 1)


def test_copy_plan_at_tp1_is_whole_tensors():
    from minitp.weight_loader import copy_plan

    cfg = _cfg()
    s = _hf_state(cfg)
    for c in copy_plan(cfg):
        t = s[c.src]
        assert c.start == 0 and c.length == t.shape[c.dim], c


def test_copy_plan_refuses_other_tensor_parallel_layouts():
    from minitp.weight_loader import copy_plan

    with pytest.raises(NotImplementedError):
        copy_plan(_cfg(), rank=1, tp=2)
