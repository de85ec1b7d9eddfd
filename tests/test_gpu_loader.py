"""Checkpoint to greedy ids: the tiny model written as a Hugging Face Qwen2
checkpoint (separate q/k/v and gate/up tensors), loaded by each loader onto
the GPU, must generate the reference's golden ids bit for bit (fp32), and the
direct-to-device load must equal the host loads.
"""

import json
import os

import numpy as np
import pytest
import torch

from tests.conftest import GOLDEN

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _write_hf_checkpoint(path, shape, state):
    """Unpack the packed reference state into HF tensor names."""
    from safetensors.torch import save_file

    hq, hkv, d, inter = shape.num_attention_heads, shape.num_key_value_heads, shape.head_dim, shape.intermediate_size
    out = {"model.embed_tokens.weight": state["model.embed_tokens.weight"], "model.norm.weight": state["model.norm.weight"]}
    for i in range(shape.num_hidden_layers):
        p = f"model.layers.{i}."
        a, m = p + "self_attn.", p + "mlp."
        for n in ("input_layernorm", "post_attention_layernorm"):
            out[f"{p}{n}.weight"] = state[f"{p}{n}.weight"]
        for kind in ("weight", "bias"):
            q, k, v = torch.split(state[a + f"qkv_proj.{kind}"], [hq * d, hkv * d, hkv * d])
            out[a + f"q_proj.{kind}"], out[a + f"k_proj.{kind}"], out[a + f"v_proj.{kind}"] = q, k, v
        out[a + "o_proj.weight"] = state[a + "o_proj.weight"]
        gate, up = torch.split(state[m + "gate_up_proj.weight"], [inter, inter])
        out[m + "gate_proj.weight"], out[m + "up_proj.weight"] = gate, up
        out[m + "down_proj.weight"] = state[m + "down_proj.weight"]
    if not shape.tie_word_embeddings:
        out["lm_head.weight"] = state["lm_head.weight"]
    os.makedirs(path, exist_ok=True)
    save_file({k: v.contiguous().clone() for k, v in out.items()}, os.path.join(path, "model.safetensors"))
    cfg = {"hidden_size": shape.hidden_size, "intermediate_size": inter, "num_hidden_layers": shape.num_hidden_layers,
           "num_attention_heads": hq, "num_key_value_heads": hkv, "head_dim": d, "vocab_size": shape.vocab_size,
           "rms_norm_eps": shape.rms_norm_eps, "rope_theta": shape.rope_theta,
           "max_position_embeddings": shape.max_position_embeddings,
           "tie_word_embeddings": shape.tie_word_embeddings}
    with open(os.path.join(path, "config.json"), "w") as f:
        json.dump(cfg, f)


def test_checkpoint_load_generates_golden_ids(tmp_path):
    from oracle import qwen2_ref

    from minitp.generation import generate_greedy
    from minitp.weight_loader import load_config, load_qwen2_tp

    from minitp.distributed.context import ParallelContext

    shape = qwen2_ref.TINY
    _write_hf_checkpoint(str(tmp_path), shape, qwen2_ref.synthetic_state(shape, seed=0, dtype=torch.float32))
    cfg = load_config(str(tmp_path))
    ctx = ParallelContext(0, 0, 1, 0, 1, torch.device(DEV), None)
    fx = np.load(os.path.join(GOLDEN, "tiny_fp32.npz"))
    prompt = torch.from_numpy(fx["prompt"]).to(DEV)
    n = fx["ids"].shape[1] - prompt.shape[1]
    models = {ld: load_qwen2_tp(str(tmp_path), cfg, ctx, dtype=torch.float32, loader=ld).eval()
              for ld in ("selective", "direct_gpu", "legacy")}
    ref_sd = models["selective"].state_dict()
    for ld, model in models.items():
        assert next(model.parameters()).device.type == "cuda", ld
        for k, v in model.state_dict().items():
            assert torch.equal(v, ref_sd[k]), (ld, k)
        ids = generate_greedy(model, prompt, n, early_stop=False)
        assert np.array_equal(ids.cpu().numpy(), fx["ids"]), ld
    bf = load_qwen2_tp(str(tmp_path), cfg, ctx, dtype=torch.bfloat16, loader="direct_gpu")
    for k, v in bf.state_dict().items():
        assert torch.equal(v, ref_sd[k].to(torch.bfloat16)), k
