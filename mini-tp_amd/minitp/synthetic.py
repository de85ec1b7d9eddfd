"""Seeded synthetic Qwen2 models and prompts, generated on the GPU.

Weights and q/k/v biases are N(0, 0.02), RMSNorm weights 1, prompt ids
uniform over the vocab; each tensor has its own generator stream (stream
ids below). The HIP generator reproduces the CPU generator spec bit for
bit, so a multi-GB model never has to be shipped or copied from the host.
"""

from __future__ import annotations

import torch

from minitp import kernels as K
from minitp.config import ModelConfig
from minitp.distributed.context import ParallelContext
from minitp.layer import TPQwen2ForCausalLM

STREAM_EMBED = 1
STREAM_LM_HEAD = 2
STREAM_PROMPT = 3


def layer_stream(layer: int, which: str) -> int:
    slot = {"qkv_w": 0, "qkv_b": 1, "o_w": 2, "gate_up_w": 3, "down_w": 4}[which]
    return 16 + 8 * layer + slot


# Workload shapes: the tiny parity model, Qwen2.5-0.5B and Qwen2.5-7B.
TINY = ModelConfig(64, 128, 2, 4, 2, 16, 1000, 1e-6, 1e6, 256, True)
QWEN05B = ModelConfig(896, 4864, 24, 14, 2, 64, 151936, 1e-6, 1e6, 32768, True)
QWEN7B = ModelConfig(3584, 18944, 28, 28, 4, 128, 152064, 1e-6, 1e6, 32768, False)
SHAPES = {"tiny": TINY, "qwen2.5-0.5b": QWEN05B, "qwen2.5-7b": QWEN7B}


@torch.no_grad()
def fill_synthetic_(model: TPQwen2ForCausalLM, seed: int = 0, std: float = 0.02) -> TPQwen2ForCausalLM:
    """Overwrite every parameter in place with the seeded synthetic values."""
    m = model.model
    K.fill_normal_(m.embed_tokens.weight, seed, STREAM_EMBED, std)
    for i, layer in enumerate(m.layers):
        a, mlp = layer.self_attn, layer.mlp
        K.fill_(layer.input_layernorm.weight, 1.0)
        K.fill_(layer.post_attention_layernorm.weight, 1.0)
        K.fill_normal_(a.qkv_proj.weight, seed, layer_stream(i, "qkv_w"), std)
        K.fill_normal_(a.qkv_proj.bias, seed, layer_stream(i, "qkv_b"), std)
        K.fill_normal_(a.o_proj.weight, seed, layer_stream(i, "o_w"), std)
        K.fill_normal_(mlp.gate_up_proj.weight, seed, layer_stream(i, "gate_up_w"), std)
        K.fill_normal_(mlp.down_proj.weight, seed, layer_stream(i, "down_w"), std)
    K.fill_(m.norm.weight, 1.0)
    if model.lm_head.weight is not m.embed_tokens.weight:
        K.fill_normal_(model.lm_head.weight, seed, STREAM_LM_HEAD, std)
    return model


def build_synthetic_model(cfg: ModelConfig, dtype: torch.dtype = torch.bfloat16, device: str | torch.device = "cuda",
                          seed: int = 0) -> TPQwen2ForCausalLM:
    """TPQwen2ForCausalLM on `device` in `dtype`, filled from the seeded generator."""
    device = torch.device(device)
    ctx = ParallelContext(0, 0, 1, 0, 1, device, None)
    with torch.device("meta"):
        model = TPQwen2ForCausalLM(cfg, ctx, init_weights=False)
    model = model.to_empty(device=device).to(dtype)
    if cfg.tie_word_embeddings:
        model.lm_head.weight = model.model.embed_tokens.weight
    return fill_synthetic_(model.eval(), seed)


def synthetic_prompt(vocab_size: int, batch: int, prompt_len: int, seed: int = 0,
                     device: str | torch.device = "cuda") -> torch.Tensor:
    return K.uniform_ids(batch * prompt_len, vocab_size, seed, STREAM_PROMPT, device).view(batch, prompt_len)
