"""CPU restatement of mini-tp's TP=1 Qwen2 forward and greedy token loop.

ORACLE / TEST INFRASTRUCTURE ONLY. Only ``tests/``, ``__graft_entry__.smoke()``
and ``bench.py``'s CPU-baseline leg may import this module, and only as the
checker or the timed CPU baseline. The product path never calls it.

Every function restates one reference function with the same torch ops, in the
same order and with the same dtype casts, so that on the CPU it reproduces the
reference's bits (pinned by tests/golden fixtures written from the reference
itself). Citations are ``file:line`` in the reference repository.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F

from oracle import synth


@dataclass(frozen=True)
class Qwen2Shape:
    """Fields of ``ModelConfig`` (minitp/config.py:17-30) the forward reads."""

    hidden_size: int
    intermediate_size: int
    num_hidden_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    head_dim: int
    vocab_size: int
    rms_norm_eps: float
    rope_theta: float
    max_position_embeddings: int
    tie_word_embeddings: bool = True


# ---------------------------------------------------------------------------
# RoPE — minitp/rope.py


def rope_tables(head_dim: int, theta: float, max_seq_len: int) -> tuple[torch.Tensor, torch.Tensor]:
    """fp32 cos/sin tables [max_seq_len, head_dim] (rope.py:27-35)."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
    pos = torch.arange(max_seq_len, dtype=torch.float32)
    freqs = pos[:, None] * inv_freq[None, :]
    emb = torch.cat([freqs, freqs], dim=-1)
    return emb.cos(), emb.sin()


def _rotate_half(x: torch.Tensor) -> torch.Tensor:
    # rope.py:57-59: pairs are (i, i + D/2)
    x1, x2 = x.float().chunk(2, dim=-1)
    return torch.cat([-x2, x1], dim=-1)


def rope_apply(cos_cache, sin_cache, q, k, positions):
    """RotaryEmbedding.apply (rope.py:47-64); q/k are [B, H, T, D]."""
    cos, sin = cos_cache[positions], sin_cache[positions]  # rope.py:45 (IndexError if out of range)
    cos = cos[None, None]
    sin = sin[None, None]

    def rotate(x):
        return (x.float() * cos + _rotate_half(x) * sin).to(x.dtype)

    return rotate(q), rotate(k)


def rope_apply_uncached(q, k, positions, theta: float):
    """apply_rope (rope.py:67-88)."""
    head_dim = q.shape[-1]
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
    freqs = positions.float()[:, None] * inv_freq[None, :]
    emb = torch.cat([freqs, freqs], dim=-1)
    cos, sin = emb.cos()[None, None], emb.sin()[None, None]

    def rotate(x):
        return (x.float() * cos + _rotate_half(x) * sin).to(x.dtype)

    return rotate(q), rotate(k)


# ---------------------------------------------------------------------------
# RMSNorm — minitp/layer.py:36-42 ("reference" implementation)


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    dtype = x.dtype
    x = x.float()
    x = x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps)
    return (x * weight.float()).to(dtype)


# ---------------------------------------------------------------------------
# KV cache — minitp/kv_cache.py:8-63


class OracleKVCache:
    def __init__(self, num_layers, batch_size, kv_heads, head_dim, max_seq_len, dtype, init="empty"):
        if init not in ("empty", "zeros"):
            raise ValueError(f"init must be 'empty' or 'zeros', got {init!r}")
        self.max_seq_len = max_seq_len
        self.seq_len = 0
        alloc = torch.empty if init == "empty" else torch.zeros
        self.k = [alloc(batch_size, kv_heads, max_seq_len, head_dim, dtype=dtype) for _ in range(num_layers)]
        self.v = [alloc(batch_size, kv_heads, max_seq_len, head_dim, dtype=dtype) for _ in range(num_layers)]

    def update(self, layer_idx, k_new, v_new):
        """kv_cache.py:43-55: write at the cursor, return the valid prefix."""
        t = k_new.shape[2]
        end = self.seq_len + t
        if end > self.max_seq_len:
            raise ValueError(f"KV cache overflow: seq {self.seq_len}+{t} > max_seq_len={self.max_seq_len}")
        self.k[layer_idx][:, :, self.seq_len : end] = k_new
        self.v[layer_idx][:, :, self.seq_len : end] = v_new
        return self.k[layer_idx][:, :, :end], self.v[layer_idx][:, :, :end]

    def advance(self, tokens):
        self.seq_len += tokens


# ---------------------------------------------------------------------------
# Model — minitp/layer.py, attention.py, mlp.py, parallel/*.py at tp_size=1


class OracleQwen2:
    """Holds reference-named tensors (state-dict keys of TPQwen2ForCausalLM)."""

    def __init__(self, shape: Qwen2Shape, state: dict[str, torch.Tensor]):
        self.cfg = shape
        self.sd = state
        self.cos_cache = None
        self.sin_cache = None
        self.use_rotary_cache = True

    # -- submodules -------------------------------------------------------
    def attention(self, i, x, positions, kv, rotary):
        """TPQwen2Attention.forward (attention.py:49-106)."""
        c = self.cfg
        b, t, _ = x.shape
        hq, hkv, hd = c.num_attention_heads, c.num_key_value_heads, c.head_dim
        p = f"model.layers.{i}.self_attn."
        y = F.linear(x, self.sd[p + "qkv_proj.weight"], self.sd[p + "qkv_proj.bias"])  # fused.py:58
        q, k, v = torch.split(y, [hq * hd, hkv * hd, hkv * hd], dim=-1)  # fused.py:60
        q = q.view(b, t, hq, hd).transpose(1, 2)
        k = k.view(b, t, hkv, hd).transpose(1, 2)
        v = v.view(b, t, hkv, hd).transpose(1, 2)
        if rotary:
            q, k = rope_apply(self.cos_cache, self.sin_cache, q, k, positions)
        else:
            q, k = rope_apply_uncached(q, k, positions, c.rope_theta)
        if kv is not None:
            cache_len = kv.seq_len
            k, v = kv.update(i, k, v)
        else:
            cache_len = 0
        if hq != hkv:  # attention.py:77-90
            group = hq // hkv
            if hkv == 1:
                k = k.expand(b, hq, k.shape[2], hd)
                v = v.expand(b, hq, v.shape[2], hd)
            else:
                k = k.repeat_interleave(group, dim=1)
                v = v.repeat_interleave(group, dim=1)
        if t == 1:  # attention.py:92-103
            out = F.scaled_dot_product_attention(q, k, v)
        elif cache_len == 0:
            out = F.scaled_dot_product_attention(q, k, v, is_causal=True)
        else:
            total = k.shape[2]
            mask = torch.ones(t, total, dtype=torch.bool).tril(diagonal=cache_len)
            out = F.scaled_dot_product_attention(q, k, v, attn_mask=mask)
        out = out.transpose(1, 2).reshape(b, t, hq * hd)
        return F.linear(out, self.sd[p + "o_proj.weight"])  # linear.py:117, no bias

    def mlp(self, i, x):
        """TPQwen2MLP.forward (mlp.py:34-38) with the fused gate/up (fused.py:102-104)."""
        p = f"model.layers.{i}.mlp."
        gate, up = torch.chunk(F.linear(x, self.sd[p + "gate_up_proj.weight"]), 2, dim=-1)
        return F.linear(F.silu(gate) * up, self.sd[p + "down_proj.weight"])

    def layer(self, i, x, positions, kv, rotary):
        """TPQwen2DecoderLayer.forward (layer.py:55-65)."""
        eps = self.cfg.rms_norm_eps
        p = f"model.layers.{i}."
        x = x + self.attention(i, rms_norm(x, self.sd[p + "input_layernorm.weight"], eps), positions, kv, rotary)
        x = x + self.mlp(i, rms_norm(x, self.sd[p + "post_attention_layernorm.weight"], eps))
        return x

    def forward(self, input_ids, positions=None, kv_cache=None):
        """TPQwen2ForCausalLM.forward (layer.py:91-124) -> logits [B, T, V]."""
        c = self.cfg
        b, t = input_ids.shape
        if positions is None:  # layer.py:99-101
            offset = kv_cache.seq_len if kv_cache is not None and t == 1 else 0
            positions = torch.arange(offset, offset + t)
        x = F.embedding(input_ids, self.sd["model.embed_tokens.weight"])  # embedding.py:46
        if self.use_rotary_cache and self.cos_cache is None:  # layer.py:103-111
            self.cos_cache, self.sin_cache = rope_tables(c.head_dim, c.rope_theta, c.max_position_embeddings)
        for i in range(c.num_hidden_layers):
            x = self.layer(i, x, positions, kv_cache, self.use_rotary_cache)
        if kv_cache is not None:
            kv_cache.advance(t)
        x = rms_norm(x, self.sd["model.norm.weight"], c.rms_norm_eps)
        return F.linear(x, self.sd["lm_head.weight"])  # embedding.py:88

    __call__ = forward

    def make_kv_cache(self, batch_size, max_seq_len, init="empty"):
        """generation.py:36-51."""
        c = self.cfg
        dtype = self.sd["model.embed_tokens.weight"].dtype
        return OracleKVCache(c.num_hidden_layers, batch_size, c.num_key_value_heads, c.head_dim, max_seq_len, dtype, init)


# ---------------------------------------------------------------------------
# Token loop — minitp/generation.py


def select_token(logits: torch.Tensor) -> torch.Tensor:
    """TP=1 path of select_token / distributed_argmax (generation.py:54-59,
    embedding.py:146-147): argmax of the last position."""
    return logits[:, -1].argmax(dim=-1, keepdim=True).squeeze(-1)


class OracleGenerationState:
    """GenerationState (generation.py:70-130)."""

    def __init__(self, model: OracleQwen2, input_ids, max_new_tokens, kv=None, kv_init="empty"):
        self.model = model
        b, t = input_ids.shape
        self.prompt_len = t
        self.max_new_tokens = max_new_tokens
        self.total = t + max_new_tokens
        self.kv = kv if kv is not None else model.make_kv_cache(b, self.total, init=kv_init)
        self.out_ids = torch.empty(b, self.total, dtype=torch.long)
        self.out_ids[:, :t] = input_ids
        self.positions_buf = torch.arange(self.total)
        self.cursor = t

    def prefill(self):
        return self.model(self.out_ids[:, : self.prompt_len], positions=self.positions_buf[: self.prompt_len], kv_cache=self.kv)

    def select_next(self, logits):
        return select_token(logits)

    def append(self, tok):
        self.out_ids[:, self.cursor] = tok
        pos = self.positions_buf[self.cursor]
        self.cursor += 1
        return pos

    def decode_step(self, tok, pos):
        return self.model(tok.unsqueeze(-1), positions=pos.unsqueeze(-1), kv_cache=self.kv)


@torch.inference_mode()
def generate_greedy(model, input_ids, max_new_tokens, eos_token_id=None, early_stop=True, kv=None,
                    kv_init="empty", on_logits=None):
    """generate_greedy (generation.py:133-171). ``on_logits(step, logits)``
    (oracle-only hook) sees the logits each selection reads."""
    state = OracleGenerationState(model, input_ids, max_new_tokens, kv=kv, kv_init=kv_init)
    b = input_ids.shape[0]
    finished = None
    eos = -1
    if early_stop and eos_token_id is not None:
        eos = eos_token_id
        finished = torch.zeros(b, dtype=torch.bool)
    logits = state.prefill()
    eos_tok = torch.tensor(eos)
    for step in range(max_new_tokens):
        if on_logits is not None:
            on_logits(step, logits)
        tok = state.select_next(logits)
        if finished is not None:
            tok = torch.where(finished, eos_tok, tok)
            finished = finished | (tok == eos)
        pos = state.append(tok)
        if finished is not None and bool(finished.all()):
            break
        if step + 1 < max_new_tokens:
            logits = state.decode_step(tok, pos)
    return state.out_ids[:, : state.cursor] if early_stop else state.out_ids


# ---------------------------------------------------------------------------
# Synthetic models (seeded N(0, 0.02) weights and biases, unit norms)


def synthetic_state(shape: Qwen2Shape, seed: int = 0, dtype=torch.float32, std: float = 0.02) -> dict[str, torch.Tensor]:
    """Reference state-dict keys (weight_loader.py:208-226) filled from the
    oracle generator. fp32 values, rounded to ``dtype`` by ``Tensor.to``."""
    c = shape
    hq, hkv, hd, h, inter = c.num_attention_heads, c.num_key_value_heads, c.head_dim, c.hidden_size, c.intermediate_size
    qkv_rows = (hq + 2 * hkv) * hd

    def normal(stream, *dims):
        n = 1
        for d in dims:
            n *= d
        return torch.from_numpy(synth.normal_f32_c(seed, stream, n, std)).view(*dims).to(dtype)

    sd: dict[str, torch.Tensor] = {}
    sd["model.embed_tokens.weight"] = normal(synth.STREAM_EMBED, c.vocab_size, h)
    for i in range(c.num_hidden_layers):
        p = f"model.layers.{i}."
        sd[p + "input_layernorm.weight"] = torch.ones(h, dtype=dtype)
        sd[p + "post_attention_layernorm.weight"] = torch.ones(h, dtype=dtype)
        sd[p + "self_attn.qkv_proj.weight"] = normal(synth.layer_stream(i, "qkv_w"), qkv_rows, h)
        sd[p + "self_attn.qkv_proj.bias"] = normal(synth.layer_stream(i, "qkv_b"), qkv_rows)
        sd[p + "self_attn.o_proj.weight"] = normal(synth.layer_stream(i, "o_w"), h, hq * hd)
        sd[p + "mlp.gate_up_proj.weight"] = normal(synth.layer_stream(i, "gate_up_w"), 2 * inter, h)
        sd[p + "mlp.down_proj.weight"] = normal(synth.layer_stream(i, "down_w"), h, inter)
    sd["model.norm.weight"] = torch.ones(h, dtype=dtype)
    if c.tie_word_embeddings:
        sd["lm_head.weight"] = sd["model.embed_tokens.weight"]
    else:
        sd["lm_head.weight"] = normal(synth.STREAM_LM_HEAD, c.vocab_size, h)
    return sd


def synthetic_prompt(vocab_size: int, batch: int, prompt_len: int, seed: int = 0) -> torch.Tensor:
    return torch.from_numpy(synth.uniform_ids_c(seed, synth.STREAM_PROMPT, batch * prompt_len, vocab_size)).view(batch, prompt_len)


# Workload shapes (sizes as stated by the workloads; max_position_embeddings
# only sizes the RoPE table, whose rows do not depend on it).
TINY = Qwen2Shape(64, 128, 2, 4, 2, 16, 1000, 1e-6, 1e6, 256, True)
QWEN05B = Qwen2Shape(896, 4864, 24, 14, 2, 64, 151936, 1e-6, 1e6, 32768, True)
QWEN7B = Qwen2Shape(3584, 18944, 28, 28, 4, 128, 152064, 1e-6, 1e6, 32768, False)
