"""Greedy token loop over the KV cache (minitp/generation.py:36-171).

Same objects and methods as the reference. ``GenerationState`` is the one
hot path: ``prefill`` runs the native whole-model program, ``decode_step``
replays the program's decode hipGraph (one graph launch per token), and the
greedy token of every step is written by the LM-head kernel straight into
``out_ids[:, cursor]``, so ``select_next`` on the logits a step just
produced returns that column and ``append`` has nothing left to copy.
Fixed-length mode (``early_stop=False``) therefore issues no host sync and
no extra kernels per token.

The decode logits buffer [B, 1, V] is reused: logits returned by one
``decode_step`` are overwritten by the next.
"""

from __future__ import annotations

import torch

from minitp.kv_cache import KVCache
from minitp.layer import TPQwen2ForCausalLM


def _kv_heads_local(model: TPQwen2ForCausalLM) -> int:
    return model.model.layers[0].self_attn.kv_heads_local


def make_kv_cache(model: TPQwen2ForCausalLM, batch_size: int, max_seq_len: int, init: str = "empty") -> KVCache:
    p = next(model.parameters())
    return KVCache(num_layers=model.cfg.num_hidden_layers, batch_size=batch_size,
                   kv_heads_local=_kv_heads_local(model), head_dim=model.cfg.head_dim, max_seq_len=max_seq_len,
                   dtype=p.dtype, device=p.device, init=init)


def select_token(model: TPQwen2ForCausalLM, logits: torch.Tensor, distributed_argmax: bool = True) -> torch.Tensor:
    """Greedy pick from the last position's logits (generation.py:54-67)."""
    if distributed_argmax:
        return model.lm_head.distributed_argmax(logits[:, -1]).squeeze(-1)
    if model.ctx.tp_size == 1:
        from minitp import kernels as K

        return K.argmax(logits[:, -1])
    raise NotImplementedError("tp_size > 1 is not built on MI355X")


class GenerationState:
    """KV cache + positions buffer + output buffer (generation.py:70-130)."""

    def __init__(self, model: TPQwen2ForCausalLM, input_ids: torch.Tensor, max_new_tokens: int,
                 kv: KVCache | None = None, distributed_argmax: bool = True, kv_init: str = "empty") -> None:
        self.model = model
        self.distributed_argmax = distributed_argmax
        b, t = input_ids.shape
        self.prompt_len = t
        self.max_new_tokens = max_new_tokens
        self.total = t + max_new_tokens
        self.kv = kv if kv is not None else make_kv_cache(model, b, self.total, init=kv_init)
        device = input_ids.device
        self.out_ids = torch.empty(b, self.total, dtype=torch.long, device=device)
        self.out_ids[:, :t] = input_ids
        self.positions_buf = torch.arange(self.total, device=device)  # the only arange
        self.cursor = t
        self.finished: torch.Tensor | None = None
        self.eos = -1
        self._native = model.native_path() and device.type == "cuda"
        self._last_logits: torch.Tensor | None = None
        self._last_tok: torch.Tensor | None = None
        self._decode_logits: torch.Tensor | None = None

    def _next_column(self) -> torch.Tensor | None:
        return self.out_ids[:, self.cursor] if self.cursor < self.total else None

    def _check_position(self, last: int) -> None:
        limit = self.model.cfg.max_position_embeddings
        if last >= limit:
            raise IndexError(f"position {last} out of range for RoPE table of {limit} rows")

    def prefill(self) -> torch.Tensor:
        """Prompt forward; positions come from the buffer (0..T-1)."""
        positions = self.positions_buf[: self.prompt_len]
        ids = self.out_ids[:, : self.prompt_len]
        if not self._native:
            return self.model(ids, positions=positions, kv_cache=self.kv)
        self._check_position(self.prompt_len - 1)
        col = self._next_column()
        logits = self.model._native(ids, positions, self.kv, next_tok=col)
        self._last_logits, self._last_tok = logits, col
        return logits

    def select_next(self, logits: torch.Tensor) -> torch.Tensor:
        if logits is self._last_logits and self._last_tok is not None:
            return self._last_tok
        return select_token(self.model, logits, self.distributed_argmax)

    def append(self, tok: torch.Tensor) -> torch.Tensor:
        """Write the token at the cursor; return its absolute position tensor."""
        col = self.out_ids[:, self.cursor]
        if not (tok.data_ptr() == col.data_ptr() and tok.shape == col.shape and tok.stride() == col.stride()):
            self.out_ids[:, self.cursor] = tok
        pos = self.positions_buf[self.cursor]
        self.cursor += 1
        return pos

    def decode_step(self, tok: torch.Tensor, pos: torch.Tensor) -> torch.Tensor:
        if not self._native:
            return self.model(tok.unsqueeze(-1), positions=pos.unsqueeze(-1), kv_cache=self.kv)
        b = tok.shape[0]
        if pos.data_ptr() == self.positions_buf.data_ptr() + (self.cursor - 1) * 8:
            self._check_position(self.cursor - 1)  # pos is positions_buf[cursor - 1]: value known
        if self._decode_logits is None or self._decode_logits.shape[0] != b:
            self._decode_logits = torch.empty(b, 1, self.model.cfg.vocab_size, dtype=self.kv.k_buf.dtype,
                                              device=self.out_ids.device)
        if tok.dtype != torch.long:
            tok = tok.long()
        col = self._next_column()
        logits = self.model.decode_native(tok, pos.reshape(()), self.kv, self._decode_logits, col)
        self._last_logits, self._last_tok = logits, col
        return logits


@torch.inference_mode()
def generate_greedy(model: TPQwen2ForCausalLM, input_ids: torch.Tensor, max_new_tokens: int,
                    eos_token_id: int | None = None, distributed_argmax: bool = True, early_stop: bool = True,
                    kv: KVCache | None = None, kv_init: str = "empty") -> torch.Tensor:
    """Greedy decode through GenerationState (generation.py:133-171): trimmed at
    the first step where every row has produced EOS when ``early_stop``;
    exactly prompt + max_new_tokens columns otherwise."""
    state = GenerationState(model, input_ids, max_new_tokens, kv=kv, distributed_argmax=distributed_argmax,
                            kv_init=kv_init)
    b = input_ids.shape[0]
    if early_stop and eos_token_id is not None:
        state.eos = eos_token_id
        state.finished = torch.zeros(b, dtype=torch.bool, device=input_ids.device)
    logits = state.prefill()
    eos_tok = torch.tensor(state.eos, device=input_ids.device)
    for step in range(max_new_tokens):
        tok = state.select_next(logits)
        if state.finished is not None:
            tok = torch.where(state.finished, eos_tok, tok)
            state.finished = state.finished | (tok == state.eos)
        pos = state.append(tok)
        if state.finished is not None and bool(state.finished.all()):
            break
        if step + 1 < max_new_tokens:
            logits = state.decode_step(tok, pos)
    return state.out_ids[:, : state.cursor] if early_stop else state.out_ids
