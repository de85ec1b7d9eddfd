"""Greedy token loop over the KV cache (minitp/generation.py:36-171).

Same objects and methods as the reference. ``GenerationState`` is the one
hot path: ``prefill`` runs the native whole-model program, ``decode_step``
replays the program's decode hipGraph (one graph launch per token), and the
greedy token of every step is written by the LM-head kernel straight into
``out_ids[:, cursor]``, so ``select_next`` on the logits a step just
produced returns that column and ``append`` has nothing left to copy.
Fixed-length mode (``early_stop=False``) therefore issues no host sync and
no extra kernels per token.

Early stop on an EOS token keeps the reference's finished mask on the
device: one more kernel after each token selection applies
``tok = where(finished, eos, tok); finished |= tok == eos`` and, once every
row has finished, records the stop column and writes it to a pinned host
word. The host reads that word instead of a blocking ``finished.all()``
copy each step; it keeps at most ``EOS_LAG`` steps queued ahead of the GPU,
and the steps it queued past the stop write no KV rows, so the result, the
cursor and ``kv.seq_len`` are the reference's.

Each ``decode_step`` returns a new logits tensor [B, 1, V], as the
reference does. ``reuse_decode_logits=True`` (what ``generate_greedy`` and
the benchmark use, since they only read the token the step picked) writes
every step's logits into one buffer instead, so the logits a step returned
are overwritten by the next step.

``prefill`` returns every prompt position's logits [B, T, V], as the
reference does, unless the state was made with ``prefill_logits="last"``:
then [B, 1, V] of the last position, the only row a token is picked from.
``generate_greedy`` uses that form, which skips T - 1 of the T LM-head rows
of the prompt (the greedy ids are the same).
"""

from __future__ import annotations

import collections
import ctypes

import torch

from minitp import _native as N
from minitp.kv_cache import KVCache
from minitp.layer import TPQwen2ForCausalLM

EOS_LAG = 2  # decode steps the host may queue before it reads the stop word


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
                 kv: KVCache | None = None, distributed_argmax: bool = True, kv_init: str = "empty",
                 prefill_logits: str = "all", reuse_decode_logits: bool = False) -> None:
        if prefill_logits not in ("all", "last"):
            raise ValueError(f"prefill_logits must be 'all' or 'last', got {prefill_logits!r}")
        self.model = model
        self.prefill_logits = prefill_logits
        self.reuse_decode_logits = reuse_decode_logits
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
        self._eos_dev: torch.Tensor | None = None  # [B + 2] finished flags, halted, stop column
        self._eos_host: torch.Tensor | None = None  # pinned stop column (0 = running)
        self._eos_host_dev: int | None = None

    def _enable_device_eos(self, eos: int) -> None:
        """Keep generate_greedy's finished mask and stop test on the device."""
        b = self.out_ids.shape[0]
        self.eos = eos
        self._eos_dev = torch.zeros(b + 2, dtype=torch.long, device=self.out_ids.device)
        self._eos_host = torch.zeros(1, dtype=torch.long, pin_memory=True)
        dev = ctypes.c_void_p()
        N.check(N.lib().minitp_host_device_pointer(self._eos_host.data_ptr(), ctypes.byref(dev)), "host_device_pointer")
        self._eos_host_dev = dev.value

    def _eos_args(self) -> tuple | None:
        if self._eos_dev is None:
            return None
        return (self._eos_dev.data_ptr(), self.eos, self.cursor, self._eos_host_dev)

    def _eos_stop(self) -> int:
        """Stop column the device recorded (0 while some row is running)."""
        return int(self._eos_host[0])

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
        logits = self.model._native(ids, positions, self.kv, next_tok=col, eos=self._eos_args(),
                                    last_only=self.prefill_logits == "last")
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
        else:
            # any other position tensor: read its value (one host sync, off the
            # generate_greedy path) so that it indexes the RoPE table as the
            # reference's gather does: past the table raises IndexError, a
            # negative position wraps (rope.py:37-45)
            from minitp.rope import _check_positions

            limit = self.model.cfg.max_position_embeddings
            _check_positions(pos, limit)
            pos = torch.where(pos < 0, pos + limit, pos)
        if not self.reuse_decode_logits or self._decode_logits is None or self._decode_logits.shape[0] != b:
            self._decode_logits = torch.empty(b, 1, self.model.cfg.vocab_size, dtype=self.kv.k_buf.dtype,
                                              device=self.out_ids.device)
        if tok.dtype != torch.long:
            tok = tok.long()
        col = self._next_column()
        logits = self.model.decode_native(tok, pos.reshape(()), self.kv, self._decode_logits, col,
                                          eos=self._eos_args())
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
                            kv_init=kv_init, prefill_logits="last", reuse_decode_logits=True)
    b = input_ids.shape[0]
    if early_stop and eos_token_id is not None and state._native and max_new_tokens > 0:
        return _generate_device_eos(state, eos_token_id, max_new_tokens)
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


def _generate_device_eos(state: GenerationState, eos: int, max_new_tokens: int) -> torch.Tensor:
    """generate_greedy's early-stop loop with the finished mask on the device."""
    if eos < 0:
        raise ValueError(f"eos_token_id must be >= 0, got {eos}")
    state._enable_device_eos(eos)
    kv_start = state.kv.seq_len
    logits = state.prefill()
    inflight: collections.deque = collections.deque()
    for step in range(max_new_tokens):
        tok = state.select_next(logits)
        pos = state.append(tok)
        if step + 1 >= max_new_tokens:
            break
        while len(inflight) >= EOS_LAG:
            inflight.popleft().synchronize()
        if state._eos_stop():
            break
        logits = state.decode_step(tok, pos)
        ev = torch.cuda.Event()
        ev.record()
        inflight.append(ev)
    torch.cuda.current_stream().synchronize()
    stop = state._eos_stop()
    if stop:
        # every column after the stop was a step the device ran halted
        state.cursor = stop
        state.kv.seq_len = kv_start + stop - 1  # the prompt, then one decode per column before the stop
    state.finished = state._eos_dev[: state.out_ids.shape[0]].bool()
    return state.out_ids[:, : state.cursor]
