"""RMSNorm, decoder layer and the Qwen2 causal LM (minitp/layer.py:19-124).

``TPQwen2ForCausalLM.forward`` keeps the reference signature and semantics
(full [B, T, V] logits, one cursor advance per forward). With the default
toggles it runs the whole forward as one native program (libminitp's
minitp_qwen2_forward: fused norm/QKV/RoPE/KV-write, attention, o_proj +
residual, norm/gate-up/SwiGLU, down + residual per layer). When an ablation
toggle is changed, or profiling labels are on, it walks the modules instead;
that path runs the same kernels one op at a time.
"""

from __future__ import annotations

import ctypes

import torch
import torch.nn as nn

from minitp import _native as N
from minitp import kernels as K
from minitp.attention import TPQwen2Attention
from minitp.config import ModelConfig
from minitp.distributed.context import ParallelContext
from minitp.kv_cache import KVCache
from minitp.mlp import TPQwen2MLP
from minitp.parallel.embedding import VocabParallelEmbedding, VocabParallelLMHead
from minitp.profiling import is_enabled as _profiling_enabled
from minitp.profiling import scope
from minitp.rope import RotaryEmbedding


class RMSNorm(nn.Module):
    """``(x * rsqrt(mean(x^2) + eps)) * w`` in fp32, cast back (layer.py:19-42)."""

    def __init__(self, hidden_size: int, eps: float, init_weights: bool = True) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.ones(hidden_size) if init_weights else torch.empty(hidden_size))
        self.eps = eps
        # The reference runs F.rms_norm for "functional" and its own fp32 math
        # for every other value (layer.py:36-42). F.rms_norm (torch 2.10)
        # computes in fp32 as well and rounds once, after the weight: the same
        # rounding as the reference math, so one kernel serves both (checked
        # against F.rms_norm on the device in the GPU tests).
        self.implementation = "reference"

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return K.rmsnorm(x, self.weight, self.eps)


class TPQwen2DecoderLayer(nn.Module):
    def __init__(self, cfg: ModelConfig, ctx: ParallelContext, init_weights: bool = True) -> None:
        super().__init__()
        self.input_layernorm = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps, init_weights=init_weights)
        self.post_attention_layernorm = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps, init_weights=init_weights)
        self.self_attn = TPQwen2Attention(cfg, ctx, init_weights=init_weights)
        self.mlp = TPQwen2MLP(cfg, ctx, init_weights=init_weights)

    def forward(self, x: torch.Tensor, positions: torch.Tensor, kv_cache: KVCache | None, layer_idx: int,
                rotary: RotaryEmbedding | None = None) -> torch.Tensor:
        x = K.add(x, self.self_attn(self.input_layernorm(x), positions, kv_cache, layer_idx, rotary))
        x = K.add(x, self.mlp(self.post_attention_layernorm(x)))
        return x


class _Program:
    """Owns one minitp_qwen2 handle built from the model's parameter pointers."""

    def __init__(self, model: "TPQwen2ForCausalLM") -> None:
        cfg = model.cfg
        lib = N.lib()
        params = []
        for layer in model.model.layers:
            a, m = layer.self_attn, layer.mlp
            params += [layer.input_layernorm.weight, layer.post_attention_layernorm.weight, a.qkv_proj.weight,
                       a.qkv_proj.bias, a.o_proj.weight, m.gate_up_proj.weight, m.down_proj.weight]
        head = [model.model.embed_tokens.weight, model.lm_head.weight, model.model.norm.weight]
        for p in params + head:
            if p is None or not p.is_cuda or not p.is_contiguous():
                raise RuntimeError("minitp: the native program needs contiguous ROCm parameters (and a QKV bias)")
        self.tensors = params + head + [model.rotary.cos_cache, model.rotary.sin_cache]
        self.signature = tuple(t.data_ptr() for t in self.tensors)
        c = N.Qwen2Config(N.dtype_code(model.model.embed_tokens.weight.dtype), cfg.num_hidden_layers, cfg.hidden_size,
                          model.model.layers[0].self_attn.q_heads_local, model.model.layers[0].self_attn.kv_heads_local,
                          cfg.head_dim, model.model.layers[0].mlp.intermediate_local, cfg.vocab_size,
                          model.rotary.max_seq_len, cfg.rms_norm_eps)
        arr = (ctypes.c_void_p * len(params))(*[p.data_ptr() for p in params])
        w = N.Qwen2Weights(head[0].data_ptr(), head[1].data_ptr(), head[2].data_ptr(),
                           model.rotary.cos_cache.data_ptr(), model.rotary.sin_cache.data_ptr(),
                           ctypes.cast(arr, ctypes.POINTER(ctypes.c_void_p)))
        h = ctypes.c_void_p()
        N.check(lib.minitp_qwen2_create(ctypes.byref(c), ctypes.byref(w), ctypes.byref(h)), "qwen2_create")
        self.handle = h
        self.cfg = c
        self.device = head[0].device
        self.dtype = head[0].dtype
        self.fwd_ws: torch.Tensor | None = None
        self.decode_ws: dict[tuple[int, int], torch.Tensor] = {}

    def decode_path_name(self, batch: int = 1) -> str:
        """The decode form that serves a step of `batch` rows."""
        return ("one hipGraph replay per token: embedding; per layer norm+QKV+RoPE+KV write, attention, "
                "o_proj+residual, norm+gate/up+SwiGLU, down+residual; norm+LM head+argmax partials, merge")

    def check_cache(self, kv: KVCache, batch: int) -> None:
        """The cache must be this model's: [L, batch, Hkv, S, D] buffers (S =
        its capacity) in the model dtype on the model's device (the kernels
        index it with those sizes)."""
        c = self.cfg
        want = (c.num_layers, batch, c.kv_heads, kv.capacity, c.head_dim)
        for buf in (kv.k_buf, kv.v_buf):
            if tuple(buf.shape) != want or buf.dtype != self.dtype or buf.device != self.device or \
                    not buf.is_contiguous():
                raise ValueError(f"KV cache {tuple(buf.shape)} {buf.dtype} on {buf.device} does not fit this model: "
                                 f"need a contiguous {want} {self.dtype} cache on {self.device}")

    def check_decode(self) -> None:
        """Synchronise and raise IndexError if a forward on any of this
        program's workspaces ran at a position outside the RoPE table (the
        sticky error word of the step state; cleared by the check)."""
        for ws in list(self.decode_ws.values()) + ([self.fwd_ws] if self.fwd_ws is not None else []):
            N.check(N.lib().minitp_qwen2_decode_check(self.handle, N.stream(), ws.data_ptr()), "qwen2_decode")

    def valid_for(self, model: "TPQwen2ForCausalLM") -> bool:
        return tuple(t.data_ptr() for t in self.tensors) == self.signature and \
            model.rotary.cos_cache.data_ptr() == self.tensors[-2].data_ptr()

    def workspace_bytes(self, tokens: int, batch: int, max_seq: int) -> int:
        return N.lib().minitp_qwen2_workspace_bytes(self.handle, tokens, batch, max_seq)

    def forward_ws(self, tokens: int, batch: int, max_seq: int) -> torch.Tensor:
        need = self.workspace_bytes(tokens, batch, max_seq)
        if self.fwd_ws is None or self.fwd_ws.numel() < need:
            self.fwd_ws = torch.zeros(need, dtype=torch.uint8, device=self.device)
        return self.fwd_ws

    def decode_workspace(self, batch: int, max_seq: int) -> torch.Tensor:
        # One buffer per (batch, max_seq) for the life of the program: the
        # decode graph recorded for that shape points into it.
        key = (batch, max_seq)
        ws = self.decode_ws.get(key)
        if ws is None:
            ws = torch.zeros(self.workspace_bytes(batch, batch, max_seq), dtype=torch.uint8, device=self.device)
            self.decode_ws[key] = ws
        return ws

    def __del__(self) -> None:
        h = getattr(self, "handle", None)
        if h is not None and h.value:
            try:
                N.lib().minitp_qwen2_destroy(h)
            except Exception:
                pass


class TPQwen2ForCausalLM(nn.Module):
    def __init__(self, cfg: ModelConfig, ctx: ParallelContext, init_weights: bool = True) -> None:
        super().__init__()
        if ctx.tp_size != 1:
            raise NotImplementedError(f"tp_size={ctx.tp_size}: this MI355X build runs tensor parallelism 1 only")
        self.cfg = cfg
        self.ctx = ctx
        self.init_weights = init_weights
        self.rotary: RotaryEmbedding | None = None  # built on first forward
        self.use_rotary_cache = True  # ablation toggle (layer.py:75)
        self.model = nn.Module()
        self.model.embed_tokens = VocabParallelEmbedding(cfg.vocab_size, cfg.hidden_size, ctx,
                                                         init_weights=init_weights)
        self.model.layers = nn.ModuleList(TPQwen2DecoderLayer(cfg, ctx, init_weights=init_weights)
                                          for _ in range(cfg.num_hidden_layers))
        self.model.norm = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps, init_weights=init_weights)
        self.lm_head = VocabParallelLMHead(cfg.hidden_size, cfg.vocab_size, ctx, init_weights=init_weights)
        if cfg.tie_word_embeddings:
            self.lm_head.weight = self.model.embed_tokens.weight
        self._prog: _Program | None = None

    # -- helpers -------------------------------------------------------------
    def _ensure_rotary(self, device: torch.device) -> RotaryEmbedding:
        if self.rotary is None or self.rotary.cos_cache.device != device:
            self.rotary = RotaryEmbedding(self.cfg.head_dim, self.cfg.rope_theta, self.cfg.max_position_embeddings,
                                          device)
        return self.rotary

    def native_path(self) -> bool:
        """True when the whole-model program serves forward (default toggles)."""
        if not self.use_rotary_cache or _profiling_enabled():
            return False
        for layer in self.model.layers:
            if not (layer.self_attn.use_fused_qkv and layer.mlp.use_fused_gateup):
                return False
        return self.model.embed_tokens.weight.dtype in (torch.float32, torch.bfloat16)

    def program(self) -> _Program:
        dev = self.model.embed_tokens.weight.device
        self._ensure_rotary(dev)
        if self._prog is None or not self._prog.valid_for(self) or self._prog.dtype != \
                self.model.embed_tokens.weight.dtype:
            self._prog = _Program(self)
        return self._prog

    def _native(self, input_ids: torch.Tensor, positions: torch.Tensor, kv_cache: KVCache | None,
                next_tok: torch.Tensor | None = None, eos: tuple | None = None,
                last_only: bool = False) -> torch.Tensor:
        """Whole-model forward on the native program. Logits [B, T, V], or
        [B, 1, V] of the last position when ``last_only`` (one LM-head row per
        sequence instead of T)."""
        prog = self.program()
        b, t = input_ids.shape
        dev = prog.device
        N.require_gpu(input_ids, positions, next_tok, what="TPQwen2ForCausalLM.forward")
        if kv_cache is not None:
            self._check_kv(prog, kv_cache, b)
        ids = input_ids if (input_ids.dtype == torch.long and input_ids.stride(-1) == 1) else \
            input_ids.long().contiguous()
        pos = positions if (positions.dtype == torch.long and positions.is_contiguous()) else \
            positions.long().contiguous()
        kv = kv_cache
        if kv is None:
            a = self.model.layers[0].self_attn
            kv = KVCache(self.cfg.num_hidden_layers, b, a.kv_heads_local, self.cfg.head_dim, t, prog.dtype, dev)
        kv.check_room(t)
        all_rows = t > 1 and not last_only
        logits = torch.empty(b, t if all_rows else 1, self.cfg.vocab_size, dtype=prog.dtype, device=dev)
        ws = prog.forward_ws(b * t, b, kv.capacity)
        step = N.Qwen2Step(ids.data_ptr(), ids.stride(0), pos.data_ptr(), b, t, kv.seq_len, kv.k_buf.data_ptr(),
                           kv.v_buf.data_ptr(), kv.capacity, logits.data_ptr(), 1 if all_rows else 0,
                           N.ptr(next_tok), next_tok.stride(0) if next_tok is not None else 0, ws.data_ptr(),
                           ws.numel(), *(eos or (None, 0, 0, None)))
        N.check(N.lib().minitp_qwen2_forward(prog.handle, N.stream(), ctypes.byref(step)), "qwen2_forward")
        if kv_cache is not None:
            kv_cache.advance(t)
        return logits

    def decode_native(self, tok: torch.Tensor, pos: torch.Tensor, kv_cache: KVCache, logits: torch.Tensor,
                      next_tok: torch.Tensor | None, eos: tuple | None = None) -> torch.Tensor:
        """One T == 1 step replayed from the program's decode hipGraph.
        tok [B] (any stride), pos 0-d long, logits [B, 1, V] written in place.
        eos: (state pointer, token, cursor, host word pointer) of the
        on-device early stop, or None."""
        prog = self._prog if self._prog is not None else self.program()
        b = tok.shape[0]
        N.require_gpu(tok, pos, next_tok, what="GenerationState.decode_step")
        if pos.dtype != torch.long or pos.numel() != 1:
            raise ValueError(f"decode_step: pos must be one int64 position, got {pos.dtype} of {pos.numel()}")
        self._check_kv(prog, kv_cache, b)
        kv_cache.check_room(1)
        ws = prog.decode_workspace(b, kv_cache.capacity)
        step = N.Qwen2Step(tok.data_ptr(), tok.stride(0), pos.data_ptr(), b, 1, kv_cache.seq_len,
                           kv_cache.k_buf.data_ptr(), kv_cache.v_buf.data_ptr(), kv_cache.capacity,
                           logits.data_ptr(), 0, N.ptr(next_tok), next_tok.stride(0) if next_tok is not None else 0,
                           ws.data_ptr(), ws.numel(), *(eos or (None, 0, 0, None)))
        N.check(N.lib().minitp_qwen2_decode(prog.handle, N.stream(), ctypes.byref(step)), "qwen2_decode")
        kv_cache.advance(1)
        return logits

    @staticmethod
    def _check_kv(prog: _Program, kv: KVCache, batch: int) -> None:
        """Once per (cache, program, batch): the cache's buffers must be the
        [L, batch, Hkv, S, D] model-dtype tensors the kernels index."""
        key = (id(prog), batch)
        if getattr(kv, "_minitp_fits", None) != key:
            prog.check_cache(kv, batch)
            kv._minitp_fits = key

    # -- reference API ---------------------------------------------------------
    def forward(self, input_ids: torch.Tensor, positions: torch.Tensor | None = None,
                kv_cache: KVCache | None = None, gather_logits: bool = False) -> torch.Tensor:
        b, t = input_ids.shape
        N.require_gpu(input_ids, self.model.embed_tokens.weight, what="TPQwen2ForCausalLM.forward")
        limit = self.cfg.max_position_embeddings
        if positions is None:  # layer.py:99-101
            offset = kv_cache.seq_len if kv_cache is not None and t == 1 else 0
            if offset + t > limit:
                raise IndexError(f"position {offset + t - 1} out of range for RoPE table of {limit} rows")
            positions = torch.arange(offset, offset + t, device=input_ids.device)
        else:
            # explicit positions index the RoPE table as the reference's
            # cos_cache[positions] does: negative ones wrap, others past the
            # table raise (rope.py:37-45). One host read of min / max.
            from minitp.rope import _check_positions

            _check_positions(positions, limit)
            positions = positions.to(input_ids.device).long()
            positions = torch.where(positions < 0, positions + limit, positions)
        if kv_cache is not None:
            kv_cache.check_room(t)
        if self.native_path():
            return self._native(input_ids, positions, kv_cache)
        x = self.model.embed_tokens(input_ids)
        rotary = self._ensure_rotary(x.device) if self.use_rotary_cache else None
        for i, layer in enumerate(self.model.layers):
            with scope(f"mini_tp.layer_{i}"):
                x = layer(x, positions, kv_cache, i, rotary)
        if kv_cache is not None:
            kv_cache.advance(t)
        with scope("mini_tp.final_norm_lm_head"):
            x = self.model.norm(x)
            if gather_logits:
                self.lm_head.gather_logits = True
                logits = self.lm_head(x)
                self.lm_head.gather_logits = False
                return logits
            return self.lm_head(x)
