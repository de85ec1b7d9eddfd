"""Local safetensors checkpoints into the packed parameters (minitp/weight_loader.py).

Hugging Face Qwen2 checkpoints keep q/k/v and gate/up as separate tensors.
This model keeps them packed: ``qkv_proj`` rows are ``[q; k; v]`` with the
bias packed the same way, and ``gate_up_proj`` rows are ``[gate; up]``
(fused.py:57-61, 102-104), because the decode kernels pair rows inside one
matrix. Loading is therefore one copy plan, a list of "rows [start, start+n)
of checkpoint tensor X (along dim d) go to parameter Y at row r", built once
by :func:`copy_plan` and carried out by three executors that cannot disagree
(weight_loader.py:172-269):

* ``"selective"`` (default): per-slice reads through ``safetensors.safe_open``
  (memory-mapped; the full state dict is never materialised), into a host
  model that is then moved to the target device;
* ``"direct_gpu"``: the model is built on the device with uninitialised
  parameters and each slice goes straight into its device parameter. A slice
  crosses PCIe in the checkpoint's dtype and is converted on the device;
* ``"legacy"``: the whole state dict is loaded on the host, then sliced.

The model runs ``tp_size == 1`` only, so every plan entry is a whole
checkpoint tensor (the reference's per-rank slicing, weight_loader.py:40-67,
has no counterpart here and a plan for another ``tp`` is refused). Every
parameter must be written by the plan, or loading raises.
"""

from __future__ import annotations

import json
import os
from dataclasses import dataclass
from types import SimpleNamespace

import torch

from minitp.config import ModelConfig
from minitp.distributed.context import ParallelContext
from minitp.layer import TPQwen2ForCausalLM

INDEX_FILE = "model.safetensors.index.json"
SINGLE_FILE = "model.safetensors"


# ---------------------------------------------------------------------------
# the copy plan


@dataclass(frozen=True)
class Copy:
    dest: str  # parameter name in the model's state dict
    dest_row: int  # first destination row (dim 0)
    src: str  # checkpoint tensor name
    dim: int  # dimension of the checkpoint tensor that is sliced
    start: int
    length: int
    optional: bool = False  # biases: a checkpoint without them leaves zeros


def copy_plan(cfg: ModelConfig, rank: int = 0, tp: int = 1, qkv_bias: bool = True) -> list[Copy]:
    """Every copy that fills the parameters from a Qwen2 checkpoint (tp 1)."""
    if tp != 1 or rank != 0:
        raise NotImplementedError(f"copy plan for rank {rank} of tp {tp}: this build loads tensor parallelism 1 only")
    plan: list[Copy] = []
    h, inter = cfg.hidden_size, cfg.intermediate_size
    plan.append(Copy("model.embed_tokens.weight", 0, "model.embed_tokens.weight", 0, 0, cfg.vocab_size))
    q_rows = cfg.num_attention_heads * cfg.head_dim
    kv_rows = cfg.num_key_value_heads * cfg.head_dim
    q0, qn, k0, kn, h0, hn, i0, inn = 0, q_rows, 0, kv_rows, 0, h, 0, inter
    for i in range(cfg.num_hidden_layers):
        p = f"model.layers.{i}."
        for norm in ("input_layernorm", "post_attention_layernorm"):
            plan.append(Copy(f"{p}{norm}.weight", 0, f"{p}{norm}.weight", 0, 0, h))
        packed = ((f"{p}self_attn.q_proj", 0, q0, qn), (f"{p}self_attn.k_proj", q_rows, k0, kn),
                  (f"{p}self_attn.v_proj", q_rows + kv_rows, k0, kn))
        for src, row, start, n in packed:
            plan.append(Copy(f"{p}self_attn.qkv_proj.weight", row, f"{src}.weight", 0, start, n))
        if qkv_bias:
            for src, row, start, n in packed:
                plan.append(Copy(f"{p}self_attn.qkv_proj.bias", row, f"{src}.bias", 0, start, n, optional=True))
        plan.append(Copy(f"{p}self_attn.o_proj.weight", 0, f"{p}self_attn.o_proj.weight", 1, h0, hn))
        plan.append(Copy(f"{p}mlp.gate_up_proj.weight", 0, f"{p}mlp.gate_proj.weight", 0, i0, inn))
        plan.append(Copy(f"{p}mlp.gate_up_proj.weight", inter, f"{p}mlp.up_proj.weight", 0, i0, inn))
        plan.append(Copy(f"{p}mlp.down_proj.weight", 0, f"{p}mlp.down_proj.weight", 1, i0, inn))
    plan.append(Copy("model.norm.weight", 0, "model.norm.weight", 0, 0, h))
    if not cfg.tie_word_embeddings:
        plan.append(Copy("lm_head.weight", 0, "lm_head.weight", 0, 0, cfg.vocab_size))
    return plan


# ---------------------------------------------------------------------------
# checkpoint access (single file or index-sharded)


class SelectiveTensorReader:
    """Reads tensors, or row/column ranges of them, from a checkpoint
    directory without materialising the state dict (weight_loader.py:74-165).
    Handles ``model.safetensors`` and ``model.safetensors.index.json``."""

    def __init__(self, model_dir: str) -> None:
        from safetensors import safe_open

        self._open = safe_open
        self._handles: dict[str, object] = {}
        index = os.path.join(model_dir, INDEX_FILE)
        if os.path.exists(index):
            with open(index) as f:
                self._files = {k: os.path.join(model_dir, v) for k, v in json.load(f)["weight_map"].items()}
            self._single = None
        else:
            self._files = {}
            self._single = os.path.join(model_dir, SINGLE_FILE)
            if not os.path.exists(self._single):
                raise FileNotFoundError(f"no {SINGLE_FILE} or {INDEX_FILE} in {model_dir}")

    def __enter__(self) -> SelectiveTensorReader:
        return self

    def __exit__(self, *exc) -> None:
        self.close()

    def _handle(self, path: str):
        h = self._handles.get(path)
        if h is None:
            h = self._handles[path] = self._open(path, framework="pt", device="cpu")
        return h

    def _path(self, name: str) -> str:
        if self._single is not None:
            return self._single
        try:
            return self._files[name]
        except KeyError:
            raise KeyError(f"tensor {name!r} not in checkpoint index") from None

    def names(self) -> list[str]:
        return list(self._handle(self._single).keys()) if self._single is not None else list(self._files)

    def has(self, name: str) -> bool:
        if self._single is not None:
            return name in self._handle(self._single).keys()
        return name in self._files

    def get(self, name: str) -> torch.Tensor:
        h = self._handle(self._path(name))
        if name not in h.keys():
            raise KeyError(f"tensor {name!r} not in checkpoint")
        return h.get_tensor(name)

    def get_slice(self, name: str, dim: int, start: int, length: int) -> torch.Tensor:
        """``tensor.narrow(dim, start, length)`` read from the file. 1-D
        tensors (norms, biases) are read whole, then narrowed."""
        h = self._handle(self._path(name))
        if name not in h.keys():
            raise KeyError(f"tensor {name!r} not in checkpoint")
        sl = h.get_slice(name)
        shape = sl.get_shape()
        if len(shape) == 1:
            return h.get_tensor(name).narrow(0, start, length)
        idx = [slice(None)] * len(shape)
        idx[dim] = slice(start, start + length)
        return sl[tuple(idx)]

    def close(self) -> None:
        self._handles.clear()


def _load_full_state(model_dir: str) -> dict[str, torch.Tensor]:
    from safetensors.torch import load_file

    index = os.path.join(model_dir, INDEX_FILE)
    if os.path.exists(index):
        with open(index) as f:
            files = sorted(set(json.load(f)["weight_map"].values()))
        state: dict[str, torch.Tensor] = {}
        for name in files:
            state.update(load_file(os.path.join(model_dir, name)))
        return state
    return load_file(os.path.join(model_dir, SINGLE_FILE))


def load_config(model_dir: str, tp_size: int = 1) -> ModelConfig:
    """ModelConfig from the checkpoint's ``config.json`` (the fields
    ``ModelConfig.from_hf`` reads; no transformers import needed)."""
    with open(os.path.join(model_dir, "config.json")) as f:
        return ModelConfig.from_hf(SimpleNamespace(**json.load(f)), tp_size=tp_size)


# ---------------------------------------------------------------------------
# executors


def _execute(plan: list[Copy], params: dict[str, torch.Tensor], read, dtype: torch.dtype) -> None:
    written: dict[str, int] = {}
    for c in plan:
        try:
            src = read(c)
        except KeyError:
            if c.optional:
                continue
            raise
        dest = params[c.dest]
        if tuple(src.shape[1:]) != tuple(dest.shape[1:]) or c.dest_row + src.shape[0] > dest.shape[0]:
            raise ValueError(f"{c.src} slice {tuple(src.shape)} does not fit {c.dest} {tuple(dest.shape)} "
                             f"at row {c.dest_row}")
        if src.device != dest.device:
            src = src.to(dest.device)  # checkpoint dtype over the bus, converted below
        dest[c.dest_row : c.dest_row + src.shape[0]].copy_(src.to(dtype) if src.dtype != dtype else src)
        written[c.dest] = written.get(c.dest, 0) + src.shape[0]
    for name, p in params.items():
        if written.get(name, 0) != p.shape[0] and not name.endswith("qkv_proj.bias"):
            raise RuntimeError(f"checkpoint load left {name} incomplete ({written.get(name, 0)} of {p.shape[0]} rows)")


def load_qwen2_tp(model_dir: str, cfg: ModelConfig, ctx: ParallelContext, dtype: torch.dtype = torch.float32,
                  device: torch.device | None = None, loader: str = "selective") -> TPQwen2ForCausalLM:
    """Build the model and fill it from a local checkpoint
    (weight_loader.py:172-236). All loaders give identical parameters. A
    checkpoint without q/k/v biases leaves the packed bias at zero."""
    if loader not in ("selective", "legacy", "direct_gpu"):
        raise ValueError(f"unknown loader {loader!r}")
    target = torch.device(device) if device is not None else torch.device(ctx.device)
    build = target if loader == "direct_gpu" and target.type == "cuda" else torch.device("cpu")
    with torch.device(build):
        model = TPQwen2ForCausalLM(cfg, ctx, init_weights=False)
    model = model.to(dtype=dtype)
    params = {k: v for k, v in model.state_dict(keep_vars=True).items()}
    if cfg.tie_word_embeddings:
        params.pop("lm_head.weight")  # the embedding's Parameter
    params = {k: v.data for k, v in params.items()}
    for name in params:
        if name.endswith("qkv_proj.bias"):
            params[name].zero_()
    plan = copy_plan(cfg, ctx.tp_rank, ctx.tp_size)
    with torch.no_grad():
        if loader == "legacy":
            state = _load_full_state(model_dir)

            def read(c: Copy) -> torch.Tensor:
                if c.src not in state:
                    raise KeyError(f"tensor {c.src!r} not in checkpoint")
                return state[c.src].narrow(c.dim, c.start, c.length)

            _execute(plan, params, read, dtype)
            del state
        else:
            with SelectiveTensorReader(model_dir) as reader:
                _execute(plan, params, lambda c: reader.get_slice(c.src, c.dim, c.start, c.length), dtype)
    return model.to(target)
