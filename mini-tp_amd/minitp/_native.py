"""ctypes binding of libminitp.so (the C ABI in include/minitp.h).

There is no CPU fallback: every op here runs a HIP kernel on the tensor's
ROCm device, and a missing library or a CPU tensor raises immediately.
Status codes map to the exceptions the reference raises for the same
condition (``ValueError`` for overflow / divisibility, ``IndexError`` for
out-of-range indices).
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib", "libminitp.so")

OK, ERR_ARG, ERR_HIP, ERR_OVERFLOW, ERR_RANGE, ERR_UNSUPPORTED, ERR_DIVISIBLE = 0, -1, -2, -3, -4, -5, -6
F32, BF16 = 0, 1
EPI_NONE, EPI_RESID, EPI_SWIGLU = 0, 1, 2
W_PER_LAYER = 7

_DTYPES = {torch.float32: F32, torch.bfloat16: BF16}

_vp, _i64, _i32, _u64, _f32, _f64, _int = (
    ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_uint64, ctypes.c_float, ctypes.c_double, ctypes.c_int,
)

# name -> (restype, argtypes); mirrors include/minitp.h
SIGNATURES = {
    "minitp_status_string": (ctypes.c_char_p, [_int]),
    "minitp_last_error": (ctypes.c_char_p, []),
    "minitp_abi_version": (_int, []),
    "minitp_fill_normal": (_int, [_vp, _int, _vp, _i64, _u64, _u64, _f64]),
    "minitp_fill_uniform_ids": (_int, [_vp, _vp, _i64, _u64, _u64, _i64]),
    "minitp_fill": (_int, [_vp, _int, _vp, _i64, _f32]),
    "minitp_embedding": (_int, [_vp, _int, _vp, _vp, _vp, _i64, _i64, _i64]),
    "minitp_rmsnorm": (_int, [_vp, _int, _vp, _vp, _vp, _i64, _i64, _f32]),
    "minitp_add": (_int, [_vp, _int, _vp, _vp, _vp, _i64, _i64]),
    "minitp_silu_mul": (_int, [_vp, _int, _vp, _vp, _i64, _vp, _i64, _i64, _i64]),
    "minitp_cast_f32_bf16": (_int, [_vp, _vp, _vp, _i64]),
    "minitp_host_device_pointer": (_int, [_vp, ctypes.POINTER(_vp)]),
    "minitp_linear": (_int, [_vp, _int, _vp, _i64, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _int, _vp]),
    "minitp_rmsnorm_linear": (_int, [_vp, _int, _vp, _i64, _vp, _f32, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _int,
                                     _vp]),
    "minitp_add_rmsnorm_linear_parts": (_int, [_vp, _int, _vp, _vp, _i32, _vp, _vp, _f32, _vp, _vp, _i64, _i64,
                                               _int]),
    "minitp_rope": (_int, [_vp, _int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64]),
    "minitp_kv_write": (_int, [_vp, _int, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64]),
    "minitp_rope_kv_write": (_int, [_vp, _int, _vp, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64,
                                    _i64, _i64, _i64, _i64]),
    "minitp_attention_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64, _i64, _i64]),
    "minitp_attention": (_int, [_vp, _int, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _vp,
                                _i64]),
    "minitp_argmax_workspace_bytes": (_i64, [_i64, _i64]),
    "minitp_argmax": (_int, [_vp, _int, _vp, _i64, _i64, _i64, _vp, _i64, _vp, _i64]),
    "minitp_argmax_static_max_bytes": (_i64, []),
    "minitp_argmax_static": (_int, [_vp, _int, _vp, _i64, _i64, _i64, _vp, _i64]),
    "minitp_qwen2_create": (_int, [_vp, _vp, ctypes.POINTER(_vp)]),
    "minitp_qwen2_destroy": (_int, [_vp]),
    "minitp_qwen2_workspace_bytes": (_i64, [_vp, _i64, _i64, _i64]),
    "minitp_qwen2_forward": (_int, [_vp, _vp, _vp]),
    "minitp_qwen2_decode": (_int, [_vp, _vp, _vp]),
    "minitp_qwen2_decode_check": (_int, [_vp, _vp, _vp]),
}


class Qwen2Config(ctypes.Structure):
    _fields_ = [("dtype", _i32), ("num_layers", _i32), ("hidden", _i32), ("heads", _i32), ("kv_heads", _i32),
                ("head_dim", _i32), ("intermediate", _i32), ("vocab", _i32), ("max_pos", _i32), ("eps", _f32)]


class Qwen2Weights(ctypes.Structure):
    _fields_ = [("embed", _vp), ("lm_head", _vp), ("final_norm", _vp), ("rope_cos", _vp), ("rope_sin", _vp),
                ("layers", ctypes.POINTER(_vp))]


class Qwen2Step(ctypes.Structure):
    _fields_ = [("ids", _vp), ("ids_ld", _i64), ("positions", _vp), ("batch", _i64), ("tokens", _i64),
                ("cache_len", _i64), ("k_cache", _vp), ("v_cache", _vp), ("max_seq", _i64), ("logits", _vp),
                ("logits_all", _i32), ("next_tok", _vp), ("next_tok_ld", _i64), ("workspace", _vp),
                ("workspace_bytes", _i64), ("eos_state", _vp), ("eos_token", _i64), ("cursor", _i64),
                ("eos_host", _vp)]


_lib = None
_lock = threading.Lock()


def lib() -> ctypes.CDLL:
    """Load the HIP library once; raise if it has not been built."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not os.path.exists(LIB_PATH):
                    raise RuntimeError(
                        f"minitp: native library {LIB_PATH} is missing; build it with "
                        "`python -c 'import __graft_entry__ as g; g.build()'` (or make -C mini-tp_amd/csrc)")
                handle = ctypes.CDLL(LIB_PATH)
                for name, (res, args) in SIGNATURES.items():
                    fn = getattr(handle, name)
                    fn.restype = res
                    fn.argtypes = args
                _lib = handle
    return _lib


def last_error() -> str:
    msg = lib().minitp_last_error()
    return msg.decode() if msg else ""


def check(status: int, what: str) -> None:
    if status == OK:
        return
    detail = last_error()
    msg = f"{what}: {detail}" if detail else f"{what}: {lib().minitp_status_string(status).decode()}"
    if status == ERR_OVERFLOW or status == ERR_DIVISIBLE:
        raise ValueError(detail or msg)
    if status == ERR_RANGE:
        raise IndexError(msg)
    if status == ERR_UNSUPPORTED:
        raise NotImplementedError(msg)
    if status == ERR_ARG:
        raise ValueError(msg)
    raise RuntimeError(msg)


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPES[dtype]
    except KeyError:
        raise TypeError(f"minitp kernels support float32 and bfloat16, got {dtype}") from None


def require_gpu(*tensors: torch.Tensor, what: str = "op") -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError(
                f"minitp: {what} runs only as a HIP kernel on a ROCm GPU; got a {t.device.type} tensor "
                "(this build has no CPU path)")


def stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


# ---------------------------------------------------------------------------
# Zeroed scratch buffers. The kernels that use completion counters leave them
# at zero when they finish, so a buffer is zeroed once when allocated and
# then reused; all users run on one stream in program order.
_scratch: dict[tuple, torch.Tensor] = {}


def scratch(device: torch.device, key: str, nbytes: int) -> torch.Tensor:
    k = (device, key)
    buf = _scratch.get(k)
    if buf is None or buf.numel() < nbytes:
        buf = torch.zeros(max(nbytes, 256), dtype=torch.uint8, device=device)
        _scratch[k] = buf
    return buf
