"""Tensor-level wrappers of the minitp HIP kernels (one per C-ABI entry point).

All inputs must live on a ROCm device; outputs are allocated here unless the
caller passes them. Launches go to torch's current stream.
"""

from __future__ import annotations

import torch

from minitp import _native as N


def _lib():
    return N.lib()


def fill_normal_(t: torch.Tensor, seed: int, stream_id: int, std: float = 0.02) -> torch.Tensor:
    """Seeded N(0, std) fill, bit-identical to the CPU generator spec."""
    N.require_gpu(t, what="fill_normal_")
    assert t.is_contiguous()
    N.check(_lib().minitp_fill_normal(N.stream(), N.dtype_code(t.dtype), t.data_ptr(), t.numel(), seed, stream_id,
                                      std), "fill_normal")
    return t


def uniform_ids(count: int, vocab: int, seed: int, stream_id: int, device) -> torch.Tensor:
    out = torch.empty(count, dtype=torch.long, device=device)
    N.require_gpu(out, what="uniform_ids")
    N.check(_lib().minitp_fill_uniform_ids(N.stream(), out.data_ptr(), count, seed, stream_id, vocab), "uniform_ids")
    return out


def fill_(t: torch.Tensor, value: float) -> torch.Tensor:
    N.require_gpu(t, what="fill_")
    assert t.is_contiguous()
    N.check(_lib().minitp_fill(N.stream(), N.dtype_code(t.dtype), t.data_ptr(), t.numel(), float(value)), "fill")
    return t


def embedding(ids: torch.Tensor, table: torch.Tensor) -> torch.Tensor:
    """F.embedding(ids, table)."""
    N.require_gpu(ids, table, what="embedding")
    ids_c = ids.contiguous().to(torch.long)
    out = torch.empty(*ids.shape, table.shape[1], dtype=table.dtype, device=table.device)
    N.check(_lib().minitp_embedding(N.stream(), N.dtype_code(table.dtype), table.data_ptr(), ids_c.data_ptr(),
                                    out.data_ptr(), ids_c.numel(), table.shape[1], table.shape[0]), "embedding")
    return out


def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    N.require_gpu(x, w, what="rmsnorm")
    xc = x.contiguous()
    out = torch.empty_like(xc)
    h = x.shape[-1]
    N.check(_lib().minitp_rmsnorm(N.stream(), N.dtype_code(x.dtype), xc.data_ptr(), w.contiguous().data_ptr(),
                                  out.data_ptr(), xc.numel() // h, h, eps), "rmsnorm")
    return out


def add(a: torch.Tensor, b: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    N.require_gpu(a, b, what="add")
    a, b = a.contiguous(), b.contiguous()
    if a.shape != b.shape or a.dtype != b.dtype:
        raise ValueError(f"add: shapes/dtypes differ: {a.shape}/{a.dtype} vs {b.shape}/{b.dtype}")
    out = torch.empty_like(a) if out is None else out
    N.check(_lib().minitp_add(N.stream(), N.dtype_code(a.dtype), a.data_ptr(), b.data_ptr(), out.data_ptr(),
                              a.numel(), a.numel()), "add")
    return out


def add_bias(x: torch.Tensor, bias: torch.Tensor) -> torch.Tensor:
    """x + bias broadcast over rows, rounded to the dtype (a separate add, as
    ``local + self.bias`` is in linear.py:120-121)."""
    N.require_gpu(x, bias, what="add_bias")
    x = x.contiguous()
    out = torch.empty_like(x)
    N.check(_lib().minitp_add(N.stream(), N.dtype_code(x.dtype), x.data_ptr(), bias.contiguous().data_ptr(),
                              out.data_ptr(), x.numel(), bias.numel()), "add_bias")
    return out


def silu_mul(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """F.silu(gate) * up for same-shaped row-major views sharing a row stride."""
    N.require_gpu(gate, up, what="silu_mul")
    n = gate.shape[-1]
    if gate.stride(-1) != 1 or up.stride(-1) != 1 or gate.stride()[:-1] != up.stride()[:-1]:
        gate, up = gate.contiguous(), up.contiguous()
    rows = gate.numel() // n
    ld_in = gate.stride(-2) if gate.dim() > 1 else n
    # rows of a [.., T, n] view are uniformly strided only if flattenable
    if gate.dim() > 2 and not _rows_uniform(gate):
        gate, up = gate.contiguous(), up.contiguous()
        ld_in = n
    out = torch.empty(*gate.shape, dtype=gate.dtype, device=gate.device)
    N.check(_lib().minitp_silu_mul(N.stream(), N.dtype_code(gate.dtype), gate.data_ptr(), up.data_ptr(), ld_in,
                                   out.data_ptr(), n, rows, n), "silu_mul")
    return out


def _rows_uniform(t: torch.Tensor) -> bool:
    # every leading dim steps by (size of the next dim) * its stride
    for d in range(t.dim() - 2):
        if t.stride(d) != t.stride(d + 1) * t.shape[d + 1]:
            return False
    return True


def _as_rows(x: torch.Tensor) -> tuple[torch.Tensor, int, int]:
    """View x [..., K] as M rows with a uniform row stride (copy if needed)."""
    k = x.shape[-1]
    vec = 4 if x.dtype == torch.float32 else 8
    ld = x.stride(-2) if x.dim() > 1 else k
    ok = x.stride(-1) == 1 and (x.dim() == 1 or _rows_uniform(x)) and x.data_ptr() % 16 == 0 and ld % vec == 0
    if not ok:
        x = x.contiguous()
        ld = k
    return x, _rows(x), ld


def _rows(x: torch.Tensor) -> int:
    m = 1
    for s in x.shape[:-1]:
        m *= s
    return m


def linear(x: torch.Tensor, w: torch.Tensor, bias: torch.Tensor | None = None, *, out: torch.Tensor | None = None,
           epilogue: int = N.EPI_NONE, aux: torch.Tensor | None = None) -> torch.Tensor:
    """F.linear(x, w, bias) with fp32 accumulation, rounded to the dtype.

    ``out`` may be a column slice of a wider row-major buffer (its row stride
    is passed through), which is how the unfused ablation paths write q/k/v
    or gate/up next to each other.
    """
    N.require_gpu(x, w, bias, what="linear")
    if x.dtype != w.dtype or (bias is not None and bias.dtype != w.dtype):
        raise TypeError(f"linear: dtype mismatch x={x.dtype} w={w.dtype}")
    w = w.contiguous()
    xr, m, ldx = _as_rows(x)
    n_out = w.shape[0] // 2 if epilogue == N.EPI_SWIGLU else w.shape[0]
    if out is None:
        out = torch.empty(*x.shape[:-1], n_out, dtype=x.dtype, device=x.device)
        ldy = n_out
    else:
        ldy = out.stride(-2) if out.dim() > 1 else n_out
    N.check(_lib().minitp_linear(N.stream(), N.dtype_code(x.dtype), xr.data_ptr(), ldx, w.data_ptr(),
                                 N.ptr(bias.contiguous() if bias is not None else None), out.data_ptr(), ldy, m,
                                 n_out, w.shape[1], epilogue, N.ptr(aux)), "linear")
    return out


def rmsnorm_linear(x: torch.Tensor, norm_w: torch.Tensor, eps: float, w: torch.Tensor,
                   bias: torch.Tensor | None = None, *, out: torch.Tensor | None = None, epilogue: int = N.EPI_NONE,
                   aux: torch.Tensor | None = None) -> torch.Tensor:
    """linear(rmsnorm(x, norm_w, eps), w, bias) as one GEMV pass over ``w``
    (decode shapes: at most 4 rows). Equal to the two-call form up to the
    norm's summation order."""
    N.require_gpu(x, norm_w, w, bias, what="rmsnorm_linear")
    if x.dtype != w.dtype or norm_w.dtype != w.dtype or (bias is not None and bias.dtype != w.dtype):
        raise TypeError(f"rmsnorm_linear: dtype mismatch x={x.dtype} norm={norm_w.dtype} w={w.dtype}")
    w = w.contiguous()
    xr, m, ldx = _as_rows(x)
    n_out = w.shape[0] // 2 if epilogue == N.EPI_SWIGLU else w.shape[0]
    if out is None:
        out = torch.empty(*x.shape[:-1], n_out, dtype=x.dtype, device=x.device)
        ldy = n_out
    else:
        ldy = out.stride(-2) if out.dim() > 1 else n_out
    N.check(_lib().minitp_rmsnorm_linear(N.stream(), N.dtype_code(x.dtype), xr.data_ptr(), ldx,
                                         norm_w.contiguous().data_ptr(), float(eps), w.data_ptr(),
                                         N.ptr(bias.contiguous() if bias is not None else None), out.data_ptr(), ldy,
                                         m, n_out, w.shape[1], epilogue, N.ptr(aux)), "rmsnorm_linear")
    return out


def add_rmsnorm_linear_parts(x: torch.Tensor, parts: torch.Tensor, norm_w: torch.Tensor, eps: float,
                             w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """One row: x_out = x + (sum of the fp32 partial rows ``parts`` [P, K],
    in row order), each rounded to the dtype (layer.py:63), then
    silu(gate) * up of rmsnorm(x_out) W^T (layer.py:64-67, mlp.py:34-38).
    Returns (x_out [K], y [N])."""
    N.require_gpu(x, parts, norm_w, w, what="add_rmsnorm_linear_parts")
    if parts.dtype != torch.float32 or x.dtype != w.dtype or norm_w.dtype != w.dtype:
        raise TypeError(f"add_rmsnorm_linear_parts: dtypes x={x.dtype} parts={parts.dtype} w={w.dtype}")
    k = x.numel()
    x, parts, w, norm_w = x.contiguous(), parts.contiguous(), w.contiguous(), norm_w.contiguous()
    x_out = torch.empty_like(x)
    y = torch.empty(w.shape[0] // 2, dtype=x.dtype, device=x.device)
    N.check(_lib().minitp_add_rmsnorm_linear_parts(N.stream(), N.dtype_code(x.dtype), x.data_ptr(), parts.data_ptr(),
                                                   parts.shape[0], x_out.data_ptr(), norm_w.data_ptr(), float(eps),
                                                   w.data_ptr(), y.data_ptr(), y.numel(), k, N.EPI_SWIGLU),
            "add_rmsnorm_linear_parts")
    return x_out, y


def rope(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, positions: torch.Tensor):
    """RotaryEmbedding.apply on contiguous [B, H, T, D] q and k."""
    N.require_gpu(q, k, cos, sin, positions, what="rope")
    q, k = q.contiguous(), k.contiguous()
    qo, ko = torch.empty_like(q), torch.empty_like(k)
    b, hq, t, d = q.shape
    N.check(_lib().minitp_rope(N.stream(), N.dtype_code(q.dtype), q.data_ptr(), k.data_ptr(), qo.data_ptr(),
                               ko.data_ptr(), cos.data_ptr(), sin.data_ptr(), positions.contiguous().data_ptr(), b, hq,
                               k.shape[1], t, d), "rope")
    return qo, ko


def cache_rows(k_cache: torch.Tensor, v_cache: torch.Tensor) -> int:
    """Row stride S of [B, Hkv, S, D] cache views whose rows are contiguous
    (a KVCache layer view may show fewer rows than its buffer holds)."""
    for c in (k_cache, v_cache):
        b, h, s, d = c.shape
        if c.stride(3) != 1 or c.stride(2) != d or c.stride(0) != h * c.stride(1) or c.stride(1) % d:
            raise ValueError(f"KV cache view {tuple(c.shape)} with strides {c.stride()} is not a [B, Hkv, S, D] "
                             "layout with contiguous rows")
    if k_cache.stride() != v_cache.stride():
        raise ValueError("K and V caches have different layouts")
    return k_cache.stride(1) // k_cache.shape[3]


def kv_write(k_new: torch.Tensor, v_new: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
             cache_len: int) -> None:
    N.require_gpu(k_new, v_new, k_cache, v_cache, what="KVCache.update")
    k_new, v_new = k_new.contiguous(), v_new.contiguous()
    b, h, t, d = k_new.shape
    if cache_len + t > k_cache.shape[2]:
        raise ValueError(f"KV cache overflow: seq {cache_len}+{t} > max_seq_len={k_cache.shape[2]}")
    N.check(_lib().minitp_kv_write(N.stream(), N.dtype_code(k_cache.dtype), k_new.data_ptr(), v_new.data_ptr(),
                                   k_cache.data_ptr(), v_cache.data_ptr(), b, h, t, d, cache_rows(k_cache, v_cache),
                                   cache_len),
            "kv_write")


def rope_kv_write(qkv: torch.Tensor, q_out: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                  cos: torch.Tensor, sin: torch.Tensor, positions: torch.Tensor, hq: int, hkv: int, cache_len: int):
    """qkv [B, T, (hq+2hkv)*D] -> rotated q_out [B, T, hq, D]; k, v into caches [B, hkv, S, D]."""
    N.require_gpu(qkv, q_out, k_cache, v_cache, what="rope_kv_write")
    b, t, _ = qkv.shape
    d = q_out.shape[-1]
    N.check(_lib().minitp_rope_kv_write(N.stream(), N.dtype_code(qkv.dtype), qkv.data_ptr(), qkv.stride(1),
                                        q_out.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), cos.data_ptr(),
                                        sin.data_ptr(), positions.contiguous().data_ptr(), cos.shape[0], b, t, hq,
                                        hkv, d, cache_rows(k_cache, v_cache), cache_len), "rope_kv_write")


def attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, cache_len: int) -> torch.Tensor:
    """q [B, T, Hq, D]; caches [B, Hkv, S, D] with cache_len + T rows filled -> [B, T, Hq * D]."""
    N.require_gpu(q, k_cache, v_cache, what="attention")
    q = q.contiguous()
    b, t, hq, d = q.shape
    hkv, s = k_cache.shape[1], cache_rows(k_cache, v_cache)
    out = torch.empty(b, t, hq * d, dtype=q.dtype, device=q.device)
    nbytes = _lib().minitp_attention_workspace_bytes(b, t, hq, hkv, d, s)
    ws = N.scratch(q.device, "attention", nbytes)
    N.check(_lib().minitp_attention(N.stream(), N.dtype_code(q.dtype), q.data_ptr(), k_cache.data_ptr(),
                                    v_cache.data_ptr(), out.data_ptr(), b, t, hq, hkv, d, s, cache_len, ws.data_ptr(),
                                    ws.numel()), "attention")
    return out


def argmax(logits: torch.Tensor) -> torch.Tensor:
    """logits [..., V] -> long [...]; torch.argmax order (first max, NaN wins)."""
    N.require_gpu(logits, what="argmax")
    v = logits.shape[-1]
    x = logits if logits.stride(-1) == 1 and (logits.dim() == 1 or _rows_uniform(logits)) else logits.contiguous()
    rows = _rows(x)
    ld = x.stride(-2) if x.dim() > 1 else v
    out = torch.empty(x.shape[:-1], dtype=torch.long, device=x.device)
    nbytes = _lib().minitp_argmax_workspace_bytes(rows, v)
    ws = N.scratch(x.device, "argmax", nbytes)
    N.check(_lib().minitp_argmax(N.stream(), N.dtype_code(x.dtype), x.data_ptr(), ld, rows, v, out.data_ptr(), 1,
                                 ws.data_ptr(), ws.numel()), "argmax")
    return out


def cast_bf16(x: torch.Tensor) -> torch.Tensor:
    """x.to(torch.bfloat16) for a contiguous fp32 tensor, on the library's
    conversion (round to nearest even)."""
    N.require_gpu(x, what="cast_bf16")
    if x.dtype != torch.float32:
        raise TypeError(f"cast_bf16: expected float32, got {x.dtype}")
    x = x.contiguous()
    out = torch.empty(x.shape, dtype=torch.bfloat16, device=x.device)
    N.check(_lib().minitp_cast_f32_bf16(N.stream(), x.data_ptr(), out.data_ptr(), x.numel()), "cast_f32_bf16")
    return out
