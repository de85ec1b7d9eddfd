"""Seeded synthetic model and prompt generator: the CPU statement of the spec.

ORACLE / TEST INFRASTRUCTURE ONLY. Nothing in the product package imports
this file; the product generates the same bits on the GPU with the
``minitp_fill_normal`` / ``minitp_fill_uniform_ids`` HIP kernels, and a GPU
test checks the two agree bit for bit.

The reference initialises weights with kaiming-uniform, leaves biases as
uninitialised memory and zeroes the embedding (``minitp/parallel/linear.py:52-56``,
``minitp/parallel/fused.py:48-52``, ``minitp/parallel/embedding.py:38-41``), so a
synthetic model must be generated outside the model and copied in through
``state_dict`` the way ``tests/test_qwen_tiny.py:53-82`` copies HF weights.
The workloads ask for N(0, 0.02) weights and biases, unit RMSNorm weights and
uniform prompt ids. This generator produces them from (seed, stream, index)
alone, with integer hashing plus IEEE-754 double ``+ - * / sqrt`` (each
correctly rounded, no fused multiply-add), so the bits are identical on any
CPU and on the GPU, and multi-GB models never have to be shipped.

Spec
----
``splitmix(key, c) = mix64(key + c * 0x9E3779B97F4A7C15)`` (mod 2**64) with the
splitmix64 finaliser ``mix64``. ``key(seed, stream) = mix64(seed * GAMMA +
stream * 0xD1B54A32D192ED03 + 1)``.

Normal element ``i`` of stream ``s``: for attempt ``j = 0..63`` draw
``h1 = splitmix(key, 2c)``, ``h2 = splitmix(key, 2c + 1)`` with ``c = 64 i + j``;
``X = 2 (h1 >> 11) 2**-53 - 1``, ``Y`` likewise; ``S = X*X + Y*Y``; accept the
first attempt with ``0 < S < 1`` (Marsaglia's polar method) and return
``X * sqrt((-2 ln S) / S)``. ``ln`` is :func:`det_log` below (exponent split
plus an atanh series), so no libm routine is involved. The weight is
``float32(std * z)``; bf16 models round that float32 to nearest-even.

Uniform id element ``i``: ``((splitmix(key, i) >> 32) * V) >> 32``.
"""

from __future__ import annotations

import numpy as np

GAMMA = 0x9E3779B97F4A7C15
STREAM_MUL = 0xD1B54A32D192ED03
MASK64 = (1 << 64) - 1
LN2 = 0.6931471805599453  # 0x1.62e42fefa39efp-1
SQRT2 = 1.4142135623730951  # 0x1.6a09e667f3bcdp+0
MAX_ATTEMPTS = 64
# atanh series coefficients 1/(2k+1), k = 0..11, each an IEEE division
LOG_COEFFS = [1.0 / (2 * k + 1) for k in range(12)]

# stream ids (shared with the HIP generator in mini-tp_amd/csrc)
STREAM_EMBED = 1
STREAM_LM_HEAD = 2
STREAM_PROMPT = 3


def layer_stream(layer: int, which: str) -> int:
    slot = {"qkv_w": 0, "qkv_b": 1, "o_w": 2, "gate_up_w": 3, "down_w": 4}[which]
    return 16 + 8 * layer + slot


def _mix64_int(z: int) -> int:
    z &= MASK64
    z ^= z >> 30
    z = (z * 0xBF58476D1CE4E5B9) & MASK64
    z ^= z >> 27
    z = (z * 0x94D049BB133111EB) & MASK64
    z ^= z >> 31
    return z


def stream_key(seed: int, stream: int) -> int:
    return _mix64_int(seed * GAMMA + stream * STREAM_MUL + 1)


def _mix64(z: np.ndarray) -> np.ndarray:
    z = z ^ (z >> np.uint64(30))
    z = z * np.uint64(0xBF58476D1CE4E5B9)
    z = z ^ (z >> np.uint64(27))
    z = z * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def _splitmix(key: int, ctr: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        return _mix64(np.uint64(key) + ctr * np.uint64(GAMMA))


def det_log(s: np.ndarray) -> np.ndarray:
    """ln(s) for normal positive float64 ``s`` using only exact integer ops and
    correctly rounded + - * /, evaluated in a fixed order."""
    bits = s.view(np.uint64)
    e = ((bits >> np.uint64(52)) & np.uint64(0x7FF)).astype(np.int64) - 1023
    m = ((bits & np.uint64(0x000FFFFFFFFFFFFF)) | np.uint64(0x3FF0000000000000)).view(np.float64)
    big = m > SQRT2
    m = np.where(big, m * 0.5, m)
    e = np.where(big, e + 1, e)
    f = (m - 1.0) / (m + 1.0)
    f2 = f * f
    p = np.full_like(f, LOG_COEFFS[11])
    for k in range(10, -1, -1):
        p = p * f2 + LOG_COEFFS[k]
    return e.astype(np.float64) * LN2 + (2.0 * f) * p


def normal_f64(seed: int, stream: int, start: int, count: int) -> np.ndarray:
    """Standard normals for element indices [start, start + count)."""
    key = stream_key(seed, stream)
    idx = np.arange(start, start + count, dtype=np.uint64)
    out = np.zeros(count, dtype=np.float64)
    pending = np.arange(count)
    for j in range(MAX_ATTEMPTS):
        if pending.size == 0:
            break
        c = idx[pending] * np.uint64(64) + np.uint64(j)
        with np.errstate(over="ignore"):
            h1 = _splitmix(key, c * np.uint64(2))
            h2 = _splitmix(key, c * np.uint64(2) + np.uint64(1))
        x = (h1 >> np.uint64(11)).astype(np.float64) * (2.0 ** -53) * 2.0 - 1.0
        y = (h2 >> np.uint64(11)).astype(np.float64) * (2.0 ** -53) * 2.0 - 1.0
        s = x * x + y * y
        ok = (s > 0.0) & (s < 1.0)
        if ok.any():
            sa = s[ok]
            out[pending[ok]] = x[ok] * np.sqrt((-2.0 * det_log(sa)) / sa)
        pending = pending[~ok]
    return out


def normal_f32(seed: int, stream: int, count: int, std: float = 0.02, chunk: int = 1 << 22) -> np.ndarray:
    """float32(std * z) for elements [0, count) of a stream."""
    out = np.empty(count, dtype=np.float32)
    for s0 in range(0, count, chunk):
        n = min(chunk, count - s0)
        out[s0 : s0 + n] = (std * normal_f64(seed, stream, s0, n)).astype(np.float32)
    return out


def uniform_ids(seed: int, stream: int, count: int, vocab: int) -> np.ndarray:
    """Uniform integers in [0, vocab) as int64."""
    key = stream_key(seed, stream)
    h = _splitmix(key, np.arange(count, dtype=np.uint64))
    return (((h >> np.uint64(32)) * np.uint64(vocab)) >> np.uint64(32)).astype(np.int64)


def bf16_round(x: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 (round to nearest even) -> float32, for finite input."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16)
    return (u << np.uint64(16)).astype(np.uint32).view(np.float32)


# ---------------------------------------------------------------------------
# C statement of the same spec (oracle/csrc/synth.c), for multi-GB models.
_LIB = None


def _clib():
    global _LIB
    if _LIB is None:
        import ctypes
        import os

        path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_build", "libsynth.so")
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} missing: run `make -C oracle`")
        lib = ctypes.CDLL(path)
        u64 = ctypes.c_uint64
        lib.synth_normal_f32.argtypes = [u64, u64, u64, u64, ctypes.c_double, ctypes.c_void_p]
        lib.synth_normal_f32.restype = None
        lib.synth_uniform_ids.argtypes = [u64, u64, u64, u64, ctypes.c_void_p]
        lib.synth_uniform_ids.restype = None
        _LIB = lib
    return _LIB


def normal_f32_c(seed: int, stream: int, count: int, std: float = 0.02, start: int = 0) -> np.ndarray:
    out = np.empty(count, dtype=np.float32)
    _clib().synth_normal_f32(seed, stream, start, count, std, out.ctypes.data)
    return out


def uniform_ids_c(seed: int, stream: int, count: int, vocab: int) -> np.ndarray:
    out = np.empty(count, dtype=np.int64)
    _clib().synth_uniform_ids(seed, stream, count, vocab, out.ctypes.data)
    return out
