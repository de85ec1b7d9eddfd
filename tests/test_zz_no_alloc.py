"""The allocation-free argmax (minitp_argmax_static) through the C ABI.

It must return what minitp_argmax (workspace form) returns on the same
logits, call after call on the static scratch: here two calls in a row, the
second with a smaller input, each checked against the workspace form and
torch.argmax. Requests beyond the scratch are refused on the host.
"""

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _argmax_workspace(logits: torch.Tensor) -> torch.Tensor:
    from minitp import _native as N

    b, v = logits.shape
    out = torch.full((b,), -7, dtype=torch.long, device=DEV)
    nbytes = N.lib().minitp_argmax_workspace_bytes(b, v)
    ws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=DEV)
    N.check(N.lib().minitp_argmax(N.stream(), N.dtype_code(logits.dtype), logits.data_ptr(), logits.stride(0), b, v,
                                  out.data_ptr(), 1, ws.data_ptr(), ws.numel()), "argmax")
    return out


def _argmax_static(logits: torch.Tensor) -> torch.Tensor:
    from minitp import _native as N

    b, v = logits.shape
    out = torch.full((b,), -7, dtype=torch.long, device=DEV)
    N.check(N.lib().minitp_argmax_static(N.stream(), N.dtype_code(logits.dtype), logits.data_ptr(), logits.stride(0),
                                         b, v, out.data_ptr(), 1), "argmax_static")
    return out


def _logits(b: int, v: int, dtype: torch.dtype, seed: int) -> torch.Tensor:
    g = torch.Generator(device="cpu").manual_seed(seed)
    x = torch.randn(b, v, generator=g)
    # ties across slices (first maximum must win) and a NaN row (NaN wins)
    x[0, 5] = x[0, v - 3] = 50.0
    if b > 2:
        x[2, v // 2] = float("nan")
        x[2, v - 1] = float("nan")
    return x.to(DEV, dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_argmax_static_equals_workspace_form_on_two_calls(dtype):
    first = _logits(37, 151936, dtype, seed=1)
    second = _logits(3, 1000, dtype, seed=2)
    got1 = _argmax_static(first)
    got2 = _argmax_static(second)  # smaller input: fewer partials than the first call left behind
    torch.cuda.synchronize()
    for logits, got in ((first, got1), (second, got2)):
        want = _argmax_workspace(logits)
        assert torch.equal(got, want)
        assert torch.equal(got.cpu(), logits.float().cpu().argmax(dim=-1))
    assert got1[0].item() == 5 and got1[2].item() == first.shape[1] // 2


def test_argmax_static_refuses_requests_beyond_its_scratch():
    from minitp import _native as N

    limit = N.lib().minitp_argmax_static_max_bytes()
    assert limit == 1 << 20
    v = 151936
    rows = limit // (12 * ((v + 4095) // 4096)) + 1  # one row more than fits
    logits = torch.empty(rows, v, dtype=torch.bfloat16, device=DEV)
    out = torch.empty(rows, dtype=torch.long, device=DEV)
    rc = N.lib().minitp_argmax_static(N.stream(), N.BF16, logits.data_ptr(), v, rows, v, out.data_ptr(), 1)
    assert rc == N.ERR_ARG and "static scratch" in N.last_error()
