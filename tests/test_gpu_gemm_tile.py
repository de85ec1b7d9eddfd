"""The 256 x 256 MFMA tile GEMM that serves bf16 prompt products (F.linear,
fused.py:57-61, linear.py:117; gate/up + SwiGLU, mlp.py:34-38), through the
C ABI (minitp_linear).

Bars: each output within half a bf16 ulp of the float64 product plus the
fp32 accumulation error (|ref| 2^-8 + 1e-3 * sum |x||w|); the SwiGLU
epilogue bitwise equal to the unfused product followed by minitp_silu_mul
(the same fixed-order sums, the same rounding points); results identical
from run to run. Shapes cover ragged M and N (not multiples of 256), K not
a multiple of the 64-wide K step, and the 7B prefill shapes at full size
(against torch's fp32 matmul on the GPU).
"""

import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _k():
    from minitp import kernels

    return kernels


def _served(m, n, k, swiglu=False):
    import math

    tiles = math.ceil(m / 256) * math.ceil(n / (128 if swiglu else 256))
    return m >= 256 and tiles >= 96


def _operands(m, n, k, seed, w_rows=None):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    w = (torch.randn(w_rows or n, k, generator=g) * 0.02).to(torch.bfloat16)
    b = (torch.randn(n, generator=g) * 0.02).to(torch.bfloat16)
    return x, w, b


@pytest.mark.parametrize("m,n,k", [(2000, 3000, 904), (4111, 1536, 896), (2304, 4608, 3584), (300, 24832, 136)])
@pytest.mark.parametrize("with_bias", [False, True])
def test_tile_gemm_against_float64(m, n, k, with_bias):
    assert _served(m, n, k)
    x, w, b = _operands(m, n, k, seed=m + n + k)
    bias = b if with_bias else None
    got = _k().linear(x.to(DEV), w.to(DEV), bias.to(DEV) if with_bias else None)
    again = _k().linear(x.to(DEV), w.to(DEV), bias.to(DEV) if with_bias else None)
    assert torch.equal(got, again), "not deterministic"
    ref = F.linear(x.double(), w.double(), None if bias is None else bias.double())
    scale = x.double().abs() @ w.double().abs().T
    err = (got.cpu().double() - ref).abs()
    bound = ref.abs() * 2 ** -8 + 1e-3 * scale.max().item()
    assert (err <= bound).all(), err.max().item()


@pytest.mark.parametrize("m,inter,k", [(2000, 3000, 904), (1024, 4864, 896), (512, 18944, 3584)])
def test_tile_swiglu_equals_unfused_product_then_silu_mul(m, inter, k):
    from minitp import _native as N

    assert _served(m, inter, k, swiglu=True) and _served(m, 2 * inter, k)
    x, w, _ = _operands(m, inter, k, seed=k + inter, w_rows=2 * inter)
    x, w = x.to(DEV), w.to(DEV)
    fused = _k().linear(x, w, epilogue=N.EPI_SWIGLU)
    y = _k().linear(x, w)
    split = _k().silu_mul(y[:, :inter], y[:, inter:])
    assert fused.shape == (m, inter)
    assert torch.equal(fused, split)
    # and the split form against torch's ops on the same bf16 products
    yc = y.cpu().float()
    ref = (F.silu(yc[:, :inter]).to(torch.bfloat16).float() * yc[:, inter:]).to(torch.bfloat16)
    torch.testing.assert_close(split.cpu().float(), ref.float(), atol=1e-6, rtol=2 ** -7)


@pytest.mark.parametrize("n,k", [(4608, 3584), (3584, 3584), (3584, 18944)])
def test_tile_gemm_7b_prefill_shapes_full_size(n, k):
    """M = 4 x 4096 rows of the 7B prefill: QKV, o_proj and down."""
    m = 16384
    g = torch.Generator(device=DEV).manual_seed(n + k)
    x = torch.randn(m, k, device=DEV, generator=g).to(torch.bfloat16)
    w = (torch.randn(n, k, device=DEV, generator=g) * 0.02).to(torch.bfloat16)
    got = _k().linear(x, w).float()
    ref = x.float() @ w.float().T
    scale = (x.float().abs().amax(dim=1, keepdim=True) * w.float().abs().sum(dim=1)).max().item()
    err = (got - ref).abs()
    assert (err <= ref.abs() * 2 ** -8 + 1e-4 * scale).all(), err.max().item()


def test_tile_swiglu_7b_gate_up_full_size():
    """gate/up + SwiGLU of the 7B prefill (16,384 x 2 x 18,944 x 3,584):
    bitwise the unfused product (checked against torch by the test above)
    followed by minitp_silu_mul."""
    from minitp import _native as N

    m, inter, k = 16384, 18944, 3584
    g = torch.Generator(device=DEV).manual_seed(5)
    x = torch.randn(m, k, device=DEV, generator=g).to(torch.bfloat16)
    w = (torch.randn(2 * inter, k, device=DEV, generator=g) * 0.02).to(torch.bfloat16)
    fused = _k().linear(x, w, epilogue=N.EPI_SWIGLU)
    y = _k().linear(x, w)
    split = _k().silu_mul(y[:, :inter], y[:, inter:])
    assert torch.equal(fused, split)
    assert torch.isfinite(fused).all()
