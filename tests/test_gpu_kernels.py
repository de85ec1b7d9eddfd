"""HIP kernels vs the CPU oracle / torch fp32 references, one op at a time.

Tolerances: fp32 results within a few ulps of an fp32 reference that sums in
another order; bf16 results within one bf16 rounding of the reference value.
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _k():
    from minitp import kernels

    return kernels


# ---------------------------------------------------------------------------
# synthetic generator: GPU bits == CPU spec bits


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("stream_id", [1, 16, 211])
def test_fill_normal_bitwise_equals_cpu_spec(dtype, stream_id):
    from oracle import synth

    n = 1_000_003
    t = torch.empty(n, dtype=dtype, device=DEV)
    _k().fill_normal_(t, seed=0, stream_id=stream_id, std=0.02)
    ref = torch.from_numpy(synth.normal_f32_c(0, stream_id, n, 0.02)).to(dtype)
    got = t.cpu()
    assert torch.equal(got.view(torch.int16 if dtype == torch.bfloat16 else torch.int32),
                       ref.view(torch.int16 if dtype == torch.bfloat16 else torch.int32))


def test_fill_normal_matches_numpy_statement_of_spec():
    from oracle import synth

    t = torch.empty(20_000, dtype=torch.float32, device=DEV)
    _k().fill_normal_(t, seed=5, stream_id=77, std=0.02)
    assert np.array_equal(t.cpu().numpy().view(np.uint32), synth.normal_f32(5, 77, 20_000).view(np.uint32))


def test_uniform_ids_equal_cpu_spec():
    from oracle import synth

    got = _k().uniform_ids(4096, 151936, seed=0, stream_id=3, device=DEV).cpu().numpy()
    assert np.array_equal(got, synth.uniform_ids(0, 3, 4096, 151936))


# ---------------------------------------------------------------------------
# RMSNorm


@pytest.mark.parametrize("hidden", [64, 896, 3584])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_rmsnorm(hidden, dtype):
    from oracle.qwen2_ref import rms_norm

    g = torch.Generator().manual_seed(hidden)
    x = (torch.randn(5, hidden, generator=g) * 3).to(dtype)
    w = (torch.rand(hidden, generator=g) + 0.5).to(dtype)
    ref = rms_norm(x, w, 1e-6)
    got = _k().rmsnorm(x.to(DEV), w.to(DEV), 1e-6).cpu()
    if dtype == torch.float32:
        torch.testing.assert_close(got, ref, atol=1e-6, rtol=1e-5)
    else:  # within one bf16 rounding of the oracle
        torch.testing.assert_close(got.float(), ref.float(), atol=0, rtol=2 ** -7)


def test_rmsnorm_constant_row_closed_form():
    # x = c everywhere: out = c / sqrt(c^2 + eps) * w
    c, eps = 0.75, 1e-6
    x = torch.full((1, 896), c, device=DEV)
    w = torch.full((896,), 2.0, device=DEV)
    got = _k().rmsnorm(x, w, eps).cpu()
    want = torch.full((1, 896), 2.0 * c / math.sqrt(c * c + eps))
    torch.testing.assert_close(got, want, atol=1e-6, rtol=1e-6)


# ---------------------------------------------------------------------------
# linear (GEMV for M <= 4, MFMA GEMM beyond)


def _ref_linear(x, w, b=None):
    return F.linear(x.double(), w.double(), None if b is None else b.double())


@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 8, 16, 32, 33, 130])
@pytest.mark.parametrize("n,k", [(64, 64), (1152, 896), (1000, 64), (896, 4864), (300, 136)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_linear_shapes(m, n, k, dtype):
    g = torch.Generator().manual_seed(m * 1000 + n + k)
    x = torch.randn(m, k, generator=g).to(dtype)
    w = (torch.randn(n, k, generator=g) * 0.02).to(dtype)
    b = (torch.randn(n, generator=g) * 0.02).to(dtype)
    got = _k().linear(x.to(DEV), w.to(DEV), b.to(DEV)).cpu().double()
    ref = _ref_linear(x, w, b)
    scale = (x.double().abs() @ w.double().abs().T).max().item()
    if dtype == torch.float32:
        assert (got - ref).abs().max().item() <= 1e-5 * scale + 1e-7
    else:
        assert ((got - ref).abs() <= ref.abs() * 2 ** -8 + 1e-3 * scale).all()


@pytest.mark.parametrize("m", [1, 3, 19, 32, 40])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_linear_residual_epilogue(m, dtype):
    from minitp import _native as N

    g = torch.Generator().manual_seed(m)
    x = torch.randn(m, 896, generator=g).to(dtype)
    w = (torch.randn(896, 896, generator=g) * 0.02).to(dtype)
    r = torch.randn(m, 896, generator=g).to(dtype)
    y = r.clone().to(DEV)
    _k().linear(x.to(DEV), w.to(DEV), out=y, epilogue=N.EPI_RESID, aux=y)
    # reference: r + dtype(x W^T), each add rounded to the dtype (layer.py:63-64)
    lin = _k().linear(x.to(DEV), w.to(DEV)).cpu()
    torch.testing.assert_close(y.cpu(), (r.float() + lin.float()).to(dtype), atol=0, rtol=0)


@pytest.mark.parametrize("m", [1, 2, 4, 7, 32])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_linear_swiglu_epilogue_equals_split(m, dtype):
    from minitp import _native as N

    if dtype == torch.float32 and m >= 4:
        pytest.skip("fp32 rows of K=896 take the GEMV register path only up to M=2; SWIGLU is GEMV-only")
    g = torch.Generator().manual_seed(7 + m)
    inter, k = 256, 896
    x = torch.randn(m, k, generator=g).to(dtype).to(DEV)
    w = (torch.randn(2 * inter, k, generator=g) * 0.05).to(dtype).to(DEV)
    fused = _k().linear(x, w, epilogue=N.EPI_SWIGLU)
    y = _k().linear(x, w)
    split = _k().silu_mul(y[:, :inter], y[:, inter:])
    assert torch.equal(fused, split)
    ref = (F.silu(y[:, :inter].cpu().float()).to(dtype).float() * y[:, inter:].cpu().float()).to(dtype)
    torch.testing.assert_close(split.cpu().float(), ref.float(), atol=1e-6, rtol=2 ** -7)


@pytest.mark.parametrize("m,k", [(1, 896), (2, 896), (4, 896), (1, 4864), (2, 4864), (7, 896), (32, 896), (32, 1024)])
@pytest.mark.parametrize("epilogue", ["none", "bias", "swiglu", "resid"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_rmsnorm_linear_matches_two_step_reference(m, k, epilogue, dtype):
    """The fused norm + GEMV against float64 linear of the dtype-rounded norm
    output (layer.py:39-42 then linear.py:57-58)."""
    from minitp import _native as N

    if dtype == torch.float32 and (m >= 4 or k == 4864) and m > 1:
        pytest.skip("fp32 rows this long take the register GEMV path only for fewer rows")
    g = torch.Generator().manual_seed(m * 31 + k + len(epilogue))
    n = 512
    eps = 1e-6
    x = torch.randn(m, k, generator=g).to(dtype)
    nw = (1 + 0.1 * torch.randn(k, generator=g)).to(dtype)
    w = (torch.randn(2 * n if epilogue == "swiglu" else n, k, generator=g) * 0.02).to(dtype)
    b = (torch.randn(n, generator=g) * 0.02).to(dtype) if epilogue == "bias" else None
    r = torch.randn(m, n, generator=g).to(dtype)
    xn = (x.float() * torch.rsqrt(x.float().pow(2).mean(-1, keepdim=True) + eps) * nw.float()).to(dtype)
    lin = xn.double() @ w.double().T
    if b is not None:
        lin = lin + b.double()
    epi = {"none": N.EPI_NONE, "bias": N.EPI_NONE, "swiglu": N.EPI_SWIGLU, "resid": N.EPI_RESID}[epilogue]
    kw = {}
    if epilogue == "resid":
        kw = {"out": r.clone().to(DEV), "aux": r.clone().to(DEV)}
    got = _k().rmsnorm_linear(x.to(DEV), nw.to(DEV), eps, w.to(DEV), None if b is None else b.to(DEV),
                              epilogue=epi, **kw).cpu().double()
    if epilogue == "swiglu":
        gate, up = lin[:, :n].to(dtype).double(), lin[:, n:].to(dtype).double()
        ref = (F.silu(gate.float()).to(dtype).double() * up)
        scale = (xn.double().abs() @ w.double().abs().T).max().item()
        tol = ref.abs() * 2 ** -7 + 2e-3 * scale if dtype == torch.bfloat16 else ref.abs() * 1e-5 + 1e-5 * scale
    elif epilogue == "resid":
        ref = r.double() + lin
        scale = (xn.double().abs() @ w.double().abs().T).max().item() + r.double().abs().max().item()
        tol = ref.abs() * 2 ** -7 + 2e-3 * scale if dtype == torch.bfloat16 else ref.abs() * 1e-6 + 1e-5 * scale
    else:
        ref = lin
        scale = (xn.double().abs() @ w.double().abs().T).max().item()
        tol = ref.abs() * 2 ** -8 + 2e-3 * scale if dtype == torch.bfloat16 else ref.abs() * 1e-6 + 1e-5 * scale
    assert ((got - ref).abs() <= tol).all(), (got - ref).abs().max().item()


@pytest.mark.parametrize("m,n,k,epilogue", [(32, 4864, 896, "swiglu"), (5, 4104, 896, "swiglu"), (17, 8272, 1024, "none"),
                                             (32, 151936, 896, "none"), (9, 9000, 136, "none"), (32, 8200, 896, "resid"),
                                             (13, 8232, 896, "bias")])
@pytest.mark.parametrize("norm", [True, False])
def test_mfma_gemv_many_tuples_equals_column_blocks(m, n, k, epilogue, norm):
    """Products with 512 or more 16-row tuples run the tuple-loop MFMA form
    (each block normalizes the input rows once for several tuples); the same
    product cut into column blocks of under 512 tuples runs one tuple per
    block. Every output is the same fixed-order sum, so the two agree
    bitwise; the float64 check bounds both."""
    from minitp import _native as N

    g = torch.Generator().manual_seed(m + n + k)
    eps = 1e-6
    x = torch.randn(m, k, generator=g).to(torch.bfloat16).to(DEV)
    nw = (1 + 0.1 * torch.randn(k, generator=g)).to(torch.bfloat16).to(DEV)
    w = (torch.randn(2 * n if epilogue == "swiglu" else n, k, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    r = torch.randn(m, n, generator=g).to(torch.bfloat16).to(DEV)
    b = (torch.randn(n, generator=g) * 0.02).to(torch.bfloat16).to(DEV) if epilogue == "bias" else None
    epi = {"none": N.EPI_NONE, "bias": N.EPI_NONE, "swiglu": N.EPI_SWIGLU, "resid": N.EPI_RESID}[epilogue]

    def run(wb, rb, bb):
        kw = {"out": rb.clone(), "aux": rb.clone()} if epilogue == "resid" else {}
        if norm:
            return _k().rmsnorm_linear(x, nw, eps, wb, bb, epilogue=epi, **kw)
        return _k().linear(x, wb, bb, epilogue=epi, **kw)

    whole = run(w, r, b)
    step = 4096 if epilogue != "swiglu" else 2048  # under 512 tuples a block of columns
    parts = []
    for c0 in range(0, n, step):
        c1 = min(n, c0 + step)
        wb = torch.cat([w[c0:c1], w[n + c0:n + c1]]) if epilogue == "swiglu" else w[c0:c1]
        parts.append(run(wb.contiguous(), r[:, c0:c1].contiguous(), None if b is None else b[c0:c1].contiguous()))
    assert torch.equal(whole, torch.cat(parts, dim=1))
    # and against float64
    xf = x.cpu().float()
    xn = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps) * nw.cpu().float()).to(torch.bfloat16) if norm \
        else x.cpu()
    lin = xn.double() @ w.cpu().double().T
    if b is not None:
        lin = lin + b.cpu().double()
    scale = (xn.double().abs() @ w.cpu().double().abs().T).max().item()
    got = whole.cpu().double()
    if epilogue == "swiglu":
        gate, up = lin[:, :n].to(torch.bfloat16).double(), lin[:, n:].to(torch.bfloat16).double()
        ref = F.silu(gate.float()).to(torch.bfloat16).double() * up
        tol = ref.abs() * 2 ** -7 + 2e-3 * scale
    elif epilogue == "resid":
        ref = r.cpu().double() + lin
        tol = ref.abs() * 2 ** -7 + 2e-3 * (scale + r.abs().max().item())
    else:
        ref, tol = lin, lin.abs() * 2 ** -8 + 2e-3 * scale
    assert ((got - ref).abs() <= tol).all(), (got - ref).abs().max().item()


@pytest.mark.parametrize("k,nparts", [(896, 14), (64, 4), (1024, 16), (896, 1), (512, 7)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_add_rmsnorm_linear_parts(k, nparts, dtype):
    """The gate/up prologue that takes o_proj as fp32 partial rows: x_out is
    exactly dtype(x + dtype(p0 + p1 + ...)) with the rows added in order in
    fp32 (layer.py:63), and y is bitwise the fused norm + gate/up GEMV run on
    x_out (the same kernel code past the prologue; that GEMV has its float64
    check in test_rmsnorm_linear_matches_two_step_reference)."""
    from minitp import _native as N

    g = torch.Generator().manual_seed(k + nparts)
    n, eps = 768, 1e-6
    x = torch.randn(k, generator=g).to(dtype)
    parts = torch.randn(nparts, k, generator=g) * 0.5
    nw = (1 + 0.1 * torch.randn(k, generator=g)).to(dtype)
    w = (torch.randn(2 * n, k, generator=g) * 0.02).to(dtype)
    s = parts[0].clone()
    for p in range(1, nparts):
        s = s + parts[p]  # fp32, row order
    want_x = (x.float() + s.to(dtype).float()).to(dtype)
    x_out, y = _k().add_rmsnorm_linear_parts(x.to(DEV), parts.to(DEV), nw.to(DEV), eps, w.to(DEV))
    assert torch.equal(x_out.cpu(), want_x)
    y_ref = _k().rmsnorm_linear(want_x.to(DEV).reshape(1, k), nw.to(DEV), eps, w.to(DEV), None,
                                epilogue=N.EPI_SWIGLU)
    assert torch.equal(y.cpu(), y_ref.reshape(-1).cpu())


def test_rmsnorm_linear_refuses_prefill_shapes():
    x = torch.randn(8, 896, device=DEV)
    nw = torch.ones(896, device=DEV)
    w = torch.randn(64, 896, device=DEV)
    with pytest.raises(NotImplementedError, match="decode shape"):
        _k().rmsnorm_linear(x, nw, 1e-6, w)


# ---------------------------------------------------------------------------
# RoPE and KV writes


@pytest.mark.parametrize("t,offset", [(1, 0), (2, 1), (7, 95), (33, 0)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_rope_matches_oracle(t, offset, dtype):
    from minitp.rope import RotaryEmbedding
    from oracle.qwen2_ref import rope_apply, rope_tables

    d = 64
    g = torch.Generator().manual_seed(t + offset)
    q = torch.randn(2, 14, t, d, generator=g).to(dtype)
    k = torch.randn(2, 2, t, d, generator=g).to(dtype)
    pos = torch.arange(offset, offset + t)
    cos, sin = rope_tables(d, 1e6, 256)
    rq, rk = rope_apply(cos, sin, q, k, pos)
    rot = RotaryEmbedding(d, 1e6, 256, torch.device(DEV))
    assert torch.equal(rot.cos_cache.cpu(), cos) and torch.equal(rot.sin_cache.cpu(), sin)
    gq, gk = rot.apply(q.to(DEV), k.to(DEV), pos.to(DEV))
    assert torch.equal(gq.cpu(), rq) and torch.equal(gk.cpu(), rk)


def test_rope_kv_write_layout_and_values():
    from oracle.qwen2_ref import rope_apply, rope_tables

    b, t, hq, hkv, d, s, cache_len = 2, 5, 4, 2, 16, 12, 3
    g = torch.Generator().manual_seed(3)
    qkv = torch.randn(b, t, (hq + 2 * hkv) * d, generator=g)
    cos, sin = rope_tables(d, 1e6, 64)
    pos = torch.arange(cache_len, cache_len + t)
    kc = torch.full((b, hkv, s, d), float("nan"), device=DEV)
    vc = kc.clone()
    q = torch.empty(b, t, hq, d, device=DEV)
    _k().rope_kv_write(qkv.to(DEV), q, kc, vc, cos.to(DEV), sin.to(DEV), pos.to(DEV), hq, hkv, cache_len)
    qv, kv, vv = torch.split(qkv, [hq * d, hkv * d, hkv * d], dim=-1)
    rq, rk = rope_apply(cos, sin, qv.view(b, t, hq, d).transpose(1, 2), kv.view(b, t, hkv, d).transpose(1, 2), pos)
    assert torch.equal(q.cpu(), rq.transpose(1, 2))
    assert torch.equal(kc.cpu()[:, :, cache_len:cache_len + t], rk)
    assert torch.equal(vc.cpu()[:, :, cache_len:cache_len + t], vv.view(b, t, hkv, d).transpose(1, 2))
    assert torch.isnan(kc.cpu()[:, :, :cache_len]).all() and torch.isnan(kc.cpu()[:, :, cache_len + t:]).all()


def test_kv_write_overflow_raises():
    kc = torch.zeros(1, 2, 4, 16, device=DEV)
    new = torch.ones(1, 2, 3, 16, device=DEV)
    with pytest.raises(ValueError, match="overflow"):
        _k().kv_write(new, new, kc, kc.clone(), cache_len=2)


# ---------------------------------------------------------------------------
# attention


def _ref_attention(q, kc, vc, cache_len):
    """attention.py:77-103 semantics on the CPU in fp64: q [B,T,Hq,D]."""
    b, t, hq, d = q.shape
    hkv = kc.shape[1]
    total = cache_len + t
    k = kc[:, :, :total].double().repeat_interleave(hq // hkv, dim=1)
    v = vc[:, :, :total].double().repeat_interleave(hq // hkv, dim=1)
    qq = q.double().transpose(1, 2)
    mask = torch.ones(t, total, dtype=torch.bool).tril(diagonal=cache_len)
    out = F.scaled_dot_product_attention(qq, k, v, attn_mask=mask)
    return out.transpose(1, 2).reshape(b, t, hq * d)


@pytest.mark.parametrize("ctx", [1, 7, 256, 257, 600, 2560])
@pytest.mark.parametrize("hq,hkv,d", [(14, 2, 64), (28, 4, 128), (4, 2, 16), (8, 8, 32)])
def test_decode_attention_fp32(ctx, hq, hkv, d):
    b, s = 2, ctx + 3
    g = torch.Generator().manual_seed(ctx + hq)
    q = torch.randn(b, 1, hq, d, generator=g)
    kc = torch.randn(b, hkv, s, d, generator=g)
    vc = torch.randn(b, hkv, s, d, generator=g)
    got = _k().attention(q.to(DEV), kc.to(DEV), vc.to(DEV), cache_len=ctx - 1).cpu()
    ref = _ref_attention(q, kc, vc, ctx - 1)
    assert (got.double() - ref).abs().max().item() < 2e-5


@pytest.mark.parametrize("ctx", [1, 5, 16, 17, 130, 384, 513, 767, 2304])
@pytest.mark.parametrize("b,hq,hkv,d", [(3, 14, 2, 64), (1, 28, 4, 128), (2, 8, 8, 64), (1, 4, 2, 16)])
def test_decode_attention_bf16(ctx, b, hq, hkv, d):
    """bf16 decode (fp32 scores, softmax and P V; the output rounded to bf16
    once): within one bf16 rounding of a float64 reference on the same bf16
    inputs, at short and split contexts, with the cache rows past the
    context poisoned."""
    g = torch.Generator().manual_seed(ctx * 31 + d)
    q = torch.randn(b, 1, hq, d, generator=g).bfloat16()
    kc = torch.randn(b, hkv, ctx + 2, d, generator=g).bfloat16()
    kc[:, :, ctx:] = float("nan")  # rows past the context must not be read
    vc = torch.randn(b, hkv, ctx + 2, d, generator=g).bfloat16()
    vc[:, :, ctx:] = float("nan")
    got = _k().attention(q.to(DEV), kc.to(DEV), vc.to(DEV), cache_len=ctx - 1).cpu().double()
    ref = _ref_attention(q, kc, vc, ctx - 1)
    assert ((got - ref).abs() <= ref.abs() * 2 ** -8 + 1e-6).all(), (got - ref).abs().max().item()


@pytest.mark.parametrize("ctx", [1, 5, 31, 32, 33, 130, 767, 2304, 2559])
@pytest.mark.parametrize("b,hq,hkv,d", [(32, 14, 2, 64), (16, 28, 4, 128), (64, 16, 2, 64)])
def test_decode_attention_bf16_grouped_mfma(ctx, b, hq, hkv, d):
    """The grouped MFMA form (bf16, batch rows x KV heads >= 64): P is
    rounded to bf16 (unit roundoff 2^-8) for its product with V, so the bar
    adds 2^-8 of the attention-weighted mean of |V| (the bound of that
    rounding) to the output rounding's |ref| 2^-8; cache rows past the
    context poisoned. (A float64 emulation of exactly these two roundings
    reaches 0.0079 at context 5 for the first shape, inside this bar and
    outside a 2^-9 one.)"""
    g = torch.Generator().manual_seed(ctx * 17 + d + b)
    q = torch.randn(b, 1, hq, d, generator=g).bfloat16()
    kc = torch.randn(b, hkv, ctx + 2, d, generator=g).bfloat16()
    kc[:, :, ctx:] = float("nan")
    vc = torch.randn(b, hkv, ctx + 2, d, generator=g).bfloat16()
    vc[:, :, ctx:] = float("nan")
    got = _k().attention(q.to(DEV), kc.to(DEV), vc.to(DEV), cache_len=ctx - 1).cpu().double()
    ref = _ref_attention(q, kc, vc, ctx - 1)
    vabs = vc.abs()
    vabs[:, :, ctx:] = 0
    ref_abs = _ref_attention(q, kc, vabs, ctx - 1)
    err = (got - ref).abs()
    assert torch.isfinite(got).all()
    assert (err <= (ref.abs() + ref_abs) * 2 ** -8 + 1e-6).all(), err.max().item()


@pytest.mark.parametrize("ctx,b,hq,hkv,d", [(16384, 1, 14, 2, 64), (32768, 1, 14, 2, 64), (32768, 1, 28, 4, 128),
                                            (8192, 16, 14, 2, 64)])
def test_decode_attention_bf16_long_context(ctx, b, hq, hkv, d):
    """Decode at contexts up to the 0.5B / 7B RoPE table's 32,768 positions
    (the most splits and the longest per-split spans; batch 16 x 2 KV heads on
    the grouped MFMA form), against float64, cache rows past the context
    poisoned; the bar of the grouped-form test."""
    g = torch.Generator().manual_seed(ctx + b + d)
    q = torch.randn(b, 1, hq, d, generator=g).bfloat16()
    kc = torch.randn(b, hkv, ctx + 2, d, generator=g).bfloat16()
    kc[:, :, ctx:] = float("nan")
    vc = torch.randn(b, hkv, ctx + 2, d, generator=g).bfloat16()
    vc[:, :, ctx:] = float("nan")
    got = _k().attention(q.to(DEV), kc.to(DEV), vc.to(DEV), cache_len=ctx - 1).cpu().double()
    ref = _ref_attention(q, kc, vc, ctx - 1)
    vabs = vc.abs()
    vabs[:, :, ctx:] = 0
    ref_abs = _ref_attention(q, kc, vabs, ctx - 1)
    err = (got - ref).abs()
    assert torch.isfinite(got).all()
    assert (err <= (ref.abs() + ref_abs) * 2 ** -8 + 1e-6).all(), err.max().item()


def test_decode_attention_single_key_returns_v_and_zero_q_averages():
    b, hq, hkv, d, s = 1, 14, 2, 64, 10
    kc = torch.randn(b, hkv, s, d)
    vc = torch.randn(b, hkv, s, d)
    q = torch.randn(b, 1, hq, d)
    out = _k().attention(q.to(DEV), kc.to(DEV), vc.to(DEV), cache_len=0).cpu().view(b, hq, d)
    for h in range(hq):  # ctx == 1: output is V[0] of the head's KV group
        torch.testing.assert_close(out[0, h], vc[0, h // 7, 0], atol=1e-6, rtol=0)
    zero = _k().attention(torch.zeros_like(q).to(DEV), kc.to(DEV), vc.to(DEV), cache_len=s - 1).cpu().view(b, hq, d)
    for h in range(hq):  # q == 0: uniform weights, output is mean(V)
        torch.testing.assert_close(zero[0, h], vc[0, h // 7].mean(0), atol=1e-5, rtol=0)


@pytest.mark.parametrize("t,cache_len", [(2, 0), (8, 0), (65, 0), (128, 0), (6, 5), (70, 33)])
@pytest.mark.parametrize("hq,hkv,d", [(14, 2, 64), (4, 2, 16), (28, 4, 128)])
def test_prefill_attention_causal(t, cache_len, hq, hkv, d):
    b = 2
    s = cache_len + t + 2
    g = torch.Generator().manual_seed(t * 7 + cache_len)
    q = torch.randn(b, t, hq, d, generator=g)
    kc = torch.randn(b, hkv, s, d, generator=g)
    vc = torch.randn(b, hkv, s, d, generator=g)
    got = _k().attention(q.to(DEV), kc.to(DEV), vc.to(DEV), cache_len=cache_len).cpu()
    ref = _ref_attention(q, kc, vc, cache_len)
    assert (got.double() - ref).abs().max().item() < 2e-5


@pytest.mark.parametrize("t,cache_len", [(2, 0), (16, 0), (65, 0), (128, 0), (6, 5), (70, 33), (300, 17)])
@pytest.mark.parametrize("hq,hkv,d", [(14, 2, 64), (4, 2, 16), (28, 4, 128), (8, 8, 32)])
def test_prefill_attention_causal_bf16(t, cache_len, hq, hkv, d):
    """bf16 prefill runs on matrix cores with P rounded to bf16 as the MFMA
    operand; against a float64 reference on the same bf16 inputs the output
    (values of order 1) agrees to a few bf16 steps: atol 3e-2."""
    b = 2
    s = cache_len + t + 2
    g = torch.Generator().manual_seed(t * 11 + cache_len + d)
    q = torch.randn(b, t, hq, d, generator=g).bfloat16()
    kc = torch.randn(b, hkv, s, d, generator=g).bfloat16()
    vc = torch.randn(b, hkv, s, d, generator=g).bfloat16()
    got = _k().attention(q.to(DEV), kc.to(DEV), vc.to(DEV), cache_len=cache_len).cpu()
    assert got.dtype == torch.bfloat16
    ref = _ref_attention(q.double(), kc.double(), vc.double(), cache_len)
    assert (got.double() - ref).abs().max().item() < 3e-2


@pytest.mark.parametrize("b,t,cache_len,hq,hkv,d", [(2, 1200, 37, 28, 4, 128), (4, 1200, 100, 14, 2, 64),
                                                    (5, 1100, 0, 12, 3, 128), (4, 1100, 64, 16, 16, 32)])
def test_prefill_attention_causal_bf16_long(b, t, cache_len, hq, hkv, d):
    """Prompts long enough for the long-prompt kernel (128-query blocks of
    two-strip waves, double-buffered K / V tiles), with key offsets that do
    and do not fall on a strip boundary, head counts with and without the
    per-XCD head grouping (B * Hq a multiple of 8 or not), and the rows past
    the keys poisoned; same bar as the short cases."""
    s = cache_len + t + 3
    g = torch.Generator().manual_seed(t + d)
    q = torch.randn(b, t, hq, d, generator=g).bfloat16()
    kc = torch.randn(b, hkv, s, d, generator=g).bfloat16()
    vc = torch.randn(b, hkv, s, d, generator=g).bfloat16()
    kc[:, :, cache_len + t:] = float("nan")
    vc[:, :, cache_len + t:] = float("nan")
    got = _k().attention(q.to(DEV), kc.to(DEV), vc.to(DEV), cache_len=cache_len).cpu().double()
    ref = _ref_attention(q.double(), kc.double(), vc.double(), cache_len)
    assert (got - ref).abs().max().item() < 3e-2


# ---------------------------------------------------------------------------
# argmax (torch.argmax order: first maximum, NaN wins)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("v", [8, 1000, 1001, 151936, 200000])  # 1001: rows off 16-byte alignment
def test_argmax_matches_torch(dtype, v):
    g = torch.Generator().manual_seed(v)
    x = torch.randn(5, v, generator=g).to(dtype)
    x[0, v - 1] = x[0].max() + 1  # unique max in the last element of a 16-byte-aligned row (the tail vector)
    x[1, v // 3] = x[1].max() + 1  # unique max
    x[2, 3] = x[2, v - 1] = x[2].max() + 1  # tie -> smaller id
    x[3] = -x[3].abs() - 1  # all negative
    got = _k().argmax(x.to(DEV)).cpu()
    assert torch.equal(got, x.argmax(dim=-1))


def test_argmax_reference_known_answers():
    # test_vocab_layers.py:134-162: {2,5} tie -> 2; ids 12095/50000/150000; tie 4242 vs 150000 -> 4242
    x = torch.zeros(1, 8)
    x[0, 5] = x[0, 2] = 2.0
    assert _k().argmax(x.to(DEV)).item() == 2
    for vid in (12095, 50000, 150000):
        x = torch.zeros(1, 200000)
        x[0, vid] = 3.5
        assert _k().argmax(x.to(DEV)).item() == vid
    x = torch.zeros(1, 200000)
    x[0, 150000] = x[0, 4242] = 1.0
    assert _k().argmax(x.to(DEV)).item() == 4242


def test_argmax_nan_wins_like_torch():
    x = torch.randn(3, 5000)
    x[0, 4000] = float("nan")
    x[1, 10] = float("nan")
    x[1, 20] = float("nan")
    x[2, 7] = float("inf")
    got = _k().argmax(x.to(DEV)).cpu()
    assert torch.equal(got, x.argmax(dim=-1)), (got, x.argmax(dim=-1))


def test_embedding_gathers_rows():
    table = torch.randn(1000, 64)
    ids = torch.tensor([[0, 999, 17], [5, 5, 3]])
    got = _k().embedding(ids.to(DEV), table.to(DEV)).cpu()
    assert torch.equal(got, F.embedding(ids, table))


# ---------------------------------------------------------------------------
# fp32 -> bf16 rounding (the conversion every bf16 kernel uses)


def test_bf16_rounding_matches_torch_bitwise():
    """Every exponent, both signs, halfway and odd/even ties, subnormals, inf
    and NaN: bit-identical to torch's CPU Tensor.to(torch.bfloat16), NaN
    staying NaN."""
    g = torch.Generator().manual_seed(3)
    bits = torch.randint(-(2**31), 2**31, (1 << 24,), generator=g, dtype=torch.int64)
    halves = (torch.arange(0, 1 << 16, dtype=torch.int64) << 16) | 0x8000  # exact ties
    odd = halves + 0x10000
    special = torch.tensor([0, 0x80000000, 0x7F800000, 0xFF800000, 0x00000001, 0x007FFFFF, 0x7F7FFFFF,
                            0x7F7F8000, 0x3F808000, 0x3F818000, 0x7FC00000, 0x7F800001], dtype=torch.int64)
    u = torch.cat([bits, halves, odd, special]) & 0xFFFFFFFF
    f = (u - ((u >> 31) << 32)).to(torch.int32).view(torch.float32)
    got = _k().cast_bf16(f.to(DEV)).cpu()
    ref = f.to(torch.bfloat16)
    nan = torch.isnan(f)
    assert torch.isnan(got[nan].float()).all()
    assert torch.equal(got[~nan].view(torch.int16), ref[~nan].view(torch.int16))
