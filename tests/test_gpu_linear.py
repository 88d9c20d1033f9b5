"""The few-row projection kernels (csrc/linear.hip) through fused_ops.

  pkv_linear           against the fp32 product of the same bf16 / fp16 /
                       fp32 inputs: within one unit in the last place of the
                       storage type plus the fp32 summation-order slack
                       (4e-6 * sqrt(k) absolute for N(0, 1) inputs); rows
                       1 .. 256, features not a multiple of the 16-wide tile,
                       k from 32 to 4096, strided x rows, bias.
  pkv_linear_swiglu    bit-identical to pkv_linear into [m, 2n] followed by
                       the stand-alone SwiGLU kernel (the same sums).
  pkv_linear_rope_qkv  bit-identical to pkv_linear followed by the
                       stand-alone RoPE kernel on the three column ranges;
                       a position past the tables sets PKV_STATUS_BAD_POS.
  pkv_linear_residual  bit-identical to pkv_linear followed by the
                       framework add (resid + y rounded to the dtype).
  pkv_linear_swiglu_rmsnorm, pkv_linear_rope_qkv_rmsnorm
                       bit-identical to pkv_rms_norm followed by the
                       unfused projection (the prologue sums squares in the
                       stand-alone kernel's order); k above 1024 is refused
                       by the library and composed by the wrappers.
  Determinism          two launches give identical bits.
"""
import math

import pytest
import torch

from serving import _native, fused_ops
from serving.layers import RoPE

pytestmark = pytest.mark.gpu
DEV = "cuda"


def ulp(x: torch.Tensor) -> torch.Tensor:
    mant = {torch.bfloat16: 7, torch.float16: 10, torch.float32: 23}[x.dtype]
    xf = x.float().abs().clamp_min(torch.finfo(x.dtype).tiny)
    return torch.exp2(torch.floor(torch.log2(xf)) - mant)


def rand(shape, dtype, seed, scale=1.0):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return (scale * torch.randn(shape, generator=g, device=DEV)).to(dtype)


def check_linear(y, x, w, b):
    ref = x.float() @ w.float().t()
    if b is not None:
        ref = ref + b.float()
    slack = 4e-6 * math.sqrt(x.shape[-1]) * max(1.0, float(x.float().abs().max()))
    err = (y.float() - ref).abs()
    lim = ulp(ref.to(y.dtype)) * 1.0001 + slack
    assert bool((err <= lim).all()), f"max err {float(err.max()):.3e}"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("m,n,k,bias,strided", [
    (128, 1024, 1024, False, False),
    (128, 1152, 1024, True, False),
    (1, 64, 32, False, False),
    (17, 1000, 96, True, True),
    (256, 48, 4096, False, False),
    (5, 3, 1024, True, False),
    (200, 2048, 544, False, True),
    (64, 4200, 64, True, False),   # two 16-feature tiles per workgroup, a partial last one
    (16, 64, 256, False, False),   # one K step per wavefront: the skipped steps add nothing
    (9, 48, 768, True, False),     # three K steps per wavefront
])
def test_linear_vs_fp32_product(dtype, m, n, k, bias, strided):
    print(f"[linear] {dtype} m={m} n={n} k={k} bias={bias} strided={strided}", flush=True)
    base = rand((m, k + (64 if strided else 0)), dtype, m + n)
    x = base[:, 32:32 + k] if strided else base
    w = rand((n, k), dtype, k, scale=0.05)
    b = rand((n,), dtype, 3) if bias else None
    y = fused_ops.linear(x, w, b)
    torch.cuda.synchronize()
    assert y.shape == (m, n)
    check_linear(y, x, w, b)
    y2 = fused_ops.linear(x, w, b)
    assert torch.equal(y, y2), "not deterministic"


def test_linear_routes_unsupported_shapes_to_library_gemm():
    x = rand((300, 64), torch.bfloat16, 1)   # more rows than the kernel takes
    w = rand((64, 64), torch.bfloat16, 2)
    torch.testing.assert_close(fused_ops.linear(x, w), torch.nn.functional.linear(x, w))
    x = rand((4, 40), torch.bfloat16, 3)     # k not a multiple of 32
    w = rand((8, 40), torch.bfloat16, 4)
    torch.testing.assert_close(fused_ops.linear(x, w), torch.nn.functional.linear(x, w))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("m,h,k,bias", [(128, 1024, 1024, False), (7, 100, 64, True),
                                        (33, 2816, 1024, False)])
def test_linear_swiglu_equals_linear_then_gate(dtype, m, h, k, bias):
    x = rand((m, k), dtype, 11)
    w = rand((2 * h, k), dtype, 12, scale=0.1)
    b = rand((2 * h,), dtype, 13) if bias else None
    got = fused_ops.linear_swiglu(x, w, b)
    gu = torch.empty((m, 2 * h), dtype=dtype, device=DEV)
    rc = _native.lib().pkv_linear(gu.data_ptr(), x.data_ptr(), w.data_ptr(), _native.ptr(b), m,
                                  2 * h, k, k, _native.dtype_code(dtype),
                                  _native.stream_ptr(x.device))
    assert rc == 0
    expect = fused_ops.silu_mul(gu[:, :h], gu[:, h:])
    torch.cuda.synchronize()
    bad = (got != expect).nonzero()
    if len(bad):
        i, j = (int(v) for v in bad[0])
        g, u = gu[i, j].item(), gu[i, h + j].item()
        raise AssertionError(f"{len(bad)} of {got.numel()} differ; first at {(i, j)}: "
                             f"gate {g!r} up {u!r} fused {got[i, j].item()!r} "
                             f"two-step {expect[i, j].item()!r}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("m,hq,hkv,d,k,bias", [(128, 16, 1, 64, 1024, False),
                                               (9, 32, 2, 128, 512, True),
                                               (40, 4, 1, 6, 64, False)])
def test_linear_rope_qkv_equals_linear_then_rope(dtype, m, hq, hkv, d, k, bias):
    print(f"[linear_rope] {dtype} m={m} hq={hq} hkv={hkv} d={d}", flush=True)
    n = (hq + 2 * hkv) * d
    x = rand((m, k), dtype, 21)
    w = rand((n, k), dtype, 22, scale=0.1)
    b = rand((n,), dtype, 23) if bias else None
    rope = RoPE(d, max_seq_len=4096).to(DEV)
    cos, sin = rope._tables_fp32()
    pos = torch.randint(0, 4096, (m,), device=DEV, dtype=torch.int32)
    q, kk, v = fused_ops.linear_rope_qkv(x, w, b, pos, cos, sin, hq, hkv, d)
    qkv = torch.empty((m, n), dtype=dtype, device=DEV)
    rc = _native.lib().pkv_linear(qkv.data_ptr(), x.data_ptr(), w.data_ptr(), _native.ptr(b), m,
                                  n, k, k, _native.dtype_code(dtype),
                                  _native.stream_ptr(x.device))
    assert rc == 0
    eq, ek, ev = fused_ops.rope(qkv[:, :hq * d], qkv[:, hq * d:(hq + hkv) * d], pos, cos, sin,
                                v=qkv[:, (hq + hkv) * d:], hq=hq, hkv=hkv, d=d)
    torch.cuda.synchronize()
    assert torch.equal(q, eq) and torch.equal(kk, ek) and torch.equal(v, ev)


def test_linear_rope_position_past_table_flags_status():
    hq, hkv, d, k, m = 4, 1, 32, 64, 3
    x = rand((m, k), torch.bfloat16, 31)
    w = rand(((hq + 2 * hkv) * d, k), torch.bfloat16, 32)
    rope = RoPE(d, max_seq_len=8).to(DEV)
    cos, sin = rope._tables_fp32()
    pos = torch.tensor([1, 8, 7], dtype=torch.int32, device=DEV)
    outs = [torch.empty((m, h, d), dtype=torch.bfloat16, device=DEV) for h in (hq, hkv, hkv)]
    status = torch.zeros(1, dtype=torch.int32, device=DEV)
    rc = _native.lib().pkv_linear_rope_qkv(
        outs[0].data_ptr(), outs[1].data_ptr(), outs[2].data_ptr(), x.data_ptr(), w.data_ptr(),
        None, m, k, k, pos.data_ptr(), cos.data_ptr(), sin.data_ptr(), 8, hq, hkv, d,
        _native.dtype_code(torch.bfloat16), status.data_ptr(), _native.stream_ptr(x.device))
    assert rc == 0
    torch.cuda.synchronize()
    assert int(status.item()) == _native.PKV_STATUS_BAD_POS


def _first_diff(got, expect):
    bad = (got != expect).nonzero()
    if not len(bad):
        return None
    idx = tuple(int(v) for v in bad[0])
    return (f"{len(bad)} of {got.numel()} differ; first at {idx}: fused {got[idx].item()!r} "
            f"two-step {expect[idx].item()!r}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("m,n,k,bias,strided", [(128, 1024, 1024, False, False),
                                                (1, 64, 32, True, False),
                                                (17, 1000, 2816, False, True),
                                                (256, 48, 96, True, False),
                                                (96, 3000, 64, True, False)])
def test_linear_residual_equals_linear_then_add(dtype, m, n, k, bias, strided):
    print(f"[linear_residual] {dtype} m={m} n={n} k={k} bias={bias}", flush=True)
    base = rand((m, k + (64 if strided else 0)), dtype, 41)
    x = base[:, 32:32 + k] if strided else base
    w = rand((n, k), dtype, 42, scale=0.05)
    b = rand((n,), dtype, 43) if bias else None
    resid = rand((m, n), dtype, 44, scale=4.0)
    expect = resid + fused_ops.linear(x, w, b)
    got = resid.clone()
    out = fused_ops.linear_residual_(got, x, w, b)
    torch.cuda.synchronize()
    assert out is got
    msg = _first_diff(got, expect)
    assert msg is None, msg


def _norm_inputs(dtype, m, k, seed, strided):
    base = rand((m, k + (64 if strided else 0)), dtype, seed, scale=3.0)
    x = base[:, 32:32 + k] if strided else base
    g = torch.Generator(device=DEV).manual_seed(seed + 1)
    nw = (1.0 + 0.2 * torch.randn(k, generator=g, device=DEV)).to(dtype)
    return x, nw


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("m,h,k,bias,strided", [(128, 2816, 1024, False, False),
                                                (1, 100, 32, True, False),
                                                (7, 256, 96, False, True),
                                                (64, 512, 640, True, False)])
def test_linear_swiglu_rmsnorm_equals_norm_then_projection(dtype, m, h, k, bias, strided):
    print(f"[linear_swiglu_rmsnorm] {dtype} m={m} h={h} k={k}", flush=True)
    x, nw = _norm_inputs(dtype, m, k, 51, strided)
    w = rand((2 * h, k), dtype, 52, scale=0.1)
    b = rand((2 * h,), dtype, 53) if bias else None
    got = fused_ops.linear_swiglu_rmsnorm(x, nw, 1e-5, w, b)
    expect = fused_ops.linear_swiglu(fused_ops.rms_norm(x, nw, 1e-5), w, b)
    torch.cuda.synchronize()
    msg = _first_diff(got, expect)
    assert msg is None, msg


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("m,hq,hkv,d,k,bias,strided", [(128, 16, 1, 64, 1024, False, False),
                                                       (9, 4, 2, 128, 512, True, True),
                                                       (1, 8, 1, 64, 64, False, False)])
def test_linear_rope_qkv_rmsnorm_equals_norm_then_projection(dtype, m, hq, hkv, d, k, bias,
                                                             strided):
    print(f"[linear_rope_qkv_rmsnorm] {dtype} m={m} hq={hq} hkv={hkv} d={d} k={k}", flush=True)
    n = (hq + 2 * hkv) * d
    x, nw = _norm_inputs(dtype, m, k, 61, strided)
    w = rand((n, k), dtype, 62, scale=0.1)
    b = rand((n,), dtype, 63) if bias else None
    rope = RoPE(d, max_seq_len=4096).to(DEV)
    cos, sin = rope._tables_fp32()
    pos = torch.randint(0, 4096, (m,), device=DEV, dtype=torch.int32)
    got = fused_ops.linear_rope_qkv_rmsnorm(x, nw, 1e-6, w, b, pos, cos, sin, hq, hkv, d)
    expect = fused_ops.linear_rope_qkv(fused_ops.rms_norm(x, nw, 1e-6), w, b, pos, cos, sin,
                                       hq, hkv, d)
    torch.cuda.synchronize()
    for g_, e_ in zip(got, expect):
        msg = _first_diff(g_, e_)
        assert msg is None, msg


def test_fused_norm_past_1024_features_refused_then_composed():
    m, h, k = 4, 64, 1056
    x, nw = _norm_inputs(torch.bfloat16, m, k, 71, False)
    w = rand((2 * h, k), torch.bfloat16, 72, scale=0.1)
    out = torch.empty((m, h), dtype=torch.bfloat16, device=DEV)
    rc = _native.lib().pkv_linear_swiglu_rmsnorm(
        out.data_ptr(), x.data_ptr(), nw.data_ptr(), 1e-5, w.data_ptr(), None, m, h, k, k,
        _native.dtype_code(torch.bfloat16), _native.stream_ptr(x.device))
    assert rc == _native.PKV_ERR_UNSUPPORTED
    got = fused_ops.linear_swiglu_rmsnorm(x, nw, 1e-5, w, None)
    expect = fused_ops.linear_swiglu(fused_ops.rms_norm(x, nw, 1e-5), w, None)
    torch.cuda.synchronize()
    assert torch.equal(got, expect)
