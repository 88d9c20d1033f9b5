"""The decoder block's element-wise HIP kernels (csrc/layers.hip, through
serving/fused_ops.py) against the framework formulas they replace.

  RoPE      bit-exact against the reference module's formula evaluated by
            torch on the CPU (models/rope.py:21-47: cos/sin cast to the
            dtype, every product and sum rounded to it), fp32 / bf16 / fp16,
            contiguous and strided (fused-projection) inputs, head dims 32 /
            64 / 128 and an odd pair count (vector and element paths); the
            value rows are copied exactly; a position past the tables sets
            PKV_STATUS_BAD_POS.
  RMSNorm   against the fp32 formula (models/rmsnorm.py:14-17): fp32 within
            1e-5 relative; bf16 / fp16 within one unit in the last place of
            the storage type (the fp32 sum of squares is reduced in another
            order than torch's), and mostly bit-identical. With the fused
            residual, the stored sum x + delta is bit-exact.
  SwiGLU    against g * sigmoid(g) * u in fp32 rounded once
            (kernels/fused_swiglu/kernel.py:17-18): fp32 within 1e-6
            relative, bf16 / fp16 within one unit in the last place.
  Model     the fused forward_step (residual adds inside the norms) gives
            bit-identical logits and pool contents to the per-layer module
            composition (PagedBlock.forward_meta), bf16.
"""
import numpy as np
import pytest
import torch

from serving import _native, fused_ops
from serving.layers import ModelConfig, RoPE
from serving.kv_pool import KVPool
from serving.paged_meta import pack_batch_meta
from serving.paged_model import PagedTransformer
from serving import workloads

pytestmark = pytest.mark.gpu
DEV = "cuda"
DTYPES = [torch.float32, torch.bfloat16, torch.float16]


def ulp(x: torch.Tensor) -> torch.Tensor:
    """One unit in the last place of x's dtype at |x| (fp32 tensor)."""
    mant = {torch.bfloat16: 7, torch.float16: 10, torch.float32: 23}[x.dtype]
    xf = x.float().abs().clamp_min(torch.finfo(x.dtype).tiny)
    return torch.exp2(torch.floor(torch.log2(xf)) - mant)


def within_one_ulp(got, ref):
    diff = (got.float() - ref.float()).abs()
    return bool((diff <= ulp(ref) * 1.0001).all())


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("d,hq,hkv,fused", [(64, 16, 1, True), (128, 32, 2, False),
                                             (32, 4, 1, True), (6, 2, 1, False)])
def test_rope_bit_exact_vs_reference_formula(dtype, d, hq, hkv, fused):
    print(f"[rope] {dtype} d={d} hq={hq} hkv={hkv} fused={fused}", flush=True)
    T = 37
    rope = RoPE(d, max_seq_len=3000)
    g = torch.Generator().manual_seed(d + hq)
    pos = torch.randint(0, 3000, (T,), generator=g)
    if fused:
        qkv = torch.randn(T, (hq + 2 * hkv) * d, generator=g).to(dtype)
        q = qkv[:, :hq * d].view(T, hq, d)
        k = qkv[:, hq * d:(hq + hkv) * d].view(T, hkv, d)
        v = qkv[:, (hq + hkv) * d:].view(T, hkv, d)
    else:
        q = torch.randn(T, hq, d, generator=g).to(dtype)
        k = torch.randn(T, hkv, d, generator=g).to(dtype)
        v = torch.randn(T, hkv, d, generator=g).to(dtype)
    eq, ek = rope.forward_tokens(q, k, pos)  # CPU tensors: the torch formula
    rope_d = rope.to(DEV)
    if fused:
        qkvd = qkv.to(DEV)
        qd = qkvd[:, :hq * d].view(T, hq, d)
        kd = qkvd[:, hq * d:(hq + hkv) * d].view(T, hkv, d)
        vd = qkvd[:, (hq + hkv) * d:].view(T, hkv, d)
    else:
        qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    gq, gk, gv = rope_d.forward_tokens(qd, kd, pos.to(DEV, torch.int32), v=vd)
    torch.cuda.synchronize()
    assert gq.is_contiguous() and gk.is_contiguous() and gv.is_contiguous()
    assert torch.equal(gq.cpu(), eq), "rotated q differs"
    assert torch.equal(gk.cpu(), ek), "rotated k differs"
    assert torch.equal(gv.cpu(), v), "v copy differs"


def test_rope_tables_in_model_dtype_bit_exact():
    """A module moved to bf16 holds bf16 tables (as the reference's does);
    the kernel gives the torch formula's result for those tables."""
    d, T = 64, 9
    rope = RoPE(d, max_seq_len=512).to(torch.bfloat16)
    q = torch.randn(T, 4, d).to(torch.bfloat16)
    k = torch.randn(T, 1, d).to(torch.bfloat16)
    pos = torch.randint(0, 512, (T,))
    eq, ek = rope.forward_tokens(q, k, pos)
    rope_d = rope.to(DEV)
    gq, gk = rope_d.forward_tokens(q.to(DEV), k.to(DEV), pos.to(DEV))
    assert torch.equal(gq.cpu(), eq) and torch.equal(gk.cpu(), ek)


def test_rope_position_past_table_flags_status():
    d, T = 64, 4
    rope = RoPE(d, max_seq_len=16).to(DEV)
    q = torch.randn(T, 2, d, device=DEV)
    k = torch.randn(T, 1, d, device=DEV)
    pos = torch.tensor([0, 5, 16, 15], dtype=torch.int32, device=DEV)
    qo, ko = torch.empty_like(q), torch.empty_like(k)
    status = torch.zeros(1, dtype=torch.int32, device=DEV)
    rc = _native.lib().pkv_rope(qo.data_ptr(), ko.data_ptr(), None, q.data_ptr(), k.data_ptr(),
                                None, 2 * d, d, 0, pos.data_ptr(), rope.cos.data_ptr(),
                                rope.sin.data_ptr(), 16, T, 2, 1, d, 0, status.data_ptr(),
                                _native.stream_ptr(q.device))
    assert rc == 0
    torch.cuda.synchronize()
    assert int(status.item()) == _native.PKV_STATUS_BAD_POS
    # the bad row is rotated by angle 0 (copied); the others are rotated
    assert torch.equal(qo[2], q[2]) and torch.equal(ko[2], k[2])
    eq, _ = RoPE(d, max_seq_len=16).forward_tokens(q[[1]].cpu(), k[[1]].cpu(),
                                                    torch.tensor([5]))
    assert torch.equal(qo[1].cpu(), eq[0])


def rms_ref32(x, w, eps):
    x32 = x.float()
    return x32 * torch.rsqrt(x32.square().mean(-1, keepdim=True) + eps) * w.float()


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("rows,dim,strided", [(1, 128, False), (128, 1024, False),
                                              (7, 4096, True), (5, 1000, False), (3, 12, True),
                                              (2, 8192, False), (2, 9216, True), (4, 96, False)])
def test_rms_norm_vs_fp32_formula(dtype, rows, dim, strided):
    print(f"[rms_norm] {dtype} rows={rows} dim={dim} strided={strided}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(rows * dim)
    base = torch.randn(rows, dim + (8 if strided else 0), generator=g, device=DEV).to(dtype)
    x = base[:, 4:4 + dim] if strided else base
    w = (1.0 + 0.1 * torch.randn(dim, generator=g, device=DEV)).to(dtype)
    y = fused_ops.rms_norm(x, w, 1e-5)
    ref = rms_ref32(x, w, 1e-5)
    torch.cuda.synchronize()
    if dtype == torch.float32:
        torch.testing.assert_close(y, ref, rtol=1e-5, atol=1e-6)
    else:
        r = ref.to(dtype)
        assert within_one_ulp(y, r)
        assert (y == r).float().mean().item() > 0.98


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("rows,dim", [(128, 1024), (3, 136), (2, 10)])
def test_add_rms_norm_residual_exact(dtype, rows, dim):
    g = torch.Generator(device=DEV).manual_seed(dim)
    x = torch.randn(rows, dim, generator=g, device=DEV).to(dtype)
    delta = torch.randn(rows, dim, generator=g, device=DEV).to(dtype)
    w = (1.0 + 0.1 * torch.randn(dim, generator=g, device=DEV)).to(dtype)
    expect_sum = x + delta  # framework add: rounded to dtype
    x_in = x.clone()
    y = fused_ops.add_rms_norm_(x_in, delta, w, 1e-6)
    y_plain = fused_ops.rms_norm(expect_sum, w, 1e-6)
    torch.cuda.synchronize()
    assert torch.equal(x_in, expect_sum), "residual sum differs"
    assert torch.equal(y, y_plain), "norm of the fused sum differs from the plain kernel"
    ref = rms_ref32(expect_sum, w, 1e-6)
    if dtype == torch.float32:
        torch.testing.assert_close(y, ref, rtol=1e-5, atol=1e-6)
    else:
        assert within_one_ulp(y, ref.to(dtype))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("rows,h,split", [(128, 1024, True), (9, 100, False), (1, 2816, True)])
def test_silu_mul_vs_fp32_formula(dtype, rows, h, split):
    g = torch.Generator(device=DEV).manual_seed(h)
    if split:
        gu = (3 * torch.randn(rows, 2 * h, generator=g, device=DEV)).to(dtype)
        gate, up = gu[:, :h], gu[:, h:]
    else:
        gate = (3 * torch.randn(rows, h, generator=g, device=DEV)).to(dtype)
        up = torch.randn(rows, h, generator=g, device=DEV).to(dtype)
    out = fused_ops.silu_mul(gate, up)
    g32, u32 = gate.float(), up.float()
    ref = g32 * torch.sigmoid(g32) * u32
    torch.cuda.synchronize()
    if dtype == torch.float32:
        torch.testing.assert_close(out, ref, rtol=1e-6, atol=1e-7)
    else:
        assert within_one_ulp(out, ref.to(dtype))


def test_fused_step_matches_module_composition_bf16():
    """forward_step (fused residual + norm chain, qkv and gate/up GEMMs)
    against PagedBlock.forward_meta layer by layer on a copy of the batch:
    identical logits and pools."""
    cfg = ModelConfig(vocab_size=4096, d_model=1024, num_layers=3, num_heads=16,
                      num_kv_heads=1, max_seq_len=4096)
    torch.manual_seed(0)
    model = PagedTransformer(cfg).to(DEV, torch.bfloat16).eval()
    dev = torch.device(DEV)
    n, bs, nb = 24, 16, 4096
    lens = workloads.lengths_uniform(n, 100, 1500, seed=5)
    tables = workloads.permuted_tables([int(x) + 1 for x in lens], bs, nb, 5)
    pools = []
    for _ in range(2):
        p = KVPool(cfg.num_layers, bs, nb, 1, cfg.head_dim, torch.bfloat16, dev)
        p.kv.copy_(torch.randn(p.kv.shape, generator=torch.Generator().manual_seed(1)).to(
            dev, torch.bfloat16))
        pools.append(p)
    meta = pack_batch_meta(tables, list(range(n + 1)), [int(x) for x in lens], n, dev, bs)
    ids = torch.randint(0, cfg.vocab_size, (n,), generator=torch.Generator().manual_seed(2)).to(dev)
    with torch.no_grad():
        fused = model.forward_step(ids, pools[0], meta)
        x = model.embedding(ids)
        for layer in model.layers:
            x = layer.forward_meta(x, pools[1], meta)
        plain = model.lm_head(model.final_norm(x))
    torch.cuda.synchronize()
    assert torch.equal(fused, plain), f"max diff {(fused.float() - plain.float()).abs().max()}"
    assert torch.equal(pools[0].kv, pools[1].kv)
