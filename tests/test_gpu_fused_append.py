"""pkv_paged_attention_append (append fused into the decode attention)
against the two calls it replaces, KVPool.write_from_table followed by
paged_attention_meta (serving/paged_mqa.py:98-110), on identical copies of
a decode batch:

  - outputs and lse bit-identical (the fused kernels read the new row from
    k_new / v_new, the two-call path from the pool, the same bytes);
  - pools bit-identical afterwards (each new row written exactly once);
  - both MFMA decode kernels (partition: config-4 shape, persistent:
    config-5 shape with a long-context bound), block boundaries crossed;
  - the small-group kernel (fp32 config-2 shape; bf16 with sequences split
    over several partitions and merged in the kernel; fp16 d 128);
  - a new row whose table entry is block 0 (reserved): skipped and flagged
    PKV_STATUS_BAD_BLOCK exactly like the stand-alone append.
"""
import numpy as np
import pytest
import torch

from serving import _native, workloads
from serving.fake_paged_attn import paged_attention_append_meta, paged_attention_meta
from serving.kv_pool import KVPool
from serving.paged_meta import pack_batch_meta

pytestmark = pytest.mark.gpu
DEV = "cuda"


def batch(n, hq, d, dtype, lo, hi, bs, nb, seed):
    dev = torch.device(DEV)
    lens = workloads.lengths_uniform(n, lo, hi, seed=seed)
    tables = workloads.permuted_tables([int(x) + 1 for x in lens], bs, nb, seed)
    pool = KVPool(1, bs, nb, 1, d, dtype, dev)
    g = torch.Generator(device=dev).manual_seed(seed)
    pool.kv.normal_(generator=g)
    meta = pack_batch_meta(tables, list(range(n + 1)), [int(x) for x in lens], n, dev, bs)
    q = torch.randn(n, hq, d, generator=g, device=dev).to(dtype)
    k = torch.randn(n, 1, d, generator=g, device=dev).to(dtype)
    v = torch.randn(n, 1, d, generator=g, device=dev).to(dtype)
    return pool, meta, q, k, v


def copy_pool(pool):
    p2 = KVPool(1, pool.block_size, pool.num_blocks, 1, pool.head_dim, pool.dtype, pool.device)
    p2.kv.copy_(pool.kv)
    return p2


@pytest.mark.parametrize("name,n,hq,d,dtype,lo,hi,bound", [
    ("partition-cfg4", 128, 16, 64, torch.bfloat16, 256, 2048, 0),
    ("persistent-cfg5", 96, 32, 128, torch.bfloat16, 100, 3000, 8192),
    ("persistent-g16d128", 64, 16, 128, torch.float16, 1, 700, 4096),
    ("small-fp32", 24, 8, 32, torch.float32, 1, 300, 0),
    ("small-g4-bf16-split", 40, 4, 64, torch.bfloat16, 1, 3000, 0),
    ("small-g2-fp16-d128", 16, 2, 128, torch.float16, 300, 900, 0),
])
def test_fused_equals_two_calls(name, n, hq, d, dtype, lo, hi, bound):
    print(f"[fused append] {name}", flush=True)
    pool_a, meta, q, k, v = batch(n, hq, d, dtype, lo, hi, 16, 16384, seed=21)
    pool_b = copy_pool(pool_a)
    if bound:
        meta.max_kv_len = bound  # selects the persistent kernel
    lse_a = torch.empty(n, hq, device=DEV)
    lse_b = torch.empty(n, hq, device=DEV)
    pool_a.write_from_table(0, k, v, meta)
    out_a = paged_attention_meta(q, pool_a.kv[0, 0], pool_a.kv[0, 1], meta, lse=lse_a)
    out_b = paged_attention_append_meta(q, k, v, pool_b, 0, meta, lse=lse_b)
    torch.cuda.synchronize()
    assert torch.equal(pool_a.kv, pool_b.kv), f"{name}: pools differ"
    assert torch.equal(out_a, out_b), f"{name}: outputs differ " \
        f"(max {(out_a.float() - out_b.float()).abs().max().item():.3e})"
    assert torch.equal(lse_a, lse_b), f"{name}: lse differs"


@pytest.mark.parametrize("hq,d,dtype", [(16, 64, torch.bfloat16), (4, 32, torch.float32)])
def test_fused_bad_block_is_skipped_and_flagged(hq, d, dtype):
    pool, meta, q, k, v = batch(8, hq, d, dtype, 40, 90, 16, 256, seed=22)
    # the new row of sequence 3 falls into a table entry set to block 0
    s = 3
    pos = int(meta.start_pos[s].item())
    meta.block_tables[s, pos // 16] = 0
    pool.debug = True
    before = pool.kv.clone()
    with pytest.raises(AssertionError):
        paged_attention_append_meta(q, k, v, pool, 0, meta)
    torch.cuda.synchronize()
    # nothing was written for sequence 3; every other new row was
    changed = (pool.kv != before).any(dim=-1).any(dim=-1)  # [1, 2, NB, BS]
    slots = torch.nonzero(changed[0, 0].flatten()).flatten().cpu().numpy()
    tables = meta.block_tables.cpu().numpy()
    starts = meta.start_pos.cpu().numpy()
    expect = sorted(int(tables[i, starts[i] // 16]) * 16 + int(starts[i]) % 16
                    for i in range(8) if i != s)
    assert np.array_equal(np.sort(slots), np.array(expect)), (slots, expect)
