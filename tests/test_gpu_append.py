"""KV append (slot-mapped scatter) and gather on the GPU, bit-exact against
the oracle (numpy index_put restatement) and torch's own index_put_.

64 sequences x 128 prompt tokens of K/V (Hkv=1, D=64,
bf16, N(0,1)) into a 4096-block pool (block_size 16), blocks handed out by
the allocator from a shuffled free list; then 64 single-token appends at
ragged positions, some crossing a block boundary.
"""
import numpy as np
import pytest
import torch

from oracle import paged_ref as ref
from serving.allocator import BlockAllocator
from serving.kv_pool import KVPool
from serving.paged_meta import pack_batch_meta
from serving.sequence import Sequence

pytestmark = pytest.mark.gpu
DEV = "cuda"


def bits(t):
    """Raw bit pattern (so -0.0 / NaN payloads are compared exactly)."""
    t = t.detach().cpu().contiguous()
    return t.view(torch.int16 if t.element_size() == 2 else torch.int32).numpy()


def shuffled_allocator(num_blocks, seed):
    """An allocator that hands its blocks out in a random order: every block
    is taken once and returned in a shuffled order (freed blocks come back
    most recently freed first), through the public interface only."""
    a = BlockAllocator(num_blocks)
    rng = np.random.default_rng(seed)
    ids = a.allocate_n(a.num_free)
    a.free([int(x) for x in rng.permutation(ids)])
    return a


def oracle_pool(pool):
    """numpy copy of the pool as [L, 2, NB*BS, Hkv, D] raw bits."""
    return bits(pool.kv).reshape(pool.num_layers, 2, -1, pool.num_kv_heads, pool.head_dim).copy()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16])
def test_cfg3_prefill_then_ragged_decode_bit_exact(dtype):
    print(f"[cfg3 append] dtype={dtype}", flush=True)
    torch.manual_seed(0)
    NB, BS, HKV, D = 4096, 16, 1, 64
    pool = KVPool(1, BS, NB, HKV, D, dtype, DEV)
    alloc = shuffled_allocator(NB, seed=0)
    seqs = [Sequence(i, [0] * 128, BS) for i in range(64)]
    for s in seqs:
        s.ensure_blocks(alloc)
    expect = oracle_pool(pool)

    # prefill: one write per sequence through make_slot_mapping
    g = torch.Generator(device=DEV).manual_seed(1)
    for s in seqs:
        k = torch.randn(128, HKV, D, generator=g, device=DEV).to(dtype)
        v = torch.randn(128, HKV, D, generator=g, device=DEV).to(dtype)
        slots = pool.make_slot_mapping(0, 128, s.block_table)
        pool.write(0, slots, k, v)
        ref.append(expect[0, 0], expect[0, 1],
                   ref.make_slot_mapping(0, 128, s.block_table, BS), bits(k), bits(v))
    torch.cuda.synchronize()
    assert np.array_equal(oracle_pool(pool), expect)

    # ragged decode: sequences grow by 0..31 tokens first so the next
    # position is ragged; 1 in 4 lands exactly on a block boundary
    rng = np.random.default_rng(2)
    for i, s in enumerate(seqs):
        extra = 16 if i % 4 == 0 else int(rng.integers(0, 32))
        s.token_ids.extend([0] * extra)
        s.append_token(0)
        s.ensure_blocks(alloc)
    positions = [s.num_tokens - 1 for s in seqs]
    assert sum(p % BS == 0 for p in positions) >= 16
    k = torch.randn(64, HKV, D, generator=g, device=DEV).to(dtype)
    v = torch.randn(64, HKV, D, generator=g, device=DEV).to(dtype)
    slots = torch.cat([pool.make_slot_mapping(p, 1, s.block_table) for p, s in zip(positions, seqs)])
    pool.write(0, slots, k, v)
    host_slots = np.concatenate([ref.make_slot_mapping(p, 1, s.block_table, BS)
                                 for p, s in zip(positions, seqs)])
    ref.append(expect[0, 0], expect[0, 1], host_slots, bits(k), bits(v))
    torch.cuda.synchronize()
    assert np.array_equal(oracle_pool(pool), expect)
    # block 0 (reserved) and every unallocated block are still zero
    assert not bits(pool.kv[0, :, 0]).any()

    # the same decode step through device metadata (in-kernel slots)
    pool2 = KVPool(1, BS, NB, HKV, D, dtype, DEV)
    pool2.kv.copy_(pool.kv)
    tables = [s.block_table for s in seqs]
    meta = pack_batch_meta(tables, list(range(65)), positions, 64, DEV, BS)
    k2 = torch.randn(64, HKV, D, generator=g, device=DEV).to(dtype)
    v2 = torch.randn(64, HKV, D, generator=g, device=DEV).to(dtype)
    pool2.write_from_table(0, k2, v2, meta)
    ref.append(expect[0, 0], expect[0, 1], host_slots, bits(k2), bits(v2))
    torch.cuda.synchronize()
    assert np.array_equal(oracle_pool(pool2), expect)


def test_write_from_table_prefill_matches_write():
    print("[append_from_table prefill]", flush=True)
    NB, BS, HKV, D = 512, 16, 2, 32
    alloc = shuffled_allocator(NB, seed=3)
    lens = [1, 15, 16, 17, 40, 100, 3]
    seqs = [Sequence(i, [0] * n, BS) for i, n in enumerate(lens)]
    for s in seqs:
        s.ensure_blocks(alloc)
    T = sum(lens)
    g = torch.Generator(device=DEV).manual_seed(4)
    k = torch.randn(T, HKV, D, generator=g, device=DEV)
    v = torch.randn(T, HKV, D, generator=g, device=DEV)
    qsl = np.concatenate([[0], np.cumsum(lens)]).tolist()
    positions = [p for n in lens for p in range(n)]
    pa = KVPool(2, BS, NB, HKV, D, torch.float32, DEV)
    pb = KVPool(2, BS, NB, HKV, D, torch.float32, DEV)
    meta = pack_batch_meta([s.block_table for s in seqs], qsl, positions, T, DEV, BS)
    pa.write_from_table(1, k, v, meta)
    slots = torch.cat([pb.make_slot_mapping(0, n, s.block_table) for n, s in zip(lens, seqs)])
    pb.write(1, slots, k, v)
    torch.cuda.synchronize()
    assert torch.equal(pa.kv, pb.kv)
    assert not pa.kv[0].any()  # other layer untouched


def test_roundtrip_and_untouched_block_zero():
    # reference tests/test_kv_pool.py:33-67 on the device
    pool = KVPool(2, 16, 16, 2, 4, torch.float32, DEV)
    bt = [9, 3, 12]
    slots = pool.make_slot_mapping(0, 40, bt)
    k = torch.randn(40, 2, 4, device=DEV)
    v = torch.randn(40, 2, 4, device=DEV)
    pool.write(0, slots, k, v)
    ko, vo = pool.gather(0, bt, 40)
    assert torch.equal(ko, k) and torch.equal(vo, v)
    assert torch.all(pool.kv[0, 0, 0] == 0) and torch.all(pool.kv[1] == 0)
    # gather matches torch indexing of the pool exactly
    ek = pool.kv[0, 0][torch.tensor(bt, device=DEV)].reshape(-1, 2, 4)[:40]
    assert torch.equal(ko, ek)


def test_append_matches_torch_index_put_with_negative_slots():
    pool = KVPool(1, 16, 8, 1, 8, torch.bfloat16, DEV)
    slots = torch.tensor([-1, 3, -128, 127, 20], device=DEV)
    k = torch.randn(5, 1, 8, device=DEV).bfloat16()
    v = torch.randn(5, 1, 8, device=DEV).bfloat16()
    expect_k = pool.flat_k[0].clone()
    expect_k[slots] = k
    pool.write(0, slots, k, v)
    torch.cuda.synchronize()
    assert np.array_equal(bits(pool.flat_k[0]), bits(expect_k))


def test_out_of_range_slot_is_skipped_and_reported():
    pool = KVPool(1, 16, 8, 1, 8, torch.float32, DEV)
    pool.debug = True
    k = torch.ones(2, 1, 8, device=DEV)
    with pytest.raises(IndexError):
        pool.write(0, torch.tensor([5, 128], device=DEV), k, k)
    # the in-range row was written, nothing outside the pool was touched
    assert torch.equal(pool.flat_k[0][5], k[0]) and pool.kv.sum().item() == 16.0


def test_odd_row_widths_use_narrow_pieces():
    # row = hkv * d * 2 bytes = 24 bytes: not a multiple of 16
    pool = KVPool(1, 4, 8, 3, 4, torch.float16, DEV)
    slots = pool.make_slot_mapping(1, 9, [2, 5, 7])
    k = torch.randn(9, 3, 4, device=DEV).half()
    pool.write(0, slots, k, -k)
    ko, vo = pool.gather(0, [2, 5, 7], 10)
    assert torch.equal(ko[1:], k) and torch.equal(vo[1:], -k)
