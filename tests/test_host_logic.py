"""Host-side logic of the drop-in serving package (no GPU needed).

Known-answer tests restated from the reference's tests/test_block_allocator.py,
tests/test_sequence.py and tests/test_kv_pool.py, plus the block-table order
of BASELINE config 1 (2 sequences x 16-token prompts, 80 greedy tokens).
"""
import pytest
import torch
import torch.nn as nn

from serving.allocator import BlockAllocator
from serving.batch import build_batch_step
from serving.generation import generate_batched
from serving.kv_pool import KVPool
from serving.paged_meta import pack_batch_meta
from serving.scheduler import Scheduler
from serving.sequence import Sequence, blocks_for


# --- allocator (reference tests/test_block_allocator.py) -------------------

def test_alloc_all_then_free_all():
    a = BlockAllocator(8)
    blocks = a.allocate_n(a.num_usable)
    assert a.num_free == 0 and 0 not in blocks and len(set(blocks)) == 7
    a.free(blocks)
    assert a.num_free == 7


def test_out_of_blocks():
    a = BlockAllocator(4)
    assert not a.can_allocate(4)
    a.allocate_n(3)
    with pytest.raises(RuntimeError):
        a.allocate()
    with pytest.raises(RuntimeError):
        a.allocate_n(1)


def test_double_free_and_block_zero():
    a = BlockAllocator(4)
    b = a.allocate()
    a.free([b])
    with pytest.raises(ValueError):
        a.free([b])
    with pytest.raises(ValueError):
        a.free([0])
    with pytest.raises(ValueError):
        a.free([4])


def test_failed_free_changes_nothing():
    a = BlockAllocator(4)
    b = a.allocate()
    before = a.num_free
    with pytest.raises(ValueError):
        a.free([b, 0])
    with pytest.raises(ValueError):
        a.free([b, b])
    assert a.num_free == before


def test_failed_free_rolls_back_and_names_first_bad_id():
    # the first bad id in list order decides the message (the reference
    # validates in list order); the ids before it stay in use
    a = BlockAllocator(8)
    b1, b2, b3 = a.allocate_n(3)
    with pytest.raises(ValueError, match=f"double free of block {b2}"):
        a.free([b1, b2, b3, b2])
    with pytest.raises(ValueError, match="invalid block id 9"):
        a.free([b3, 9, b1])
    assert a.num_free == 4
    # nothing was released: the next allocation is a fresh id, and every
    # original id can still be freed exactly once
    assert a.allocate() == 4
    a.free([b3, b1, b2])
    assert [a.allocate() for _ in range(3)] == [b2, b1, b3]


def test_allocation_order_is_ascending_then_lifo(kats):
    c = kats["allocator_order"]
    a = BlockAllocator(c["num_blocks"])
    assert a.allocate_n(len(c["first"])) == c["first"]
    a.free(c["free"])
    assert [a.allocate() for _ in c["then"]] == c["then"]


# --- sequence (reference tests/test_sequence.py) ----------------------------

def test_blocks_for(kats):
    c = kats["blocks_for"]
    for n, expected in c["cases"]:
        assert blocks_for(n, c["block_size"]) == expected, n


def test_growth_at_boundary():
    a = BlockAllocator(10)
    s = Sequence(0, list(range(16)), block_size=16)
    s.ensure_blocks(a)
    assert len(s.block_table) == 1
    s.append_token(99)
    assert s.num_new_blocks_needed() == 1
    s.ensure_blocks(a)
    assert len(s.block_table) == 2


def test_release_and_no_shared_blocks():
    a = BlockAllocator(10)
    s1 = Sequence(1, list(range(20)), 16)
    s1.ensure_blocks(a)
    s2 = Sequence(2, list(range(20)), 16)
    s2.ensure_blocks(a)
    assert not set(s1.block_table) & set(s2.block_table)
    s1.release(a)
    s2.release(a)
    assert a.num_free == a.num_usable


# --- KV pool host parts (reference tests/test_kv_pool.py) ------------------

def make_tiny_pool():
    return KVPool(num_layers=2, block_size=16, num_blocks=16, num_kv_heads=2, head_dim=4,
                  dtype=torch.float32, device="cpu")


def test_pool_shapes():
    pool = make_tiny_pool()
    assert pool.kv.shape == (2, 2, 16, 16, 2, 4)
    assert pool.flat_k[0].shape == (16 * 16, 2, 4)
    assert pool.flat_k[0].data_ptr() == pool.kv[0, 0].data_ptr()
    assert pool.flat_v[1].data_ptr() == pool.kv[1, 1].data_ptr()
    assert not pool.kv.any()


def test_pool_slot_mapping_kat(kats):
    pool = make_tiny_pool()
    for c in kats["slot_mapping"]:
        slots = pool.make_slot_mapping(start=c["start"], n=c["n"], block_table=c["block_table"])
        assert slots.dtype == torch.long and slots.tolist() == c["slots"]


def test_pool_slot_mapping_asserts():
    pool = make_tiny_pool()
    with pytest.raises(AssertionError, match="too short"):
        pool.make_slot_mapping(10, 7, [3])
    with pytest.raises(AssertionError, match="block 0"):
        pool.make_slot_mapping(0, 20, [4, 0])
    # a block id past the pool: the reference's index_put would raise at
    # write time; here the mapping refuses it (the device write would skip it)
    with pytest.raises(IndexError, match="out of range"):
        pool.make_slot_mapping(0, 20, [4, 16])


def test_pool_write_checks_then_refuses_cpu():
    pool = make_tiny_pool()
    slots = pool.make_slot_mapping(0, 4, [5])
    k = torch.zeros(4, 2, 4)
    with pytest.raises(AssertionError):
        pool.write(0, slots.int(), k, k)
    with pytest.raises(AssertionError):
        pool.write(0, slots, k.double(), k.double())
    with pytest.raises(AssertionError):
        pool.write(0, slots[:3], k, k)
    # the write itself is a HIP kernel: no CPU path, fails loudly
    with pytest.raises(RuntimeError, match="GPU"):
        pool.write(0, slots, k, k)


def test_from_config():
    from types import SimpleNamespace
    cfg = SimpleNamespace(num_layers=3, block_size=32, num_gpu_blocks=8, num_kv_heads=1,
                          head_dim=64, kv_dtype=torch.bfloat16)
    pool = KVPool.from_config(cfg, "cpu")
    assert pool.kv.shape == (3, 2, 8, 32, 1, 64) and pool.kv.dtype == torch.bfloat16


# --- batch step / metadata packing -----------------------------------------

def test_build_batch_step_kat():
    a = BlockAllocator(16)
    s0 = Sequence(0, [5, 6, 7], 16)
    s0.ensure_blocks(a)
    s1 = Sequence(1, list(range(20)), 16)
    s1.ensure_blocks(a)
    b = build_batch_step([(s0, s0.token_ids), (s1, [19])], "cpu")
    assert b.input_ids.tolist() == [5, 6, 7, 19]
    assert b.positions == [0, 1, 2, 19]
    assert b.query_start_loc == [0, 3, 4]
    assert b.block_tables == [[1], [2, 3]]
    assert b.seq_lens == [3, 20]
    assert b.num_seqs == 2


def test_pack_batch_meta_kat():
    m = pack_batch_meta([[5, 2], [7], []], [0, 3, 4, 4], [17, 18, 19, 5], 4, "cpu", 16)
    assert m.block_tables.tolist() == [[5, 2], [7, 0], [0, 0]]
    assert m.seq_lens.tolist() == [20, 6, 0]
    assert m.query_start_loc.tolist() == [0, 3, 4, 4]
    assert m.start_pos.tolist() == [17, 5, 0]
    assert m.positions.tolist() == [17, 18, 19, 5]
    assert (m.max_q_len, m.max_kv_len, m.max_blocks, m.num_seqs, m.num_tokens) == (3, 20, 2, 3, 4)
    assert not m.is_decode
    d = pack_batch_meta([[1], [2]], [0, 1, 2], [3, 9], 2, "cpu", 16)
    assert d.is_decode


def test_pack_batch_meta_errors():
    with pytest.raises(ValueError, match="num_seqs \\+ 1"):
        pack_batch_meta([[1]], [0], [0], 1, "cpu", 16)
    with pytest.raises(ValueError, match="start at 0"):
        pack_batch_meta([[1]], [0, 2], [0], 1, "cpu", 16)
    with pytest.raises(ValueError, match="length T"):
        pack_batch_meta([[1]], [0, 1], [0, 1], 1, "cpu", 16)
    with pytest.raises(ValueError, match="exceeds"):
        pack_batch_meta([[1]], [0, 1], [16], 1, "cpu", 16)
    with pytest.raises(AssertionError, match="block 0"):
        pack_batch_meta([[3, 0]], [0, 1], [17], 1, "cpu", 16)


# --- generation / scheduler with a model that never touches the pool -------

class FixedLogitModel(nn.Module):
    """Records each step's batch; logits favour token (step + row) % vocab."""

    def __init__(self, vocab=50):
        super().__init__()
        self.p = nn.Parameter(torch.zeros(1))
        self.vocab = vocab
        self.batches = []

    def forward_batch(self, batch, pool):
        # snapshot: the batch shares the sequences' live block-table lists
        batch.block_tables = [list(bt) for bt in batch.block_tables]
        self.batches.append(batch)
        n = batch.num_seqs
        logits = torch.zeros(n, self.vocab)
        for i in range(n):
            logits[i, (len(self.batches) + i) % self.vocab] = 10.0
        return logits


def test_config1_block_tables_kat(kats):
    # 2 sequences, 16-token prompts, 80 greedy tokens, block_size 16,
    # 256 blocks: prefill allocates 1, 2; each 16-token boundary allocates
    # seq0 then seq1; final kv length 16 + 79 = 95 -> 6 blocks each
    model = FixedLogitModel()
    a = BlockAllocator(256)
    out = generate_batched(model, [list(range(16)), list(range(16, 32))], 80, None, a)
    assert [len(o) for o in out] == [80, 80]
    last = model.batches[-1]
    c = kats["config1_block_tables"]
    assert last.block_tables == c["tables"]
    assert last.positions == c["last_positions"] and last.seq_lens == c["last_seq_lens"]
    assert len(model.batches) == 80
    assert a.num_free == a.num_usable  # released in the finally block
    assert out[0][:3] == [1, 2, 3] and out[1][:3] == [2, 3, 4]


def test_generate_batched_argument_errors():
    model = FixedLogitModel()
    a = BlockAllocator(8)
    with pytest.raises(ValueError):
        generate_batched(model, [[1]], -1, None, a)
    with pytest.raises(ValueError):
        generate_batched(model, [[1], []], 2, None, a)
    assert generate_batched(model, [], 3, None, a) == []
    assert generate_batched(model, [[1]], 0, None, a) == [[]]


def test_scheduler_admission_headroom_and_release():
    from types import SimpleNamespace
    model = FixedLogitModel(vocab=8)
    a = BlockAllocator(6)  # 5 usable
    sched = Scheduler(model, None, a, SimpleNamespace(eos_token_id=7), block_size=16,
                      temperature=1.0, top_k=1, top_p=1.0)
    sched.add_request(list(range(20)), 2)  # needs 2 blocks
    sched.add_request(list(range(17)), 2)  # needs 2 blocks
    sched.add_request(list(range(5)), 1)   # needs 1 block
    res = sched.step()
    # first: 5 - 2 >= 1 admitted; second: 3 - 2 >= 2 fails -> waits
    assert [r[0] for r in res] == [0]
    assert len(sched.running) == 1 and len(sched.waiting) == 2
    res = sched.step()
    assert res[0][2] is True  # reached max_new_tokens
    while sched.running or sched.waiting:
        sched.step()
    assert a.num_free == a.num_usable
