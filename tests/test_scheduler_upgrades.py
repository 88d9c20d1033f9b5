"""Scheduler with a SchedulerConfig (serving/scheduler.py): token budget,
sequence cap, chunked prefill and recompute preemption. CPU only, with a
model stub that behaves like a paged KV cache: every computed token is
written to its pool slot (block_table[pos // bs] * bs + pos % bs) and the
next token is a hash of the whole context read back through the block
table, so a chunk computed at the wrong positions, a skipped chunk or a
preempted sequence that is not fully recomputed yields a different stream
than the plain greedy recurrence."""
from types import SimpleNamespace

import pytest
import torch

from serving.allocator import BlockAllocator
from serving.layers import SchedulerConfig
from serving.scheduler import Scheduler

VOCAB = 97
EOS = 96


def next_token(context):
    h = 0
    for j, t in enumerate(context):
        h = (h * 1000003 + (j + 1) * (t + 7)) % 2147483647
    return h % (VOCAB - 1)  # never EOS: requests run to max_new_tokens


class PagedStub(torch.nn.Module):
    def __init__(self, bs):
        super().__init__()
        self.p = torch.nn.Parameter(torch.zeros(1))
        self.bs = bs
        self.kv = {}
        self.batches = []

    def forward_batch(self, batch, pool):
        self.batches.append(batch)
        ids = batch.input_ids.tolist()
        out = torch.full((batch.num_seqs, VOCAB), -1.0)
        for i in range(batch.num_seqs):
            a, b = batch.query_start_loc[i], batch.query_start_loc[i + 1]
            table = batch.block_tables[i]
            for t, pos in zip(ids[a:b], batch.positions[a:b]):
                self.kv[table[pos // self.bs] * self.bs + pos % self.bs] = t
            ctx = [self.kv[table[j // self.bs] * self.bs + j % self.bs]
                   for j in range(batch.seq_lens[i])]
            out[i, next_token(ctx)] = 1.0
        return out


def expected(prompt, n):
    toks = list(prompt)
    for _ in range(n):
        toks.append(next_token(toks))
    return toks[len(prompt):]


def run(sched):
    got = {}
    steps = 0
    while sched.running or sched.waiting:
        for sid, tok, done in sched.step():
            got.setdefault(sid, []).append(tok)
        steps += 1
        assert steps < 10000
    return got


def prompts():
    g = torch.Generator().manual_seed(0)
    lens = [40, 5, 90, 17, 33, 64, 8, 120]
    return [torch.randint(0, VOCAB - 1, (n,), generator=g).tolist() for n in lens]


@pytest.mark.parametrize("chunked,budget,max_seqs,blocks", [
    (True, 24, 3, 64),     # chunked prefill, plenty of blocks
    (True, 16, 4, 20),     # chunked prefill and preemption
    (False, 128, 2, 24),   # whole prompts
    (True, 512, 8, 400),   # budget never binds
])
def test_budgeted_scheduler_matches_greedy_recurrence(chunked, budget, max_seqs, blocks):
    bs = 8
    model = PagedStub(bs)
    alloc = BlockAllocator(blocks)
    sc = SchedulerConfig(max_num_seqs=max_seqs, max_num_batched_tokens=budget,
                         enable_chunked_prefill=chunked,
                         cudagraph_batch_sizes=[1, 2])
    sched = Scheduler(model, None, alloc, SimpleNamespace(eos_token_id=EOS), block_size=bs,
                      temperature=1.0, top_k=1, top_p=1.0, sched_cfg=sc)
    ps = prompts()
    new = [12, 30, 7, 25, 18, 9, 40, 3]
    for p, n in zip(ps, new):
        sched.add_request(p, n)
    got = run(sched)
    for sid, (p, n) in enumerate(zip(ps, new)):
        assert got[sid] == expected(p, n), f"request {sid}"
    assert alloc.num_free == alloc.num_usable
    for b in model.batches:
        assert len(b.positions) <= budget and b.num_seqs <= max_seqs
    if blocks <= 20:
        assert sched.num_preemptions > 0
    if chunked and budget < 120:
        # some prompt was split: a batch computed a prefix of a longer prompt
        assert any(len(b.positions) == budget for b in model.batches)


@pytest.mark.parametrize("chunked", [False, True])
def test_recompute_preemption_under_decode_growth(chunked):
    """Four 30-token prompts admitted together (4 blocks each of a 23-block
    pool), each generating 60 tokens (8 more blocks): decode growth must
    preempt and recompute, and every stream still follows the recurrence."""
    bs = 8
    model = PagedStub(bs)
    alloc = BlockAllocator(24)
    sc = SchedulerConfig(max_num_seqs=4, max_num_batched_tokens=64 if chunked else 96,
                         enable_chunked_prefill=chunked, cudagraph_batch_sizes=[1])
    sched = Scheduler(model, None, alloc, SimpleNamespace(eos_token_id=EOS), block_size=bs,
                      top_k=1, sched_cfg=sc)
    g = torch.Generator().manual_seed(3)
    ps = [torch.randint(0, VOCAB - 1, (30,), generator=g).tolist() for _ in range(4)]
    for p in ps:
        sched.add_request(p, 60)
    got = run(sched)
    assert sched.num_preemptions > 0
    for sid, p in enumerate(ps):
        assert got[sid] == expected(p, 60), f"request {sid}"
    assert alloc.num_free == alloc.num_usable


def test_budgeted_scheduler_rejects_what_cannot_run():
    alloc = BlockAllocator(10)
    sc = SchedulerConfig(max_num_seqs=2, max_num_batched_tokens=16, cudagraph_batch_sizes=[1])
    sched = Scheduler(PagedStub(8), None, alloc, SimpleNamespace(eos_token_id=EOS),
                      block_size=8, top_k=1, sched_cfg=sc)
    with pytest.raises(ValueError):
        sched.add_request(list(range(20)), 1)   # longer than the budget, no chunking
    with pytest.raises(ValueError):
        sched.add_request(list(range(10)), 7)   # a recompute could not fit the budget
    with pytest.raises(ValueError):
        sched.add_request(list(range(10)), 70)  # can never fit the pool
    with pytest.raises(AssertionError):
        SchedulerConfig(max_num_seqs=8, max_num_batched_tokens=4)


def test_reference_mode_unchanged_without_config():
    alloc = BlockAllocator(64)
    sched = Scheduler(PagedStub(16), None, alloc, SimpleNamespace(eos_token_id=EOS),
                      block_size=16, top_k=1)
    sched.add_request(list(range(20)), 3)
    res = sched.step()
    seq = sched.running[0]
    # the prompt is in the pool; the sampled token is next
    assert [r[0] for r in res] == [0] and sched.computed_tokens(seq) == seq.num_tokens - 1
