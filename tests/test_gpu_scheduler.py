"""The Scheduler with a SchedulerConfig on the real paged model (BASELINE
config-1 shape, fp32): chunked prefill through the MFMA-less fp32 attention
path's varlen kernel and recompute preemption in a pool too small for all
requests must give, under greedy sampling (top_k = 1), exactly the tokens
each prompt produces alone with generate_batched."""
from types import SimpleNamespace

import pytest
import torch

from serving.allocator import BlockAllocator
from serving.generation import generate_batched
from serving.kv_pool import KVPool
from serving.layers import ModelConfig, SchedulerConfig
from serving.paged_model import PagedTransformer
from serving.scheduler import Scheduler

pytestmark = pytest.mark.gpu
DEV = "cuda"


def test_chunked_prefill_and_preemption_match_single_sequence_greedy():
    print("[scheduler] chunked prefill + preemption, fp32 cfg1 model", flush=True)
    cfg = ModelConfig(vocab_size=50257, d_model=128, num_layers=4, num_heads=4, num_kv_heads=1,
                      max_seq_len=128)
    torch.manual_seed(0)
    model = PagedTransformer(cfg).to(DEV).eval()
    g = torch.Generator().manual_seed(5)
    lens, new = [20, 24, 18, 30], [40, 40, 40, 40]
    prompts = [torch.randint(0, 50257, (n,), generator=g).tolist() for n in lens]

    expect = []
    for p, n in zip(prompts, new):
        pool = KVPool(cfg.num_layers, 16, 64, 1, cfg.head_dim, torch.float32, DEV)
        expect.append(generate_batched(model, [p], n, pool, BlockAllocator(64))[0])

    nb = 8  # 7 usable blocks of 16 tokens for ~250 tokens of requests
    pool = KVPool(cfg.num_layers, 16, nb, 1, cfg.head_dim, torch.float32, DEV)
    alloc = BlockAllocator(nb)
    sc = SchedulerConfig(max_num_seqs=4, max_num_batched_tokens=24, enable_chunked_prefill=True,
                         cudagraph_batch_sizes=[1, 2])
    sched = Scheduler(model, pool, alloc, SimpleNamespace(eos_token_id=-1), block_size=16,
                      temperature=1.0, top_k=1, top_p=1.0, sched_cfg=sc)
    for p, n in zip(prompts, new):
        sched.add_request(p, n)
    got, steps, biggest = {}, 0, 0
    while sched.running or sched.waiting:
        for sid, tok, done in sched.step():
            got.setdefault(sid, []).append(tok)
        biggest = max(biggest, sched.last_batch_tokens)
        steps += 1
        assert steps < 2000
    assert sched.num_preemptions > 0
    assert biggest == 24  # a prompt was split over steps
    for sid in range(len(prompts)):
        assert got[sid] == expect[sid], f"request {sid}"
    assert alloc.num_free == alloc.num_usable
