"""the reference's CPU model shape, random init from seed
0, fp32: d_model 128, 4 layers, 4 query heads, 1 KV head (head_dim 32),
RMSNorm, RoPE, SwiGLU, vocab 50257, max_seq_len 128. Two 16-token prompts
drawn uniformly from [0, 50257) (seed 0), 80 greedy tokens each,
block_size 16, 256 pool blocks.

Greedy tokens from the GPU paged path must equal the CPU fp32 oracle's
exactly; every step's logits agree within 1e-5 relative (of the logit
scale); the final block tables are the hand-derived
seq0 = [1,3,5,7,9,11], seq1 = [2,4,6,8,10,12].
"""
import numpy as np
import pytest
import torch

from oracle import torch_ref
from serving.allocator import BlockAllocator
from serving.batch import build_batch_step
from serving.generation import generate_batched
from serving.kv_pool import KVPool
from serving.layers import ModelConfig
from serving.paged_model import PagedTransformer
from serving.sequence import Sequence

pytestmark = pytest.mark.gpu
DEV = "cuda"


def cfg1():
    return ModelConfig(vocab_size=50257, d_model=128, num_layers=4, num_heads=4,
                       num_kv_heads=1, max_seq_len=128)


def build_model(cfg, seed=0):
    torch.manual_seed(seed)
    return PagedTransformer(cfg)  # constructed on the CPU, as the reference does


def prompts(seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, 50257, (2, 16), generator=g).tolist()


def test_cfg1_greedy_tokens_identical_fp32():
    print("[cfg1 greedy]", flush=True)
    cfg = cfg1()
    model = build_model(cfg)
    sd = {k: v.clone() for k, v in model.state_dict().items()}
    model = model.to(DEV).eval()
    p = prompts()
    pool = KVPool(cfg.num_layers, 16, 256, cfg.num_kv_heads, cfg.head_dim, torch.float32, DEV)
    alloc = BlockAllocator(256)

    # product path, recording every step's logits
    seqs = [Sequence(i, list(x), 16) for i, x in enumerate(p)]
    got_tok = [[] for _ in seqs]
    got_logits = []
    for s in seqs:
        s.ensure_blocks(alloc)
    batch = build_batch_step([(s, s.token_ids) for s in seqs], DEV)
    for step in range(80):
        logits = model.forward_batch(batch, pool)
        got_logits.append(logits.cpu())
        nxt = logits.argmax(-1).tolist()
        for o, t in zip(got_tok, nxt):
            o.append(t)
        if step == 79:
            break
        for s, t in zip(seqs, nxt):
            s.append_token(t)
            s.ensure_blocks(alloc)
        batch = build_batch_step([(s, [t]) for s, t in zip(seqs, nxt)], DEV)
    assert [s.block_table for s in seqs] == [[1, 3, 5, 7, 9, 11], [2, 4, 6, 8, 10, 12]]

    ref_model = torch_ref.RefModel(sd, cfg.num_layers, cfg.num_heads, cfg.num_kv_heads,
                                   cfg.max_seq_len)
    ref_tok, ref_logits = torch_ref.generate_batched_ref(ref_model, p, 80)
    assert got_tok == ref_tok
    for step in range(80):
        expect = torch.stack([ref_logits[0][step], ref_logits[1][step]])
        scale = float(expect.abs().max())
        torch.testing.assert_close(got_logits[step], expect, rtol=1e-5, atol=1e-5 * scale)

    # the library's own greedy loop gives the same tokens and frees its blocks
    alloc2 = BlockAllocator(256)
    pool2 = KVPool(cfg.num_layers, 16, 256, cfg.num_kv_heads, cfg.head_dim, torch.float32, DEV)
    assert generate_batched(model, p, 80, pool2, alloc2) == ref_tok
    assert alloc2.num_free == alloc2.num_usable


def test_single_sequence_generate_paged_matches_batched():
    from serving.generation import generate_paged
    cfg = cfg1()
    model = build_model(cfg).to(DEV).eval()
    p = prompts(1)[0]
    pool = KVPool(cfg.num_layers, 16, 64, 1, cfg.head_dim, torch.float32, DEV)
    a = BlockAllocator(64)
    single = generate_paged(model, p, 12, pool, a)
    batched = generate_batched(model, [p], 12, pool, a)[0]
    assert single == batched
