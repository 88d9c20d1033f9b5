"""Paged MQA layer == contiguous-cache MQA (the invariant of the reference's
tests/test_paged_mqa.py:9-71), fp32, atol 1e-5.

The contiguous side is the oracle's CPU restatement: same weights,
interleaved RoPE at absolute positions, a growing dense K/V cache and
bottom-right causal SDPA.
"""
from types import SimpleNamespace

import pytest
import torch
import torch.nn.functional as F

from oracle import torch_ref
from serving.allocator import BlockAllocator
from serving.kv_pool import KVPool
from serving.paged_mqa import MQA_Paged
from serving.sequence import Sequence

pytestmark = pytest.mark.gpu
DEV = "cuda"
CFG = SimpleNamespace(d_model=256, num_heads=8, num_kv_heads=1, bias=False, dropout=0.0,
                      max_seq_len=512)


class ContiguousMQA:
    """CPU fp32 MQA with a dense per-sequence cache (MQA_Cached semantics)."""

    def __init__(self, mqa):
        self.w = {k: v.detach().cpu().float() for k, v in mqa.state_dict().items()}
        self.hq, self.hkv, self.d = mqa.num_heads, mqa.num_kv_heads, mqa.headdim
        self.cos, self.sin = torch_ref.rope_tables(self.d, CFG.max_seq_len)
        self.k = self.v = None

    def step(self, x, start):
        x = x.cpu().float().reshape(-1, CFG.d_model)
        T = x.shape[0]
        pos = torch.arange(start, start + T)
        q = F.linear(x, self.w["q_proj.weight"]).view(T, self.hq, self.d)
        k = F.linear(x, self.w["k_proj.weight"]).view(T, self.hkv, self.d)
        v = F.linear(x, self.w["v_proj.weight"]).view(T, self.hkv, self.d)
        c, s = self.cos[pos], self.sin[pos]
        q = torch_ref.rope_rotate(q.transpose(0, 1), c, s).transpose(0, 1)
        k = torch_ref.rope_rotate(k.transpose(0, 1), c, s).transpose(0, 1)
        self.k = k if self.k is None else torch.cat([self.k, k])
        self.v = v if self.v is None else torch.cat([self.v, v])
        o = torch_ref.sdpa_one(q, self.k, self.v, causal=True)
        return F.linear(o.reshape(T, -1), self.w["out.weight"])


@pytest.mark.parametrize("prompt_len", [1, 16, 17, 20])
def test_paged_matches_contiguous(prompt_len):
    print(f"[paged mqa] prompt_len={prompt_len}", flush=True)
    torch.manual_seed(0)
    mqa = MQA_Paged(CFG, backend="pytorch").to(DEV).eval()
    ref = ContiguousMQA(mqa)
    alloc = BlockAllocator(64)
    pool = KVPool(1, 16, 64, 1, 32, torch.float32, DEV)
    seq = Sequence(0, [0] * prompt_len, 16)
    seq.ensure_blocks(alloc)
    with torch.no_grad():
        x = torch.randn(1, prompt_len, 256, device=DEV)
        out = mqa.forward_paged(x, pool, 0, seq.block_table, start=0)
        torch.testing.assert_close(out.cpu().reshape(prompt_len, -1), ref.step(x, 0),
                                   rtol=0, atol=1e-5)
        for _ in range(20):
            x = torch.randn(1, 1, 256, device=DEV)
            seq.append_token(0)
            seq.ensure_blocks(alloc)
            start = seq.num_tokens - 1
            out = mqa.forward_paged(x, pool, 0, seq.block_table, start=start)
            torch.testing.assert_close(out.cpu().reshape(1, -1), ref.step(x, start),
                                       rtol=0, atol=1e-5)


def test_two_interleaved_sequences():
    torch.manual_seed(0)
    mqa = MQA_Paged(CFG, backend="pytorch").to(DEV).eval()
    alloc = BlockAllocator(64)
    pool = KVPool(1, 16, 64, 1, 32, torch.float32, DEV)
    seqs = [Sequence(i, [0] * 16, 16) for i in range(2)]
    refs = [ContiguousMQA(mqa) for _ in range(2)]
    for s in seqs:
        s.ensure_blocks(alloc)
    assert [s.block_table for s in seqs] == [[1], [2]]
    with torch.no_grad():
        for s, r in zip(seqs, refs):
            x = torch.randn(1, 16, 256, device=DEV)
            out = mqa.forward_paged(x, pool, 0, s.block_table, start=0)
            torch.testing.assert_close(out.cpu().reshape(16, -1), r.step(x, 0), rtol=0, atol=1e-5)
        for _ in range(40):
            for s, r in zip(seqs, refs):
                x = torch.randn(1, 1, 256, device=DEV)
                s.append_token(0)
                s.ensure_blocks(alloc)
                start = s.num_tokens - 1
                out = mqa.forward_paged(x, pool, 0, s.block_table, start=start)
                torch.testing.assert_close(out.cpu().reshape(1, -1), r.step(x, start),
                                           rtol=0, atol=1e-5)
    a, b = seqs
    assert set(a.block_table).isdisjoint(b.block_table)
    assert any(y - x != 1 for x, y in zip(a.block_table, a.block_table[1:]))


def test_batched_ragged_step_matches_per_sequence():
    # one forward_paged_batched over a mixed prefill/decode batch equals the
    # same tokens run sequence by sequence
    torch.manual_seed(1)
    mqa = MQA_Paged(CFG).to(DEV).eval()
    alloc = BlockAllocator(64)
    pool_a = KVPool(1, 16, 64, 1, 32, torch.float32, DEV)
    pool_b = KVPool(1, 16, 64, 1, 32, torch.float32, DEV)
    lens = [5, 33, 1]
    seqs = [Sequence(i, [0] * n, 16) for i, n in enumerate(lens)]
    for s in seqs:
        s.ensure_blocks(alloc)
    x = torch.randn(sum(lens), 256, device=DEV)
    qsl = [0, 5, 38, 39]
    positions = [p for n in lens for p in range(n)]
    with torch.no_grad():
        out = mqa.forward_paged_batched(x, pool_a, 0, positions, qsl,
                                        [s.block_table for s in seqs])
        parts = [mqa.forward_paged(x[qsl[i]:qsl[i + 1]][None], pool_b, 0, s.block_table, 0)[0]
                 for i, s in enumerate(seqs)]
    torch.testing.assert_close(out, torch.cat(parts), rtol=0, atol=1e-6)
    # K/V come from projections of differently sized batches, which round
    # differently in the last bit; the rows must land in the same slots
    torch.testing.assert_close(pool_a.kv, pool_b.kv, rtol=0, atol=1e-6)
    assert torch.equal(pool_a.kv != 0, pool_b.kv != 0)
