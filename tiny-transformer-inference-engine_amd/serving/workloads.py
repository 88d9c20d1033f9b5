"""Synthetic, seeded workloads of the benchmark configurations (shared by the
parity tests and bench.py). All lengths, tables and values are drawn from
explicit seeds so every run sees identical inputs.

  cfg2  isolated decode op: N=32, Hq=8, Hkv=1, D=32, BS=16, pool 1024
        blocks, context U[64, 256], tables a random non-overlapping
        permutation of pool blocks.
  cfg3  append: 64 x 128-token prefill, Hkv=1, D=64, pool 4096 blocks,
        blocks from a shuffled free list; then 64 ragged single-token appends.
  cfg4  model decode step: N=128, context U[256, 2048], Hq=16, Hkv=1, D=64,
        pool 16384 blocks.
  cfg5  long-context stress: N=256, Hq=32, Hkv=1, D=128, lognormal context
        (mean 1024, sigma 1, capped at 8192), block size 16 or 32, tables
        fragmented by a seeded interleaved allocate/free trace.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch

from .allocator import BlockAllocator


def lengths_uniform(n, lo, hi, seed):
    return np.random.default_rng(seed).integers(lo, hi + 1, size=n).astype(np.int64)


def lengths_lognormal(n, mean, cap, seed, sigma=1.0):
    """Lognormal with the given mean (mu = ln(mean) - sigma^2/2), >= 1, capped."""
    mu = math.log(mean) - sigma * sigma / 2.0
    x = np.random.default_rng(seed).lognormal(mu, sigma, size=n)
    return np.clip(np.rint(x), 1, cap).astype(np.int64)


def permuted_tables(lens, bs, num_blocks, seed):
    """Non-overlapping tables from a random permutation of blocks 1..NB-1."""
    nblk = [(int(x) + bs - 1) // bs for x in lens]
    perm = np.random.default_rng(seed).permutation(np.arange(1, num_blocks))
    if sum(nblk) > len(perm):
        raise ValueError(f"pool of {num_blocks} blocks too small for {sum(nblk)} blocks")
    tables, cur = [], 0
    for nb in nblk:
        tables.append(perm[cur:cur + nb].tolist())
        cur += nb
    return tables


def fragmented_tables(lens, bs, num_blocks, seed, filler_frac=0.35):
    """Block tables grown the way a serving engine grows them under churn:
    filler requests are admitted and retired at random while the real
    sequences grow one block at a time, round-robin, so each table ends up
    scattered over the pool (BlockAllocator's LIFO reuse order)."""
    rng = np.random.default_rng(seed)
    alloc = BlockAllocator(num_blocks)
    need = [(int(x) + bs - 1) // bs for x in lens]
    tables = [[] for _ in lens]
    fillers = []
    budget = int(filler_frac * (num_blocks - 1 - sum(need)))
    while True:
        active = [i for i in range(len(lens)) if len(tables[i]) < need[i]]
        if not active:
            break
        for i in active:
            tables[i].append(alloc.allocate())
            r = rng.random()
            if r < 0.05 and alloc.num_free > sum(need) - sum(map(len, tables)) + 8:
                held = sum(len(f) for f in fillers)
                if held < budget:
                    fillers.append(alloc.allocate_n(int(rng.integers(1, 5))))
            elif r < 0.09 and fillers:
                alloc.free(fillers.pop(int(rng.integers(0, len(fillers)))))
    return tables


def tables_tensor(tables, device, width=None):
    width = max(len(t) for t in tables) if width is None else width
    out = np.zeros((len(tables), max(width, 1)), dtype=np.int32)
    for i, t in enumerate(tables):
        out[i, :len(t)] = t
    return torch.from_numpy(out).to(device)


@dataclass
class DecodeProblem:
    q: torch.Tensor            # [N, Hq, D]
    k_pool: torch.Tensor       # [NB, BS, Hkv, D]
    v_pool: torch.Tensor
    block_tables: torch.Tensor  # int32 [N, max_blk]
    seq_lens: torch.Tensor      # int32 [N]
    lens: np.ndarray
    tables: list
    hq: int
    hkv: int
    d: int
    bs: int

    @property
    def n_seq(self):
        return len(self.lens)

    def kv_bytes(self):
        return int(self.lens.sum()) * self.hkv * self.d * 2 * self.k_pool.element_size()


def decode_problem(lens, hq, hkv, d, bs, num_blocks, dtype, device, seed,
                   fragmented=False, garbage=None):
    """Random paged decode problem: Q, K, V ~ N(0,1) (seeded, generated on
    `device`), one query per sequence. With `garbage`, every slot no sequence
    owns (other blocks and the tail of each last block) holds that value."""
    lens = np.asarray(lens, dtype=np.int64)
    tables = (fragmented_tables(lens, bs, num_blocks, seed) if fragmented
              else permuted_tables(lens, bs, num_blocks, seed))
    g = torch.Generator(device=device).manual_seed(seed)
    shape = (num_blocks, bs, hkv, d)
    k_pool = torch.randn(shape, generator=g, device=device, dtype=torch.float32).to(dtype)
    v_pool = torch.randn(shape, generator=g, device=device, dtype=torch.float32).to(dtype)
    if garbage is not None:
        owned = torch.zeros(num_blocks * bs, dtype=torch.bool, device=device)
        for t, n in zip(tables, lens):
            idx = (torch.as_tensor(t, device=device, dtype=torch.long)[:, None] * bs
                   + torch.arange(bs, device=device)).reshape(-1)[:int(n)]
            owned[idx] = True
        k_pool.view(-1, hkv, d)[~owned] = garbage
        v_pool.view(-1, hkv, d)[~owned] = garbage
    q = torch.randn((len(lens), hq, d), generator=g, device=device, dtype=torch.float32).to(dtype)
    return DecodeProblem(q=q, k_pool=k_pool, v_pool=v_pool,
                         block_tables=tables_tensor(tables, device),
                         seq_lens=torch.as_tensor(lens, dtype=torch.int32, device=device),
                         lens=lens, tables=tables, hq=hq, hkv=hkv, d=d, bs=bs)


def cfg2_problem(dtype, device, seed=0):
    return decode_problem(lengths_uniform(32, 64, 256, seed), 8, 1, 32, 16, 1024, dtype,
                          device, seed)


def cfg4_problem(device, seed=0, dtype=torch.bfloat16):
    return decode_problem(lengths_uniform(128, 256, 2048, seed), 16, 1, 64, 16, 16384,
                          dtype, device, seed)


def cfg5_problem(device, seed=0, bs=16, dtype=torch.bfloat16):
    lens = lengths_lognormal(256, 1024, 8192, seed)
    need = int(sum((int(x) + bs - 1) // bs for x in lens))
    num_blocks = 1 << max(10, math.ceil(math.log2(need * 1.6 + 1)))
    return decode_problem(lens, 32, 1, 128, bs, num_blocks, dtype, device, seed,
                          fragmented=True)


@dataclass
class MixedProblem:
    pool: object      # KVPool (one layer)
    meta: object      # PagedBatchMeta of the step
    q: torch.Tensor   # [T, 32, 128]
    k: torch.Tensor   # [T, 1, 128] rows appended this step
    v: torch.Tensor
    dec_lens: np.ndarray  # decode contexts before the step
    chunk: int
    n_new: int


def cfg5_mixed_problem(device, chunk=128, n_new=4, seed=0, bs=16, dtype=torch.bfloat16):
    """One config-5 step: the 256 decode sequences (lognormal contexts) each
    append one token and attend over it, and n_new new sequences append and
    attend over their first `chunk` prompt tokens (chunked prefill), in one
    batch; tables fragmented as in cfg5_problem, from one allocator."""
    from .kv_pool import KVPool
    from .paged_meta import pack_batch_meta

    dec = lengths_lognormal(256, 1024, 8192, seed)
    starts = [int(x) for x in dec] + [0] * n_new
    q_lens = [1] * len(dec) + [chunk] * n_new
    ends = [s + q for s, q in zip(starts, q_lens)]
    need = int(sum((e + bs - 1) // bs for e in ends))
    num_blocks = 1 << max(10, math.ceil(math.log2(need * 1.6 + 1)))
    tables = fragmented_tables(ends, bs, num_blocks, seed)
    dev = torch.device(device)
    pool = KVPool(1, bs, num_blocks, 1, 128, dtype, dev)
    g = torch.Generator(device=dev).manual_seed(seed)
    pool.kv.normal_(generator=g)
    T = sum(q_lens)
    qsl = np.concatenate([[0], np.cumsum(q_lens)]).tolist()
    positions = [p for s, q in zip(starts, q_lens) for p in range(s, s + q)]
    meta = pack_batch_meta(tables, qsl, positions, T, dev, bs)
    q = torch.randn(T, 32, 128, generator=g, device=dev).to(dtype)
    k = torch.randn(T, 1, 128, generator=g, device=dev).to(dtype)
    v = torch.randn(T, 1, 128, generator=g, device=dev).to(dtype)
    return MixedProblem(pool=pool, meta=meta, q=q, k=k, v=v, dec_lens=dec, chunk=chunk,
                        n_new=n_new)
