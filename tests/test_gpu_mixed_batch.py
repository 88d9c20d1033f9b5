"""Batches that mix decode sequences (one query token) with chunked-prefill
sequences (many), as in BASELINE config 5's step (256 decodes + a 512-token
chunked-prefill append for 4 new sequences). One library call splits such a
batch: the decode sequences run on an MFMA decode kernel, the prefill
sequences on the prefill kernel.

  - outputs and lse against the fp64 oracle (bf16 / fp16: 2e-2 absolute),
    with the decode part on the split-K partition kernel, the persistent
    kernel, and the automatic choice;
  - fused append (pkv_paged_attention_append) of such a batch against
    KVPool.write_from_table + attention: pools and outputs bit-identical;
  - sequences without a query this step inside the mixed batch.
"""
import numpy as np
import pytest
import torch

from oracle import paged_ref as ref
from serving import _native, workloads
from serving.fake_paged_attn import paged_attention_append_meta, paged_attention_meta
from serving.kv_pool import KVPool
from serving.paged_meta import pack_batch_meta

pytestmark = pytest.mark.gpu
DEV = "cuda"


def np64(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def mixed_batch(n_dec, chunks, hq, d, dtype, bs, seed, empty=(), hkv=1, shuffle=False):
    """n_dec decode sequences (lognormal contexts, one new token each) then
    len(chunks) prefill sequences; chunks[i] = (prior context, chunk tokens).
    Sequences listed in `empty` get no query this step; shuffle: the
    sequences in a seeded random order instead (decode and prefill mixed)."""
    dec_lens = workloads.lengths_lognormal(n_dec, 600, 3000, seed)
    q_lens, starts = [], []
    for i, L in enumerate(dec_lens):
        q_lens.append(0 if i in empty else 1)
        starts.append(int(L))
    for prior, n in chunks:
        q_lens.append(n)
        starts.append(prior)
    if shuffle:
        perm = np.random.default_rng(seed).permutation(len(q_lens))
        q_lens = [q_lens[i] for i in perm]
        starts = [starts[i] for i in perm]
    ends = [s + q for s, q in zip(starts, q_lens)]
    tables = workloads.permuted_tables([max(e, s + 1) for s, e in zip(starts, ends)], bs,
                                       1 << 15, seed)
    pool = KVPool(1, bs, 1 << 15, hkv, d, dtype, torch.device(DEV))
    g = torch.Generator(device=DEV).manual_seed(seed)
    pool.kv.normal_(generator=g)
    T = sum(q_lens)
    qsl = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int64).tolist()
    positions = [p for s, q in zip(starts, q_lens) for p in range(s, s + q)]
    meta = pack_batch_meta(tables, qsl, positions, T, torch.device(DEV), bs)
    q = torch.randn(T, hq, d, generator=g, device=DEV).to(dtype)
    k = torch.randn(T, hkv, d, generator=g, device=DEV).to(dtype)
    v = torch.randn(T, hkv, d, generator=g, device=DEV).to(dtype)
    return pool, meta, q, k, v


def oracle(pool, meta, q):
    return ref.paged_attention(np64(q), np64(pool.kv[0, 0]), np64(pool.kv[0, 1]),
                               meta.block_tables.cpu().numpy(), meta.seq_lens.cpu().numpy(),
                               meta.query_start_loc.cpu().numpy())


@pytest.mark.parametrize("part_tokens", [0, 512, _native.PART_PERSISTENT],
                         ids=["auto", "partition", "persistent"])
@pytest.mark.parametrize("hq,d,dtype", [(32, 128, torch.bfloat16), (16, 64, torch.float16)])
def test_mixed_batch_vs_oracle(part_tokens, hq, d, dtype):
    print(f"[mixed] hq={hq} d={d} {dtype} part_tokens={part_tokens}", flush=True)
    # 4 new sequences' 128-token chunks (no prior context) and one later
    # chunk of a longer prompt
    pool, meta, q, k, v = mixed_batch(48, [(0, 128), (0, 128), (0, 128), (0, 128), (700, 96)],
                                      hq, d, dtype, 16, seed=31, empty=(5,))
    pool.write_from_table(0, k, v, meta)
    lse = torch.empty(q.shape[0], hq, device=DEV)
    out = torch.empty_like(q)
    from serving.fake_paged_attn import _launch
    _launch(q, pool.kv[0, 0], pool.kv[0, 1], meta.block_tables, meta.seq_lens,
            meta.query_start_loc, meta.num_seqs, meta.max_q_len, meta.max_kv_len, 0.0, True,
            out, lse, part_tokens)
    torch.cuda.synchronize()
    eo, el = oracle(pool, meta, q)
    got = np64(out)
    assert np.all(np.isfinite(got))
    err = np.abs(got - eo).max()
    assert err <= 2e-2, f"max err {err:.3e}"
    fin = np.isfinite(el)
    np.testing.assert_allclose(lse.cpu().numpy()[fin], el[fin], rtol=0, atol=2e-2)


@pytest.mark.parametrize("bound", [0, 8192])
def test_mixed_batch_fused_append_equals_two_calls(bound):
    print(f"[mixed fused] bound={bound}", flush=True)
    pool_a, meta, q, k, v = mixed_batch(64, [(0, 128), (0, 128), (300, 128), (0, 128)], 32, 128,
                                        torch.bfloat16, 16, seed=32)
    if bound:
        meta.max_kv_len = bound  # the persistent decode kernel
    pool_b = KVPool(1, 16, pool_a.num_blocks, 1, 128, torch.bfloat16, torch.device(DEV))
    pool_b.kv.copy_(pool_a.kv)
    lse_a = torch.empty(q.shape[0], 32, device=DEV)
    lse_b = torch.empty(q.shape[0], 32, device=DEV)
    pool_a.write_from_table(0, k, v, meta)
    out_a = paged_attention_meta(q, pool_a.kv[0, 0], pool_a.kv[0, 1], meta, lse=lse_a)
    out_b = paged_attention_append_meta(q, k, v, pool_b, 0, meta, lse=lse_b)
    torch.cuda.synchronize()
    assert torch.equal(pool_a.kv, pool_b.kv), "pools differ"
    assert torch.equal(out_a, out_b), "outputs differ"
    assert torch.equal(lse_a, lse_b), "lse differs"
    eo, _ = oracle(pool_a, meta, q)
    assert np.abs(np64(out_b) - eo).max() <= 2e-2


# The fused mixed call with the persistent decode kernel at head dim 128 runs
# as one launch (decode shares and prefill pairs in one grid, the decode
# shares taking their new rows from k_new / v_new); the two-call form runs
# the same kernels' code on rows read back from the pool. Both are bit for
# bit the same: every (sequence, kv head) gets the same shares of the
# persistent kernel's cost line either way.
@pytest.mark.parametrize("hq,hkv,dtype,bs,shuffle", [
    (32, 1, torch.bfloat16, 16, False),
    (32, 1, torch.float16, 32, True),
    (16, 1, torch.bfloat16, 8, True),
    (64, 2, torch.bfloat16, 16, True),
    (32, 2, torch.float16, 16, False),
], ids=["g32-bf16-bs16", "g32-f16-bs32-shuffled", "g16-bf16-bs8-shuffled",
        "g32x2-bf16-bs16-shuffled", "g16x2-f16-bs16"])
def test_mixed_one_launch_equals_two_calls(hq, hkv, dtype, bs, shuffle):
    print(f"[mixed one launch] hq={hq} hkv={hkv} {dtype} bs={bs} shuffle={shuffle}", flush=True)
    pool_a, meta, q, k, v = mixed_batch(
        96, [(0, 128), (0, 77), (500, 128), (0, 1), (0, 256)], hq, 128, dtype, bs, seed=33,
        empty=(3, 40), hkv=hkv, shuffle=shuffle)
    meta.max_kv_len = 8192  # the persistent decode kernel
    pool_b = KVPool(1, bs, pool_a.num_blocks, hkv, 128, dtype, torch.device(DEV))
    pool_b.kv.copy_(pool_a.kv)
    lse_a = torch.empty(q.shape[0], hq, device=DEV)
    lse_b = torch.empty(q.shape[0], hq, device=DEV)
    pool_a.write_from_table(0, k, v, meta)
    out_a = paged_attention_meta(q, pool_a.kv[0, 0], pool_a.kv[0, 1], meta, lse=lse_a)
    out_b = paged_attention_append_meta(q, k, v, pool_b, 0, meta, lse=lse_b)
    # the same call again: the arrival counters were left at zero
    out_c = paged_attention_append_meta(q, k, v, pool_b, 0, meta)
    torch.cuda.synchronize()
    assert torch.equal(pool_a.kv, pool_b.kv), "pools differ"
    assert torch.equal(out_a, out_b), "outputs differ"
    assert torch.equal(lse_a, lse_b), "lse differs"
    assert torch.equal(out_b, out_c), "a repeated call differs"
    eo, el = oracle(pool_a, meta, q)
    assert np.abs(np64(out_b) - eo).max() <= 2e-2
    fin = np.isfinite(el)
    np.testing.assert_allclose(lse_b.cpu().numpy()[fin], el[fin], rtol=0, atol=2e-2)


# max_q_len is a bound: a fused mixed call whose batch holds no sequence
# with more than one query token still appends every row (the prefill
# kernel, which appends the decode rows of a mixed batch, has no pair to
# run), with the two-call form as reference.
@pytest.mark.parametrize("bound", [0, 8192], ids=["partition", "persistent"])
def test_mixed_call_without_prefill_rows_still_appends(bound):
    print(f"[mixed no prefill] bound={bound}", flush=True)
    pool_a, meta, q, k, v = mixed_batch(40, [], 32, 128, torch.bfloat16, 16, seed=34, empty=(7,))
    meta.max_q_len = 4
    if bound:
        meta.max_kv_len = bound
    pool_b = KVPool(1, 16, pool_a.num_blocks, 1, 128, torch.bfloat16, torch.device(DEV))
    pool_b.kv.copy_(pool_a.kv)
    pool_a.write_from_table(0, k, v, meta)
    out_a = paged_attention_meta(q, pool_a.kv[0, 0], pool_a.kv[0, 1], meta)
    out_b = paged_attention_append_meta(q, k, v, pool_b, 0, meta)
    torch.cuda.synchronize()
    assert torch.equal(pool_a.kv, pool_b.kv), "pools differ"
    assert torch.equal(out_a, out_b), "outputs differ"


# The one-launch form at its edges: no decode sequence at all (the decode
# workgroups find nothing to do), a single one, and a single prefill
# sequence beside many decodes.
@pytest.mark.parametrize("n_dec,chunks", [
    (0, [(0, 128), (300, 64)]),
    (1, [(0, 128), (0, 200)]),
    (130, [(50, 40)]),
], ids=["prefill-only", "one-decode", "one-prefill"])
def test_mixed_one_launch_edges(n_dec, chunks):
    print(f"[mixed one launch edges] n_dec={n_dec} chunks={chunks}", flush=True)
    pool_a, meta, q, k, v = mixed_batch(n_dec, chunks, 32, 128, torch.bfloat16, 16, seed=35)
    meta.max_kv_len = 8192  # the persistent decode kernel
    pool_b = KVPool(1, 16, pool_a.num_blocks, 1, 128, torch.bfloat16, torch.device(DEV))
    pool_b.kv.copy_(pool_a.kv)
    pool_a.write_from_table(0, k, v, meta)
    out_a = paged_attention_meta(q, pool_a.kv[0, 0], pool_a.kv[0, 1], meta)
    out_b = paged_attention_append_meta(q, k, v, pool_b, 0, meta)
    torch.cuda.synchronize()
    assert torch.equal(pool_a.kv, pool_b.kv), "pools differ"
    assert torch.equal(out_a, out_b), "outputs differ"
    eo, _ = oracle(pool_a, meta, q)
    assert np.abs(np64(out_b) - eo).max() <= 2e-2


def test_mixed_one_launch_graph_replays():
    """The one-launch mixed call captured in a HIP graph (with a private
    workspace): several replays, with eager calls of the same step in
    between, each give the eager step's pool and output bit for bit."""
    print("[mixed one launch graph]", flush=True)
    pool, meta, q, k, v = mixed_batch(80, [(0, 128), (200, 96)], 32, 128, torch.bfloat16, 16,
                                      seed=36)
    meta.max_kv_len = 8192  # the persistent decode kernel: one launch
    base = pool.kv.clone()
    ref = paged_attention_append_meta(q, k, v, pool, 0, meta)
    torch.cuda.synchronize()
    ref_pool = pool.kv.clone()
    ws = _native.Workspace()
    out = torch.empty_like(q)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with _native.workspace_scope(ws), torch.cuda.stream(side):
        paged_attention_append_meta(q, k, v, pool, 0, meta, out=out)  # warm-up
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with _native.workspace_scope(ws), torch.cuda.graph(g):
        paged_attention_append_meta(q, k, v, pool, 0, meta, out=out)
    for r in range(3):
        pool.kv.copy_(base)
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {r}: outputs differ"
        assert torch.equal(pool.kv, ref_pool), f"replay {r}: pools differ"
        eager = paged_attention_append_meta(q, k, v, pool, 0, meta)  # eager work between
        torch.cuda.synchronize()
        assert torch.equal(eager, ref)
