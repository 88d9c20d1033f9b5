"""fp8 KV pools (CacheConfig.kv_dtype = torch.float8_e4m3fn, reference
models/model_config.py:49, :77-88; the pool stores what index_put into a
float8 tensor stores, serving/kv_pool.py:57-70).

  - append: rows of bf16 / fp16 / fp32 (with NaN, infinities, overflow,
    subnormals and rounding ties planted) written through KVPool.write and
    write_from_table: the pool bytes equal the oracle's rounding
    (oracle.paged_ref.e4m3_codes, pinned against torch on the CPU) and
    torch's own index_put into a float8 pool on the GPU, bit for bit;
  - gather returns the pool's bytes;
  - decode attention (split-K partition and persistent kernels, 16 and 32
    heads, D 64 and 128) against the fp64 oracle on the fp8 values of the
    pools, within 2e-2 absolute;
  - the fused append + attention call equals the two-call path (pool bytes
    and outputs bit for bit), and a mixed decode + chunked-prefill step
    matches the oracle;
  - a model decode step on an fp8 pool replayed from a HIP graph equals the
    eager step bit for bit.
"""
import numpy as np
import pytest
import torch

from oracle import paged_ref as ref
from serving import _native, workloads
from serving.allocator import BlockAllocator
from serving.fake_paged_attn import (paged_attention_append_meta, paged_attention_meta,
                                     paged_mqa_decode)
from serving.kv_pool import KVPool
from serving.paged_meta import pack_batch_meta

pytestmark = pytest.mark.gpu
DEV = "cuda"
FP8 = torch.float8_e4m3fn
TOL = 2e-2
SPECIAL = [0.0, -0.0, 448.0, -448.0, 464.0, -464.0, 470.0, 480.0, 1e6, float("inf"),
           float("-inf"), float("nan"), 2.0 ** -9, 2.0 ** -10, 3 * 2.0 ** -10, 2.0 ** -6,
           1.0625, 1.1875, -1.0625, 0.01, 1e-5, 240.0, 232.0]


def _bytes(t):
    return t.detach().contiguous().view(torch.uint8).cpu().numpy()


def _rows(n, hkv, d, dtype, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    x = torch.randn(n, hkv, d, generator=g, device=DEV) * torch.exp(
        3 * torch.randn(n, hkv, d, generator=g, device=DEV))
    flat = x.view(-1)
    flat[:len(SPECIAL)] = torch.tensor(SPECIAL, device=DEV)
    return x.to(dtype)


def _fp8_values(t):
    """float64 values of an fp8 tensor through the oracle's widening."""
    return ref.e4m3_values(_bytes(t)).reshape(tuple(t.shape))


@pytest.mark.parametrize("src", [torch.bfloat16, torch.float16, torch.float32])
def test_fp8_append_bit_exact(src):
    print(f"[fp8 append] rows {src}", flush=True)
    NB, BS, HKV, D = 512, 16, 2, 64
    pool = KVPool(1, BS, NB, HKV, D, FP8, DEV)
    alloc = BlockAllocator(NB)
    tables = [alloc.allocate_n(3) for _ in range(8)]
    slots = torch.cat([pool.make_slot_mapping(0, 40, t) for t in tables])
    k = _rows(slots.numel(), HKV, D, src, 1)
    v = _rows(slots.numel(), HKV, D, src, 2)
    pool.write(0, slots, k, v)
    torch.cuda.synchronize()
    # the oracle's rounding into a zero pool
    ek = np.zeros((NB * BS, HKV, D), dtype=np.uint8)
    ev = np.zeros_like(ek)
    ref.append(ek, ev, slots.cpu().numpy(), ref.e4m3_codes(k.float().cpu().numpy()),
               ref.e4m3_codes(v.float().cpu().numpy()))
    assert np.array_equal(_bytes(pool.flat_k[0]), ek)
    assert np.array_equal(_bytes(pool.flat_v[0]), ev)
    # torch's index_put into a float8 pool on the GPU
    tk = torch.zeros(NB * BS, HKV, D, dtype=FP8, device=DEV)
    tk[slots] = k.to(FP8)
    assert np.array_equal(_bytes(pool.flat_k[0]), _bytes(tk))

    # the same rows through device metadata (in-kernel slots), one layer up
    pool2 = KVPool(2, BS, NB, HKV, D, FP8, DEV)
    meta = pack_batch_meta(tables, [40 * i for i in range(9)], list(range(40)) * 8, 320, DEV, BS)
    pool2.write_from_table(1, k, v, meta)
    torch.cuda.synchronize()
    assert np.array_equal(_bytes(pool2.flat_k[1]), ek)
    assert np.array_equal(_bytes(pool2.flat_v[1]), ev)
    assert not _bytes(pool2.kv[0]).any()

    # gather: the pool's bytes
    gk, gv = pool.gather(0, tables[3], 40)
    assert gk.dtype == FP8
    assert np.array_equal(_bytes(gk), _bytes(pool.flat_k[0][slots[120:160]]))
    assert np.array_equal(_bytes(gv), _bytes(pool.flat_v[0][slots[120:160]]))


def _fp8_problem(lens, g, d, nb, seed):
    p = workloads.decode_problem(lens, g, 1, d, 16, nb, torch.bfloat16, DEV, seed=seed)
    return p, p.k_pool.to(FP8), p.v_pool.to(FP8)


@pytest.mark.parametrize("g,d", [(16, 64), (32, 128), (16, 128), (32, 64)])
@pytest.mark.parametrize("part", [512, _native.PART_PERSISTENT])
def test_fp8_decode_against_oracle(g, d, part):
    print(f"[fp8 decode] g={g} d={d} part={part}", flush=True)
    rng = np.random.default_rng(g + d)
    lens = np.minimum(rng.lognormal(np.log(700), 1.0, size=48).astype(int) + 1, 5000)
    lens[::11] = 0
    nb = 1 << int(np.ceil(np.log2(sum((int(x) + 15) // 16 + 1 for x in lens) * 1.3)))
    p, k8, v8 = _fp8_problem(np.maximum(lens, 1), g, d, nb, seed=g * d)
    seq_lens = torch.as_tensor(lens, dtype=torch.int32, device=DEV)
    lse = torch.empty(len(lens), g, device=DEV)
    out = paged_mqa_decode(p.q, k8, v8, p.block_tables, seq_lens, lse=lse, part_tokens=part,
                           max_kv_len=int(lens.max()))
    torch.cuda.synchronize()
    eo, el = ref.paged_attention(p.q.double().cpu().numpy(), _fp8_values(k8), _fp8_values(v8),
                                 p.block_tables.cpu().numpy(), lens, None)
    got = out.double().cpu().numpy()
    assert np.all(np.isfinite(got))
    assert np.abs(got - eo).max() <= TOL
    L = lse.cpu().numpy()
    fin = np.isfinite(el)
    assert np.array_equal(np.isinf(L), ~fin)
    np.testing.assert_allclose(L[fin], el[fin], rtol=0, atol=TOL)


def test_fp8_fused_append_equals_two_calls():
    """cfg4 head shape: the decode step's append fused into the partition
    kernel against KVPool.write_from_table + paged_attention_meta."""
    print("[fp8 fused append]", flush=True)
    N, HQ, D, BS, NB = 64, 16, 64, 16, 8192
    lens = workloads.lengths_uniform(N, 200, 1500, seed=5)
    tables = workloads.permuted_tables([int(x) + 1 for x in lens], BS, NB, seed=5)
    pools = [KVPool(1, BS, NB, 1, D, FP8, DEV) for _ in range(2)]
    g = torch.Generator(device=DEV).manual_seed(5)
    init = (torch.randn(1, 2, NB, BS, 1, D, generator=g, device=DEV) * 2).to(FP8)
    for pl in pools:
        pl.kv.copy_(init)
    meta = pack_batch_meta(tables, list(range(N + 1)), [int(x) for x in lens], N, DEV, BS)
    q = torch.randn(N, HQ, D, generator=g, device=DEV).bfloat16()
    # new rows of moderate size with rounding ties and subnormals planted
    # (NaN / overflow rows are the append test's: attention over them is NaN)
    kn = (torch.randn(N, 1, D, generator=g, device=DEV) * 2).bfloat16()
    vn = (torch.randn(N, 1, D, generator=g, device=DEV) * 2).bfloat16()
    ties = torch.tensor([1.0625, 1.1875, -1.0625, 2.0 ** -10, 3 * 2.0 ** -10, 2.0 ** -9],
                        device=DEV).bfloat16()
    kn.view(-1)[:ties.numel()] = ties
    vn.view(-1)[:ties.numel()] = ties
    a = paged_attention_append_meta(q, kn, vn, pools[0], 0, meta)
    pools[1].write_from_table(0, kn, vn, meta)
    b = paged_attention_meta(q, pools[1].kv[0, 0], pools[1].kv[0, 1], meta)
    torch.cuda.synchronize()
    assert np.array_equal(_bytes(pools[0].kv), _bytes(pools[1].kv)), "pools differ"
    assert torch.equal(a.view(torch.int16), b.view(torch.int16)), "outputs differ"
    # and both against the oracle for a sample of sequences
    sample = list(range(0, N, 8))
    kv = _fp8_values(pools[0].kv[0])
    eo, _ = ref.paged_attention(q[sample].double().cpu().numpy(), kv[0], kv[1],
                                meta.block_tables.cpu().numpy()[sample],
                                meta.seq_lens.cpu().numpy()[sample], None)
    assert np.abs(a[sample].double().cpu().numpy() - eo).max() <= TOL


@pytest.mark.parametrize("bs", [16, 32])
def test_fp8_mixed_step_against_oracle(bs):
    print(f"[fp8 mixed] bs={bs}", flush=True)
    p = workloads.cfg5_mixed_problem(torch.device(DEV), chunk=128, n_new=4, seed=3, bs=bs)
    pool = KVPool(1, bs, p.pool.num_blocks, 1, 128, FP8, DEV)
    pool.kv.copy_(p.pool.kv.to(FP8))
    before = _bytes(pool.kv[0])
    lse = torch.empty(p.q.shape[0], 32, device=DEV)
    out = paged_attention_append_meta(p.q, p.k, p.v, pool, 0, p.meta, lse=lse)
    torch.cuda.synchronize()
    meta = p.meta
    ek, ev = before[0].reshape(-1, 1, 128).copy(), before[1].reshape(-1, 1, 128).copy()
    ref.append_from_table(ek, ev, ref.e4m3_codes(p.k.float().cpu().numpy()),
                          ref.e4m3_codes(p.v.float().cpu().numpy()),
                          meta.block_tables.cpu().numpy(), meta.query_start_loc.cpu().numpy(),
                          meta.start_pos.cpu().numpy(), bs)
    assert np.array_equal(_bytes(pool.flat_k[0]), ek)
    assert np.array_equal(_bytes(pool.flat_v[0]), ev)
    n_dec = len(p.dec_lens)
    seqs = list(range(0, n_dec, 16)) + list(range(n_dec, n_dec + 4))
    qsl = meta.query_start_loc.cpu().numpy()
    rows = np.concatenate([np.arange(qsl[s], qsl[s + 1]) for s in seqs])
    sub_qsl = np.concatenate([[0], np.cumsum([qsl[s + 1] - qsl[s] for s in seqs])])
    # the blocks these sequences use, as a small float64 pool
    tabs = meta.block_tables.cpu().numpy()[seqs]
    used, small = np.unique(tabs, return_inverse=True)
    small = small.reshape(tabs.shape).astype(np.int32)
    blk = torch.as_tensor(used, dtype=torch.long, device=DEV)
    kp = ref.e4m3_values(_bytes(pool.kv[0, 0][blk]))
    vp = ref.e4m3_values(_bytes(pool.kv[0, 1][blk]))
    eo, el = ref.paged_attention(p.q[torch.as_tensor(rows, device=DEV)].double().cpu().numpy(),
                                 kp, vp, small, meta.seq_lens.cpu().numpy()[seqs], sub_qsl)
    got = out[torch.as_tensor(rows, device=DEV)].double().cpu().numpy()
    assert np.all(np.isfinite(got))
    assert np.abs(got - eo).max() <= TOL
    np.testing.assert_allclose(lse[torch.as_tensor(rows, device=DEV)].cpu().numpy(), el,
                               rtol=0, atol=TOL)


def test_fp8_model_step_graph_equals_eager():
    from serving.graph_step import DecodeStepGraph
    from serving.layers import CacheConfig, EngineConfig, ModelConfig, SchedulerConfig
    from serving.paged_model import PagedTransformer
    print("[fp8 model graph]", flush=True)
    ecfg = EngineConfig(model=ModelConfig(vocab_size=4096, d_model=1024, num_layers=2,
                                          num_heads=16, num_kv_heads=1, max_seq_len=4096,
                                          dtype=torch.bfloat16),
                        cache=CacheConfig(block_size=16, num_gpu_blocks=4096, kv_dtype=FP8),
                        sched=SchedulerConfig(max_num_batched_tokens=4096))
    cfg = ecfg.model
    torch.manual_seed(0)
    model = PagedTransformer(cfg).to(DEV, torch.bfloat16).eval()
    n, steps = 32, 4
    lens = workloads.lengths_uniform(n, 256, 2048, seed=9)
    tables = workloads.permuted_tables([int(x) + steps + 2 for x in lens], 16, 4096, seed=9)
    pools = [KVPool.from_engine_config(ecfg, torch.device(DEV)) for _ in range(2)]
    assert pools[0].dtype == FP8 and ecfg.bytes_per_block == 2 * 2 * 16 * 64
    g = torch.Generator(device=DEV).manual_seed(9)
    init = torch.randn(pools[0].kv.shape, generator=g, device=DEV).to(FP8)
    metas = []
    for pl in pools:
        pl.kv.copy_(init)
        m = pack_batch_meta(tables, list(range(n + 1)), [int(x) for x in lens], n, DEV, 16)
        m.max_kv_len = int(max(lens)) + steps + 2
        metas.append(m)
    ids = torch.randint(0, cfg.vocab_size, (n,), generator=g, device=DEV)
    graph = DecodeStepGraph(model, pools[1], metas[1], ids.clone(), warmup=1)
    ids_a = ids
    for k in range(steps + 1):
        with torch.no_grad():
            logits = model.forward_step(ids_a, pools[0], metas[0])
        ids_a = logits.argmax(-1)
        for t in (metas[0].positions, metas[0].start_pos, metas[0].seq_lens):
            t.add_(1)
        if k == 0:
            torch.cuda.synchronize()
            assert torch.equal(graph.ids, ids_a), "warm-up step differs"
            continue
        toks = graph.replay()
        torch.cuda.synchronize()
        assert torch.isfinite(logits.float()).all()
        assert torch.equal(toks, ids_a), f"replay {k}: tokens differ"
        assert torch.equal(graph.logits, logits), f"replay {k}: logits differ"
    assert np.array_equal(_bytes(pools[0].kv), _bytes(pools[1].kv)), "pools differ"
