"""The greedy decode step captured as a HIP graph (serving/graph_step.py)
against the same step run eagerly.

Two identical copies of a batch (pool, metadata, tokens) advance in
lock-step: one by DecodeStepGraph.replay(), one by the eager
forward_step + argmax. Every replay must produce exactly the eager step's
tokens and logits, and the pools must stay bit-identical, with unrelated
eager work and host synchronisations between the replays. Covered in fp32
(BASELINE config-1 model shape) and in bf16 with the MFMA decode kernel
(config-4 head shape, a smaller model); contexts grow across block
boundaries during the replays.
"""
import pytest
import torch

from serving import workloads
from serving.graph_step import DecodeStepGraph
from serving.kv_pool import KVPool
from serving.layers import ModelConfig
from serving.paged_meta import pack_batch_meta
from serving.paged_model import PagedTransformer

pytestmark = pytest.mark.gpu
DEV = "cuda"


def make_batch(cfg, dtype, n_seq, lens, bs, nb, steps, seed):
    dev = torch.device(DEV)
    tables = workloads.permuted_tables([int(x) + steps + 2 for x in lens], bs, nb, seed)
    pool = KVPool(cfg.num_layers, bs, nb, cfg.num_kv_heads, cfg.head_dim, dtype, dev)
    g = torch.Generator(device=dev).manual_seed(seed)
    for l in range(cfg.num_layers):
        pool.kv[l].normal_(generator=g)
    meta = pack_batch_meta(tables, list(range(n_seq + 1)), [int(x) for x in lens], n_seq, dev, bs)
    meta.max_kv_len = int(max(lens)) + steps + 2
    ids = torch.randint(0, cfg.vocab_size, (n_seq,), generator=g, device=dev)
    return pool, meta, ids


def clone_batch(pool, meta, ids):
    p2 = KVPool(pool.num_layers, pool.block_size, pool.num_blocks, pool.num_kv_heads,
                pool.head_dim, pool.dtype, pool.device)
    p2.kv.copy_(pool.kv)
    m2 = type(meta)(**{f: (getattr(meta, f).clone() if torch.is_tensor(getattr(meta, f))
                           else getattr(meta, f)) for f in meta.__dataclass_fields__})
    return p2, m2, ids.clone()


@pytest.mark.parametrize("dtype,cfg,n_seq,lo,hi", [
    (torch.float32, ModelConfig(vocab_size=50257, d_model=128, num_layers=4, num_heads=4,
                                num_kv_heads=1, max_seq_len=512), 4, 20, 200),
    (torch.bfloat16, ModelConfig(vocab_size=4096, d_model=1024, num_layers=2, num_heads=16,
                                 num_kv_heads=1, max_seq_len=4096), 32, 256, 2048),
])
def test_graph_replays_match_eager_steps(dtype, cfg, n_seq, lo, hi):
    print(f"[graph step] {dtype} layers={cfg.num_layers} n_seq={n_seq}", flush=True)
    steps = 6
    torch.manual_seed(0)
    model = PagedTransformer(cfg).to(DEV, dtype).eval()
    lens = workloads.lengths_uniform(n_seq, lo, hi, seed=3)
    pool_a, meta_a, ids_a = make_batch(cfg, dtype, n_seq, lens, 16, 4096, steps, seed=5)
    pool_b, meta_b, ids_b = clone_batch(pool_a, meta_a, ids_a)

    def eager_step():
        nonlocal ids_a
        with torch.no_grad():
            logits = model.forward_step(ids_a, pool_a, meta_a)
        ids_a = logits.argmax(-1)
        meta_a.positions.add_(1)
        meta_a.start_pos.add_(1)
        meta_a.seq_lens.add_(1)
        return logits

    graph = DecodeStepGraph(model, pool_b, meta_b, ids_b, warmup=1)  # one real step
    eager_step()
    torch.cuda.synchronize()
    assert torch.equal(graph.ids, ids_a), "warm-up step differs"
    junk = torch.randn(1 << 16, device=DEV)
    for k in range(steps):
        toks = graph.replay()
        torch.cuda.synchronize()
        ref_logits = eager_step()
        junk = junk * 1.0001 + 1.0       # unrelated eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(toks, ids_a), f"replay {k}: tokens differ"
        assert torch.equal(graph.logits, ref_logits), f"replay {k}: logits differ"
        assert torch.equal(meta_b.seq_lens, meta_a.seq_lens), f"replay {k}: metadata differs"
    assert torch.equal(pool_b.kv, pool_a.kv), "pools differ after the replays"


def test_graph_rejects_prefill_batch():
    cfg = ModelConfig(vocab_size=128, d_model=64, num_layers=1, num_heads=4, num_kv_heads=1,
                      max_seq_len=64)
    model = PagedTransformer(cfg).to(DEV).eval()
    pool = KVPool(1, 16, 64, 1, cfg.head_dim, torch.float32, torch.device(DEV))
    meta = pack_batch_meta([[1, 2]], [0, 3], [0, 1, 2], 3, torch.device(DEV), 16)
    with pytest.raises(ValueError):
        DecodeStepGraph(model, pool, meta, torch.zeros(3, dtype=torch.long, device=DEV))


def test_graph_keeps_its_workspace_when_eager_calls_grow_theirs():
    """Capture, then an unrelated eager attention call that needs a larger
    process-wide workspace (so the caching allocator frees the old one),
    then allocations that may reuse the freed memory (filled with non-zero
    words, which would look like dirty arrival counters): every replay must
    still equal the eager step bit for bit."""
    from serving.fake_paged_attn import paged_mqa_decode
    dtype = torch.bfloat16
    cfg = ModelConfig(vocab_size=4096, d_model=1024, num_layers=2, num_heads=16,
                      num_kv_heads=1, max_seq_len=4096)
    n_seq, steps = 32, 4
    print(f"[graph step] workspace growth after capture, n_seq={n_seq}", flush=True)
    torch.manual_seed(0)
    model = PagedTransformer(cfg).to(DEV, dtype).eval()
    lens = workloads.lengths_uniform(n_seq, 256, 2048, seed=4)
    pool_a, meta_a, ids_a = make_batch(cfg, dtype, n_seq, lens, 16, 4096, steps, seed=6)
    pool_b, meta_b, ids_b = clone_batch(pool_a, meta_a, ids_a)
    graph = DecodeStepGraph(model, pool_b, meta_b, ids_b, warmup=1)
    with torch.no_grad():
        logits = model.forward_step(ids_a, pool_a, meta_a)
    ids_a = logits.argmax(-1)
    for t in (meta_a.positions, meta_a.start_pos, meta_a.seq_lens):
        t.add_(1)
    # grow the process-wide workspace (persistent-kernel problem, ~9 MB of
    # scratch), release the old buffer, and reuse freed memory
    prob = workloads.cfg5_problem(torch.device(DEV), seed=1, bs=16)
    paged_mqa_decode(prob.q, prob.k_pool, prob.v_pool, prob.block_tables, prob.seq_lens,
                     max_kv_len=int(prob.lens.max()))
    torch.cuda.synchronize()
    del prob
    torch.cuda.empty_cache()
    junk = [torch.full((1 << 18,), 7, dtype=torch.int32, device=DEV) for _ in range(64)]
    torch.cuda.synchronize()
    for k in range(steps):
        toks = graph.replay()
        torch.cuda.synchronize()
        with torch.no_grad():
            ref = model.forward_step(ids_a, pool_a, meta_a)
        ids_a = ref.argmax(-1)
        for t in (meta_a.positions, meta_a.start_pos, meta_a.seq_lens):
            t.add_(1)
        torch.cuda.synchronize()
        assert torch.equal(toks, ids_a), f"replay {k}: tokens differ"
        assert torch.equal(graph.logits, ref), f"replay {k}: logits differ"
    assert torch.equal(pool_b.kv, pool_a.kv), "pools differ after the replays"
    del junk
