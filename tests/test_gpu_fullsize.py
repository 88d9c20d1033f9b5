"""BASELINE's two largest workloads at their full size, checked against the
oracle (not only HIP against HIP).

cfg4 decode step: the 12-layer, d_model 1024, vocab 50257 bf16 model at
batch 128 (contexts U[256, 2048], block size 16) through forward_step.
Every layer's library call (append + attention) is intercepted: the pool
layer after it must equal the layer before it with the step's K/V rows
written by oracle.paged_ref.append_from_table, bit for bit; the attention
output of all 128 sequences must match the reference's gather + SDPA path
(oracle.torch_ref.paged_attention_sdpa, fp32) on the updated pool, and 16
sampled sequences plus the shortest and the longest
oracle.paged_ref.paged_attention (fp64), within 2e-2 absolute (bf16
storage, bf16 P in the PV product). The
same step is then captured as a HIP graph and replayed against eager steps:
tokens, logits and pools bit-identical.

cfg5 mixed step: 256 decode queries (lognormal contexts, mean 1024, cap
8192) each appending one token, plus 4 new sequences appending and
attending over a 512-token prompt chunk, one fused call, at block sizes 16
and 32. Every pool slot no sequence owns holds 1e3 (the reference's
tests/test.py garbage fill), so a key read past a context or through a
wrong table entry shows. Pool rows bit-exact against the oracle's append;
every row (256 decode rows and the 4 x 512 prefill rows, causal,
bottom-right aligned: pagedattn.cu:196-207) against gather + SDPA in fp32;
the 4 prefill sequences in full and 32 decode sequences against the fp64
oracle, outputs and lse within 2e-2.
"""
import numpy as np
import pytest
import torch

from oracle import paged_ref as ref
from oracle import torch_ref
from serving import workloads
from serving.fake_paged_attn import paged_attention_append_meta
from serving.graph_step import DecodeStepGraph
from serving.kv_pool import KVPool
from serving.layers import ModelConfig
from serving.paged_meta import pack_batch_meta
from serving.paged_model import PagedTransformer
import serving.paged_mqa as paged_mqa

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = 2e-2


def _layer_cpu(pool, layer):
    """(K, V) of one pool layer as CPU bf16/fp16 tensors [slots, hkv, d]."""
    return pool.flat_k[layer].detach().cpu().clone(), pool.flat_v[layer].detach().cpu().clone()


def _bits(t):
    return t.contiguous().view(torch.int16).numpy()


def _expected_after_append(before_k, before_v, k_new, v_new, meta, bs):
    """The oracle's append (serving/paged_mqa.py:87-99 semantics) applied to
    raw bit copies of the layer."""
    ek, ev = _bits(before_k).copy(), _bits(before_v).copy()
    ref.append_from_table(ek, ev, _bits(k_new.detach().cpu()), _bits(v_new.detach().cpu()),
                          meta.block_tables.cpu().numpy(), meta.query_start_loc.cpu().numpy(),
                          meta.start_pos.cpu().numpy(), bs)
    return ek, ev


def _compact(k_flat, v_flat, tables, seqs, bs):
    """The blocks the chosen sequences' tables name, as a small float64 pool,
    and their tables renumbered into it."""
    rows = [np.asarray(tables[s]) for s in seqs]
    used = np.unique(np.concatenate(rows))
    remap = {int(b): i for i, b in enumerate(used)}
    hkv, d = k_flat.shape[1], k_flat.shape[2]
    kb = k_flat.view(-1, bs, hkv, d)[torch.as_tensor(used, dtype=torch.long)]
    vb = v_flat.view(-1, bs, hkv, d)[torch.as_tensor(used, dtype=torch.long)]
    width = max(len(r) for r in rows)
    small = np.zeros((len(seqs), width), dtype=np.int32)
    for i, r in enumerate(rows):
        small[i, :len(r)] = [remap[int(b)] for b in r]
    return (kb.float().numpy().astype(np.float64), vb.float().numpy().astype(np.float64), small)


def _close(got, want, what):
    got = got.astype(np.float64)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    err = np.abs(got - want).max()
    assert err <= TOL, f"{what}: max err {err:.3e}"


def _clone(pool, meta, ids):
    p2 = KVPool(pool.num_layers, pool.block_size, pool.num_blocks, pool.num_kv_heads,
                pool.head_dim, pool.dtype, pool.device)
    p2.kv.copy_(pool.kv)
    m2 = type(meta)(**{f: (getattr(meta, f).clone() if torch.is_tensor(getattr(meta, f))
                           else getattr(meta, f)) for f in meta.__dataclass_fields__})
    return p2, m2, ids.clone()


def test_cfg4_model_step_full_size_against_oracle_and_graph(monkeypatch):
    cfg = ModelConfig(vocab_size=50257, d_model=1024, num_layers=12, num_heads=16,
                      num_kv_heads=1, max_seq_len=4096)
    N, BS, NB, steps = 128, 16, 16384, 3
    print(f"[cfg4 full] layers={cfg.num_layers} batch={N} vocab={cfg.vocab_size}", flush=True)
    dev = torch.device(DEV)
    torch.manual_seed(0)
    model = PagedTransformer(cfg).to(dev, torch.bfloat16).eval()
    lens = workloads.lengths_uniform(N, 256, 2048, seed=0)
    tables = workloads.permuted_tables([int(x) + steps + 2 for x in lens], BS, NB, seed=0)
    pool = KVPool(cfg.num_layers, BS, NB, 1, cfg.head_dim, torch.bfloat16, dev)
    g = torch.Generator(device=dev).manual_seed(1)
    for l in range(cfg.num_layers):
        pool.kv[l].normal_(generator=g)
    meta = pack_batch_meta(tables, list(range(N + 1)), [int(x) for x in lens], N, dev, BS)
    meta.max_kv_len = int(max(lens)) + steps + 2
    ids = torch.randint(0, cfg.vocab_size, (N,), generator=g, device=dev)
    pool_b, meta_b, ids_b = _clone(pool, meta, ids)

    rng = np.random.default_rng(4)
    sample = sorted(set(rng.choice(N, 16, replace=False).tolist())
                    | {int(np.argmin(lens)), int(np.argmax(lens))})
    seen = []
    real = paged_mqa.paged_attention_append_meta

    def checked(q, k, v, pool_, layer, meta_, **kw):
        bk, bv = _layer_cpu(pool_, layer)
        out = real(q, k, v, pool_, layer, meta_, **kw)
        torch.cuda.synchronize()
        ak, av = _layer_cpu(pool_, layer)
        ek, ev = _expected_after_append(bk, bv, k, v, meta_, BS)
        assert np.array_equal(_bits(ak), ek), f"layer {layer}: K pool differs from the oracle append"
        assert np.array_equal(_bits(av), ev), f"layer {layer}: V pool differs from the oracle append"
        # every sequence against gather + SDPA in fp32
        nb_ = ak.shape[0] // BS
        sdpa = torch_ref.paged_attention_sdpa(q.detach().cpu(), ak.view(nb_, BS, *ak.shape[1:]),
                                              av.view(nb_, BS, *av.shape[1:]),
                                              meta_.block_tables.cpu(), meta_.seq_lens.cpu(),
                                              dtype=torch.float32)
        _close(out.detach().float().cpu().numpy(), sdpa.numpy().astype(np.float64),
               f"layer {layer} attention, all {N} rows vs SDPA")
        kp, vp, small = _compact(ak, av, tables, sample, BS)
        qs = q[sample].detach().float().cpu().numpy().astype(np.float64)
        sl = meta_.seq_lens.cpu().numpy()[sample]
        eo, _ = ref.paged_attention(qs, kp, vp, small, sl, None)
        _close(out[sample].detach().float().cpu().numpy(), eo, f"layer {layer} attention")
        seen.append(layer)
        return out

    with monkeypatch.context() as m:
        m.setattr(paged_mqa, "paged_attention_append_meta", checked)
        with torch.no_grad():
            logits = model.forward_step(ids, pool, meta)
    assert seen == list(range(cfg.num_layers)), seen
    assert torch.isfinite(logits.float()).all()
    ids_a = logits.argmax(-1)
    for t in (meta.positions, meta.start_pos, meta.seq_lens):
        t.add_(1)

    # the same step as a HIP graph (its warm-up is that first step)
    graph = DecodeStepGraph(model, pool_b, meta_b, ids_b, warmup=1)
    torch.cuda.synchronize()
    assert torch.equal(graph.ids, ids_a), "graph warm-up step differs from the checked step"
    assert torch.equal(pool_b.kv, pool.kv), "pools differ after the first step"
    for k in range(steps):
        toks = graph.replay()
        torch.cuda.synchronize()
        with torch.no_grad():
            ref_logits = model.forward_step(ids_a, pool, meta)
        ids_a = ref_logits.argmax(-1)
        for t in (meta.positions, meta.start_pos, meta.seq_lens):
            t.add_(1)
        torch.cuda.synchronize()
        assert torch.equal(toks, ids_a), f"replay {k}: tokens differ"
        assert torch.equal(graph.logits, ref_logits), f"replay {k}: logits differ"
    assert torch.equal(pool_b.kv, pool.kv), "pools differ after the replays"


@pytest.mark.parametrize("bs", [16, 32])
def test_cfg5_mixed_step_full_size_against_oracle(bs):
    chunk, n_new = 512, 4
    print(f"[cfg5 mixed full] bs={bs} 256 decodes + {n_new} x {chunk}", flush=True)
    dev = torch.device(DEV)
    p = workloads.cfg5_mixed_problem(dev, chunk=chunk, n_new=n_new, seed=0, bs=bs)
    meta, pool = p.meta, p.pool
    tables = list(meta.block_tables.cpu().numpy())  # rows padded with block 0
    ends = meta.seq_lens.cpu().numpy()
    n_seq = len(ends)
    # garbage in every slot no sequence owns once the step has appended
    owned = np.zeros(pool.num_blocks * bs, dtype=bool)
    for s in range(n_seq):
        pos = np.arange(int(ends[s]))
        owned[tables[s][pos // bs].astype(np.int64) * bs + pos % bs] = True
    free = torch.as_tensor(~owned, device=dev)
    pool.flat_k[0][free] = 1e3
    pool.flat_v[0][free] = 1e3
    torch.cuda.synchronize()

    bk, bv = _layer_cpu(pool, 0)
    lse = torch.empty(p.q.shape[0], p.q.shape[1], device=dev)
    out = paged_attention_append_meta(p.q, p.k, p.v, pool, 0, meta, lse=lse)
    torch.cuda.synchronize()
    ak, av = _layer_cpu(pool, 0)
    ek, ev = _expected_after_append(bk, bv, p.k, p.v, meta, bs)
    assert np.array_equal(_bits(ak), ek), "K pool differs from the oracle append"
    assert np.array_equal(_bits(av), ev), "V pool differs from the oracle append"

    # every row (decode and prefill) against gather + SDPA in fp32
    nb_ = ak.shape[0] // bs
    sdpa = torch_ref.paged_attention_sdpa(p.q.cpu(), ak.view(nb_, bs, *ak.shape[1:]),
                                          av.view(nb_, bs, *av.shape[1:]), meta.block_tables.cpu(),
                                          meta.seq_lens.cpu(), meta.query_start_loc.cpu(),
                                          dtype=torch.float32)
    assert sdpa.shape == out.shape
    _close(out.float().cpu().numpy(), sdpa.numpy().astype(np.float64),
           f"bs {bs}: all {out.shape[0]} rows vs SDPA")

    n_dec = len(p.dec_lens)
    rng = np.random.default_rng(bs)
    dec = sorted(set(rng.choice(n_dec, 32, replace=False).tolist())
                 | {int(np.argmax(p.dec_lens)), int(np.argmin(p.dec_lens))})
    seqs = dec + list(range(n_dec, n_seq))
    qsl = meta.query_start_loc.cpu().numpy()
    rows = np.concatenate([np.arange(qsl[s], qsl[s + 1]) for s in seqs])
    sub_qsl = np.concatenate([[0], np.cumsum([qsl[s + 1] - qsl[s] for s in seqs])])
    kp, vp, small = _compact(ak, av, tables, seqs, bs)
    qs = p.q[torch.as_tensor(rows, device=dev)].float().cpu().numpy().astype(np.float64)
    eo, el = ref.paged_attention(qs, kp, vp, small, ends[seqs], sub_qsl)
    got = out[torch.as_tensor(rows, device=dev)].float().cpu().numpy()
    _close(got[:len(dec)], eo[:len(dec)], f"bs {bs}: decode rows")
    _close(got[len(dec):], eo[len(dec):], f"bs {bs}: prefill rows")
    L = lse[torch.as_tensor(rows, device=dev)].cpu().numpy()
    assert np.all(np.isfinite(L)) and np.all(np.isfinite(el))
    np.testing.assert_allclose(L, el, rtol=0, atol=TOL, err_msg=f"bs {bs}: lse")
