"""The MFMA prefill / chunked-prefill kernel (csrc/prefill_mfma.hip) against
the fp64 oracle (bf16 / fp16: 2e-2 absolute, lse too).

Shapes: 16 or 32 query heads per KV head (8 or 4 query tokens per tile; 8
with two 16-head row tiles per wavefront for long runs at 32), head dim 64 / 128, 1 or 2 KV heads, block size 16 / 32; query runs
not a multiple of the tile's tokens, runs longer than the context
(kv_len < q_len), an empty context, a one-sequence batch (no decode split),
causal and not, a custom scale.
"""
import numpy as np
import pytest
import torch

from oracle import paged_ref as ref
from serving import workloads
from serving.fake_paged_attn import paged_attn_fwd

pytestmark = pytest.mark.gpu
DEV = "cuda"


def np64(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def problem(seqs, hq, hkv, d, bs, dtype, seed):
    q_lens = [a for a, _ in seqs]
    kv_lens = [b for _, b in seqs]
    p = workloads.decode_problem(kv_lens, hq, hkv, d, bs,
                                 sum((k + bs - 1) // bs for k in kv_lens) + 16,
                                 dtype, DEV, seed, garbage=1e3)
    g = torch.Generator(device=DEV).manual_seed(seed + 7)
    q = torch.randn(sum(q_lens), hq, d, generator=g, device=DEV).to(dtype)
    qsl = torch.tensor(np.concatenate([[0], np.cumsum(q_lens)]), dtype=torch.int32, device=DEV)
    return p, q, qsl, max(q_lens)


CASES = {
    # new sequences' chunks, ragged tails (q_len % TQ != 0)
    "chunks": [(128, 128), (77, 77), (130, 130), (5, 5)],
    # later chunks of long prompts
    "continued": [(64, 700), (33, 1000), (128, 2100)],
    # more queries than keys (seq_lens below q_len) and an empty context
    "short_kv": [(40, 20), (16, 0), (50, 50)],
    # a single sequence: no decode split
    "single": [(300, 1300)],
    # query runs of 256+ tokens over 512+ keys: 8-token tiles at 32 heads per kv head
    "wide": [(512, 512), (260, 900), (7, 7)],
}


@pytest.mark.parametrize("case", list(CASES))
@pytest.mark.parametrize("hq,hkv,d,bs,dtype", [
    (32, 1, 128, 16, torch.bfloat16),
    (16, 1, 64, 16, torch.bfloat16),
    (32, 2, 64, 32, torch.float16),
    (64, 2, 128, 16, torch.bfloat16),
])
def test_prefill_vs_oracle(case, hq, hkv, d, bs, dtype):
    print(f"[prefill] {case} hq={hq} hkv={hkv} d={d} bs={bs} {dtype}", flush=True)
    p, q, qsl, mql = problem(CASES[case], hq, hkv, d, bs, dtype, seed=41)
    O, L = paged_attn_fwd(q, p.k_pool, p.v_pool, p.block_tables, p.seq_lens, qsl, mql)
    torch.cuda.synchronize()
    eo, el = ref.paged_attention(np64(q), np64(p.k_pool), np64(p.v_pool),
                                 p.block_tables.cpu().numpy(), p.seq_lens.cpu().numpy(),
                                 qsl.cpu().numpy())
    got = np64(O)
    assert np.all(np.isfinite(got))
    assert np.abs(got - eo).max() <= 2e-2, f"max err {np.abs(got - eo).max():.3e}"
    Ln = L.cpu().numpy()
    fin = np.isfinite(el)
    assert np.array_equal(np.isfinite(Ln), fin), "+inf lse rows differ"
    np.testing.assert_allclose(Ln[fin], el[fin], rtol=0, atol=2e-2)


@pytest.mark.parametrize("causal,scale", [(False, 0.0), (True, 0.05), (False, 0.2)])
def test_prefill_noncausal_and_scale(causal, scale):
    p, q, qsl, mql = problem([(96, 300), (17, 17), (64, 64)], 32, 1, 128, 16, torch.bfloat16,
                             seed=42)
    O, L = paged_attn_fwd(q, p.k_pool, p.v_pool, p.block_tables, p.seq_lens, qsl, mql,
                          scale=scale, causal=causal)
    torch.cuda.synchronize()
    eo, el = ref.paged_attention(np64(q), np64(p.k_pool), np64(p.v_pool),
                                 p.block_tables.cpu().numpy(), p.seq_lens.cpu().numpy(),
                                 qsl.cpu().numpy(), scale=scale if scale > 0 else None,
                                 causal=causal)
    assert np.abs(np64(O) - eo).max() <= 2e-2
    np.testing.assert_allclose(L.cpu().numpy(), el, rtol=0, atol=2e-2)
