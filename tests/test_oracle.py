"""Pins the CPU oracle (oracle/) before anything is compared against it.

Each oracle function is checked against a reference known-answer test, a
library routine, a closed form, or a brute force, chosen so that a plausible
mistake fails: the planted-mistake tests at the bottom run the oracle with a
deliberate error and require one of these checks to reject it.
"""
import math

import numpy as np
import pytest
import torch

from oracle import paged_ref as ref
from oracle import torch_ref


# ---------------------------------------------------------------------------
# slot mapping / append / gather
# ---------------------------------------------------------------------------

def test_slot_mapping_reference_kat(kats):
    # tests/test_kv_pool.py:25-30 of the reference
    for c in kats["slot_mapping"]:
        got = ref.make_slot_mapping(c["start"], c["n"], c["block_table"], c["block_size"])
        assert got.tolist() == c["slots"]


def test_slot_mapping_closed_form():
    rng = np.random.default_rng(0)
    bt = rng.permutation(np.arange(1, 64))[:9].tolist()
    slots = ref.make_slot_mapping(5, 120, bt, 16)
    for i, s in enumerate(slots):
        p = 5 + i
        assert s == bt[p // 16] * 16 + p % 16


def test_slot_mapping_asserts():
    with pytest.raises(AssertionError, match="too short"):
        ref.make_slot_mapping(10, 7, [3], 16)
    with pytest.raises(AssertionError, match="block 0"):
        ref.make_slot_mapping(0, 20, [4, 0], 16)


def _pool(nb=16, bs=16, hkv=2, d=4, seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.zeros(nb * bs, hkv, d), torch.zeros(nb * bs, hkv, d), g


def test_append_matches_index_put_bit_exact():
    fk, fv, g = _pool()
    slots = torch.randperm(16 * 16, generator=g)[:100]
    k = torch.randn(100, 2, 4, generator=g)
    v = torch.randn(100, 2, 4, generator=g)
    nk, nv = fk.numpy().copy(), fv.numpy().copy()
    ref.append(nk, nv, slots.numpy(), k.numpy(), v.numpy())
    tk, tv = fk.clone(), fv.clone()
    tk.index_put_((slots,), k)
    tv.index_put_((slots,), v)
    assert np.array_equal(nk, tk.numpy()) and np.array_equal(nv, tv.numpy())


def test_append_negative_slot_wraps_like_torch():
    fk, fv, g = _pool()
    slots = torch.tensor([-1, -256, 5])
    k = torch.randn(3, 2, 4, generator=g)
    nk, nv = fk.numpy().copy(), fv.numpy().copy()
    ref.append(nk, nv, slots.numpy(), k.numpy(), k.numpy())
    tk = fk.clone()
    tk[slots] = k
    assert np.array_equal(nk, tk.numpy())
    with pytest.raises(IndexError):
        ref.append(nk, nv, np.array([256]), k[:1].numpy(), k[:1].numpy())


def test_write_gather_roundtrip_and_untouched_zero():
    # tests/test_kv_pool.py:33-67 of the reference
    kv = np.zeros((2, 2, 16, 16, 2, 4), dtype=np.float32)
    fk, fv = kv[0, 0].reshape(-1, 2, 4), kv[0, 1].reshape(-1, 2, 4)
    rng = np.random.default_rng(1)
    bt = [9, 3, 12]
    k = rng.standard_normal((40, 2, 4)).astype(np.float32)
    v = rng.standard_normal((40, 2, 4)).astype(np.float32)
    ref.append(fk, fv, ref.make_slot_mapping(0, 40, bt, 16), k, v)
    ko, vo = ref.gather(kv[0, 0], kv[0, 1], bt, 40)
    assert np.array_equal(ko, k) and np.array_equal(vo, v)
    assert not kv[0, 0, 0].any() and not kv[1].any()


def test_gather_matches_torch_index_select():
    g = torch.Generator().manual_seed(2)
    pool = torch.randn(32, 16, 1, 8, generator=g)
    bt = [5, 17, 2]
    k, _ = ref.gather(pool.numpy(), pool.numpy(), bt, 37)
    expect = pool.index_select(0, torch.tensor(bt)).reshape(-1, 1, 8)[:37]
    assert np.array_equal(k, expect.numpy())


# ---------------------------------------------------------------------------
# metadata packing
# ---------------------------------------------------------------------------

def test_pack_metadata_kat(kats):
    for c in kats["pack_metadata"]:
        table, lens, qloc, mql = ref.pack_metadata(c["block_tables"], c["query_start_loc"],
                                                   c["positions"], c["T"], c["block_size"])
        assert table.tolist() == c["table"]
        assert lens.tolist() == c["seq_lens"]
        assert qloc.tolist() == c["query_start_loc"]
        assert mql == c["max_q_len"]


def test_pack_metadata_errors():
    with pytest.raises(ValueError, match="num_seqs \\+ 1"):
        ref.pack_metadata([[1]], [0], [0], 1, 16)
    with pytest.raises(ValueError, match="start at 0"):
        ref.pack_metadata([[1]], [0, 2], [0], 1, 16)
    with pytest.raises(ValueError, match="length T"):
        ref.pack_metadata([[1]], [0, 1], [0, 1], 1, 16)
    with pytest.raises(ValueError, match="exceeds"):
        ref.pack_metadata([[1]], [0, 1], [16], 1, 16)


# ---------------------------------------------------------------------------
# paged attention
# ---------------------------------------------------------------------------

def make_problem(q_lens, kv_lens, hq, hkv, d, bs, seed=0, garbage=1e3, extra_blocks=4,
                 dtype=np.float64):
    """Random paged problem with shuffled physical blocks and garbage in every
    slot no sequence owns (methodology of the reference's tests/test.py:61-114)."""
    rng = np.random.default_rng(seed)
    nblk = [max(1, math.ceil(kv / bs)) for kv in kv_lens]
    nb = sum(nblk) + extra_blocks
    k_pool = np.full((nb, bs, hkv, d), garbage, dtype=dtype)
    v_pool = np.full((nb, bs, hkv, d), garbage, dtype=dtype)
    perm = rng.permutation(nb)
    table = np.zeros((len(q_lens), max(nblk)), dtype=np.int32)
    cur = 0
    dense = []
    for s, kv in enumerate(kv_lens):
        ids = perm[cur:cur + nblk[s]]
        cur += nblk[s]
        table[s, :nblk[s]] = ids
        k = rng.standard_normal((kv, hkv, d)).astype(dtype)
        v = rng.standard_normal((kv, hkv, d)).astype(dtype)
        dense.append((k, v))
        for b in range(nblk[s]):
            lo, hi = b * bs, min((b + 1) * bs, kv)
            if hi > lo:
                k_pool[ids[b], :hi - lo] = k[lo:hi]
                v_pool[ids[b], :hi - lo] = v[lo:hi]
    q = rng.standard_normal((sum(q_lens), hq, d)).astype(dtype)
    qsl = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    return dict(q=q, k_pool=k_pool, v_pool=v_pool, table=table,
                seq_lens=np.asarray(kv_lens, dtype=np.int32), qsl=qsl, dense=dense,
                q_lens=list(q_lens), kv_lens=list(kv_lens), hq=hq, hkv=hkv, d=d, bs=bs)


def brute_force(p, causal=True, scale=None):
    """Pure-Python loops over the dense per-sequence K/V (no pool, no numpy
    linear algebra): the textbook definition."""
    hq, hkv, d = p["hq"], p["hkv"], p["d"]
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    out = np.zeros_like(p["q"])
    lse = np.full(p["q"].shape[:2], np.inf)
    for s, (ql, kv) in enumerate(zip(p["q_lens"], p["kv_lens"])):
        k, v = p["dense"][s]
        q0 = int(p["qsl"][s])
        for i in range(ql):
            qpos = kv - ql + i
            for h in range(hq):
                kvh = h // (hq // hkv)
                keys = [j for j in range(kv) if (not causal or j <= qpos)]
                if not keys:
                    continue
                sc = [scale * sum(float(p["q"][q0 + i, h, t]) * float(k[j, kvh, t]) for t in range(d))
                      for j in keys]
                m = max(sc)
                w = [math.exp(x - m) for x in sc]
                z = sum(w)
                for t in range(d):
                    out[q0 + i, h, t] = sum(wj * float(v[j, kvh, t]) for wj, j in zip(w, keys)) / z
                lse[q0 + i, h] = m + math.log(z)
    return out, lse


TINY = dict(q_lens=[1, 3, 2, 1], kv_lens=[5, 7, 2, 9], hq=4, hkv=2, d=8, bs=4)


def _oracle(p, **kw):
    return ref.paged_attention(p["q"], p["k_pool"], p["v_pool"], p["table"], p["seq_lens"],
                               p["qsl"], **kw)


@pytest.mark.parametrize("causal", [True, False])
def test_attention_vs_brute_force(causal):
    p = make_problem(**TINY, seed=3)
    out, lse = _oracle(p, causal=causal)
    bo, bl = brute_force(p, causal=causal)
    np.testing.assert_allclose(out, bo, rtol=0, atol=1e-12)
    np.testing.assert_allclose(lse, bl, rtol=0, atol=1e-12)


def test_attention_vs_golden_fixture(attention_golden):
    # tests/golden/attention_small.npz: textbook outputs written by
    # tests/golden/make_attention_golden.py, independent of the oracle
    for name, c in attention_golden.items():
        out, lse = ref.paged_attention(c["q"], c["k_pool"], c["v_pool"], c["block_table"],
                                       c["seq_lens"], c["query_start_loc"])
        np.testing.assert_allclose(out, c["out"], rtol=0, atol=1e-12, err_msg=name)
        fin = np.isfinite(c["lse"])
        assert np.array_equal(np.isfinite(lse), fin), name
        np.testing.assert_allclose(lse[fin], c["lse"][fin], rtol=0, atol=1e-12, err_msg=name)


@pytest.mark.parametrize("hq,hkv,d,bs", [(8, 1, 32, 16), (8, 8, 64, 16), (16, 4, 128, 16),
                                         (14, 2, 80, 16), (8, 1, 64, 32)])
def test_attention_vs_torch_sdpa(hq, hkv, d, bs):
    # scenarios of the reference's tests/test.py:33-38 (shortened)
    q_lens = [1, 1, 64, 33, 1, 100]
    kv_lens = [37, 513, 700, 1000, 16, 100]
    p = make_problem(q_lens, kv_lens, hq, hkv, d, bs, seed=4)
    out, _ = _oracle(p)
    sd = torch_ref.paged_attention_sdpa(torch.from_numpy(p["q"]), torch.from_numpy(p["k_pool"]),
                                        torch.from_numpy(p["v_pool"]), p["table"].tolist(),
                                        p["kv_lens"], p["qsl"].tolist())
    np.testing.assert_allclose(out, sd.numpy(), rtol=0, atol=1e-10)


def test_attention_closed_forms():
    p = make_problem([1, 1, 2], [1, 6, 5], 4, 1, 16, 4, seed=5)
    out, lse = _oracle(p)
    # kv_len = 1: softmax of one key is 1, output is that key's value
    np.testing.assert_allclose(out[0], np.broadcast_to(p["dense"][0][1][0, 0], (4, 16)), atol=1e-14)
    # lse equals logsumexp of the scaled scores
    k1 = p["dense"][1][0][:, 0]
    scores = (k1 @ p["q"][1].T) / 4.0  # [6, hq]
    m = scores.max(0)
    np.testing.assert_allclose(lse[1], m + np.log(np.exp(scores - m).sum(0)), atol=1e-12)
    # q = 0: uniform weights, output = mean of the visible values
    p2 = dict(p)
    p2["q"] = np.zeros_like(p["q"])
    out0, lse0 = _oracle(p2)
    v1 = p["dense"][1][1][:, 0]
    np.testing.assert_allclose(out0[1], np.broadcast_to(v1.mean(0), (4, 16)), atol=1e-14)
    np.testing.assert_allclose(lse0[1], math.log(6), atol=1e-14)
    # causal prefill row i of sequence 2 (q_len 2, kv 5) sees keys 0..3+i
    v2 = p["dense"][2][1][:, 0]
    np.testing.assert_allclose(out0[2], np.broadcast_to(v2[:4].mean(0), (4, 16)), atol=1e-14)
    np.testing.assert_allclose(out0[3], np.broadcast_to(v2.mean(0), (4, 16)), atol=1e-14)
    # constant V: output is that constant whatever the scores
    p3 = dict(p)
    p3["v_pool"] = np.full_like(p["v_pool"], 2.5)
    out3, _ = _oracle(p3)
    np.testing.assert_allclose(out3, 2.5, atol=1e-13)


def test_attention_empty_rows():
    p = make_problem([1, 1], [0, 3], 2, 1, 8, 4, seed=6)
    out, lse = _oracle(p)
    assert not out[0].any() and np.all(np.isinf(lse[0])) and np.all(lse[0] > 0)
    assert np.all(np.isfinite(lse[1]))


def test_attention_clamps_to_table_capacity():
    # seq_lens beyond max_blk * bs is clamped (pagedattn.cu:187-189): the
    # result equals attention over the first max_blk * bs keys
    p = make_problem([1], [8], 2, 1, 8, 4, seed=7)
    lens_big = np.array([50], dtype=np.int32)
    out_big, _ = ref.paged_attention(p["q"], p["k_pool"], p["v_pool"], p["table"], lens_big, p["qsl"])
    out, _ = _oracle(p)
    np.testing.assert_allclose(out_big, out, atol=1e-14)


def test_attention_scale_argument():
    p = make_problem([2], [6], 2, 1, 8, 4, seed=8)
    out_half, _ = _oracle(p, scale=0.5)
    bo, _ = brute_force(p, scale=0.5)
    np.testing.assert_allclose(out_half, bo, atol=1e-12)
    # scale <= 0 selects the default 1/sqrt(d) (pagedattn.cu:930-931)
    np.testing.assert_allclose(_oracle(p, scale=-1.0)[0], _oracle(p)[0], atol=0)


def test_attention_large_scores_stable():
    p = make_problem([1], [20], 2, 1, 8, 4, seed=9)
    p["q"] = p["q"] * 200.0
    out, _ = _oracle(p)
    assert np.all(np.isfinite(out))
    bo, _ = brute_force(p)
    np.testing.assert_allclose(out, bo, atol=1e-9)


# ---------------------------------------------------------------------------
# planted mistakes: each must be rejected by one of the checks above
# ---------------------------------------------------------------------------

def _fails(fn):
    try:
        fn()
    except AssertionError:
        return True
    return False


@pytest.mark.parametrize("mutation", ["topleft", "noscale", "kvhead_mod", "noclamp", "nomax"])
def test_planted_mistake_is_caught(mutation):
    p = make_problem(**TINY, seed=3)

    def vs_brute():
        out, lse = _oracle(p, _mutation=mutation)
        bo, bl = brute_force(p)
        np.testing.assert_allclose(out, bo, atol=1e-9)
        np.testing.assert_allclose(lse, bl, atol=1e-9)

    def vs_clamp():
        pc = make_problem([1], [8], 2, 1, 8, 4, seed=7)
        big = ref.paged_attention(pc["q"], pc["k_pool"], pc["v_pool"], pc["table"],
                                  np.array([50], dtype=np.int32), pc["qsl"], _mutation=mutation)[0]
        np.testing.assert_allclose(big, _oracle(pc)[0], atol=1e-12)

    def vs_large():
        pl = make_problem([1], [20], 2, 1, 8, 4, seed=9)
        pl["q"] = pl["q"] * 5000.0
        with np.errstate(over="ignore", invalid="ignore"):
            out = _oracle(pl, _mutation=mutation)[0]
        np.testing.assert_allclose(out, brute_force(pl)[0], atol=1e-9)

    assert _fails(vs_brute) or _fails(vs_clamp) or _fails(vs_large), mutation


# ---------------------------------------------------------------------------
# model restatement pieces
# ---------------------------------------------------------------------------

def test_rope_closed_forms():
    cos, sin = torch_ref.rope_tables(8, 64)
    x = torch.randn(1, 5, 8, generator=torch.Generator().manual_seed(0), dtype=torch.float64)
    # position 0 is the identity
    y0 = torch_ref.rope_rotate(x[:, :1], cos[:1].double(), sin[:1].double())
    assert torch.equal(y0, x[:, :1])
    # each (even, odd) pair is rotated: its norm is preserved
    pos = torch.tensor([3, 7, 11, 20, 63])
    y = torch_ref.rope_rotate(x, cos[pos].double(), sin[pos].double())
    nx = x[..., 0::2] ** 2 + x[..., 1::2] ** 2
    ny = y[..., 0::2] ** 2 + y[..., 1::2] ** 2
    assert torch.allclose(nx, ny, atol=1e-6)
    # q.k after rotation depends only on the position difference
    q = torch.randn(8, dtype=torch.float64)
    k = torch.randn(8, dtype=torch.float64)

    def dot_at(pq, pk):
        a = torch_ref.rope_rotate(q[None, None], cos[pq:pq + 1].double(), sin[pq:pq + 1].double())
        b = torch_ref.rope_rotate(k[None, None], cos[pk:pk + 1].double(), sin[pk:pk + 1].double())
        return float((a * b).sum())

    assert abs(dot_at(10, 4) - dot_at(30, 24)) < 1e-5
    # angle of pair i at position p is p * 10000^(-2i/8)
    assert abs(float(sin[5, 1]) - math.sin(5 * 10000 ** (-2 / 8))) < 1e-6


def test_rmsnorm_kat():
    x = torch.tensor([[3.0, 4.0]])
    y = torch_ref.rmsnorm(x, torch.tensor([1.0, 2.0]), eps=0.0)
    r = math.sqrt((9 + 16) / 2)
    assert torch.allclose(y, torch.tensor([[3 / r, 8 / r]]))


def test_e4m3_codes_match_torch_and_the_format():
    """The oracle's fp8 rounding (oracle.paged_ref.e4m3_codes) against torch's
    conversion to float8_e4m3fn on every bf16 and fp16 value and a wide
    random sample, and against the format's closed forms: the largest finite
    value, the smallest subnormal, ties to even, NaN for overflow."""
    import torch
    for x in (torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16).float(),
              torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.float16).float(),
              torch.randn(1 << 18, generator=torch.Generator().manual_seed(0))
              * torch.exp(4 * torch.randn(1 << 18, generator=torch.Generator().manual_seed(1)))):
        want = x.to(torch.float8_e4m3fn).view(torch.uint8).numpy()
        assert np.array_equal(ref.e4m3_codes(x.numpy()), want)
    c = ref.e4m3_codes
    assert c(448.0) == 0x7E and c(-448.0) == 0xFE          # largest finite
    assert c(463.9) == 0x7E and c(464.0) == 0x7E          # tie below 480 goes to even (448)
    assert c(464.01) == 0x7F and c(1e9) == 0x7F           # beyond: NaN, no infinity
    assert c(np.inf) == 0x7F and c(-np.inf) == 0xFF and c(np.nan) == 0x7F
    assert c(2.0 ** -9) == 0x01 and c(2.0 ** -10) == 0x00  # smallest subnormal; tie to even 0
    assert c(3 * 2.0 ** -10) == 0x02                        # 1.5 ulp: tie to even (2)
    assert c(1.0) == 0x38 and c(1.0625) == 0x38 and c(1.1875) == 0x3A
    v = ref.e4m3_values(np.arange(256, dtype=np.uint8))
    assert np.isnan(v[0x7F]) and np.isnan(v[0xFF]) and np.sum(np.isnan(v)) == 2
    fin = ~np.isnan(v)
    assert np.array_equal(ref.e4m3_codes(v[fin].astype(np.float32)), np.arange(256)[fin])
