"""Paged attention on the GPU against the oracle.

Tolerances (from the task's north star and the reference's own tests):
  fp32: rtol 1e-5, atol 1e-5 against the fp64 oracle and against the
        reference's PyTorch gather + SDPA path in fp32
        (tests/test_paged_mqa.py:28 of the reference uses atol=1e-5);
  bf16 / fp16: 2e-2 absolute against the fp64 oracle evaluated on the same
        (rounded) inputs.
lse (log-sum-exp of the scaled scores, natural log) is checked the same way.
"""
import math

import numpy as np
import pytest
import torch

from oracle import paged_ref as ref
from oracle import torch_ref
from serving import workloads
from serving.fake_paged_attn import (PagedVarlenAttention, paged_attn_fwd,
                                     paged_mqa_decode, paged_varlen_attention)

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = {torch.float32: dict(rtol=1e-5, atol=1e-5),
       torch.bfloat16: dict(rtol=0, atol=2e-2),
       torch.float16: dict(rtol=0, atol=2e-2)}


def np64(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def oracle(q, k_pool, v_pool, table, lens, qsl=None, scale=None, causal=True):
    return ref.paged_attention(np64(q), np64(k_pool), np64(v_pool),
                               table.cpu().numpy() if torch.is_tensor(table) else np.asarray(table),
                               lens.cpu().numpy() if torch.is_tensor(lens) else np.asarray(lens),
                               None if qsl is None else (qsl.cpu().numpy() if torch.is_tensor(qsl) else np.asarray(qsl)),
                               scale=scale, causal=causal)


def close(out, expect, dtype, what):
    got = np64(out)
    tol = TOL[dtype]
    err = np.abs(got - expect)
    bound = tol["atol"] + tol["rtol"] * np.abs(expect)
    worst = float((err - bound).max()) if err.size else 0.0
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    assert worst <= 0, f"{what}: max err {err.max():.3e} exceeds tolerance"


# ---------------------------------------------------------------------------
# committed fixture: textbook outputs (tests/golden/attention_small.npz)
# ---------------------------------------------------------------------------

def _golden_inputs(c, dtype):
    t = lambda a: torch.from_numpy(a).to(DEV, dtype)  # noqa: E731
    i = lambda a: torch.from_numpy(a).to(DEV)  # noqa: E731
    return (t(c["q"]), t(c["k_pool"]), t(c["v_pool"]), i(c["block_table"]), i(c["seq_lens"]),
            i(c["query_start_loc"]))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_golden_fixture(attention_golden, dtype):
    # the inputs are bf16-representable, so every dtype sees them exactly
    for name, c in attention_golden.items():
        print(f"[golden] {name} {dtype}", flush=True)
        q, kp, vp, table, lens, qsl = _golden_inputs(c, dtype)
        O, L = paged_attn_fwd(q, kp, vp, table, lens, qsl, c["max_q_len"])
        torch.cuda.synchronize()
        close(O, c["out"], dtype, f"{name} out")
        Ln = L.cpu().numpy().astype(np.float64)
        fin = np.isfinite(c["lse"])
        assert np.array_equal(np.isfinite(Ln), fin), f"{name}: lse +inf rows differ"
        tol = TOL[dtype]
        np.testing.assert_allclose(Ln[fin], c["lse"][fin], rtol=tol["rtol"], atol=tol["atol"],
                                   err_msg=name)


@pytest.mark.parametrize("part_tokens", [0, 32, -1], ids=["auto", "plen32", "persistent"])
def test_golden_fixture_decode_kernels(attention_golden, part_tokens):
    # the MFMA decode kernels (split-K partition and persistent) on the
    # fixture's decode cases, bf16
    for name, c in attention_golden.items():
        if c["max_q_len"] != 1:
            continue
        print(f"[golden decode] {name} part_tokens={part_tokens}", flush=True)
        q, kp, vp, table, lens, _ = _golden_inputs(c, torch.bfloat16)
        lse = torch.empty(q.shape[0], q.shape[1], device=DEV)
        out = paged_mqa_decode(q, kp, vp, table, lens, lse=lse, part_tokens=part_tokens)
        torch.cuda.synchronize()
        close(out, c["out"], torch.bfloat16, f"{name} out")
        np.testing.assert_allclose(lse.cpu().numpy(), c["lse"], rtol=0, atol=2e-2, err_msg=name)


# ---------------------------------------------------------------------------
# isolated paged MQA decode op
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_cfg2_decode_vs_oracle(dtype):
    print(f"[cfg2 decode] dtype={dtype}", flush=True)
    p = workloads.cfg2_problem(dtype, DEV, seed=0)
    lse = torch.empty(p.n_seq, p.hq, dtype=torch.float32, device=DEV)
    out = paged_mqa_decode(p.q, p.k_pool, p.v_pool, p.block_tables, p.seq_lens, lse=lse)
    torch.cuda.synchronize()
    eo, el = oracle(p.q, p.k_pool, p.v_pool, p.block_tables, p.seq_lens)
    close(out, eo, dtype, "out")
    close(lse, el, torch.float32 if dtype == torch.float32 else dtype, "lse")


def test_cfg2_fp32_vs_reference_torch_path():
    # the reference's own PyTorch paged path: gather + SDPA (tests/test.py:145-178)
    p = workloads.cfg2_problem(torch.float32, DEV, seed=1)
    out = paged_mqa_decode(p.q, p.k_pool, p.v_pool, p.block_tables, p.seq_lens)
    sd = torch_ref.paged_attention_sdpa(p.q, p.k_pool, p.v_pool, p.tables, p.lens.tolist())
    torch.testing.assert_close(out.cpu(), sd, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("part_tokens", [32, 64, 96, 4096])
def test_split_k_partitions_agree(part_tokens):
    p = workloads.cfg2_problem(torch.float32, DEV, seed=2)
    out = paged_mqa_decode(p.q, p.k_pool, p.v_pool, p.block_tables, p.seq_lens,
                           part_tokens=part_tokens)
    eo, _ = oracle(p.q, p.k_pool, p.v_pool, p.block_tables, p.seq_lens)
    close(out, eo, torch.float32, f"part_tokens={part_tokens}")


# ---------------------------------------------------------------------------
# varlen scenarios of the reference's tests/test.py:33-46, garbage-filled pools
# ---------------------------------------------------------------------------

SCENARIOS = {
    "prefill": [(128, 128), (300, 300), (77, 77)],
    "decode": [(1, 1024), (1, 37), (1, 2048), (1, 513), (1, 129), (1, 16), (1, 777)],
    "chunked": [(64, 700), (100, 100), (33, 1000), (128, 640)],
    "mixed": [(256, 256), (1, 900), (1, 5), (50, 450), (1, 2000)],
}
HEADS = [(8, 8, 64, 16), (16, 4, 128, 16), (8, 1, 64, 32), (14, 2, 80, 16), (32, 1, 128, 16),
         (16, 1, 64, 16)]


def build_varlen(seqs, hq, hkv, d, bs, dtype, seed):
    q_lens = [a for a, _ in seqs]
    kv_lens = [b for _, b in seqs]
    p = workloads.decode_problem(kv_lens, hq, hkv, d, bs,
                                 sum((k + bs - 1) // bs for k in kv_lens) + 16,
                                 dtype, DEV, seed, garbage=1e3)
    g = torch.Generator(device=DEV).manual_seed(seed + 100)
    q = torch.randn(sum(q_lens), hq, d, generator=g, device=DEV).to(dtype)
    qsl = torch.tensor(np.concatenate([[0], np.cumsum(q_lens)]), dtype=torch.int32, device=DEV)
    positions = torch.cat([torch.arange(kv - ql, kv, dtype=torch.int32, device=DEV)
                           for ql, kv in seqs])
    return p, q, qsl, positions


@pytest.mark.parametrize("scenario", list(SCENARIOS))
@pytest.mark.parametrize("heads", HEADS, ids=lambda h: "x".join(map(str, h)))
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_varlen_scenarios(scenario, heads, dtype):
    hq, hkv, d, bs = heads
    print(f"[varlen] {scenario} {heads} {dtype}", flush=True)
    seqs = SCENARIOS[scenario]
    p, q, qsl, positions = build_varlen(seqs, hq, hkv, d, bs, dtype, seed=5)
    out = paged_varlen_attention(q, p.k_pool, p.v_pool, p.block_tables, qsl, positions,
                                 num_heads=hq, num_kv_heads=hkv)
    torch.cuda.synchronize()
    eo, _ = oracle(q, p.k_pool, p.v_pool, p.block_tables, p.seq_lens, qsl)
    close(out, eo, dtype, f"{scenario} {heads}")


def test_list_metadata_and_module_form():
    hq, hkv, d, bs = 8, 1, 64, 16
    seqs = [(3, 40), (1, 17), (5, 5)]
    p, q, qsl, positions = build_varlen(seqs, hq, hkv, d, bs, torch.float32, seed=6)
    tables = [t for t in p.tables]
    mod = PagedVarlenAttention(hq, hkv)
    out = mod(q, p.k_pool, p.v_pool, tables, qsl.tolist(), positions.tolist())
    eo, _ = oracle(q, p.k_pool, p.v_pool, p.block_tables, p.seq_lens, qsl)
    close(out, eo, torch.float32, "lists")
    with pytest.raises(NotImplementedError):
        paged_varlen_attention(q, p.k_pool, p.v_pool, tables, qsl.tolist(), positions.tolist(),
                               hq, hkv, non_causal=True)
    with pytest.raises(ValueError):
        paged_varlen_attention(q, p.k_pool, p.v_pool, tables, qsl.tolist(), positions.tolist(),
                               hq + 1, hkv)


def test_native_fwd_lse_noncausal_scale_and_empty_rows():
    hq, hkv, d, bs = 4, 2, 32, 16
    seqs = [(2, 30), (1, 1), (4, 4)]
    p, q, qsl, _ = build_varlen(seqs, hq, hkv, d, bs, torch.float32, seed=7)
    lens = p.seq_lens.clone()
    lens[1] = 0  # no visible key: out 0, lse +inf
    for causal in (True, False):
        for scale in (0.0, 0.3):
            O, L = paged_attn_fwd(q, p.k_pool, p.v_pool, p.block_tables, lens, qsl, 4,
                                  scale=scale, causal=causal)
            eo, el = oracle(q, p.k_pool, p.v_pool, p.block_tables, lens, qsl,
                            scale=scale if scale > 0 else None, causal=causal)
            close(O, eo, torch.float32, f"causal={causal} scale={scale}")
            Ln = L.cpu().numpy()
            assert np.all(np.isinf(Ln[2]) & (Ln[2] > 0))
            fin = np.isfinite(el)
            np.testing.assert_allclose(Ln[fin], el[fin], rtol=1e-5, atol=1e-5)
            assert not O[2].any()


def test_kv_len_clamped_to_table_capacity():
    p = workloads.cfg2_problem(torch.float32, DEV, seed=3)
    big = p.seq_lens + 5000
    out = paged_mqa_decode(p.q, p.k_pool, p.v_pool, p.block_tables, big)
    cap = torch.full_like(p.seq_lens, p.block_tables.shape[1] * p.bs)
    eo, _ = oracle(p.q, p.k_pool, p.v_pool, p.block_tables, torch.minimum(big, cap))
    close(out, eo, torch.float32, "clamped")


@pytest.mark.parametrize("bs", [16, 32])
def test_cfg5_shape_decode_sampled(bs):
    # full BASELINE config 5 decode shape (N=256, Hq=32, D=128, bf16,
    # fragmented tables); the oracle checks a sample of 24 sequences
    print(f"[cfg5 decode] bs={bs}", flush=True)
    p = workloads.cfg5_problem(DEV, seed=0, bs=bs)
    out = paged_mqa_decode(p.q, p.k_pool, p.v_pool, p.block_tables, p.seq_lens,
                           max_kv_len=int(p.lens.max()))
    torch.cuda.synchronize()
    rng = np.random.default_rng(0)
    pick = np.sort(rng.choice(p.n_seq, 24, replace=False))
    pick = np.union1d(pick, [int(np.argmax(p.lens)), int(np.argmin(p.lens))])
    idx = torch.as_tensor(pick, device=DEV)
    eo, _ = oracle(p.q[idx], p.k_pool, p.v_pool, p.block_tables[idx], p.seq_lens[idx])
    close(out[idx], eo, torch.bfloat16, "cfg5")
