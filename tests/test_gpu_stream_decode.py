"""The wavefront-specialised persistent decode kernel (part_tokens =
PART_STREAM: producer wavefronts stream K/V into an LDS ring by LDS-DMA,
consumer wavefronts compute 16 heads x 16 tokens of every chunk, end-worker
wavefronts finish the sequences) through the C ABI with the status word:

  - config 5 in full (256 lognormal contexts, 32 heads, D 128), every row
    against the reference's gather + SDPA path in fp32 and a sample against
    the fp64 oracle, block sizes 16 and 32; no PKV_STATUS_STALLED (every
    wait between the kernel's wavefronts ended);
  - fp16, 16 heads per kv head, two kv heads;
  - a table entry outside the pool: its rows read as zeros (the zero fill of
    pagedattn.cu:47-76's asyncLOAD_PAGED_TILE) and PKV_STATUS_BAD_BLOCK;
  - repeated calls give identical bits.
bf16/fp16 tolerance 2e-2 absolute (P rounded to the 16-bit type for PV).
"""
import numpy as np
import pytest
import torch

from oracle import paged_ref as ref
from oracle import torch_ref
from serving import _native, workloads

pytestmark = pytest.mark.gpu
DEV = "cuda"
STREAM = _native.PART_STREAM


def np64(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def call(p, out, lse, status, part=STREAM):
    T, hq, d = p.q.shape
    nb, bs, hkv, _ = p.k_pool.shape
    mb = p.block_tables.shape[1]
    code = _native.kv_code(p.q.dtype, p.k_pool.dtype)
    L = _native.lib()
    wsb = L.pkv_attention_workspace_bytes(T, 1, hq, hkv, d, mb, bs, 0, part, code)
    ws = _native.current_workspace().get(p.q.device, wsb)
    rc = L.pkv_paged_attention(
        out.data_ptr(), _native.ptr(lse), p.q.data_ptr(), p.k_pool.data_ptr(),
        p.v_pool.data_ptr(), nb, bs, p.block_tables.data_ptr(), mb, p.seq_lens.data_ptr(),
        None, T, T, 1, 0, hq, hkv, d, 0.0, 1, part, code, _native.ptr(ws), wsb,
        _native.ptr(status), _native.stream_ptr(p.q.device))
    _native.check(rc, "pkv_paged_attention")


def run(p, part=STREAM):
    out = torch.empty_like(p.q)
    lse = torch.empty(p.q.shape[0], p.hq, device=DEV)
    st = torch.zeros(1, dtype=torch.int32, device=DEV)
    call(p, out, lse, st, part)
    torch.cuda.synchronize()
    return out, lse, int(st.item())


def check(out, lse, eo, el, what, tol=2e-2):
    got = np64(out)
    assert np.all(np.isfinite(got)), what
    err = np.abs(got - eo).max()
    assert err <= tol, f"{what}: max err {err:.3e}"
    if lse is not None:
        L = lse.cpu().numpy()
        fin = np.isfinite(el)
        assert np.array_equal(np.isinf(L), ~fin), f"{what}: lse infinities"
        np.testing.assert_allclose(L[fin], el[fin], rtol=0, atol=tol, err_msg=what)


@pytest.mark.parametrize("bs", [16, 32])
def test_cfg5_every_row(bs):
    print(f"[stream cfg5] bs={bs}", flush=True)
    p = workloads.cfg5_problem(DEV, seed=3, bs=bs)
    out, lse, st = run(p)
    assert st == 0, f"status {st}"
    # every row against gather + SDPA in fp32 (pinned against paged_ref by
    # tests/test_oracle.py)
    sdpa = torch_ref.paged_attention_sdpa(p.q, p.k_pool, p.v_pool, p.block_tables,
                                          p.seq_lens, dtype=torch.float32)
    err = (out.float().cpu() - sdpa).abs().max().item()
    assert err <= 2e-2, f"all rows vs SDPA: {err:.3e}"
    # a sample, with lse, against the fp64 oracle
    rows = np.r_[np.argsort(p.lens)[-3:], np.argsort(p.lens)[:3], np.arange(0, 256, 37)]
    sub = workloads.DecodeProblem(q=p.q[rows], k_pool=p.k_pool, v_pool=p.v_pool,
                                  block_tables=p.block_tables[rows], seq_lens=p.seq_lens[rows],
                                  lens=p.lens[rows], tables=None, hq=p.hq, hkv=p.hkv, d=p.d,
                                  bs=p.bs)
    eo, el = ref.paged_attention(np64(sub.q), np64(p.k_pool), np64(p.v_pool),
                                 sub.block_tables.cpu().numpy(), sub.seq_lens.cpu().numpy(), None)
    check(out[rows], lse[rows], eo, el, "sample vs fp64 oracle")


@pytest.mark.parametrize("dtype,hq,hkv", [(torch.float16, 32, 1), (torch.bfloat16, 16, 1),
                                          (torch.bfloat16, 64, 2), (torch.float16, 32, 2)])
def test_shapes(dtype, hq, hkv):
    print(f"[stream shapes] {dtype} hq={hq} hkv={hkv}", flush=True)
    lens = [700, 3, 4000, 90, 1, 2500, 33]
    p = workloads.decode_problem(lens, hq, hkv, 128, 16, 1024, dtype, DEV, seed=41)
    out, lse, st = run(p)
    assert st == 0, f"status {st}"
    eo, el = ref.paged_attention(np64(p.q), np64(p.k_pool), np64(p.v_pool),
                                 p.block_tables.cpu().numpy(), p.seq_lens.cpu().numpy(), None)
    check(out, lse, eo, el, f"{dtype} hq={hq} hkv={hkv}")


def test_bad_table_entry_reads_zeros_and_sets_status():
    lens = [3000, 500, 1700]
    p = workloads.decode_problem(lens, 32, 1, 128, 16, 1024, torch.bfloat16, DEV, seed=42)
    nb = p.k_pool.shape[0]
    used = {int(b) for t in p.tables for b in t}
    spare = next(b for b in range(1, nb) if b not in used)
    # expected: the entry points at a block of zeros
    k0, v0 = p.k_pool.clone(), p.v_pool.clone()
    k0[spare] = 0
    v0[spare] = 0
    tbl_ref = p.block_tables.clone()
    tbl_ref[0, 40] = spare
    tbl_ref[2, 0] = spare
    eo, el = ref.paged_attention(np64(p.q), np64(k0), np64(v0), tbl_ref.cpu().numpy(),
                                 p.seq_lens.cpu().numpy(), None)
    p.block_tables[0, 40] = nb + 5
    p.block_tables[2, 0] = -7
    out, lse, st = run(p)
    assert st & _native.PKV_STATUS_BAD_BLOCK, f"status {st}"
    assert not st & _native.PKV_STATUS_STALLED, f"status {st}"
    check(out, lse, eo, el, "bad entries")


def test_repeated_calls_identical_bits():
    p = workloads.cfg5_problem(DEV, seed=5, bs=16)
    a, la, sa = run(p)
    for k in range(3):
        b, lb, sb = run(p)
        assert sa == sb == 0
        assert torch.equal(a, b) and torch.equal(la, lb), f"call {k + 1} differs"
