"""The reference-side binding shown in INTEGRATION.md, executed as written.

The two ctypes stubs of INTEGRATION.md section 3 (`paged_attn_fwd`, the
drop-in for the reference's pybind11 `pagedattn` module,
kernels/pagedattn/extension.cpp:56-69, and `append_and_attend`, the fused
append + attention of serving/paged_mqa.py:98-110) are taken out of the
Markdown file, pointed at the library built in this tree, and run on split
batches (sequences long enough to be cut across workgroups, so the
workspace's arrival counters are exercised) against the fp64 oracle, twice
in a row on the stub's persistent workspace. The library's dirty-workspace
check is covered here too: a workspace whose counters are not zero raises
PKV_STATUS_DIRTY_WORKSPACE.

Tolerance: bf16, 2e-2 absolute against the oracle on the same rounded inputs
(the north star's bf16 bound).
"""
import os
import re

import numpy as np
import pytest
import torch

from oracle import paged_ref as ref
from serving import _native, workloads
from serving.kv_pool import KVPool
from serving.paged_meta import pack_batch_meta

pytestmark = pytest.mark.gpu
DEV = "cuda"
REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def shim_namespace():
    with open(os.path.join(REPO, "INTEGRATION.md")) as f:
        blocks = re.findall(r"```python\n(.*?)```", f.read(), re.S)
    stub = next(b for b in blocks if "def paged_attn_fwd" in b)
    fused = next(b for b in blocks if "def append_and_attend" in b)
    assert "/path/to/libpagedkv.so" in stub
    ns = {}
    exec(compile(stub.replace("/path/to/libpagedkv.so", _native.LIB_PATH),
                 "INTEGRATION.md:paged_attn_fwd", "exec"), ns)
    exec(compile(fused, "INTEGRATION.md:append_and_attend", "exec"), ns)
    return ns


def np64(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def check(out, expect, what):
    err = float(np.abs(np64(out) - expect).max())
    assert np.isfinite(np64(out)).all(), f"{what}: non-finite output"
    assert err <= 2e-2, f"{what}: max err {err:.3e}"


@pytest.mark.parametrize("cfg", ["cfg4", "cfg5"])
def test_shim_paged_attn_fwd_on_split_batches(cfg):
    print(f"[shim] paged_attn_fwd {cfg}", flush=True)
    ns = shim_namespace()
    dev = torch.device(DEV)
    p = (workloads.cfg4_problem(dev, seed=2) if cfg == "cfg4"
         else workloads.cfg5_problem(dev, seed=2, bs=16))
    n = p.n_seq
    qloc = torch.arange(n + 1, dtype=torch.int32, device=DEV)
    for call in range(2):  # the second call reuses the stub's workspace
        O, lse = ns["paged_attn_fwd"](p.q, p.k_pool, p.v_pool, p.block_tables, p.seq_lens,
                                      qloc, 1)
        torch.cuda.synchronize()
        # every sequence against the oracle would take minutes on the CPU:
        # check a sample that includes the longest (most split) ones
        order = np.argsort(-p.lens)
        pick = sorted(set(order[:8].tolist()) | set(range(0, n, max(1, n // 8))))
        exp, exp_lse = ref.paged_attention(
            np64(p.q[pick]), np64(p.k_pool), np64(p.v_pool),
            p.block_tables[pick].cpu().numpy(), p.lens[pick], None)
        check(O[pick], exp, f"{cfg} call {call}")
        assert np.abs(lse[pick].cpu().numpy() - exp_lse).max() < 2e-2
    # the counters are back at zero after every call
    ws = next(iter(ns["_WS"].values()))
    assert not ws[:256 * 1024].any(), "arrival counters not reset"


def test_shim_append_and_attend_matches_oracle():
    print("[shim] append_and_attend cfg4 shape", flush=True)
    ns = shim_namespace()
    dev = torch.device(DEV)
    N, HQ, D, BS, NB = 128, 16, 64, 16, 16384
    lens = workloads.lengths_uniform(N, 256, 2048, seed=3)
    tables = workloads.permuted_tables([int(x) + 1 for x in lens], BS, NB, seed=3)
    pool = KVPool(1, BS, NB, 1, D, torch.bfloat16, dev)
    g = torch.Generator(device=dev).manual_seed(3)
    pool.kv.normal_(generator=g)
    meta = pack_batch_meta(tables, list(range(N + 1)), [int(x) for x in lens], N, dev, BS)
    q = torch.randn(N, HQ, D, generator=g, device=dev).bfloat16()
    k = torch.randn(N, 1, D, generator=g, device=dev).bfloat16()
    v = torch.randn(N, 1, D, generator=g, device=dev).bfloat16()
    before_k = pool.flat_k[0].clone()
    out = ns["append_and_attend"](q, k, v, pool, 0, meta.block_tables, meta.seq_lens,
                                  meta.query_start_loc, meta.start_pos, 1, meta.max_kv_len)
    torch.cuda.synchronize()
    # the pool after the call: the new rows at their slots, nothing else changed
    fk = np64(before_k)
    slots = np.array([tables[i][int(lens[i]) // BS] * BS + int(lens[i]) % BS for i in range(N)])
    fk[slots] = np64(k)
    assert np.array_equal(np64(pool.flat_k[0]), fk), "K pool differs from the oracle append"
    pick = list(range(0, N, 8))
    exp, _ = ref.paged_attention(np64(q[pick]), np64(pool.kv[0, 0]), np64(pool.kv[0, 1]),
                                 meta.block_tables[pick].cpu().numpy(),
                                 (lens + 1)[pick], None)
    check(out[pick], exp, "append_and_attend")


def test_shim_fp8_pools():
    """The shim with float8_e4m3fn pools (CacheConfig.kv_dtype): KVPool.write
    body as INTEGRATION.md gives it is not exercised here (the product's
    KVPool is), but both attention stubs are: paged_attn_fwd on a cfg5-shaped
    batch with fp8 pools, against the oracle on the pools' fp8 values."""
    print("[shim] fp8 pools", flush=True)
    ns = shim_namespace()
    dev = torch.device(DEV)
    p = workloads.cfg5_problem(dev, seed=4, bs=16)
    k8, v8 = p.k_pool.to(torch.float8_e4m3fn), p.v_pool.to(torch.float8_e4m3fn)
    n = p.n_seq
    qloc = torch.arange(n + 1, dtype=torch.int32, device=DEV)
    O, lse = ns["paged_attn_fwd"](p.q, k8, v8, p.block_tables, p.seq_lens, qloc, 1)
    torch.cuda.synchronize()
    order = np.argsort(-p.lens)
    pick = sorted(set(order[:4].tolist()) | set(range(0, n, max(1, n // 6))))
    kv = [ref.e4m3_values(t.view(torch.uint8).cpu().numpy()) for t in (k8, v8)]
    exp, exp_lse = ref.paged_attention(np64(p.q[pick]), kv[0], kv[1],
                                       p.block_tables[pick].cpu().numpy(), p.lens[pick], None)
    check(O[pick], exp, "fp8 pools")
    assert np.abs(lse[pick].cpu().numpy() - exp_lse).max() < 2e-2


@pytest.mark.parametrize("part", [0, _native.PART_PERSISTENT])
def test_dirty_workspace_is_reported(part):
    """A workspace allocated without zero-filling (here: every byte 7) makes
    at least one workgroup see an arrival counter out of range: the call
    raises PKV_STATUS_DIRTY_WORKSPACE instead of leaving rows silently
    unwritten. A zero-filled workspace leaves the bit clear."""
    print(f"[shim] dirty workspace, part_tokens={part}", flush=True)
    dev = torch.device(DEV)
    p = workloads.cfg4_problem(dev, seed=5)
    L = _native.lib()
    hq, d, bs = p.hq, p.d, p.bs
    mk = int(p.lens.max())
    nbytes = L.pkv_attention_workspace_bytes(p.n_seq, 1, hq, 1, d, p.block_tables.shape[1], bs,
                                             mk, part, 2)
    assert nbytes > 0
    out = torch.empty_like(p.q)
    for fill, expect_dirty in ((7, True), (0, False)):
        ws = torch.full((nbytes,), fill, dtype=torch.uint8, device=DEV)
        status = torch.zeros(1, dtype=torch.int32, device=DEV)
        rc = L.pkv_paged_attention(
            out.data_ptr(), None, p.q.data_ptr(), p.k_pool.data_ptr(), p.v_pool.data_ptr(),
            p.k_pool.shape[0], bs, p.block_tables.data_ptr(), p.block_tables.shape[1],
            p.seq_lens.data_ptr(), None, p.n_seq, p.n_seq, 1, mk, hq, 1, d, 0.0, 1, part, 2,
            ws.data_ptr(), nbytes, status.data_ptr(), _native.stream_ptr(dev))
        _native.check(rc, "pkv_paged_attention")
        torch.cuda.synchronize()
        dirty = bool(int(status.item()) & _native.PKV_STATUS_DIRTY_WORKSPACE)
        assert dirty == expect_dirty, f"fill {fill}: status {int(status.item())}"
