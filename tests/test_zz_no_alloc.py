"""pkv_paged_attention_noalloc (no workspace argument: partials and arrival
counters in the library's per-device scratch array) against
pkv_paged_attention with a caller-owned workspace, both called through the
C ABI on the same inputs. Two calls in a row on the scratch array, the
second on a smaller problem (a different kernel and layout), each compared
bit for bit: same plan, same kernels, same combination order. A problem
whose workspace exceeds the scratch array is refused on the host. A fresh
process whose first noalloc call is captured into a HIP graph."""
import ctypes

import numpy as np
import pytest
import torch

from serving import _native, workloads

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _ptr(t):
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def _args(p, out, lse, part_tokens, max_kv_len):
    n = len(p.lens)
    return [_ptr(out), _ptr(lse), _ptr(p.q), _ptr(p.k_pool), _ptr(p.v_pool),
            p.k_pool.shape[0], p.bs, _ptr(p.block_tables), p.block_tables.shape[1],
            _ptr(p.seq_lens), None, n, n, 1, max_kv_len, p.hq, p.hkv, p.d, 0.0, 0,
            part_tokens, _native.DTYPE_CODES[p.q.dtype]]


def _run_both(p, part_tokens, label):
    print(f"[noalloc] {label}: n={len(p.lens)} hq={p.hq} d={p.d} part={part_tokens}",
          flush=True)
    L = _native.lib()
    n = len(p.lens)
    mk = int(p.lens.max())
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    ws_bytes = L.pkv_attention_workspace_bytes(n, 1, p.hq, p.hkv, p.d, p.block_tables.shape[1],
                                               p.bs, mk, part_tokens,
                                               _native.DTYPE_CODES[p.q.dtype])
    ws = torch.zeros(max(ws_bytes, 1), dtype=torch.uint8, device=DEV)
    st_a = torch.zeros(1, dtype=torch.int32, device=DEV)
    st_b = torch.zeros(1, dtype=torch.int32, device=DEV)
    out_a, lse_a = torch.full_like(p.q, 3.0), torch.full((n, p.hq), 3.0, device=DEV)
    out_b, lse_b = torch.full_like(p.q, 5.0), torch.full((n, p.hq), 5.0, device=DEV)
    rc = L.pkv_paged_attention(*_args(p, out_a, lse_a, part_tokens, mk), _ptr(ws),
                               ws.numel(), _ptr(st_a), stream)
    assert rc == 0, L.pkv_last_error()
    rc = L.pkv_paged_attention_noalloc(*_args(p, out_b, lse_b, part_tokens, mk), _ptr(st_b),
                                       stream)
    assert rc == 0, L.pkv_last_error()
    torch.cuda.synchronize()
    assert int(st_a.item()) == 0 and int(st_b.item()) == 0
    assert torch.equal(out_a.view(torch.int16), out_b.view(torch.int16)), f"{label}: out differs"
    assert torch.equal(lse_a, lse_b), f"{label}: lse differs"
    return ws_bytes


def test_noalloc_matches_workspace_entry_point_on_two_calls():
    # 1: persistent kernel, long lognormal contexts (sequences cut across
    #    workgroups: partials and arrival counters in the scratch array)
    lens1 = workloads.lengths_lognormal(96, 1024, 8192, 7)
    need = int(sum((int(x) + 15) // 16 for x in lens1))
    p1 = workloads.decode_problem(lens1, 32, 1, 128, 16, 1 << int(np.ceil(np.log2(need * 1.5))),
                                  torch.bfloat16, DEV, seed=7)
    b1 = _run_both(p1, _native.PART_PERSISTENT, "call 1 (persistent)")
    assert b1 > 256 * 1024
    # 2: smaller problem, split-K partition kernel (its counters at the start
    #    of the same scratch header, partials laid out differently)
    lens2 = workloads.lengths_uniform(24, 256, 2048, 8)
    p2 = workloads.decode_problem(lens2, 16, 1, 64, 16, 4096, torch.bfloat16, DEV, seed=8)
    b2 = _run_both(p2, 512, "call 2 (partition, smaller)")
    assert 0 < b2 < b1
    # and the persistent problem once more, after the other layout
    _run_both(p1, _native.PART_PERSISTENT, "call 3 (persistent again)")


def test_noalloc_refuses_a_problem_beyond_its_scratch():
    L = _native.lib()
    # 4096 sequences x 128 partitions of 32 tokens x 16 rows: far beyond 16 MiB
    need = L.pkv_attention_workspace_bytes(4096, 1, 16, 1, 128, 256, 16, 4096, 32,
                                           _native.DTYPE_CODES[torch.bfloat16])
    assert need > 16 << 20
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = L.pkv_paged_attention_noalloc(None, None, None, None, None, 1 << 16, 16, None, 256,
                                       None, None, 4096, 4096, 1, 4096, 16, 1, 128, 0.0, 0, 32,
                                       _native.DTYPE_CODES[torch.bfloat16], None, stream)
    assert rc == _native.PKV_ERR_WORKSPACE
    assert b"scratch" in L.pkv_last_error()


_CAPTURE_FIRST_CALL = r'''
import ctypes, sys, torch
from serving import _native, workloads
DEV = "cuda"
L = _native.lib()
lens = workloads.lengths_lognormal(64, 1024, 8192, 9)
nblk = 1 << int(sum((int(x) + 15) // 16 for x in lens) * 3 // 2).bit_length()
p = workloads.decode_problem(lens, 32, 1, 128, 16, nblk, torch.bfloat16, DEV, seed=9)
n, mk, part = len(lens), int(p.lens.max()), _native.PART_PERSISTENT
code = _native.DTYPE_CODES[p.q.dtype]
P = lambda t: ctypes.c_void_p(0 if t is None else t.data_ptr())
def args(out, lse):
    return [P(out), P(lse), P(p.q), P(p.k_pool), P(p.v_pool), p.k_pool.shape[0], p.bs,
            P(p.block_tables), p.block_tables.shape[1], P(p.seq_lens), None, n, n, 1, mk,
            p.hq, p.hkv, p.d, 0.0, 0, part, code]
def stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
wsb = L.pkv_attention_workspace_bytes(n, 1, p.hq, p.hkv, p.d, p.block_tables.shape[1], p.bs,
                                      mk, part, code)
ws = torch.zeros(wsb, dtype=torch.uint8, device=DEV)
out_a, lse_a = torch.empty_like(p.q), torch.empty(n, p.hq, device=DEV)
st_a = torch.zeros(1, dtype=torch.int32, device=DEV)
assert L.pkv_paged_attention(*args(out_a, lse_a), P(ws), wsb, P(st_a), stream()) == 0
torch.cuda.synchronize()
# the process's first noalloc call, under graph capture
out_b, lse_b = torch.full_like(p.q, 7.0), torch.full((n, p.hq), 7.0, device=DEV)
st_b = torch.zeros(1, dtype=torch.int32, device=DEV)
g = torch.cuda.CUDAGraph()
side = torch.cuda.Stream()
side.wait_stream(torch.cuda.current_stream())
with torch.cuda.stream(side), torch.cuda.graph(g, stream=side):
    rc = L.pkv_paged_attention_noalloc(*args(out_b, lse_b), P(st_b), stream())
assert rc == 0, L.pkv_last_error()
for rep in range(3):
    out_b.fill_(7.0)
    lse_b.fill_(7.0)
    g.replay()
    torch.cuda.synchronize()
    assert int(st_b.item()) == 0, f"replay {rep}: status {int(st_b.item())}"
    assert torch.equal(out_a.view(torch.int16), out_b.view(torch.int16)), f"replay {rep}: out"
    assert torch.equal(lse_a, lse_b), f"replay {rep}: lse"
    # eager noalloc calls between the replays share the scratch array
    out_c, lse_c = torch.empty_like(p.q), torch.empty(n, p.hq, device=DEV)
    st_c = torch.zeros(1, dtype=torch.int32, device=DEV)
    assert L.pkv_paged_attention_noalloc(*args(out_c, lse_c), P(st_c), stream()) == 0
    torch.cuda.synchronize()
    assert int(st_c.item()) == 0 and torch.equal(out_a.view(torch.int16), out_c.view(torch.int16))
print("capture-first-call ok", flush=True)
'''


def test_noalloc_first_call_of_a_process_under_graph_capture():
    """A fresh process whose first noalloc call is captured into a HIP graph
    (the scratch address is taken and the counter-header fill kernel becomes
    a node of the graph); three replays, with eager noalloc calls between
    them, each bit-identical to pkv_paged_attention."""
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ)
    env["PYTHONPATH"] = os.pathsep.join(
        [os.path.join(root, "tiny-transformer-inference-engine_amd"), root,
         env.get("PYTHONPATH", "")])
    print("[noalloc] capture of a process's first call (subprocess)", flush=True)
    r = subprocess.run([sys.executable, "-c", _CAPTURE_FIRST_CALL], cwd=root, env=env,
                       capture_output=True, text=True, timeout=100)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    assert "capture-first-call ok" in r.stdout
