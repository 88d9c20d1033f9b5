"""The MFMA decode kernels (the split-K partition form, part_tokens > 0 or
automatic below long context bounds; the persistent forms with equal shares
of all context chunks: register-staged, part_tokens = PART_PERSISTENT or
PART_STATIC, and wavefront-specialised, PART_STREAM, which falls back to the
register-staged one at head dim 64) against the fp64 oracle, on the shapes
that stress their work decomposition:

  - one very long sequence, cut by every workgroup share (all partials,
    one last-arriving merger);
  - hundreds of short sequences, many inside one share (finished in place);
  - empty contexts (kv_len = 0 -> zero row, lse = +inf) mixed with others;
  - sequences with no query this step (query_start_loc with q_len 0);
  - repeated calls on one workspace (per-sequence records of one call must
    never leak into the next, e.g. a sequence without a query this step).
bf16/fp16 tolerance 2e-2 absolute (bf16 P in the PV product).
"""
import numpy as np
import pytest
import torch

from oracle import paged_ref as ref
from serving import _native, workloads
from serving.fake_paged_attn import paged_attn_fwd, paged_mqa_decode

pytestmark = pytest.mark.gpu
SK = _native.PART_PERSISTENT
STATIC = _native.PART_STATIC
STREAM = _native.PART_STREAM
PART = 512  # the split-K partition kernel, 512-token partitions
DEV = "cuda"
SHAPES = [(16, 64), (32, 128), (16, 128), (32, 64)]  # (heads per kv head, D)


def np64(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def oracle(p, lens=None, qsl=None):
    lens = p.seq_lens if lens is None else lens
    return ref.paged_attention(np64(p.q), np64(p.k_pool), np64(p.v_pool),
                               p.block_tables.cpu().numpy(), lens.cpu().numpy(),
                               None if qsl is None else qsl.cpu().numpy())


def check(out, lse, eo, el, what):
    got = np64(out)
    assert np.all(np.isfinite(got)), what
    err = np.abs(got - eo).max()
    assert err <= 2e-2, f"{what}: max err {err:.3e}"
    if lse is not None:
        L = lse.cpu().numpy()
        fin = np.isfinite(el)
        assert np.array_equal(np.isinf(L), ~fin), f"{what}: lse infinities"
        np.testing.assert_allclose(L[fin], el[fin], rtol=0, atol=2e-2, err_msg=what)


@pytest.mark.parametrize("g,d", SHAPES)
@pytest.mark.parametrize("part_tokens", [SK, STATIC, STREAM, 0, 512])
def test_single_long_sequence(g, d, part_tokens):
    print(f"[decode long] g={g} d={d} part={part_tokens}", flush=True)
    p = workloads.decode_problem([30000], g, 1, d, 16, 2048, torch.bfloat16, DEV, seed=11)
    lse = torch.empty(1, g, device=DEV)
    out = paged_mqa_decode(p.q, p.k_pool, p.v_pool, p.block_tables, p.seq_lens, lse=lse,
                           part_tokens=part_tokens)
    torch.cuda.synchronize()
    eo, el = oracle(p)
    check(out, lse, eo, el, "long")


@pytest.mark.parametrize("g,d", SHAPES)
def test_many_short_and_empty_sequences_repeated(g, d):
    print(f"[decode short] g={g} d={d}", flush=True)
    rng = np.random.default_rng(12)
    lens = rng.integers(1, 90, size=600)
    lens[::17] = 0      # empty contexts
    lens[5] = 4000      # one long one among them
    p = workloads.decode_problem(np.maximum(lens, 1), g, 1, d, 16, 8192, torch.bfloat16,
                                 DEV, seed=12)
    seq_lens = torch.as_tensor(lens, dtype=torch.int32, device=DEV)
    eo, el = oracle(p, seq_lens)
    for rep in range(6):
        pt = (PART, STATIC, STREAM)[rep % 3]
        lse = torch.empty(len(lens), g, device=DEV)
        out = paged_mqa_decode(p.q, p.k_pool, p.v_pool, p.block_tables, seq_lens, lse=lse,
                               part_tokens=pt)
        torch.cuda.synchronize()
        check(out, lse, eo, el, f"short rep {rep} part_tokens={pt}")
    # the partition kernel agrees
    out2 = paged_mqa_decode(p.q, p.k_pool, p.v_pool, p.block_tables, seq_lens, part_tokens=256)
    check(out2, None, eo, el, "partition kernel")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_gqa_two_kv_heads_and_missing_queries(dtype):
    # hkv = 2 (32 query heads), query_start_loc with empty query ranges
    g, d, hkv = 16, 128, 2
    lens = [700, 3, 1500, 64, 1]
    p = workloads.decode_problem(lens, g * hkv, hkv, d, 32, 512, dtype, DEV, seed=13)
    qlens = [1, 0, 1, 1, 0]
    qsl = torch.tensor(np.concatenate([[0], np.cumsum(qlens)]), dtype=torch.int32, device=DEV)
    T = int(sum(qlens))
    q = p.q[:T].contiguous()
    eo, el = ref.paged_attention(np64(q), np64(p.k_pool), np64(p.v_pool),
                                 p.block_tables.cpu().numpy(), p.seq_lens.cpu().numpy(),
                                 qsl.cpu().numpy())
    for pt in (0, SK, STATIC, STREAM, PART):
        O = torch.empty_like(q)
        L = torch.empty(T, g * hkv, device=DEV)
        paged_mqa_decode(q, p.k_pool, p.v_pool, p.block_tables, p.seq_lens, out=O, lse=L,
                         query_start_loc=qsl, part_tokens=pt)
        torch.cuda.synchronize()
        check(O, L, eo, el, f"gqa part_tokens={pt}")
    

def test_cfg4_and_cfg5_kernels_agree():
    for name, p in [("cfg4", workloads.cfg4_problem(DEV)), ("cfg5", workloads.cfg5_problem(DEV))]:
        mk = int(p.lens.max())
        a = paged_mqa_decode(p.q, p.k_pool, p.v_pool, p.block_tables, p.seq_lens, max_kv_len=mk,
                             part_tokens=SK)
        b = paged_mqa_decode(p.q, p.k_pool, p.v_pool, p.block_tables, p.seq_lens, max_kv_len=mk,
                             part_tokens=512)
        torch.cuda.synchronize()
        diff = (a.float() - b.float()).abs().max().item()
        assert diff <= 2e-2, f"{name}: persistent vs partition kernel differ by {diff}"
    

@pytest.mark.parametrize("pt", [SK, STATIC, STREAM, PART])
def test_records_of_previous_call_do_not_leak(pt):
    """A call where every sequence is split across workgroups, then a call on
    the same workspace where some of those sequences have no query: rows are
    written only for the queries present (a guard row past T stays intact)."""
    g, d = 32, 128
    lens = [6000, 5000, 7000, 4000, 6500]
    p = workloads.decode_problem(lens, g, 1, d, 16, 4096, torch.bfloat16, DEV, seed=14)
    first = paged_mqa_decode(p.q, p.k_pool, p.v_pool, p.block_tables, p.seq_lens,
                             part_tokens=pt)
    torch.cuda.synchronize()
    eo, el = oracle(p)
    check(first, None, eo, el, "all queries")
    qlens = [0, 1, 0, 1, 1]
    qsl = torch.tensor(np.concatenate([[0], np.cumsum(qlens)]), dtype=torch.int32, device=DEV)
    T = int(sum(qlens))
    q = p.q[[1, 3, 4]].contiguous()
    out = torch.full((T + 1, g, d), 7.0, dtype=torch.bfloat16, device=DEV)
    lse = torch.full((T + 1, g), 7.0, device=DEV)
    paged_mqa_decode(q, p.k_pool, p.v_pool, p.block_tables, p.seq_lens, out=out[:T],
                     lse=lse[:T], part_tokens=pt, query_start_loc=qsl)
    torch.cuda.synchronize()
    eo2, el2 = ref.paged_attention(np64(q), np64(p.k_pool), np64(p.v_pool),
                                   p.block_tables.cpu().numpy(), p.seq_lens.cpu().numpy(),
                                   qsl.cpu().numpy())
    check(out[:T], lse[:T], eo2, el2, "subset of queries")
    assert torch.all(out[T] == 7.0) and torch.all(lse[T] == 7.0), "guard row overwritten"


def _counters():
    """The decode kernels' arrival counters in the library workspace on this
    device: the partition kernel's (first 8 KiB) and the persistent kernels'
    per-sequence ones (the last int of each 16-byte record after them, and
    the one before it, which the wavefront-specialised kernel uses for its
    second head group)."""
    buf = _native.WORKSPACE._bufs[(torch.cuda.current_device(), "attention")]
    recs = buf[8 * 1024: 256 * 1024].view(torch.int32).view(-1, 4)
    return torch.cat([buf[: 8 * 1024].view(torch.int32), recs[:, 3], recs[:, 2]])


@pytest.mark.parametrize("pt", [STATIC, STREAM, PART])
def test_cut_sequences_alternating_inputs_and_counters_reset(pt):
    """Pieces of long sequences are merged inside the kernel by the last
    workgroup to arrive, from partials other workgroups (on other XCDs)
    stored just before. Two problems with the same lengths and tables but different
    Q/K/V alternate on one workspace: a partial read before it was written
    this call (stale, from the previous call) would carry the other
    problem's values. Every call is checked, and the arrival counters are
    back to zero after each."""
    g, d = 32, 128
    rng = np.random.default_rng(21)
    lens = np.minimum(rng.lognormal(np.log(900), 1.0, size=96).astype(int) + 1, 6000)
    pa = workloads.decode_problem(lens, g, 1, d, 16, 16384, torch.bfloat16, DEV, seed=21)
    pb = workloads.decode_problem(lens, g, 1, d, 16, 16384, torch.bfloat16, DEV, seed=22)
    pb.block_tables.copy_(pa.block_tables)
    refs = {"a": oracle(pa), "b": oracle(pb)}
    for i in range(12):
        name, p = ("a", pa) if i % 2 == 0 else ("b", pb)
        lse = torch.empty(len(lens), g, device=DEV)
        out = paged_mqa_decode(p.q, p.k_pool, p.v_pool, p.block_tables, p.seq_lens, lse=lse,
                               part_tokens=pt)
        torch.cuda.synchronize()
        check(out, lse, *refs[name], f"call {i} ({name})")
        assert int(_counters().abs().sum()) == 0, f"call {i}: arrival counters not reset"


@pytest.mark.parametrize("seed", range(8))
def test_persistent_random_length_mixes(seed):
    """Random batch sizes and length mixes (a few sequences longer than a
    share, many shorter, empty contexts, sizes where the cost line has fewer
    units than workgroups): every way a share can start, end and be cut."""
    rng = np.random.default_rng(100 + seed)
    g, d = [(16, 64), (32, 128), (16, 128), (32, 64)][seed % 4]
    n = int(rng.choice([1, 3, 40, 300, 700]))
    kind = seed % 3
    if kind == 0:
        lens = rng.integers(0, 120, size=n)
    elif kind == 1:
        lens = np.minimum(rng.lognormal(np.log(600), 1.3, size=n).astype(int), 9000)
    else:
        lens = rng.integers(0, 40, size=n)
        lens[rng.integers(0, n, size=max(1, n // 50))] = rng.integers(2000, 12000)
    print(f"[decode mix] seed={seed} g={g} d={d} n={n} sum={int(lens.sum())}", flush=True)
    nb = 1 << max(10, int(np.ceil(np.log2(sum((int(x) + 15) // 16 + 1 for x in lens) * 1.3))))
    p = workloads.decode_problem(np.maximum(lens, 1), g, 1, d, 16, nb, torch.bfloat16, DEV,
                                 seed=200 + seed)
    seq_lens = torch.as_tensor(lens, dtype=torch.int32, device=DEV)
    eo, el = oracle(p, seq_lens)
    for rep in range(6):
        pt = (PART, STATIC, STREAM)[rep % 3]
        lse = torch.empty(n, g, device=DEV)
        out = paged_mqa_decode(p.q, p.k_pool, p.v_pool, p.block_tables, seq_lens, lse=lse,
                               part_tokens=pt)
        torch.cuda.synchronize()
        check(out, lse, eo, el, f"mix seed {seed} rep {rep} part_tokens {pt}")
        assert int(_counters().abs().sum()) == 0, "arrival counters not reset"


@pytest.mark.parametrize("pt", [STATIC, STREAM, 512])
def test_in_kernel_merges_replayed_from_a_hip_graph(pt):
    """The decode launch with its in-kernel merges (arrival counters in the
    workspace, reset by the last contributor) captured in a HIP graph and
    replayed with eager work and host synchronisations in between: every
    replay equals the eager result bit for bit, and the counters are zero
    after each."""
    g, d = 32, 128
    rng = np.random.default_rng(31)
    lens = np.minimum(rng.lognormal(np.log(900), 1.0, size=64).astype(int) + 1, 6000)
    p = workloads.decode_problem(lens, g, 1, d, 16, 16384, torch.bfloat16, DEV, seed=31)
    out = torch.empty_like(p.q)
    lse = torch.empty(len(lens), g, device=DEV)
    mk = int(max(lens))

    def call():
        paged_mqa_decode(p.q, p.k_pool, p.v_pool, p.block_tables, p.seq_lens, out=out,
                         lse=lse, max_kv_len=mk, part_tokens=pt)

    call()
    torch.cuda.synchronize()
    eo, el = out.clone(), lse.clone()
    check(eo, el, *oracle(p), "eager")
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        call()  # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call()
    torch.cuda.synchronize()
    for k in range(4):
        out.fill_(7.0)
        lse.fill_(7.0)
        _ = torch.randn(1024, 1024, device=DEV).sum()  # unrelated eager work
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eo) and torch.equal(lse, el), f"replay {k} differs"
        assert int(_counters().abs().sum()) == 0, f"replay {k}: counters not reset"


@pytest.mark.parametrize("scale", [1e5, 1e-6])
@pytest.mark.parametrize("g,d", [(32, 128), (16, 64)])
@pytest.mark.parametrize("part_tokens", [SK, STATIC, STREAM, 0, 512])
def test_bf16_value_range_through_staging_and_partials(scale, g, d, part_tokens):
    """bf16 values far outside fp16's range (1e5: past fp16's largest finite
    65504; 1e-6: among fp16's subnormals, a few bits of precision): the
    wavefront staging and the split-K partials keep bf16's exponent range.
    A long sequence cut by many shares, one of medium length, a short one.
    Tolerance 2e-2 relative to the value scale."""
    print(f"[decode bf16 range] scale={scale} g={g} d={d} part={part_tokens}", flush=True)
    p = workloads.decode_problem([30000, 3000, 17], g, 1, d, 16, 4096, torch.bfloat16, DEV,
                                 seed=17)
    p.v_pool.mul_(scale)
    lse = torch.empty(3, g, device=DEV)
    out = paged_mqa_decode(p.q, p.k_pool, p.v_pool, p.block_tables, p.seq_lens, lse=lse,
                           part_tokens=part_tokens)
    torch.cuda.synchronize()
    eo, el = oracle(p)
    got = np64(out)
    assert np.all(np.isfinite(got))
    err = np.abs(got - eo).max() / scale
    assert err <= 2e-2, f"max err {err:.3e} x scale"
    fin = np.isfinite(el)
    np.testing.assert_allclose(lse.cpu().numpy()[fin], el[fin], rtol=0, atol=2e-2)
