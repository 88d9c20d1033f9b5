"""Greedy token choice (csrc/sampling.hip, pkv_argmax_rows) against
torch.argmax on the CPU, bit-exact: the first index holding the maximum and
the framework's NaN order. Vocabulary sizes with unaligned rows (50257:
rows start off a 16-byte boundary), tiny and large rows, strided rows,
planted ties inside one 16-byte vector, across threads and across
wavefronts, NaN rows, all -inf rows; fp32 / fp16 / bf16. Also the greedy
decode-step helpers that use it (sampling.greedy).

The fused top-k / top-p sampling kernel (pkv_sample_rows) against the
float64 restatement at the same uniforms (oracle/sampling_ref.py): kept set
and drawn token, fp32 / bf16 / fp16, vocabularies of 37 to 50257, top_k 1
to 64, ties at the threshold, strided rows, the draw frequencies over a
grid of uniforms, the reference's errors and the fallback when the kernel
declines a call."""
import numpy as np
import pytest
import torch

from oracle import sampling_ref as sref
from serving import _native, fused_ops, sampling
from serving import sampling as smp

pytestmark = pytest.mark.gpu
DEV = "cuda"


def check(logits):
    got = fused_ops.argmax_rows(logits)
    torch.cuda.synchronize()
    expect = logits.cpu().argmax(-1)
    assert torch.equal(got.cpu(), expect), (got.cpu()[got.cpu() != expect][:8],
                                            expect[got.cpu() != expect][:8])


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("rows,vocab", [(128, 50257), (3, 1), (5, 7), (9, 8), (2, 100003),
                                        (64, 4096), (600, 3000), (520, 70001)])
def test_argmax_random(dtype, rows, vocab):
    print(f"[argmax] {dtype} rows={rows} vocab={vocab}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(rows * 7 + vocab)
    check((4 * torch.randn(rows, vocab, generator=g, device=DEV)).to(dtype))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_argmax_ties_nan_inf_and_strides(dtype):
    vocab = 50257
    base = torch.randn(12, vocab + 40, device=DEV).to(dtype)
    x = base[:, 3:3 + vocab]  # strided rows, unaligned starts
    x[0, 10] = x[0, 40000] = 100          # far apart: first wins
    x[1, 4097] = x[1, 4096] = 100         # neighbours (one vector or a boundary)
    x[2, 8] = x[2, 9] = x[2, 10] = 100    # inside one 16-byte vector
    x[3, 50256] = 100                     # last element (tail)
    x[4, 0] = 100                         # first element (unaligned head)
    x[5, 30000] = float("nan")
    x[5, 500] = float("nan")              # first NaN wins
    x[6, :] = float("-inf")               # no finite value: index 0
    x[7, 7] = float("inf")
    x[7, 6] = float("inf")
    x[8, 123] = float("nan")
    x[8, 50000] = float("inf")
    x[9, :] = 1.0                          # all equal
    x[10, 33] = -0.0
    x[10, :] = torch.where(x[10] > 0, -x[10], x[10])
    x[10, 33] = 0.0
    x[10, 12] = -0.0                       # +0 and -0 compare equal: first wins
    check(x)


def test_greedy_helper_uses_kernel():
    logits = torch.randn(16, 50257, device=DEV, dtype=torch.bfloat16)
    out = sampling.greedy(logits)
    assert out.shape == (16, 1) and out.dtype == torch.long
    assert torch.equal(out.cpu(), logits.cpu().argmax(-1, keepdim=True))


# ---- fused top-k / top-p sampling (pkv_sample_rows) against the float64
# restatement (oracle/sampling_ref.py) at the same uniforms; a row whose
# uniform lies within 1e-5 of a bucket edge (fp32 vs fp64 sums) is skipped,
# and most rows must be checked.


def _check_rows(logits, temperature, top_k, top_p, seed, min_checked=0.9):
    rows = logits.shape[0]
    g = torch.Generator(device=DEV).manual_seed(seed)
    u = torch.rand(rows, generator=g, device=DEV)
    ids, status = fused_ops.sample_rows(logits, temperature, top_k, top_p, u)
    torch.cuda.synchronize()
    assert int(status.item()) == 0
    x = logits.float().cpu().numpy().astype(np.float64)
    y32 = (logits.float() / temperature).cpu().numpy().astype(np.float64)
    got = ids.cpu().numpy()
    checked = 0
    for r in range(rows):
        keep, probs = sref.sample_probs(y32[r], 1.0, top_k, top_p)
        # a top-p boundary within rounding (equal masses from ties) may keep
        # one token more or less in fp32 than in fp64: such rows are skipped
        kk = sref.top_k_keep(y32[r], top_k)
        kidx = np.nonzero(kk)[0]
        order = kidx[np.lexsort((kidx, -y32[r][kidx]))]
        e = np.exp(y32[r][order] - y32[r][order[0]])
        near_p = top_p < 1.0 and np.min(np.abs(np.cumsum(e / e.sum()) - top_p)) < 1e-5
        if near_p:
            continue
        assert keep[got[r]], f"row {r}: token {got[r]} outside the top-k/top-p set"
        want, margin = sref.pick(probs, float(u[r]))
        if margin > 1e-5:
            assert got[r] == want, f"row {r}: kernel {got[r]} oracle {want}"
            checked += 1
    assert checked >= min_checked * rows, f"only {checked} of {rows} rows checked"
    del x


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows,vocab,top_k,top_p,temp", [
    (128, 50257, 32, 0.9, 1.0),
    (64, 50257, 64, 1.0, 0.7),
    (33, 1000, 5, 0.5, 1.3),
    (7, 37, 64, 0.95, 1.0),
    (16, 4096, 1, 1.0, 1.0),
])
def test_sample_rows_vs_oracle(dtype, rows, vocab, top_k, top_p, temp):
    print(f"[sample_rows] {dtype} rows={rows} vocab={vocab} k={top_k} p={top_p} t={temp}",
          flush=True)
    g = torch.Generator(device=DEV).manual_seed(rows * vocab)
    logits = (3 * torch.randn(rows, vocab, generator=g, device=DEV)).to(dtype)
    _check_rows(logits, temp, top_k, top_p, seed=rows + top_k)


def test_sample_rows_ties_and_strided_rows():
    # bf16 logits on a coarse grid: many values tie at the top-k threshold
    g = torch.Generator(device=DEV).manual_seed(5)
    base = torch.randint(0, 12, (40, 3000), generator=g, device=DEV).float() / 4
    logits = base.to(torch.bfloat16)
    _check_rows(logits, 1.0, 16, 0.77, seed=6, min_checked=0.6)
    wide = torch.zeros(40, 3200, dtype=torch.bfloat16, device=DEV)
    wide[:, 100:3100] = logits
    _check_rows(wide[:, 100:3100], 1.0, 16, 0.77, seed=6, min_checked=0.6)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("vocab", [50257, 65536, 65537, 1000])
def test_sample_top_k_1_picks_head_and_tail_maxima(dtype, vocab):
    """top_k 1 is the argmax (a single maximum) also when the maximum sits
    in a row's scalar head (before the first 16-byte boundary) or its scalar
    tail, on rows that start off the 16-byte grid; 65536 entries is the
    largest row held in registers, 65537 the smallest one that is not."""
    rows = 24
    print(f"[sample head/tail] {dtype} vocab={vocab}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(vocab)
    base = torch.randn(rows, vocab + 8, generator=g, device=DEV).to(dtype)
    x = base[:, 3:3 + vocab]
    es = x.element_size()
    for r in range(rows):
        head = min(vocab, ((16 - x[r].data_ptr() % 16) % 16) // es)
        tail = (vocab - head) % (16 // es)
        if r % 3 == 0 and head > 0:
            x[r, r % head] = 9.0
        elif r % 3 == 1 and tail > 0:
            x[r, vocab - 1 - r % tail] = 9.0
        else:
            x[r, (r * 977) % vocab] = 9.0  # (no tie: tied maxima all survive top_k 1)
    u = torch.rand(rows, generator=g, device=DEV)
    ids, st = fused_ops.sample_rows(x, 1.0, 1, 1.0, u)
    torch.cuda.synchronize()
    assert int(st.item()) == 0
    assert torch.equal(ids.cpu(), x.float().cpu().argmax(-1))


def test_sample_top_k_1_is_argmax_and_distribution_matches():
    g = torch.Generator(device=DEV).manual_seed(9)
    logits = torch.randn(256, 5000, generator=g, device=DEV)
    u = torch.rand(256, generator=g, device=DEV)
    ids, st = fused_ops.sample_rows(logits, 1.0, 1, 1.0, u)
    assert torch.equal(ids, torch.argmax(logits, dim=-1))
    # one row drawn at a grid of uniforms: the frequencies are the probabilities
    row = torch.tensor([[2.0, 1.0, 0.5, 0.0, -1.0] + [-30.0] * 59], device=DEV)
    n = 4096
    us = (torch.arange(n, device=DEV, dtype=torch.float32) + 0.5) / n
    ids, st = fused_ops.sample_rows(row.expand(n, -1).contiguous(), 1.0, 4, 1.0, us)
    freq = torch.bincount(ids, minlength=64).float().cpu().numpy() / n
    _, probs = sref.sample_probs(row[0].cpu().numpy().astype(np.float64), 1.0, 4, 1.0)
    assert np.allclose(freq, probs, atol=2e-3)


def test_sample_errors_and_overflow_fallback():
    with pytest.raises(ValueError, match="NaN or infinity"):
        smp.sample(torch.tensor([[0.0, float("nan")]], device=DEV), top_k=2)
    # every logit equal: all 5000 values reach the threshold -> the kernel
    # declines the call and sample() draws with the framework path
    flat = torch.zeros(3, 5000, device=DEV)
    u = torch.rand(3, device=DEV)
    ids, st = fused_ops.sample_rows(flat, 1.0, 32, 0.9, u)
    assert int(st.item()) & _native.PKV_STATUS_SAMPLE_OVERFLOW
    tok = smp.sample(flat, temperature=1.0, top_k=32, top_p=0.9)
    assert tok.shape == (3, 1) and bool(((tok >= 0) & (tok < 5000)).all())
    # the kernel path of sample(): tokens inside the kept set
    g = torch.Generator(device=DEV).manual_seed(11)
    logits = torch.randn(64, 50257, generator=g, device=DEV).bfloat16()
    tok = smp.sample(logits, temperature=1.0, top_k=32, top_p=0.9).squeeze(-1).cpu().numpy()
    y = logits.float().cpu().numpy().astype(np.float64)
    for r in range(64):
        keep, _ = sref.sample_probs(y[r], 1.0, 32, 0.9)
        assert keep[tok[r]]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("vocab", [50257, 1000, 20])
def test_sample_status_bits_16bit(dtype, vocab):
    """Status bits and the -1 id of a declined row, per row, against the
    per-element rule: NONFINITE for a non-finite logit, BAD_DISTRIBUTION for
    a finite logit whose scaled value is not finite, SAMPLE_OVERFLOW for more
    than 1024 values at the threshold."""
    print(f"[sample status] {dtype} vocab={vocab}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(vocab)
    base = (3 * torch.randn(6, vocab, generator=g, device=DEV)).to(dtype)
    base[1, vocab // 2] = float("nan")
    base[2, vocab - 1] = float("-inf")
    base[3, 3] = float("inf")
    base[4, 0] = float("nan")
    base[4, 1] = 60000.0 if dtype == torch.float16 else 3e38
    base[5] = 0.0
    for temp in (1.0, 1e-3, 1e-36):
        for r in range(6):
            x = base[r:r + 1].contiguous()
            xf = x.float().cpu().numpy()[0]
            fin = np.isfinite(xf)
            with np.errstate(over="ignore", invalid="ignore"):
                y = xf.astype(np.float32) / np.float32(temp)
            want = 0
            if not fin.all():
                want |= _native.PKV_STATUS_NONFINITE
            if (fin & ~np.isfinite(y)).any():
                want |= _native.PKV_STATUS_BAD_DISTRIBUTION
            if want == 0 and r == 5 and vocab > 1024:
                want = _native.PKV_STATUS_SAMPLE_OVERFLOW
            u = torch.full((1,), 0.5, device=DEV)
            ids, st = fused_ops.sample_rows(x, temp, 32, 0.9, u)
            torch.cuda.synchronize()
            assert int(st.item()) == want, f"row {r} temp {temp}: status {int(st.item())} want {want}"
            if want:
                assert int(ids.item()) == -1
            else:
                assert 0 <= int(ids.item()) < vocab


# ---- split argmax rows (several workgroups per row, through the workspace)
# against one workgroup per row (no workspace): the same ids


def _abi_argmax(logits, ws):
    rows, vocab = logits.shape
    ids = torch.full((rows,), -7, dtype=torch.long, device=DEV)
    wsb = 0 if ws is None else ws.numel()
    rc = _native.lib().pkv_argmax_rows(ids.data_ptr(), logits.data_ptr(), rows, vocab,
                                       logits.stride(0), _native.dtype_code(logits.dtype),
                                       _native.ptr(ws), wsb, _native.stream_ptr(logits.device))
    _native.check(rc, "argmax_rows")
    return ids


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows,vocab", [(128, 50257), (3, 100003), (40, 16385), (511, 20000),
                                        (2, 40000)])
def test_split_argmax_agrees_with_one_workgroup_per_row(dtype, rows, vocab):
    print(f"[split argmax] {dtype} rows={rows} vocab={vocab}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(rows + vocab)
    logits = (3 * torch.randn(rows, vocab + 5, generator=g, device=DEV)).to(dtype)[:, 2:2 + vocab]
    # planted ties across slices, NaN in a late slice, +0 / -0, -inf rows
    logits[0, 100] = logits[0, vocab - 3] = 50
    logits[1, vocab // 2] = logits[1, vocab // 2 + 1] = 50
    logits[-1, vocab - 1] = float("nan")
    logits[-1, vocab // 3] = float("nan")
    if rows > 3:
        logits[2] = -1.0
        logits[2, vocab - 1] = 0.0
        logits[2, 7] = -0.0
        logits[3] = float("-inf")
    nb = _native.lib().pkv_argmax_workspace_bytes(rows, vocab, _native.dtype_code(dtype))
    assert nb > 0
    ws = torch.zeros(nb, dtype=torch.uint8, device=DEV)
    expect = logits.cpu().argmax(-1)
    for rep in range(3):  # counters and key words are left at zero by every call
        a = _abi_argmax(logits, ws)
        b = _abi_argmax(logits, None)
        torch.cuda.synchronize()
        assert torch.equal(a.cpu(), expect), f"rep {rep}: split argmax differs from torch"
        assert torch.equal(b.cpu(), expect), f"rep {rep}: one-workgroup argmax differs"
    assert torch.equal(ws, torch.zeros_like(ws))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_argmax_negative_nan_and_slice_ends(dtype):
    """A NaN with its sign bit set is still the largest value; maxima in the
    last 16-byte vector of a slice (the vector every clamped load of the
    slice's last round re-reads) and in the scalar head and tail."""
    rows, vocab = 64, 50257
    print(f"[argmax slice ends] {dtype}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(5)
    base = (3 * torch.randn(rows, vocab + 8, generator=g, device=DEV)).to(dtype)
    logits = base[:, 1:1 + vocab]  # rows start off the 16-byte grid
    # NaN bit patterns with the sign bit set: 0xffc00001, 0xffc1, 0xfe01
    ibits = {torch.float32: (torch.int32, -0x3fffff), torch.bfloat16: (torch.int16, -0x3f),
             torch.float16: (torch.int16, -0x1ff)}[dtype]
    nn = torch.tensor([ibits[1]], dtype=ibits[0]).view(dtype)[0].to(DEV)
    assert bool(torch.isnan(nn)) and bool(torch.signbit(nn))
    logits[0, 4000] = nn
    logits[1, 4000] = nn
    logits[1, 3000] = float("nan")
    logits[2, 3000] = nn
    logits[2, 4000] = float("nan")
    es = logits.element_size()
    V = 16 // es
    nsplit = min(64, -(-vocab // (256 * 4 * V)))
    for r in range(3, rows):
        addr = logits[r].data_ptr()
        head = min(vocab, ((16 - addr % 16) % 16) // es)
        nvec = (vocab - head) // V
        per = -(-nvec // nsplit)
        k = r % (nsplit + 2)
        if k == nsplit:
            pos = max(head - 1, 0)            # the scalar head
        elif k == nsplit + 1:
            pos = vocab - 1                   # the scalar tail (or the last vector)
        else:
            pos = head + (min(nvec, (k + 1) * per) - 1) * V + (r % V)
        logits[r, pos] = 60
        if r % 2:
            logits[r, (pos * 7) % vocab] = 60  # a tie elsewhere: the first wins
    nb = _native.lib().pkv_argmax_workspace_bytes(rows, vocab, _native.dtype_code(dtype))
    ws = torch.zeros(nb, dtype=torch.uint8, device=DEV)
    expect = logits.cpu().argmax(-1)
    assert int(expect[0]) == 4000 and int(expect[1]) == 3000 and int(expect[2]) == 3000
    a = _abi_argmax(logits, ws)
    b = _abi_argmax(logits, None)
    torch.cuda.synchronize()
    assert torch.equal(a.cpu(), expect)
    assert torch.equal(b.cpu(), expect)


def test_argmax_workspace_query():
    L = _native.lib()
    bf = _native.dtype_code(torch.bfloat16)
    assert L.pkv_argmax_workspace_bytes(128, 50257, bf) == 128 * 256
    assert L.pkv_argmax_workspace_bytes(512, 50257, bf) == 0  # one workgroup per row
    assert L.pkv_argmax_workspace_bytes(128, 1000, bf) == 0   # one slice
    assert L.pkv_argmax_workspace_bytes(4, 30000, bf) == 4 * 256
