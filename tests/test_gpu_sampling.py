"""Greedy token choice (csrc/sampling.hip, pkv_argmax_rows) against
torch.argmax on the CPU, bit-exact: the first index holding the maximum and
the framework's NaN order. Vocabulary sizes with unaligned rows (50257:
rows start off a 16-byte boundary), tiny and large rows, strided rows,
planted ties inside one 16-byte vector, across threads and across
wavefronts, NaN rows, all -inf rows; fp32 / fp16 / bf16. Also the greedy
decode-step helpers that use it (sampling.greedy)."""
import pytest
import torch

from serving import fused_ops, sampling

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
                                        (64, 4096)])
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
