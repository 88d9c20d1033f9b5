"""The sampling restatement (oracle/sampling_ref.py) pinned without the
reference import: the reference's own known answers (tests/test_sampling.py
of the reference: top_k = 1 is the argmax, exactly k kept without ties,
[10, 0, 0, 0] at top_p 0.5 keeps one token, top_p = 1 keeps all), the
framework's topk / sort / softmax / cumsum on random rows (library routines,
through serving/sampling.py's apply_top_k / apply_top_p, the reference's
formulas), brute force on tiny rows, and the inverse-CDF draw against its
closed form. Also: the C ABI refuses bad sampling arguments without a
launch."""
import itertools

import numpy as np
import pytest
import torch

from oracle import sampling_ref as sr
from serving import _native
from serving.sampling import apply_top_k, apply_top_p


def test_reference_known_answers():
    k, _ = sr.sample_probs(np.array([0.0, 8.0, 2.0]), 1.0, 1, 1.0)
    assert np.nonzero(k)[0].tolist() == [1]
    k, _ = sr.sample_probs(np.arange(10.0), 1.0, 3, 1.0)
    assert np.nonzero(k)[0].tolist() == [7, 8, 9]
    k, _ = sr.sample_probs(np.array([10.0, 0.0, 0.0, 0.0]), 1.0, 0, 0.5)
    assert k.sum() == 1 and k[0]
    rng = np.random.default_rng(1)
    x = rng.standard_normal(50)
    assert sr.sample_probs(x, 1.0, 0, 1.0)[0].all()


def test_ties_at_the_threshold_are_kept():
    k, p = sr.sample_probs(np.array([3.0, 3.0, 3.0, 1.0]), 1.0, 2, 1.0)
    assert k.tolist() == [True, True, True, False]
    assert np.allclose(p[:3], 1 / 3)


@pytest.mark.parametrize("seed", range(6))
def test_masks_match_framework_routines(seed):
    rng = np.random.default_rng(seed)
    # float32 rows, as sample() hands them over (logits.float())
    x = (rng.standard_normal((4, 300)) * 2).astype(np.float32).astype(np.float64)
    top_k = [1, 7, 32, 300][seed % 4]
    top_p = [1.0, 0.9, 0.5, 0.2, 0.95, 0.7][seed]
    temp = [1.0, 0.7, 1.3][seed % 3]
    t = torch.from_numpy(x).float()
    y = (t / temp).double()  # the division in fp32, as sample() does it
    ref = apply_top_p(apply_top_k(y, top_k), top_p)
    x = y.numpy() * temp
    for r in range(4):
        keep, probs = sr.sample_probs(y[r].numpy(), 1.0, top_k, top_p)
        assert np.array_equal(keep, torch.isfinite(ref[r]).numpy()), f"row {r}"
        want = torch.softmax(ref[r], -1).numpy()
        assert np.allclose(probs, want, rtol=1e-12, atol=1e-15)


def test_brute_force_tiny_rows():
    # every row of 4 values from a small grid, every k and a few top_p:
    # the kept set is the smallest descending prefix (ties kept at the k-th
    # value) whose mass before each member is <= top_p
    grid = [-1.0, 0.0, 0.5, 2.0]
    for row in itertools.product(grid, repeat=4):
        x = np.array(row)
        for k in range(1, 5):
            for top_p in (0.3, 0.6, 1.0):
                keep, _ = sr.sample_probs(x, 1.0, k, top_p)
                kth = sorted(x, reverse=True)[k - 1]
                cand = [i for i in range(4) if x[i] >= kth]
                cand.sort(key=lambda i: (-x[i], i))
                e = np.exp(x[cand] - x[cand[0]])
                pr = e / e.sum()
                want, mass = [], 0.0
                for i, q in zip(cand, pr):
                    if not want or mass <= top_p:
                        want.append(i)
                    mass += q
                assert sorted(np.nonzero(keep)[0].tolist()) == sorted(want), (row, k, top_p)


def test_inverse_cdf_draw():
    probs = np.array([0.2, 0.0, 0.5, 0.3])
    assert sr.pick(probs, 0.1)[0] == 0
    assert sr.pick(probs, 0.2)[0] == 2   # zero-probability index 1 is never drawn
    assert sr.pick(probs, 0.69)[0] == 2
    assert sr.pick(probs, 0.71)[0] == 3
    assert sr.pick(probs, 0.999999)[0] == 3
    # over a fine grid of u the draw frequencies are the probabilities
    us = (np.arange(100000) + 0.5) / 100000
    counts = np.bincount([sr.pick(probs, u)[0] for u in us], minlength=4) / len(us)
    assert np.allclose(counts, probs, atol=1e-4)


def test_sample_rows_validation_without_gpu():
    L = _native.lib()
    # top_k outside the kernel's range, top_p / temperature outside their domains
    assert L.pkv_sample_rows(16, 16, 2, 10, 10, 1.0, 0, 0.9, 16, 0, None, None) == -2
    assert L.pkv_sample_rows(16, 16, 2, 10, 10, 1.0, 65, 0.9, 16, 0, None, None) == -2
    assert L.pkv_sample_rows(16, 16, 2, 10, 10, 1.0, 8, 0.0, 16, 0, None, None) == -1
    assert L.pkv_sample_rows(16, 16, 2, 10, 10, 0.0, 8, 0.9, 16, 0, None, None) == -1
    assert L.pkv_sample_rows(16, 16, 2, 10, 10, float("inf"), 8, 0.9, 16, 0, None, None) == -1
    assert L.pkv_sample_rows(16, 16, 2, 10, 5, 1.0, 8, 0.9, 16, 0, None, None) == -1
