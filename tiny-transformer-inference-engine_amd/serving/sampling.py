"""Token sampling used by the Scheduler (reference: sampling.py:5-137).

greedy = argmax; sample = temperature, then top-k (keep logits >= the k-th
largest), then top-p (keep the smallest prefix of the sorted distribution
whose mass reaches top_p, always at least one token), then a multinomial
draw. Errors mirror the reference's ValueErrors.
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F

from . import fused_ops


def greedy(logits):
    """[batch, vocab] -> [batch, 1] argmax; on a ROCm device one HIP kernel
    (fused_ops.argmax_rows, same ties and NaN order as torch.argmax)."""
    if logits.is_cuda and logits.dim() == 2 and logits.shape[-1] > 0:
        return fused_ops.argmax_rows(logits)[:, None]
    return torch.argmax(logits, dim=-1, keepdim=True)


def apply_top_k(logits, top_k):
    if top_k <= 0:
        return logits
    k = min(top_k, logits.shape[-1])
    kth = torch.topk(logits.float(), k, dim=-1).values[:, -1:]
    return logits.masked_fill(logits < kth, float("-inf"))


def apply_top_p(logits, top_p):
    if top_p >= 1.0:
        return logits
    if top_p <= 0.0:
        raise ValueError("top_p must be > 0")
    sorted_logits, order = torch.sort(logits, descending=True, dim=-1)
    mass_before = torch.cumsum(F.softmax(sorted_logits, dim=-1), dim=-1)
    # drop a token when the mass strictly before it already exceeds top_p
    drop = torch.zeros_like(mass_before, dtype=torch.bool)
    drop[:, 1:] = mass_before[:, :-1] > top_p
    sorted_logits = sorted_logits.masked_fill(drop, float("-inf"))
    return torch.full_like(logits, float("-inf")).scatter(-1, order, sorted_logits)


# top_k range of the fused sampling kernel (pkv_sample_rows)
KERNEL_MAX_TOP_K = 64


def sample(logits, temperature=1.0, top_k=0, top_p=1.0):
    """On a ROCm device with 1 <= top_k <= 64: one HIP kernel per step
    (fused_ops.sample_rows) draws every row by inverse CDF at a uniform from
    torch's generator; its status word is read once (the reference's own
    finiteness checks synchronise too) to raise the reference's errors, and
    a row the kernel declines (massive ties at the threshold) sends the
    call to the framework path below."""
    if logits.ndim != 2 or logits.shape[-1] == 0:
        raise ValueError("logits must have shape [batch, vocab] with non-empty vocab")
    if not math.isfinite(temperature) or temperature <= 0:
        raise ValueError("temperature must be finite and > 0")
    if top_k < 0:
        raise ValueError("top_k must be >= 0")
    if not 0 < top_p <= 1:
        raise ValueError("top_p must be in (0, 1]")
    if (logits.is_cuda and 1 <= top_k <= KERNEL_MAX_TOP_K
            and logits.dtype in (torch.float32, torch.bfloat16, torch.float16)):
        u = torch.rand(logits.shape[0], device=logits.device, dtype=torch.float32)
        ids, status = fused_ops.sample_rows(logits, temperature, top_k, top_p, u)
        flags = int(status.item())
        if flags & fused_ops._native.PKV_STATUS_NONFINITE:
            raise ValueError("logits contain NaN or infinity")
        if flags & fused_ops._native.PKV_STATUS_BAD_DISTRIBUTION:
            raise ValueError("sampling produced an invalid probability distribution")
        if not flags & fused_ops._native.PKV_STATUS_SAMPLE_OVERFLOW:
            return ids[:, None]
    logits = logits.float()
    if not torch.isfinite(logits).all():
        raise ValueError("logits contain NaN or infinity")
    logits = apply_top_p(apply_top_k(logits / temperature, top_k), top_p)
    probs = F.softmax(logits, dim=-1)
    if not torch.isfinite(probs).all() or (probs.sum(dim=-1) <= 0).any():
        raise ValueError("sampling produced an invalid probability distribution")
    return torch.multinomial(probs, num_samples=1)
