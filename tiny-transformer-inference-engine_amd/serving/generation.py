"""Paged generation loops — drop-in for serving/generation.py.

generate_batched (greedy, reference generation.py:112-148): one prefill step
for all prompts, then max_new_tokens-1 decode steps of one token per
sequence; blocks are released in a finally block. generate_paged /
prefill_seq / decode_step are the single-sequence variants (:71-110).
generate_batched_text (:11-69) additionally needs a tokenizer; the
reference's tiktoken "gpt2" encoding is used when importable, otherwise pass
`tokenizer` (any object with encode_ordinary).
"""
from __future__ import annotations

import torch

from .batch import build_batch_step
from .sampling import greedy, sample
from .sequence import Sequence


def _argmax_tokens(logits):
    # one argmax launch and one device->host copy per step for the whole batch
    return greedy(logits)[:, 0].tolist()


@torch.no_grad()
def generate_batched(model, prompts_ids, max_new_tokens, pool, alloc, block_size=16):
    """prompts_ids: list of token-id lists. Returns the greedy continuation
    of each, in order."""
    if max_new_tokens < 0:
        raise ValueError("max_new_tokens must be >= 0")
    if not prompts_ids:
        return []
    if any(not prompt for prompt in prompts_ids):
        raise ValueError("every prompt must contain at least one token")
    if max_new_tokens == 0:
        return [[] for _ in prompts_ids]
    device = next(model.parameters()).device
    seqs = [Sequence(i, list(p), block_size) for i, p in enumerate(prompts_ids)]
    outputs = [[] for _ in seqs]
    try:
        for s in seqs:
            s.ensure_blocks(alloc)
        batch = build_batch_step([(s, s.token_ids) for s in seqs], device)
        next_tokens = _argmax_tokens(model.forward_batch(batch, pool))
        for out, t in zip(outputs, next_tokens):
            out.append(t)
        for _ in range(max_new_tokens - 1):
            for s, t in zip(seqs, next_tokens):
                s.append_token(t)
                s.ensure_blocks(alloc)
            batch = build_batch_step([(s, [t]) for s, t in zip(seqs, next_tokens)], device)
            next_tokens = _argmax_tokens(model.forward_batch(batch, pool))
            for out, t in zip(outputs, next_tokens):
                out.append(t)
        return outputs
    finally:
        for s in seqs:
            s.release(alloc)


@torch.no_grad()
def prefill_seq(model, seq, pool, alloc):
    seq.ensure_blocks(alloc)
    device = next(model.parameters()).device
    ids = torch.tensor([seq.token_ids], dtype=torch.long, device=device)
    return int(model(ids, pool, seq.block_table, start=0)[0, -1].argmax())


@torch.no_grad()
def decode_step(model, seq, pool, alloc, token_id):
    seq.append_token(token_id)
    seq.ensure_blocks(alloc)
    device = next(model.parameters()).device
    x = torch.tensor([[token_id]], dtype=torch.long, device=device)
    return int(model(x, pool, seq.block_table, start=seq.num_tokens - 1)[0, -1].argmax())


@torch.no_grad()
def generate_paged(model, prompt_ids, max_new_tokens, pool, alloc, block_size=16):
    if max_new_tokens < 0:
        raise ValueError("max_new_tokens must be >= 0")
    if not prompt_ids:
        raise ValueError("prompt must contain at least one token")
    if max_new_tokens == 0:
        return []
    seq = Sequence(0, list(prompt_ids), block_size)
    try:
        out = [prefill_seq(model, seq, pool, alloc)]
        while len(out) < max_new_tokens:
            out.append(decode_step(model, seq, pool, alloc, out[-1]))
        return out
    finally:
        seq.release(alloc)


def _default_tokenizer():
    try:
        import tiktoken
    except ImportError as e:
        raise RuntimeError(
            "generate_batched_text needs a tokenizer: install tiktoken or pass tokenizer=") from e
    return tiktoken.get_encoding("gpt2")


@torch.no_grad()
def generate_batched_text(model, cfg, prompts, max_new_tokens, eos_token_id,
                          pool, alloc, temperature=1.0, top_k=32, top_p=0.9,
                          block_size=16, tokenizer=None):
    """Sampled batched generation from text prompts (reference
    generation.py:11-69): stops a sequence at eos_token_id."""
    if max_new_tokens < 0:
        raise ValueError("max_new_tokens must be >= 0")
    if not prompts:
        return []
    if temperature <= 0 or top_k < 0 or not 0 < top_p <= 1:
        raise ValueError("invalid sampling parameters")
    enc = tokenizer if tokenizer is not None else _default_tokenizer()
    device = next(model.parameters()).device
    prompt_ids = [enc.encode_ordinary(p) for p in prompts]
    if any(not ids for ids in prompt_ids):
        raise ValueError("every prompt must encode to at least one token")
    if any(len(ids) + max_new_tokens > cfg.max_seq_len for ids in prompt_ids):
        raise ValueError("prompt plus requested generation exceeds max_seq_len")
    if max_new_tokens == 0:
        return [[] for _ in prompts]

    seqs = [Sequence(i, list(ids), block_size) for i, ids in enumerate(prompt_ids)]
    outputs = [[] for _ in seqs]

    def pick(row):
        return int(sample(row.unsqueeze(0), temperature=temperature,
                          top_k=top_k, top_p=top_p).item())
    try:
        for seq in seqs:
            seq.ensure_blocks(alloc)
        logits = model.forward_batch(build_batch_step([(s, s.token_ids) for s in seqs], device), pool)
        next_tokens = {i: pick(logits[i]) for i in range(len(seqs))}
        finished = [False] * len(seqs)
        for i, token in next_tokens.items():
            finished[i] = token == eos_token_id
            if not finished[i]:
                outputs[i].append(token)
        for _ in range(max_new_tokens - 1):
            if all(finished):
                break
            active = [i for i, done in enumerate(finished) if not done]
            for i in active:
                seqs[i].append_token(next_tokens[i])
                seqs[i].ensure_blocks(alloc)
            logits = model.forward_batch(
                build_batch_step([(seqs[i], [next_tokens[i]]) for i in active], device), pool)
            current = {}
            for row, i in enumerate(active):
                token = pick(logits[row])
                current[i] = token
                finished[i] = token == eos_token_id
                if not finished[i]:
                    outputs[i].append(token)
            next_tokens = current
        return outputs
    finally:
        for seq in seqs:
            seq.release(alloc)
