"""Paged generation loops — drop-in for serving/generation.py.

Entry points and their reference counterparts:
  generate_batched      serving/generation.py:112-148  greedy, token ids in
  generate_batched_text serving/generation.py:11-69    sampled, text in,
                                                       stops a row at EOS
  generate_paged        serving/generation.py:91-110   greedy, one sequence
  prefill_seq           serving/generation.py:71-77
  decode_step           serving/generation.py:80-88

The batched entry points share one driver (_drive): a _Cohort holds the
calls' sequences, feeds the model one prefill step of whole prompts and then
at most max_new_tokens - 1 decode steps of one token per running sequence,
and returns every block to the allocator when the call ends, normally or by
an exception. Per step the next tokens of the whole batch come from one
device call (one argmax kernel, or one sampling kernel) and one
device-to-host copy, instead of one per row. A row that samples
eos_token_id stops there; the EOS token is not part of its output, and the
decode steps after it leave that row out of the batch.
"""
from __future__ import annotations

import torch

from .batch import build_batch_step
from .sampling import greedy, sample
from .sequence import Sequence


class _Cohort:
    """The sequences of one batched call.

    rows      Sequence objects, in prompt order
    produced  tokens emitted per row so far
    running   indices of the rows still generating, ascending (the row order
              of the next decode batch)
    feed      the token each running row feeds to the next decode step
    """

    def __init__(self, id_lists, block_size, alloc, device):
        self.alloc = alloc
        self.device = device
        self.rows = [Sequence(n, list(ids), block_size) for n, ids in enumerate(id_lists)]
        self.produced = [[] for _ in self.rows]
        self.running = list(range(len(self.rows)))
        self.feed = {}

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        for row in self.rows:
            row.release(self.alloc)
        return False

    def prefill_batch(self):
        for row in self.rows:
            row.ensure_blocks(self.alloc)
        return build_batch_step([(row, row.token_ids) for row in self.rows], self.device)

    def decode_batch(self):
        entries = []
        for n in self.running:
            row = self.rows[n]
            row.append_token(self.feed[n])
            row.ensure_blocks(self.alloc)
            entries.append((row, [self.feed[n]]))
        return build_batch_step(entries, self.device)

    def accept(self, tokens, stop_id):
        """tokens[i] is the pick of batch row i, i.e. of rows[running[i]]."""
        still = []
        for n, tok in zip(self.running, tokens):
            if stop_id is not None and tok == stop_id:
                continue
            self.produced[n].append(tok)
            self.feed[n] = tok
            still.append(n)
        self.running = still


def _drive(model, pool, cohort, max_new_tokens, pick, stop_id=None):
    cohort.accept(pick(model.forward_batch(cohort.prefill_batch(), pool)), stop_id)
    for _ in range(max_new_tokens - 1):
        if not cohort.running:
            break
        cohort.accept(pick(model.forward_batch(cohort.decode_batch(), pool)), stop_id)
    return cohort.produced


def _model_device(model):
    return next(model.parameters()).device


def _greedy_ids(logits):
    return greedy(logits)[:, 0].tolist()


@torch.no_grad()
def generate_batched(model, prompts_ids, max_new_tokens, pool, alloc, block_size=16):
    """prompts_ids: list of token-id lists. Returns the greedy continuation of
    each (max_new_tokens tokens, no EOS stop), in prompt order."""
    if max_new_tokens < 0:
        raise ValueError("max_new_tokens must be >= 0")
    if not prompts_ids:
        return []
    if not all(prompts_ids):
        raise ValueError("every prompt must contain at least one token")
    if max_new_tokens == 0:
        return [[] for _ in prompts_ids]
    with _Cohort(prompts_ids, block_size, alloc, _model_device(model)) as cohort:
        return _drive(model, pool, cohort, max_new_tokens, _greedy_ids)


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
    """Sampled batched generation from text prompts. Returns the token ids
    each prompt produced before it sampled eos_token_id (or before
    max_new_tokens). tokenizer: any object with encode_ordinary(str); the
    reference's tiktoken "gpt2" encoding when None."""
    if max_new_tokens < 0:
        raise ValueError("max_new_tokens must be >= 0")
    if not prompts:
        return []
    if temperature <= 0 or top_k < 0 or not 0 < top_p <= 1:
        raise ValueError("invalid sampling parameters")
    enc = tokenizer if tokenizer is not None else _default_tokenizer()
    id_lists = [enc.encode_ordinary(text) for text in prompts]
    if not all(id_lists):
        raise ValueError("every prompt must encode to at least one token")
    if max(len(ids) for ids in id_lists) + max_new_tokens > cfg.max_seq_len:
        raise ValueError("prompt plus requested generation exceeds max_seq_len")
    if max_new_tokens == 0:
        return [[] for _ in prompts]

    def pick(logits):
        return sample(logits, temperature=temperature, top_k=top_k, top_p=top_p)[:, 0].tolist()

    with _Cohort(id_lists, block_size, alloc, _model_device(model)) as cohort:
        return _drive(model, pool, cohort, max_new_tokens, pick, stop_id=eos_token_id)


def _last_position_argmax(model, seq, pool, new_ids):
    """Runs new_ids (the last len(new_ids) tokens of seq) through the
    single-sequence model call and returns the argmax at the last position."""
    x = torch.tensor([new_ids], dtype=torch.long, device=_model_device(model))
    logits = model(x, pool, seq.block_table, start=seq.num_tokens - len(new_ids))
    return int(logits[0, -1].argmax())


@torch.no_grad()
def prefill_seq(model, seq, pool, alloc):
    """Whole prompt of seq from position 0; returns its greedy next token."""
    seq.ensure_blocks(alloc)
    return _last_position_argmax(model, seq, pool, seq.token_ids)


@torch.no_grad()
def decode_step(model, seq, pool, alloc, token_id):
    """Appends token_id to seq, runs it at its position, returns the greedy
    next token."""
    seq.append_token(token_id)
    seq.ensure_blocks(alloc)
    return _last_position_argmax(model, seq, pool, [token_id])


@torch.no_grad()
def generate_paged(model, prompt_ids, max_new_tokens, pool, alloc, block_size=16):
    """Greedy single-sequence generation: one prefill call, then one decode
    call per further token."""
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
