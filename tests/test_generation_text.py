"""generate_batched_text on the CPU with a stub tokenizer and a fixed-logit
model (after the reference's tests/test_inference.py:9-20, whose
FixedLogitModel puts +100 on one token and -100 elsewhere). With top_k = 1
the draw is the argmax, so every sequence of tokens below is exact.

Covered: EOS ends a row without being emitted and drops it from later
batches; the requested length; one prefill step then at most
max_new_tokens - 1 decode steps; the reference's ValueErrors; blocks
returned to the allocator on success and on an exception.
"""
from types import SimpleNamespace

import pytest
import torch
from torch import nn

from serving.allocator import BlockAllocator
from serving.generation import generate_batched_text

EOS = 7


class StubTokenizer:
    """One token per character: ord(c) % 7 (never EOS)."""

    def encode_ordinary(self, text):
        return [ord(c) % 7 for c in text]


class ScriptedLogits(nn.Module):
    """Row r of the batch at step s (0 = prefill) gets +100 at
    script(seq_id, s) and -100 elsewhere; records every batch."""

    def __init__(self, script, vocab=8):
        super().__init__()
        self.anchor = nn.Parameter(torch.zeros(()))
        self.script = script
        self.vocab = vocab
        self.calls = []

    def forward_batch(self, batch, pool):
        step = len(self.calls)
        self.calls.append(SimpleNamespace(n=batch.num_seqs, ids=batch.input_ids.tolist(),
                                          positions=list(batch.positions),
                                          seq_lens=list(batch.seq_lens)))
        logits = torch.full((batch.num_seqs, self.vocab), -100.0)
        # rows of a decode batch are the running sequences in id order; the
        # stub recovers their ids from the sequence lengths it was given
        for r, sid in enumerate(self.row_ids(batch)):
            logits[r, self.script(sid, step)] = 100.0
        return logits

    def row_ids(self, batch):
        return self.ids_by_len[tuple(batch.seq_lens)] if hasattr(self, "ids_by_len") else \
            list(range(batch.num_seqs))


def cfg(max_seq_len=64):
    return SimpleNamespace(max_seq_len=max_seq_len, eos_token_id=EOS)


def gen(model, prompts, n, alloc=None, **kw):
    alloc = alloc if alloc is not None else BlockAllocator(32)
    out = generate_batched_text(model, cfg(kw.pop("max_seq_len", 64)), prompts, n, EOS, None,
                                alloc, temperature=1.0, top_k=1, top_p=1.0, block_size=4,
                                tokenizer=StubTokenizer(), **kw)
    return out, alloc


def test_eos_first_token_stops_every_row():
    model = ScriptedLogits(lambda sid, step: EOS)
    out, alloc = gen(model, ["ab", "xyz"], 5)
    assert out == [[], []]
    assert len(model.calls) == 1                  # the prefill step only
    assert alloc.num_free == alloc.num_usable


def test_requested_length():
    model = ScriptedLogits(lambda sid, step: 3)
    out, alloc = gen(model, ["a"], 3)
    assert out == [[3, 3, 3]]
    assert len(model.calls) == 3                  # prefill + 2 decode steps
    # decode steps feed the previous token at the next position
    assert [c.ids for c in model.calls] == [[ord("a") % 7], [3], [3]]
    assert [c.positions for c in model.calls] == [[0], [1], [2]]
    assert alloc.num_free == alloc.num_usable


def test_rows_finish_independently():
    # sequence 0 emits 1, 2, then EOS; sequence 1 emits 4 every step
    script = {0: [1, 2, EOS, 5, 5], 1: [4, 4, 4, 4, 4]}
    model = ScriptedLogits(lambda sid, step: script[sid][step])
    # prompt lengths 2 and 5: a batch's seq_lens name its rows
    model.ids_by_len = {(2, 5): [0, 1], (3, 6): [0, 1], (4, 7): [0, 1], (8,): [1], (9,): [1]}
    out, alloc = gen(model, ["ab", "cdefg"], 5)
    assert out == [[1, 2], [4, 4, 4, 4, 4]]
    assert [c.n for c in model.calls] == [2, 2, 2, 1, 1]
    assert model.calls[3].ids == [4] and model.calls[3].positions == [7]
    assert alloc.num_free == alloc.num_usable


def test_argument_errors_and_trivial_calls():
    model = ScriptedLogits(lambda sid, step: 1)
    with pytest.raises(ValueError, match="max_new_tokens"):
        gen(model, ["a"], -1)
    assert gen(model, [], 3)[0] == []
    for bad in (dict(temperature=0.0), dict(top_k=-1), dict(top_p=0.0), dict(top_p=1.5)):
        args = dict(temperature=1.0, top_k=1, top_p=1.0)
        args.update(bad)
        with pytest.raises(ValueError, match="invalid sampling"):
            generate_batched_text(model, cfg(), ["a"], 2, EOS, None, BlockAllocator(8),
                                  tokenizer=StubTokenizer(), **args)
    with pytest.raises(ValueError, match="encode to at least one token"):
        gen(model, ["a", ""], 2)
    with pytest.raises(ValueError, match="exceeds max_seq_len"):
        gen(model, ["abcdef"], 3, max_seq_len=8)
    out, _ = gen(model, ["abcde"], 3, max_seq_len=8)  # exactly max_seq_len
    assert out == [[1, 1, 1]]
    n_calls = len(model.calls)
    assert gen(model, ["a", "b"], 0)[0] == [[], []]
    assert len(model.calls) == n_calls            # no model call for 0 tokens


def test_blocks_released_when_the_model_raises():
    class Boom(ScriptedLogits):
        def forward_batch(self, batch, pool):
            if self.calls:
                raise RuntimeError("boom")
            return super().forward_batch(batch, pool)

    alloc = BlockAllocator(32)
    with pytest.raises(RuntimeError, match="boom"):
        gen(Boom(lambda sid, step: 1), ["abcdefgh", "ij"], 4, alloc=alloc)
    assert alloc.num_free == alloc.num_usable
