"""One engine step's batch description — drop-in for serving/batch.py."""
from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass
class BatchStep:
    input_ids: torch.Tensor   # [T] int64 on the model device
    positions: list           # absolute position of each of the T tokens
    query_start_loc: list     # cumulative token offsets, N + 1 entries
    block_tables: list        # per-sequence physical block ids
    seq_lens: list            # tokens per sequence after this step

    @property
    def num_seqs(self):
        return len(self.block_tables)


def build_batch_step(entries, device):
    """entries: (seq, new_token_ids) pairs — the whole prompt for a prefill,
    [last sampled token] for a decode (reference: serving/batch.py:18-36).
    The new tokens of a sequence occupy positions
    [num_tokens - len(new), num_tokens)."""
    input_ids, positions, qsl, block_tables, seq_lens = [], [], [0], [], []
    for seq, new_tokens in entries:
        first = seq.num_tokens - len(new_tokens)
        input_ids.extend(new_tokens)
        positions.extend(range(first, first + len(new_tokens)))
        qsl.append(qsl[-1] + len(new_tokens))
        block_tables.append(seq.block_table)
        seq_lens.append(seq.num_tokens)

    return BatchStep(
        input_ids=torch.tensor(input_ids, dtype=torch.long, device=device),
        positions=positions,
        query_start_loc=qsl,
        block_tables=block_tables,
        seq_lens=seq_lens,
    )
