"""Device-resident metadata of one paged step.

The reference rebuilds block tables, slot mappings and kv lengths per layer
and per sequence with host round trips (serving/paged_mqa.py:87-96,
serving/fake_paged_attn.py:52-100). Here the ragged host lists are validated
and packed once per step into a single int32 buffer, copied to the device in
one transfer, and reused by every layer's append and attention launch.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch


@dataclass
class PagedBatchMeta:
    block_tables: torch.Tensor     # int32 [N, max_blocks], zero padded
    seq_lens: torch.Tensor         # int32 [N]  kv length after this step
    query_start_loc: torch.Tensor  # int32 [N+1]
    start_pos: torch.Tensor        # int32 [N]  position of each sequence's first new token
    positions: torch.Tensor        # int32 [T]  absolute position of every new token
    num_seqs: int
    num_tokens: int
    max_blocks: int
    max_q_len: int
    max_kv_len: int
    block_size: int
    # seq_lens, start_pos and positions as one contiguous view (pack_batch_meta
    # lays them out back to back), so a decode step advances them with one add
    step_view: torch.Tensor | None = None

    @property
    def is_decode(self) -> bool:
        return self.max_q_len == 1 and self.num_tokens == self.num_seqs

    def advance_(self) -> None:
        """Every sequence one token further, on the device: seq_lens,
        start_pos and positions + 1 (one kernel when they share step_view)."""
        v = self.step_view
        n, t = self.num_seqs, self.num_tokens
        if (v is not None and v.numel() == 2 * n + t and v.dtype == torch.int32
                and self.seq_lens.data_ptr() == v.data_ptr()
                and self.start_pos.data_ptr() == v.data_ptr() + 4 * n
                and self.positions.data_ptr() == v.data_ptr() + 8 * n):
            v.add_(1)
            return
        self.positions.add_(1)
        self.start_pos.add_(1)
        self.seq_lens.add_(1)


def _as_list(x):
    if isinstance(x, torch.Tensor):
        return x.tolist()
    return list(x)


def pack_batch_meta(block_tables, query_start_loc, positions, T: int, device,
                    block_size: int, check_append: bool = True) -> PagedBatchMeta:
    """Validate and pack one step's ragged metadata.

    Checks, with the reference's exception types and messages:
      - query_start_loc / positions lengths (fake_paged_attn.py:60-66, ValueError)
      - kv_len = positions[last] + 1 fits the table (fake_paged_attn.py:86-92, ValueError)
      - with check_append: the new tokens' slots fit the table and avoid
        reserved block 0 (kv_pool.py:41-42, :52-53, AssertionError)
    """
    tables = [_as_list(bt) for bt in block_tables]
    qsl = [int(x) for x in _as_list(query_start_loc)]
    pos = [int(x) for x in _as_list(positions)]
    n = len(tables)
    if len(qsl) != n + 1:
        raise ValueError("query_start_loc must have length num_seqs + 1")
    if qsl[0] != 0 or qsl[-1] != T:
        raise ValueError("query_start_loc must start at 0 and end at T")
    if len(pos) != T:
        raise ValueError(f"positions must have length T ({T})")

    max_blocks = max((len(bt) for bt in tables), default=0)
    seq_lens = np.zeros(n, dtype=np.int32)
    start_pos = np.zeros(n, dtype=np.int32)
    max_q_len = 0
    for i, bt in enumerate(tables):
        s0, s1 = qsl[i], qsl[i + 1]
        q_len = s1 - s0
        max_q_len = max(max_q_len, q_len)
        if q_len <= 0:
            continue
        kv_len = pos[s1 - 1] + 1
        cap = len(bt) * block_size
        if kv_len > cap:
            raise ValueError(f"seq {i}: kv_len {kv_len} exceeds {len(bt)} * blocksize ({cap})")
        seq_lens[i] = kv_len
        start = pos[s0]
        start_pos[i] = start
        if check_append:
            assert start + q_len <= cap, \
                f"block table too short: need {start + q_len} slots, table gives {cap}"
            first_blk, last_blk = start // block_size, (start + q_len - 1) // block_size
            if 0 in bt[first_blk:last_blk + 1]:
                raise AssertionError("slot mapping touches block 0, which is reserved")

    # one int32 host buffer -> one H2D copy; device views carved out of it
    # (seq_lens, start_pos, positions back to back: one add advances them)
    sizes = [n * max_blocks, n + 1, n, n, T]
    buf = np.zeros(sum(sizes), dtype=np.int32)
    off = 0
    if max_blocks:
        tab = buf[:n * max_blocks].reshape(n, max_blocks)
        for i, bt in enumerate(tables):
            tab[i, :len(bt)] = bt
    off += sizes[0]
    buf[off:off + n + 1] = qsl
    off += n + 1
    buf[off:off + n] = seq_lens
    off += n
    buf[off:off + n] = start_pos
    off += n
    buf[off:off + T] = pos
    host = torch.from_numpy(buf)
    if torch.device(device).type == "cuda":
        host = host.pin_memory()
    dev = host.to(device, non_blocking=True)
    views = torch.split(dev, sizes)
    step0 = sizes[0] + sizes[1]
    return PagedBatchMeta(
        block_tables=views[0].view(n, max_blocks),
        seq_lens=views[2],
        query_start_loc=views[1],
        start_pos=views[3],
        positions=views[4],
        step_view=dev[step0:step0 + 2 * n + T],
        num_seqs=n,
        num_tokens=T,
        max_blocks=max_blocks,
        max_q_len=max_q_len,
        max_kv_len=int(seq_lens.max()) if n else 0,
        block_size=block_size,
    )
