"""Paged KV block pool — drop-in for the reference's serving/kv_pool.py.

Same constructor, attributes (`kv`, `flat_k`, `flat_v`, `device`, ...), and
methods (`make_slot_mapping`, `write`, `gather`, `from_config`) with the same
assertions; `write` and `gather` run as HIP kernels (libpagedkv.so) instead of
torch index_put / index_select. `write_from_table` is the batched append used
by the paged layer: slots are computed in-kernel from device-resident block
tables, so a step needs no per-sequence host work.

Pool layout (unchanged, so tests that index `pool.kv` keep working):
  kv[num_layers, 2, num_blocks, block_size, num_kv_heads, head_dim]
K and V of one layer are num_blocks*block_size*hkv*d elements apart; a token
slot is one contiguous row of hkv*d elements.
"""
from __future__ import annotations

import os

import numpy as np
import torch

from . import _native


def _debug_default() -> bool:
    return os.environ.get("PKV_DEBUG", "0") not in ("", "0")


class KVPool:
    """Block pool of K/V rows (reference: serving/kv_pool.py:3-82)."""

    def __init__(self, num_layers, block_size, num_blocks, num_kv_heads, head_dim, dtype, device):
        self.num_layers = num_layers
        self.block_size = block_size
        self.num_blocks = num_blocks
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.dtype = dtype

        # zero-initialised like the reference (kv_pool.py:12-16): blocks that
        # are never written, block 0 in particular, read as zeros
        self.kv = torch.zeros(
            (num_layers, 2, num_blocks, block_size, num_kv_heads, head_dim),
            dtype=dtype,
            device=device,
        )
        self.device = self.kv.device
        self._shape_check()

        self.flat_k = [self.kv[l, 0].view(-1, num_kv_heads, head_dim) for l in range(num_layers)]
        self.flat_v = [self.kv[l, 1].view(-1, num_kv_heads, head_dim) for l in range(num_layers)]
        self.debug = _debug_default()

    @classmethod
    def from_config(cls, cfg, device):
        """kv_pool.py:23-33: flat attributes num_layers, block_size,
        num_gpu_blocks, num_kv_heads, head_dim, kv_dtype."""
        return cls(
            num_layers=cfg.num_layers,
            block_size=cfg.block_size,
            num_blocks=cfg.num_gpu_blocks,
            num_kv_heads=cfg.num_kv_heads,
            head_dim=cfg.head_dim,
            dtype=cfg.kv_dtype,
            device=device,
        )

    @classmethod
    def from_engine_config(cls, ecfg, device):
        """A pool for an EngineConfig: the model's layers and heads, the
        cache's block size and block count, kv_dtype (fp8 with
        CacheConfig.kv_dtype = torch.float8_e4m3fn)."""
        m = ecfg.model
        return cls(m.num_layers, ecfg.cache.block_size, ecfg.num_blocks, m.num_kv_heads,
                   m.head_dim, ecfg.kv_dtype, device)

    def _shape_check(self):
        expected = (self.num_layers, 2, self.num_blocks, self.block_size,
                    self.num_kv_heads, self.head_dim)
        assert self.kv.shape == expected, f"shape mismatch: {self.kv.shape} vs {expected}"

    @property
    def num_slots(self) -> int:
        return self.num_blocks * self.block_size

    # ------------------------------------------------------------------
    # slot mapping (host integer work, one H2D copy)
    # ------------------------------------------------------------------
    def make_slot_mapping(self, start: int, n: int, block_table: list[int]) -> torch.Tensor:
        """slot[p] = table[p // bs] * bs + p % bs for p in [start, start+n)
        (kv_pool.py:40-55), with the reference's two assertions."""
        assert start + n <= len(block_table) * self.block_size, \
            f"block table too short: need {start+n} slots, table gives {len(block_table)*self.block_size}"
        p = np.arange(start, start + n, dtype=np.int64)
        bt = np.asarray(list(block_table), dtype=np.int64)
        slot = bt[p // self.block_size] * self.block_size + p % self.block_size
        assert np.all(slot >= self.block_size), \
            f"slot mapping touches block 0, which is reserved: {slot[slot < self.block_size]}"
        # the reference's index_put in write() raises on a slot past the
        # pool; write() here skips such a slot on the device (and raises only
        # under debug, after a synchronisation), so catch it on the host
        # where the mapping is built
        if slot.size and int(slot.max()) >= self.num_slots:
            raise IndexError(
                f"slot {int(slot.max())} out of range for a pool of {self.num_slots} slots")
        return torch.from_numpy(slot).to(self.device)

    # ------------------------------------------------------------------
    # append
    # ------------------------------------------------------------------
    def _status(self):
        return torch.zeros(1, dtype=torch.int32, device=self.device) if self.debug else None

    def _raise_status(self, status, what):
        if status is None:
            return
        bits = int(status.item())
        if bits & _native.PKV_STATUS_BAD_SLOT:
            raise IndexError(f"{what}: slot index out of range for a pool of {self.num_slots} slots")
        if bits & _native.PKV_STATUS_SHORT_TABLE:
            raise AssertionError(f"{what}: block table too short for the written positions")
        if bits & _native.PKV_STATUS_BAD_BLOCK:
            raise AssertionError(f"{what}: block table entry is block 0 or outside the pool")

    def write(self, layer: int, slot_mapping: torch.Tensor, k: torch.Tensor, v: torch.Tensor):
        """flat_k[layer][slot_mapping] = k; flat_v[layer][slot_mapping] = v
        (kv_pool.py:57-70), as one HIP scatter launch for K and V."""
        assert slot_mapping.dtype == torch.long
        assert slot_mapping.device == self.device, f"{slot_mapping.device} vs {self.device}"

        assert k.shape == v.shape, f"k/v shape mismatch: {k.shape} vs {v.shape}"
        assert k.shape[0] == slot_mapping.numel(), \
            f"k has {k.shape[0]} rows but slot_mapping has {slot_mapping.numel()} slots"
        assert k.shape[1:] == (self.num_kv_heads, self.head_dim), \
            f"k trailing dims {k.shape[1:]} != expected {(self.num_kv_heads, self.head_dim)}"
        self._check_row_dtype(k, v)

        _native.require_device(self.kv, k, v, slot_mapping, what="KVPool.write")
        if k.device != self.device or v.device != self.device:
            raise RuntimeError(f"k/v on {k.device}/{v.device}, pool on {self.device}")
        k = k.contiguous()
        v = v.contiguous()
        slots = slot_mapping.contiguous()
        status = self._status()
        rc = _native.lib().pkv_append(
            self.flat_k[layer].data_ptr(), self.flat_v[layer].data_ptr(), self.num_slots,
            k.data_ptr(), v.data_ptr(), slots.data_ptr(), k.shape[0],
            self.num_kv_heads * self.head_dim, _native.kv_code(k.dtype, self.dtype),
            _native.ptr(status), _native.stream_ptr(self.device))
        _native.check(rc, "pkv_append")
        self._raise_status(status, "KVPool.write")

    def _check_row_dtype(self, k: torch.Tensor, v: torch.Tensor) -> None:
        """Rows of the pool's dtype; an fp8 pool (kv_dtype float8_e4m3fn)
        takes float32/float16/bfloat16 rows and rounds them on the way in,
        as the reference's index_put into a float8 pool does."""
        if self.dtype == _native.FP8_KV_DTYPE:
            assert k.dtype == v.dtype and k.dtype in _native.DTYPE_CODES, \
                f"k/v dtype {k.dtype}/{v.dtype}: an fp8 pool takes float32, float16 or bfloat16 rows"
        else:
            assert k.dtype == self.dtype, f"k dtype {k.dtype} != pool dtype {self.dtype}"
            assert v.dtype == self.dtype, f"v dtype {v.dtype} != pool dtype {self.dtype}"

    def check_rows(self, k: torch.Tensor, v: torch.Tensor, meta) -> None:
        """The checks of KVPool.write (kv_pool.py:58-67) for a step's rows."""
        assert k.shape == v.shape, f"k/v shape mismatch: {k.shape} vs {v.shape}"
        assert k.shape[1:] == (self.num_kv_heads, self.head_dim), \
            f"k trailing dims {k.shape[1:]} != expected {(self.num_kv_heads, self.head_dim)}"
        self._check_row_dtype(k, v)
        assert k.shape[0] == meta.num_tokens, \
            f"k has {k.shape[0]} rows but the batch has {meta.num_tokens} tokens"

    def write_from_table(self, layer: int, k: torch.Tensor, v: torch.Tensor, meta) -> None:
        """Append the step's new K/V rows of every sequence with slots computed
        in-kernel from `meta` (a PagedBatchMeta): equivalent to
        make_slot_mapping per sequence + one write (serving/paged_mqa.py:87-99)."""
        self.check_rows(k, v, meta)
        _native.require_device(self.kv, k, v, what="KVPool.write_from_table")
        k = k.contiguous()
        v = v.contiguous()
        status = self._status()
        rc = _native.lib().pkv_append_from_table(
            self.flat_k[layer].data_ptr(), self.flat_v[layer].data_ptr(), self.num_blocks,
            self.block_size, k.data_ptr(), v.data_ptr(), meta.block_tables.data_ptr(),
            meta.max_blocks, meta.query_start_loc.data_ptr(), meta.start_pos.data_ptr(),
            meta.num_seqs, k.shape[0], self.num_kv_heads * self.head_dim,
            _native.kv_code(k.dtype, self.dtype), _native.ptr(status),
            _native.stream_ptr(self.device))
        _native.check(rc, "pkv_append_from_table")
        self._raise_status(status, "KVPool.write_from_table")

    # ------------------------------------------------------------------
    # gather
    # ------------------------------------------------------------------
    def _gather_code(self) -> int:
        if self.dtype == _native.FP8_KV_DTYPE:
            return _native.DTYPE_CODES[torch.bfloat16] | _native.PKV_KV_FP8  # byte copy
        return _native.dtype_code(self.dtype)

    def gather(self, layer: int, block_table: list[int], seq_len: int):
        """Dense copy of one sequence's first seq_len rows (kv_pool.py:72-82)."""
        assert seq_len <= len(block_table) * self.block_size, \
            f"seq_len={seq_len} exceeds capacity of block_table ({len(block_table)*self.block_size})"
        _native.require_device(self.kv, what="KVPool.gather")
        bt = torch.as_tensor(list(block_table), dtype=torch.int32).to(self.device)
        k = torch.empty((seq_len, self.num_kv_heads, self.head_dim), dtype=self.dtype, device=self.device)
        v = torch.empty_like(k)
        status = self._status()
        rc = _native.lib().pkv_gather(
            k.data_ptr(), v.data_ptr(), self.kv[layer, 0].data_ptr(), self.kv[layer, 1].data_ptr(),
            self.num_blocks, self.block_size, bt.data_ptr(), bt.numel(), seq_len,
            self.num_kv_heads * self.head_dim, self._gather_code(),
            _native.ptr(status), _native.stream_ptr(self.device))
        _native.check(rc, "pkv_gather")
        self._raise_status(status, "KVPool.gather")
        return k, v
