"""MQA_Paged — drop-in for the reference's serving/paged_mqa.py.

Multi-query attention whose K/V live in a KVPool. Same constructor
(config with d_model, num_heads, num_kv_heads, bias, dropout, max_seq_len;
`backend` accepted for compatibility), same submodules and parameter names
(q_proj, k_proj, v_proj, out, rope) so reference checkpoints load, and the
same two entry points:
  forward_paged(x [1, SQ, d_model], pool, layer_idx, block_table, start)
  forward_paged_batched(x [T, d_model], pool, layer_idx, positions,
                        query_start_loc, block_tables)
The step runs: the q/k/v projections and RoPE as one HIP kernel, the
slot-mapped K/V append and the paged attention as HIP kernels
(libpagedkv.so), then the output projection. The per-sequence slot-mapping loop of the reference
(paged_mqa.py:87-99) becomes one in-kernel slot computation from
device-resident block tables.
"""
from __future__ import annotations

import torch
import torch.nn as nn

from .fake_paged_attn import paged_attention_append_meta, paged_attention_meta
from . import fused_ops
from .fused_ops import FusedRows
from .layers import RoPE
from .paged_meta import PagedBatchMeta, pack_batch_meta


def _get_kv_pool(pool, layer_idx):
    """[num_blocks, block_size, Hkv, D] K and V tensors of one layer
    (reference: paged_mqa.py:22-43, including its alternative attribute names)."""
    if hasattr(pool, "kv"):
        return pool.kv[layer_idx, 0], pool.kv[layer_idx, 1]
    for k_name, v_name in (("k_buffer", "v_buffer"), ("k_buffers", "v_buffers"),
                           ("k_pool", "v_pool"), ("k_cache", "v_cache")):
        if hasattr(pool, k_name) and hasattr(pool, v_name):
            return getattr(pool, k_name)[layer_idx], getattr(pool, v_name)[layer_idx]
    raise AttributeError(
        f"KVPool layout not recognised: {type(pool).__name__} "
        f"has attrs {[a for a in dir(pool) if not a.startswith('_')]}")


class MQA_Paged(nn.Module):
    def __init__(self, config, backend="pytorch"):
        super().__init__()
        self.d_model = config.d_model
        self.num_heads = config.num_heads
        self.num_kv_heads = config.num_kv_heads
        self.bias = config.bias
        self.dropout = config.dropout
        self.backend = backend
        assert self.backend in ("cuda", "pytorch")
        assert self.d_model % self.num_heads == 0
        assert self.num_heads % self.num_kv_heads == 0

        self.headdim = self.d_model // self.num_heads
        self.num_groups = self.num_heads // self.num_kv_heads
        self.rotary_dim = self.headdim

        # construction order = reference MQA_Cached (models/mqa.py:123-126)
        self.q_proj = nn.Linear(self.d_model, self.num_heads * self.headdim, bias=self.bias)
        self.k_proj = nn.Linear(self.d_model, self.num_kv_heads * self.headdim, bias=self.bias)
        self.v_proj = nn.Linear(self.d_model, self.num_kv_heads * self.headdim, bias=self.bias)
        self.out = nn.Linear(self.d_model, self.d_model, bias=self.bias)
        self.rope = RoPE(self.rotary_dim, config.max_seq_len)
        self._qkv = FusedRows(self.q_proj, self.k_proj, self.v_proj)

    def forward(self, *args, **kwargs):
        raise NotImplementedError(
            "MQA_Paged runs through forward_paged / forward_paged_batched; the "
            "contiguous-cache forward of MQA_Cached is not part of this library")

    def forward_paged(self, x, pool, layer_idx, block_table, start):
        """Single sequence, SQ new tokens at positions start..start+SQ-1
        (reference: paged_mqa.py:48-62)."""
        B, SQ, _ = x.shape
        assert B == 1, "forward_paged is single-sequence only"
        out = self.forward_paged_batched(
            x.reshape(SQ, x.shape[-1]), pool, layer_idx,
            list(range(start, start + SQ)), [0, SQ], [list(block_table)])
        return out.view(B, SQ, x.shape[-1])

    def forward_paged_batched(self, x, pool, layer_idx, positions, query_start_loc,
                              block_tables):
        """Ragged batch of T tokens (reference: paged_mqa.py:64-113)."""
        T = x.shape[0]
        meta = pack_batch_meta(block_tables, query_start_loc, positions, T, x.device,
                               pool.block_size)
        return self.forward_meta(x, pool, layer_idx, meta)

    def forward_meta(self, x, pool, layer_idx, meta: PagedBatchMeta):
        """One layer of a step whose metadata is already on the device."""
        T, d_model = x.shape
        # q, k, v by one projection over the row-concatenated weights with
        # RoPE in its epilogue (contiguous rotated q, k and v)
        w, b = self._qkv.get()
        cos, sin = self.rope._tables_fp32()
        q, k, v = fused_ops.linear_rope_qkv(x, w, b, meta.positions, cos, sin, self.num_heads,
                                            self.num_kv_heads, self.headdim)

        # append + attention in one library call (fused on the decode kernels)
        out = paged_attention_append_meta(q, k, v, pool, layer_idx, meta)
        return fused_ops.linear(out.view(T, d_model), self.out.weight, self.out.bias)

    def forward_meta_residual_(self, x, norm, pool, layer_idx, meta: PagedBatchMeta):
        """x += forward_meta(norm(x), ...) in place, with the norm taken in
        the qkv projection's prologue and the residual add in the out
        projection's epilogue (the same rounded values as the separate
        norm, layer and add). Returns x."""
        T, d_model = x.shape
        w, b = self._qkv.get()
        cos, sin = self.rope._tables_fp32()
        q, k, v = fused_ops.linear_rope_qkv_rmsnorm(x, norm.weight, norm.eps, w, b,
                                                    meta.positions, cos, sin, self.num_heads,
                                                    self.num_kv_heads, self.headdim)
        out = paged_attention_append_meta(q, k, v, pool, layer_idx, meta)
        return fused_ops.linear_residual_(x, out.view(T, d_model), self.out.weight,
                                          self.out.bias)
