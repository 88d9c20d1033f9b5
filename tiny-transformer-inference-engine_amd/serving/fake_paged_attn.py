"""Paged varlen attention — drop-in for the reference's
serving/fake_paged_attn.py, backed by libpagedkv.so (HIP, gfx950).

Public API (same names, arguments and exceptions as the reference):
  paged_varlen_attention(q, k_pool, v_pool, block_tables, query_start_loc,
                         positions, num_heads, num_kv_heads, scale=None,
                         non_causal=False) -> [T, Hq, D]
  PagedVarlenAttention(num_heads, num_kv_heads, scale=None, non_causal=False)
  is_available()
plus the native-level entry the reference binds from its extension,
  paged_attn_fwd(Q, Kpool, Vpool, blocktable, seq_lens, queryloc, max_q_len,
                 scale=0.0, causal=True, return_lse=True) -> (O, Lse)
(kernels/pagedattn/extension.cpp:56-69), and a decode entry for
device-resident metadata, paged_mqa_decode(...), that needs no host sync.

Differences by design: f32 / f16 / bf16 are computed natively (the
reference casts Q and both whole pools to fp16 on every call,
fake_paged_attn.py:208-215); only the forward exists (inference), so calls
that would need a backward raise NotImplementedError.
"""
from __future__ import annotations

import math
from typing import List, Optional

import torch

from . import _native
from .paged_meta import PagedBatchMeta, pack_batch_meta

__all__ = [
    "paged_varlen_attention",
    "PagedVarlenAttention",
    "is_available",
    "paged_attn_fwd",
    "paged_attention_meta",
    "paged_mqa_decode",
]


def is_available() -> bool:
    """True if libpagedkv.so loads and a ROCm device exists
    (reference: fake_paged_attn.py:47-49)."""
    return _native.is_available()


def _check_no_grad(*ts: torch.Tensor) -> None:
    if torch.is_grad_enabled() and any(t.requires_grad for t in ts):
        raise NotImplementedError(
            "paged attention here is forward-only (inference); run it under "
            "torch.no_grad() or torch.inference_mode()")


def _launch(q, k_pool, v_pool, block_tables, seq_lens, queryloc, n_seq,
            max_q_len, max_kv_len, scale, causal, out, lse,
            part_tokens: int = 0):
    T, hq, d = q.shape
    nb, bs, hkv, _ = k_pool.shape
    max_blk = block_tables.shape[1] if block_tables.dim() == 2 else 0
    code = _native.kv_code(q.dtype, k_pool.dtype)
    L = _native.lib()
    ws_bytes = L.pkv_attention_workspace_bytes(
        n_seq, max_q_len, hq, hkv, d, max_blk, bs, max_kv_len, part_tokens, code)
    ws = _native.current_workspace().get(q.device, ws_bytes)
    rc = L.pkv_paged_attention(
        out.data_ptr(), _native.ptr(lse), q.data_ptr(), k_pool.data_ptr(),
        v_pool.data_ptr(), nb, bs, block_tables.data_ptr() if max_blk else None,
        max_blk, seq_lens.data_ptr(), _native.ptr(queryloc), n_seq, T, max_q_len,
        max_kv_len, hq, hkv, d, float(scale), int(bool(causal)), part_tokens,
        code, _native.ptr(ws), ws_bytes, None, _native.stream_ptr(q.device))
    _native.check(rc, "pkv_paged_attention")


def paged_attn_fwd(Q, Kpool, Vpool, blocktable, seq_lens, queryloc, max_q_len,
                   scale=0.0, causal=True, return_lse=True, max_kv_len=0):
    """Native forward with the reference extension's contract
    (kernels/pagedattn/pagedattn.cu:1052-1079): all tensors on the GPU and
    contiguous, int32 metadata, Q [T, Hq, D], pools [NB, BS, Hkv, D] of Q's
    dtype (f32, f16 or bf16). Returns (O, Lse) with Lse float32 [T, Hq]
    (empty when return_lse is False). Errors raise RuntimeError like the
    reference's TORCH_CHECKs (:872-894)."""
    ts = (Q, Kpool, Vpool, blocktable, seq_lens, queryloc)
    if not all(t.is_cuda for t in ts):
        raise RuntimeError("all tensors must be CUDA")
    if not (Q.dtype == Kpool.dtype == Vpool.dtype and Q.dtype in _native.DTYPE_CODES):
        raise RuntimeError("Q/Kpool/Vpool must share one dtype: float32, float16 or bfloat16")
    if not (blocktable.dtype == seq_lens.dtype == queryloc.dtype == torch.int32):
        raise RuntimeError("metadata must be int32")
    if not all(t.is_contiguous() for t in ts):
        raise RuntimeError("all tensors must be contiguous")
    if Q.dim() != 3:
        raise RuntimeError("Q must be [total_q_tokens, Hq, D]")
    if Kpool.dim() != 4 or Kpool.shape != Vpool.shape:
        raise RuntimeError("Kpool/Vpool must be [num_blocks, blocksize, Hkv, D] and equal shape")
    if Kpool.shape[3] != Q.shape[2]:
        raise RuntimeError("head dim mismatch")
    if Q.shape[1] % Kpool.shape[2] != 0:
        raise RuntimeError("Hq must be a multiple of Hkv")
    if Q.shape[2] % 8 != 0:
        raise RuntimeError("head dim must be a multiple of 8")
    bs = Kpool.shape[1]
    if bs <= 0 or bs & (bs - 1):
        raise RuntimeError("blocksize must be a power of two")
    if blocktable.dim() != 2 or blocktable.shape[0] != seq_lens.shape[0]:
        raise RuntimeError("blocktable must be [num_seqs, max_blocks_per_seq]")
    if queryloc.numel() != seq_lens.numel() + 1:
        raise RuntimeError("queryloc must be [num_seqs + 1]")
    O = torch.empty_like(Q)
    Lse = torch.empty((Q.shape[0], Q.shape[1]) if return_lse else (0,),
                      dtype=torch.float32, device=Q.device)
    n_seq = seq_lens.shape[0]
    if n_seq == 0 or max_q_len <= 0 or Q.shape[0] == 0:
        return O, Lse
    _launch(Q, Kpool, Vpool, blocktable, seq_lens, queryloc, n_seq, int(max_q_len),
            int(max_kv_len), scale if scale and scale > 0 else 0.0, causal, O,
            Lse if return_lse else None)
    return O, Lse


def _pack_metadata(block_tables, query_start_loc, positions, T, device, blocksize):
    """Reference-shaped packer (fake_paged_attn.py:52-100): returns
    (blocktable int32 [N, max_blk], seq_lens int32 [N], queryloc int32 [N+1],
    max_q_len). Lists are validated and packed on the host in one transfer;
    device tensors are packed on the device (one host sync for max_q_len)."""
    if isinstance(block_tables, torch.Tensor) and block_tables.is_cuda:
        qsl = torch.as_tensor(query_start_loc, device=device).to(torch.int32)
        pos = torch.as_tensor(positions, device=device)
        n = block_tables.shape[0]
        if qsl.numel() != n + 1:
            raise ValueError("query_start_loc must have length num_seqs + 1")
        if pos.numel() != T:
            raise ValueError(f"positions must have length T ({T})")
        q_len = qsl[1:] - qsl[:-1]
        last = (qsl[1:] - 1).clamp(min=0).long()
        seq_lens = torch.where(q_len > 0, pos[last].to(torch.int32) + 1,
                               torch.zeros_like(q_len)).to(torch.int32)
        max_q_len = int(q_len.max().item()) if n else 0
        return block_tables.to(torch.int32).contiguous(), seq_lens, qsl.contiguous(), max_q_len
    meta = pack_batch_meta(block_tables, query_start_loc, positions, T, device,
                           blocksize, check_append=False)
    return meta.block_tables, meta.seq_lens, meta.query_start_loc, meta.max_q_len


def paged_varlen_attention(
    q: torch.Tensor,                          # [T, Hq, D]
    k_pool: torch.Tensor,                     # [num_blocks, blocksize, Hkv, D]
    v_pool: torch.Tensor,                     # [num_blocks, blocksize, Hkv, D]
    block_tables: List[List[int]],
    query_start_loc: List[int],
    positions: List[int],
    num_heads: int,
    num_kv_heads: int,
    scale: Optional[float] = None,
    non_causal: bool = False,
) -> torch.Tensor:
    """Causal paged self-attention over a ragged batch
    (reference: fake_paged_attn.py:150-228). Query i of a sequence with
    kv_len keys (kv_len = its last position + 1) sees keys
    j <= kv_len - q_len + i. Output has q's dtype."""
    if not is_available():
        raise RuntimeError(
            "libpagedkv.so or a ROCm device is not available; build the "
            "library and run on an MI355X")
    if q.dim() != 3:
        raise ValueError(f"q must be [T, Hq, D], got {tuple(q.shape)}")
    T, Hq, D = q.shape
    if Hq != num_heads:
        raise ValueError(f"q H={Hq} != num_heads={num_heads}")
    if k_pool.shape[2] != num_kv_heads:
        raise ValueError(f"pool Hkv={k_pool.shape[2]} != num_kv_heads={num_kv_heads}")
    if Hq % num_kv_heads != 0:
        raise ValueError(f"Hq ({Hq}) must be a multiple of Hkv ({num_kv_heads})")
    if D % 8 != 0:
        raise ValueError(f"head_dim {D} must be a multiple of 8")
    blocksize = k_pool.shape[1]
    if blocksize & (blocksize - 1) != 0 or blocksize <= 0:
        raise ValueError(f"blocksize {blocksize} must be a power of two")
    if non_causal:
        # the reference raises here too (no bidirectional backward); the
        # forward itself is available through paged_attn_fwd(causal=False)
        raise NotImplementedError(
            "non_causal gradient path is not implemented; "
            "use paged_attn_fwd(..., causal=False) for a non-causal forward.")
    if q.device.type != "cuda":
        raise RuntimeError("paged_varlen_attention requires a CUDA tensor for q")
    _check_no_grad(q, k_pool, v_pool)

    device = q.device
    blocktable, seq_lens, queryloc, max_q_len = _pack_metadata(
        block_tables, query_start_loc, positions, T, device, blocksize)
    orig_dtype = q.dtype
    qk = q if q.dtype == k_pool.dtype else q.to(k_pool.dtype)
    kp = k_pool.contiguous()
    vp = v_pool if v_pool.dtype == k_pool.dtype else v_pool.to(k_pool.dtype)
    O, _ = paged_attn_fwd(qk.contiguous(), kp, vp.contiguous(), blocktable,
                          seq_lens, queryloc, max_q_len,
                          scale if scale is not None else 0.0, True, False)
    return O if O.dtype == orig_dtype else O.to(orig_dtype)


def paged_attention_meta(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                         meta: PagedBatchMeta, scale: Optional[float] = None,
                         causal: bool = True, out: Optional[torch.Tensor] = None,
                         lse: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Attention for a step whose metadata was packed once (pack_batch_meta):
    no host work or synchronisation per call."""
    _native.require_device(q, k_pool, v_pool, what="paged_attention_meta")
    if out is None:
        out = torch.empty_like(q)
    queryloc = None if meta.is_decode else meta.query_start_loc
    _launch(q, k_pool, v_pool, meta.block_tables, meta.seq_lens, queryloc,
            meta.num_seqs, meta.max_q_len, meta.max_kv_len,
            scale if scale is not None and scale > 0 else 0.0, causal, out, lse)
    return out


def paged_attention_append_meta(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, pool,
                                layer: int, meta: PagedBatchMeta,
                                scale: Optional[float] = None, causal: bool = True,
                                out: Optional[torch.Tensor] = None,
                                lse: Optional[torch.Tensor] = None) -> torch.Tensor:
    """pool.write_from_table(layer, k, v, meta) followed by
    paged_attention_meta(q, ..., meta) in one library call
    (pkv_paged_attention_append): on the MFMA decode kernels the append is
    fused into the attention launch. Same pool contents, outputs and errors
    as the two calls (serving/paged_mqa.py:98-110)."""
    pool.check_rows(k, v, meta)
    _native.require_device(q, k, v, pool.kv, what="paged_attention_append_meta")
    if out is None:
        out = torch.empty_like(q)
    k = k.contiguous()
    v = v.contiguous()
    T, hq, d = q.shape
    kp, vp = pool.flat_k[layer], pool.flat_v[layer]
    if k.dtype != q.dtype:
        raise TypeError(f"new K/V rows ({k.dtype}) must have the queries' dtype ({q.dtype})")
    code = _native.kv_code(q.dtype, pool.dtype)
    L = _native.lib()
    max_blk = meta.block_tables.shape[1] if meta.block_tables.dim() == 2 else 0
    ws_bytes = L.pkv_attention_workspace_bytes(
        meta.num_seqs, meta.max_q_len, hq, pool.num_kv_heads, d, max_blk, pool.block_size,
        meta.max_kv_len, 0, code)
    ws = _native.current_workspace().get(q.device, ws_bytes)
    status = pool._status()
    rc = L.pkv_paged_attention_append(
        out.data_ptr(), _native.ptr(lse), q.data_ptr(), kp.data_ptr(), vp.data_ptr(),
        pool.num_blocks, pool.block_size, meta.block_tables.data_ptr() if max_blk else None,
        max_blk, meta.seq_lens.data_ptr(), meta.query_start_loc.data_ptr(), meta.num_seqs, T,
        meta.max_q_len, meta.max_kv_len, hq, pool.num_kv_heads, d,
        float(scale if scale is not None and scale > 0 else 0.0), int(bool(causal)), 0, code,
        k.data_ptr(), v.data_ptr(), meta.start_pos.data_ptr(), _native.ptr(ws), ws_bytes,
        _native.ptr(status), _native.stream_ptr(q.device))
    _native.check(rc, "pkv_paged_attention_append")
    pool._raise_status(status, "paged_attention_append_meta")
    return out


def paged_mqa_decode(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                     block_tables: torch.Tensor, seq_lens: torch.Tensor,
                     scale: Optional[float] = None, max_kv_len: int = 0,
                     out: Optional[torch.Tensor] = None,
                     lse: Optional[torch.Tensor] = None,
                     part_tokens: int = 0,
                     query_start_loc: Optional[torch.Tensor] = None) -> torch.Tensor:
    """One decode query per sequence (q [N, Hq, D]) against device-resident
    int32 block_tables [N, max_blk] and seq_lens [N]. `max_kv_len` (0: table
    capacity) bounds the context and sizes the split-K grid. With
    `query_start_loc` (int32 [n_seq + 1], every range 0 or 1 token long) q
    holds only the sequences that have a query this step. `part_tokens`:
    0 automatic, > 0 the split-K partition length, _native.PART_PERSISTENT
    the persistent kernel."""
    _native.require_device(q, k_pool, v_pool, block_tables, seq_lens, what="paged_mqa_decode")
    if out is None:
        out = torch.empty_like(q)
    n_seq = q.shape[0] if query_start_loc is None else block_tables.shape[0]
    _launch(q, k_pool, v_pool, block_tables, seq_lens, query_start_loc, n_seq, 1,
            int(max_kv_len), scale if scale is not None and scale > 0 else 0.0,
            True, out, lse, part_tokens)
    return out


class PagedVarlenAttention(torch.nn.Module):
    """Module form of paged_varlen_attention (reference: fake_paged_attn.py:231-258)."""

    def __init__(self, num_heads: int, num_kv_heads: int,
                 scale: Optional[float] = None, non_causal: bool = False):
        super().__init__()
        self.num_heads = num_heads
        self.num_kv_heads = num_kv_heads
        self.scale = scale
        self.non_causal = non_causal

    def forward(self, q, k_pool, v_pool, block_tables, query_start_loc, positions):
        return paged_varlen_attention(
            q, k_pool, v_pool,
            block_tables, query_start_loc, positions,
            num_heads=self.num_heads,
            num_kv_heads=self.num_kv_heads,
            scale=self.scale,
            non_causal=self.non_causal,
        )
