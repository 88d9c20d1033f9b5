"""numpy restatement of the reference's paged KV path — TEST INFRASTRUCTURE ONLY.

Used by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as
the checker; never by the product. Each function cites the reference
file:line it restates (paths relative to the reference repository).
"""
from __future__ import annotations

import math
from typing import Sequence

import numpy as np


def make_slot_mapping(start: int, n: int, block_table: Sequence[int],
                      block_size: int) -> np.ndarray:
    """serving/kv_pool.py:40-55: slot[p] = bt[p // bs] * bs + p % bs for
    p in [start, start + n); asserts the table is long enough (:41-42) and
    that no slot falls in reserved block 0 (:52-53)."""
    if start + n > len(block_table) * block_size:
        raise AssertionError(
            f"block table too short: need {start + n} slots, table gives "
            f"{len(block_table) * block_size}")
    p = np.arange(start, start + n, dtype=np.int64)
    bt = np.asarray(block_table, dtype=np.int64).reshape(-1)
    slot = bt[p // block_size] * block_size + p % block_size
    if np.any(slot < block_size):
        raise AssertionError(
            f"slot mapping touches block 0, which is reserved: {slot[slot < block_size]}")
    return slot


def append(flat_k: np.ndarray, flat_v: np.ndarray, slot_mapping: np.ndarray,
           k: np.ndarray, v: np.ndarray) -> None:
    """serving/kv_pool.py:57-70: `flat_k[l][slot] = k; flat_v[l][slot] = v`
    (index_put with int64 indices; negative indices wrap, as in Python).
    flat_* are [num_slots, hkv, d] views of one layer; mutated in place."""
    slots = np.asarray(slot_mapping, dtype=np.int64)
    n = flat_k.shape[0]
    if np.any((slots < -n) | (slots >= n)):
        raise IndexError("slot out of range")
    flat_k[slots] = k
    flat_v[slots] = v


def append_from_table(flat_k, flat_v, k, v, block_tables, query_start_loc,
                      start_pos, block_size) -> None:
    """serving/paged_mqa.py:87-99: per sequence i with q tokens
    qsl[i]..qsl[i+1], make_slot_mapping(start_pos[i], n_i, table_i), then one
    write of the concatenated slots."""
    slots = []
    for i, bt in enumerate(block_tables):
        n = int(query_start_loc[i + 1] - query_start_loc[i])
        if n == 0:
            continue
        slots.append(make_slot_mapping(int(start_pos[i]), n, bt, block_size))
    if slots:
        append(flat_k, flat_v, np.concatenate(slots), k, v)


def gather(k_layer: np.ndarray, v_layer: np.ndarray, block_table: Sequence[int],
           seq_len: int):
    """serving/kv_pool.py:72-82: kv[l, 0][bt].reshape(-1, hkv, d)[:seq_len].
    k_layer/v_layer are [num_blocks, bs, hkv, d]."""
    bs = k_layer.shape[1]
    if seq_len > len(block_table) * bs:
        raise AssertionError(
            f"seq_len={seq_len} exceeds capacity of block_table ({len(block_table) * bs})")
    bt = np.asarray(block_table, dtype=np.int64)
    hkv, d = k_layer.shape[2], k_layer.shape[3]
    k = k_layer[bt].reshape(-1, hkv, d)[:seq_len]
    v = v_layer[bt].reshape(-1, hkv, d)[:seq_len]
    return k, v


def pack_metadata(block_tables, query_start_loc, positions, T: int,
                  block_size: int):
    """serving/fake_paged_attn.py:52-100: ragged lists -> blocktable int32
    [N, max_blk] zero-padded (:70-76), seq_lens[i] = positions[last_i] + 1
    (:80-92, ValueError when it exceeds the table capacity), queryloc int32
    (:94), max_q_len (:96-99). ValueErrors of :60-66 kept verbatim."""
    num_seqs = len(block_tables)
    if len(query_start_loc) != num_seqs + 1:
        raise ValueError("query_start_loc must have length num_seqs + 1")
    if query_start_loc[0] != 0 or query_start_loc[-1] != T:
        raise ValueError("query_start_loc must start at 0 and end at T")
    if len(positions) != T:
        raise ValueError(f"positions must have length T ({T})")
    max_blocks = max((len(bt) for bt in block_tables), default=0)
    table = np.zeros((num_seqs, max_blocks), dtype=np.int32)
    for i, bt in enumerate(block_tables):
        table[i, :len(bt)] = np.asarray(bt, dtype=np.int32)
    seq_lens = np.zeros(num_seqs, dtype=np.int32)
    for i in range(num_seqs):
        s0, s1 = int(query_start_loc[i]), int(query_start_loc[i + 1])
        if s1 > s0:
            seq_lens[i] = int(positions[s1 - 1]) + 1
            cap = len(block_tables[i]) * block_size
            if seq_lens[i] > cap:
                raise ValueError(
                    f"seq {i}: kv_len {seq_lens[i]} exceeds "
                    f"{len(block_tables[i])} * blocksize ({cap})")
    qloc = np.asarray(query_start_loc, dtype=np.int32)
    max_q_len = max((int(query_start_loc[i + 1]) - int(query_start_loc[i])
                     for i in range(num_seqs)), default=0)
    return table, seq_lens, qloc, int(max_q_len)


def paged_attention(q, k_pool, v_pool, block_table, seq_lens, query_start_loc,
                    scale=None, causal=True, dtype=np.float64, _mutation=None):
    """Paged attention forward, as pagedattn.forward computes it
    (kernels/pagedattn/pagedattn.cu), in `dtype` arithmetic:

      kv_len = min(seq_lens[s], max_blk * bs)                (:187-189)
      ctx    = max(kv_len - q_len, 0) if causal else 0        (:196-200)
      query i of s sees key j iff j < kv_len and j <= ctx+i   (:315-329)
      kv head of query head h = h // (hq // hkv)              (:180)
      scale <= 0 or None -> 1/sqrt(d)                         (:930-931)
      O = softmax(scale * q K^T) V; lse = m + ln(l); no
      visible key -> O = 0, lse = +inf                        (:418-446)

    Keys are read through the block table exactly as asyncLOAD_PAGED_TILE
    does (:47-53): page = j // bs, phys = table[page], slot = phys*bs + j%bs.
    q [T, hq, d]; pools [num_blocks, bs, hkv, d]; block_table [N, max_blk];
    seq_lens [N]; query_start_loc [N+1] or None (one query per sequence).
    Returns (out [T, hq, d], lse [T, hq]) in `dtype`.

    `_mutation` plants a known mistake so tests can show their checks catch
    it: "topleft" (causal mask aligned top-left, ctx = 0), "noscale"
    (scale 1), "kvhead_mod" (kv head = h % hkv), "noclamp" (kv_len not
    clamped to the table capacity), "nomax" (no max subtraction, so large
    scores overflow). Never set outside tests.
    """
    q = np.asarray(q)
    T, hq, d = q.shape
    nb, bs, hkv, _ = k_pool.shape
    table = np.asarray(block_table, dtype=np.int64)
    n_seq = table.shape[0]
    max_blk = table.shape[1] if table.ndim == 2 else 0
    qloc = (np.arange(n_seq + 1) if query_start_loc is None
            else np.asarray(query_start_loc, dtype=np.int64))
    if scale is None or scale <= 0:
        scale = 1.0 / math.sqrt(d)
    if _mutation == "noscale":
        scale = 1.0
    g = hq // hkv
    out = np.zeros((T, hq, d), dtype=dtype)
    lse = np.full((T, hq), np.inf, dtype=dtype)
    kf = np.asarray(k_pool).astype(dtype)
    vf = np.asarray(v_pool).astype(dtype)
    qf = q.astype(dtype)
    sc = dtype(scale)
    for s in range(n_seq):
        q0, q1 = int(qloc[s]), int(qloc[s + 1])
        q_len = q1 - q0
        if q_len <= 0:
            continue
        kv_len = max(0, min(int(seq_lens[s]), max_blk * bs))
        if _mutation == "noclamp":
            kv_len = int(seq_lens[s])
        ctx = max(kv_len - q_len, 0) if causal else 0
        if _mutation == "topleft":
            ctx = 0
        j = np.arange(kv_len)
        if kv_len:
            phys = table[s, np.minimum(j // bs, max_blk - 1)]
            slots = phys * bs + j % bs
            K = kf.reshape(nb * bs, hkv, d)[slots]  # [kv_len, hkv, d]
            V = vf.reshape(nb * bs, hkv, d)[slots]
        for i in range(q_len):
            vis = kv_len if not causal else min(kv_len, ctx + i + 1)
            if vis <= 0:
                continue
            for h in range(hq):
                kvh = h % hkv if _mutation == "kvhead_mod" else h // g
                sco = (K[:vis, kvh, :] @ qf[q0 + i, h]) * sc
                m = dtype(0) if _mutation == "nomax" else sco.max()
                p = np.exp(sco - m)
                l = p.sum()
                out[q0 + i, h] = (p @ V[:vis, kvh, :]) / l
                lse[q0 + i, h] = m + np.log(l)
    return out, lse


def e4m3_codes(x) -> np.ndarray:
    """fp8 e4m3 bytes (OCP, torch.float8_e4m3fn) of float32 values, as the
    reference's KVPool.write stores rows into a pool whose CacheConfig.kv_dtype
    is float8_e4m3fn (models/model_config.py:49, serving/kv_pool.py:57-70:
    index_put converts). Format: sign, 4 exponent bits (bias 7), 3 mantissa
    bits; no infinities; S.1111.111 is NaN; largest finite 1.75 * 2^8 = 448;
    below 2^-6 the values are the multiples of 2^-9. Rounding to nearest,
    ties to even; magnitudes above 464 (those that round past 448; 464
    itself is a tie and goes to 448), infinities and NaN give NaN (0x7F with
    the sign)."""
    x = np.asarray(x, dtype=np.float32)
    sign = (np.signbit(x).astype(np.uint8) << 7)
    with np.errstate(invalid="ignore"):  # signalling NaN inputs
        a = np.abs(x.astype(np.float64))
    out = np.zeros(x.shape, dtype=np.uint8)
    nan = ~np.isfinite(a)
    a = np.where(nan, 0.0, a)
    sub = a < 2.0 ** -6
    # subnormal range: m * 2^-9, m = round-half-even(a * 512) (m = 8 is 2^-6,
    # whose code 0x08 is the first normal one)
    m = np.rint(np.where(sub, a, 0.0) * 512.0)  # numpy rounds halves to even
    out = np.where(sub, m.astype(np.int64), 0).astype(np.uint8)
    # normal range: exponent e (2^e <= a < 2^(e+1)), 3-bit mantissa rounded
    e = np.floor(np.log2(np.where(sub, 1.0, a)))
    q = np.rint(np.where(sub, 1.0, a) / 2.0 ** e * 8.0)  # 8..16, halves to even
    e = np.where(q >= 16, e + 1, e)
    q = np.where(q >= 16, 8, q)
    code = ((e + 7).astype(np.int64) << 3) | (q.astype(np.int64) - 8)
    big = (~sub) & ((code > 0x7E) | (e + 7 > 15))
    out = np.where(sub, out, np.clip(code, 0, 0x7F).astype(np.uint8))
    out = np.where(big | nan, 0x7F, out).astype(np.uint8)
    return out | sign


def e4m3_values(codes) -> np.ndarray:
    """float64 values of fp8 e4m3 bytes (the exact widening the attention
    kernels read an fp8 pool with)."""
    c = np.asarray(codes, dtype=np.uint8).astype(np.int64)
    sign = np.where(c & 0x80, -1.0, 1.0)
    e = (c >> 3) & 15
    m = c & 7
    val = np.where(e == 0, m * 2.0 ** -9, (1.0 + m / 8.0) * 2.0 ** (e - 7))
    val = np.where((e == 15) & (m == 7), np.nan, val)
    return sign * val


def decode_attention_bytes(seq_lens, hq, hkv, d, elem_bytes, block_size):
    """Algorithmic HBM bytes of one paged decode attention call (one query per
    sequence): K and V rows of every visible token, Q and O, block-table
    entries actually used (4 B each) and seq_lens (4 B each)."""
    kv = int(np.sum(seq_lens))
    n = len(seq_lens)
    blocks = int(np.sum([(int(x) + block_size - 1) // block_size for x in seq_lens]))
    return kv * hkv * d * 2 * elem_bytes + 2 * n * hq * d * elem_bytes + 4 * blocks + 4 * n
