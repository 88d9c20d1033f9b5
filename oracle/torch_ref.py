"""The reference's PyTorch paged path, on the CPU — TEST INFRASTRUCTURE ONLY.

Used by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as
the checker / CPU baseline; never by the product.

  gather_kv, sdpa_one, paged_attention_sdpa
      the "gather + SDPA" reference of tests/test.py:138-178: per sequence,
      index the pool through the block table, then
      F.scaled_dot_product_attention with a bottom-right causal mask
      (query i of q_len sees key j <= kv_len - q_len + i).
  append_index_put
      KVPool.write as the reference runs it: flat[slot] = rows
      (serving/kv_pool.py:57-70).
  RefModel / generate_batched_ref
      fp32 restatement of the paged model's arithmetic
      (serving/paged_model.py:50-67, serving/paged_mqa.py:64-113,
      models/rope.py:14-35, models/rmsnorm.py:13-17 CPU branch,
      models/mlp.py:30 CPU branch) with a contiguous per-sequence KV cache,
      and greedy batched generation (serving/generation.py:112-148).
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F


def causal_mask(q_len: int, kv_len: int) -> torch.Tensor:
    """[q_len, kv_len] bool, True = visible (tests/test.py:138-142)."""
    pos = torch.arange(kv_len - q_len, kv_len).unsqueeze(1)
    j = torch.arange(kv_len).unsqueeze(0)
    return j <= pos


def gather_kv(k_pool, v_pool, table_row, kv_len):
    """Dense [kv_len, Hkv, D] K/V of one sequence (tests/test.py:145-152)."""
    bs, hkv, d = k_pool.shape[1], k_pool.shape[2], k_pool.shape[3]
    nb = math.ceil(kv_len / bs)
    ids = torch.as_tensor(table_row[:nb], dtype=torch.long)
    k = k_pool[ids].reshape(nb * bs, hkv, d)[:kv_len]
    v = v_pool[ids].reshape(nb * bs, hkv, d)[:kv_len]
    return k, v


def sdpa_one(q, k, v, causal=True, scale=None):
    """q [Lq, H, D], k/v [Lkv, Hkv, D] -> [Lq, H, D] (tests/test.py:155-165)."""
    h, hkv = q.shape[1], k.shape[1]
    g = h // hkv
    qh = q.permute(1, 0, 2).unsqueeze(0)
    kh = k.permute(1, 0, 2).repeat_interleave(g, dim=0).unsqueeze(0).contiguous()
    vh = v.permute(1, 0, 2).repeat_interleave(g, dim=0).unsqueeze(0).contiguous()
    mask = causal_mask(q.shape[0], k.shape[0]) if causal else None
    o = F.scaled_dot_product_attention(qh, kh, vh, attn_mask=mask, scale=scale)
    return o.squeeze(0).permute(1, 0, 2).contiguous()


def paged_attention_sdpa(q, k_pool, v_pool, block_tables, seq_lens, query_start_loc=None,
                         causal=True, scale=None, dtype=None):
    """Whole ragged batch through gather + SDPA (tests/test.py:168-178) on the
    CPU, in `dtype` (default: q's dtype). Sequences whose q_len exceeds
    kv_len, or with kv_len 0, are outside this reference's domain."""
    q, k_pool, v_pool = q.cpu(), k_pool.cpu(), v_pool.cpu()
    if dtype is not None:
        q, k_pool, v_pool = q.to(dtype), k_pool.to(dtype), v_pool.to(dtype)
    tables = block_tables.tolist() if isinstance(block_tables, torch.Tensor) else block_tables
    lens = [int(x) for x in (seq_lens.tolist() if isinstance(seq_lens, torch.Tensor) else seq_lens)]
    n = len(lens)
    qsl = (list(range(n + 1)) if query_start_loc is None else
           [int(x) for x in (query_start_loc.tolist() if isinstance(query_start_loc, torch.Tensor)
                             else query_start_loc)])
    outs = []
    for s in range(n):
        q0, q1 = qsl[s], qsl[s + 1]
        if q1 == q0:
            continue
        k, v = gather_kv(k_pool, v_pool, tables[s], lens[s])
        outs.append(sdpa_one(q[q0:q1], k, v, causal, scale))
    return torch.cat(outs) if outs else q[:0].clone()


def append_index_put(flat_k, flat_v, slot_mapping, k, v):
    """flat_k[slot] = k; flat_v[slot] = v, in place (serving/kv_pool.py:69-70)."""
    flat_k[slot_mapping] = k
    flat_v[slot_mapping] = v


# ---------------------------------------------------------------------------
# fp32 model restatement
# ---------------------------------------------------------------------------

def rope_tables(dim, max_seq_len, base=10000.0):
    """cos/sin [max_seq_len, dim/2] (models/rope.py:14-19)."""
    inv_freq = 1.0 / (base ** (torch.arange(0, dim, 2).float() / dim))
    ang = torch.outer(torch.arange(max_seq_len).float(), inv_freq)
    return ang.cos(), ang.sin()


def rope_rotate(x, cos, sin):
    """x [..., T, D] with cos/sin [T, D/2] broadcast (models/rope.py:21-35)."""
    y = torch.empty_like(x)
    xe, xo = x[..., 0::2], x[..., 1::2]
    y[..., 0::2] = xe * cos - xo * sin
    y[..., 1::2] = xe * sin + xo * cos
    return y


def rmsnorm(x, w, eps=1e-5):
    """models/rmsnorm.py:13-17 (CPU branch)."""
    x32 = x.float()
    y = x32 * torch.rsqrt(x32.square().mean(dim=-1, keepdim=True) + eps)
    return (y * w.float()).to(x.dtype)


class RefModel:
    """CPU restatement of PagedTransformer with contiguous per-sequence K/V.

    `sd` is a state dict with the reference parameter names
    (embedding.embedding.weight, layers.{i}.attn.{q_proj,k_proj,v_proj,out}
    .weight, layers.{i}.{attn_norm,mlp_norm}.weight, layers.{i}.mlp.
    {gate_proj,up_proj,down_proj}.weight, final_norm.weight, lm_head.weight).
    """

    def __init__(self, sd, num_layers, num_heads, num_kv_heads, max_seq_len,
                 dtype=torch.float32):
        self.sd = {k: v.detach().to("cpu", dtype) for k, v in sd.items()}
        self.L = num_layers
        self.hq = num_heads
        self.hkv = num_kv_heads
        d_model = self.sd["embedding.embedding.weight"].shape[1]
        self.d = d_model // num_heads
        cos, sin = rope_tables(self.d, max_seq_len)
        self.cos, self.sin = cos.to(dtype), sin.to(dtype)
        self.cache = {}  # seq_id -> per layer [K [n, hkv, d], V]

    def _lin(self, name, x):
        b = self.sd.get(name + ".bias")
        return F.linear(x, self.sd[name + ".weight"], b)

    def forward_seq(self, seq_id, token_ids, positions):
        """Run new tokens of one sequence (positions contiguous, continuing
        its cache); returns the last token's logits [vocab]."""
        sd = self.sd
        x = F.embedding(torch.as_tensor(token_ids, dtype=torch.long), sd["embedding.embedding.weight"])
        pos = torch.as_tensor(positions, dtype=torch.long)
        cos, sin = self.cos.index_select(0, pos), self.sin.index_select(0, pos)
        layers = self.cache.setdefault(seq_id, [[None, None] for _ in range(self.L)])
        T = x.shape[0]
        for l in range(self.L):
            p = f"layers.{l}."
            h = rmsnorm(x, sd[p + "attn_norm.weight"])
            q = self._lin(p + "attn.q_proj", h).view(T, self.hq, self.d)
            k = self._lin(p + "attn.k_proj", h).view(T, self.hkv, self.d)
            v = self._lin(p + "attn.v_proj", h).view(T, self.hkv, self.d)
            q = rope_rotate(q.transpose(0, 1), cos, sin).transpose(0, 1)
            k = rope_rotate(k.transpose(0, 1), cos, sin).transpose(0, 1)
            kc, vc = layers[l]
            kc = k if kc is None else torch.cat([kc, k])
            vc = v if vc is None else torch.cat([vc, v])
            layers[l] = [kc, vc]
            att = sdpa_one(q, kc, vc, causal=True)
            x = x + self._lin(p + "attn.out", att.reshape(T, -1))
            h = rmsnorm(x, sd[p + "mlp_norm.weight"])
            g = self._lin(p + "mlp.gate_proj", h)
            u = self._lin(p + "mlp.up_proj", h)
            x = x + self._lin(p + "mlp.down_proj", F.silu(g) * u)
        last = rmsnorm(x[-1:], sd["final_norm.weight"])
        return F.linear(last, sd["lm_head.weight"])[0]


@torch.no_grad()
def generate_batched_ref(model: RefModel, prompts_ids, max_new_tokens):
    """Greedy batched generation (serving/generation.py:112-148 semantics):
    prefill every prompt, then max_new_tokens-1 single-token steps; returns
    (tokens per sequence, logits of every step per sequence)."""
    outs = [[] for _ in prompts_ids]
    logits_log = [[] for _ in prompts_ids]
    lengths = []
    for i, p in enumerate(prompts_ids):
        lg = model.forward_seq(i, list(p), list(range(len(p))))
        logits_log[i].append(lg)
        outs[i].append(int(lg.argmax()))
        lengths.append(len(p))
    for _ in range(max_new_tokens - 1):
        for i in range(len(prompts_ids)):
            t = outs[i][-1]
            lg = model.forward_seq(i, [t], [lengths[i]])
            lengths[i] += 1
            logits_log[i].append(lg)
            outs[i].append(int(lg.argmax()))
    return outs, logits_log
