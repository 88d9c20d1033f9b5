"""Dense layers around the paged attention path.

Each keeps the reference module's constructor, parameter names and
arithmetic so that state dicts load unchanged and results match:
  RoPE            models/rope.py:5-47 (interleaved even/odd pairs)
  RMSNorm         models/rmsnorm.py:6-18 (the fp32 formula of its CPU branch)
  SwiGLU          models/mlp.py:17-32 (silu(gate) * up, then down)
  TokenEmbedding  models/embedding.py:5-15
  ModelConfig     models/model_config.py:8-41
As in the reference, which routes CUDA tensors to its own kernels
(models/rmsnorm.py:18, models/mlp.py:30), tensors on a ROCm device go to the
HIP kernels of fused_ops (RMSNorm, token-major RoPE, the SwiGLU projections
with the gate in their epilogue); CPU tensors use the PyTorch formulas.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import fused_ops


class RoPE(nn.Module):
    """Rotary embedding on interleaved (even, odd) pairs:
    out_even = x_even*cos - x_odd*sin, out_odd = x_even*sin + x_odd*cos with
    angle position * base^(-2i/dim)."""

    def __init__(self, dim, max_seq_len=2048, base=10000.0):
        super().__init__()
        assert dim % 2 == 0, "RoPE dimension must be even"
        self.dim = dim
        self.base = base
        self.max_seq_len = max_seq_len
        inv_freq = 1.0 / (base ** (torch.arange(0, dim, 2).float() / dim))
        angles = torch.outer(torch.arange(max_seq_len).float(), inv_freq)
        # [1, 1, max_seq_len, dim/2], non-persistent like the reference
        self.register_buffer("cos", angles.cos()[None, None], persistent=False)
        self.register_buffer("sin", angles.sin()[None, None], persistent=False)

    def _tables_fp32(self):
        """cos / sin as fp32 [max_seq_len, dim/2] for the HIP kernel, which
        rounds them to the activation dtype itself. A module moved to a
        lower precision holds its tables in that precision already (rounded
        once; rounding again changes nothing), so the fp32 copy is exact;
        it is cached until the buffers change."""
        key = (self.cos.data_ptr(), self.cos._version, self.sin.data_ptr(), self.sin._version)
        if getattr(self, "_t32_key", None) != key:
            half = self.dim // 2
            self._t32 = (self.cos.float().reshape(-1, half).contiguous(),
                         self.sin.float().reshape(-1, half).contiguous())
            self._t32_key = key
        return self._t32

    @staticmethod
    def _rotate(q, k, cos, sin):
        def rot(x):
            y = torch.empty_like(x)
            xe, xo = x[..., 0::2], x[..., 1::2]
            y[..., 0::2] = xe * cos - xo * sin
            y[..., 1::2] = xe * sin + xo * cos
            return y
        return rot(q), rot(k)

    def forward(self, q, k, position_offset: int = 0):
        T = q.shape[-2]
        cos = self.cos[:, :, position_offset:position_offset + T, :].to(dtype=q.dtype)
        sin = self.sin[:, :, position_offset:position_offset + T, :].to(dtype=q.dtype)
        return self._rotate(q, k, cos, sin)

    def forward_at(self, q, k, positions):
        """q, k [..., H, T, D] rotated at absolute `positions` [T]."""
        cos = self.cos.index_select(2, positions).to(dtype=q.dtype)
        sin = self.sin.index_select(2, positions).to(dtype=q.dtype)
        return self._rotate(q, k, cos, sin)

    def forward_tokens(self, q, k, positions, v=None):
        """Token-major variant: q [T, Hq, D], k [T, Hkv, D]. Same element-wise
        arithmetic as forward_at, without the head/token transposes. On a
        ROCm device one HIP kernel rotates both (and, with v, also returns v
        made contiguous: q, k, v may be strided slices of one projection)."""
        if q.is_cuda:
            cos, sin = self._tables_fp32()
            return fused_ops.rope(q, k, positions, cos, sin, v=v)
        if v is not None:
            return (*self.forward_tokens(q, k, positions), v.contiguous())
        cos = self.cos[0, 0].index_select(0, positions).to(dtype=q.dtype)[:, None, :]
        sin = self.sin[0, 0].index_select(0, positions).to(dtype=q.dtype)[:, None, :]
        return self._rotate(q, k, cos, sin)


class RMSNorm(nn.Module):
    def __init__(self, dim: int, eps: float = 1e-5):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.is_cuda:
            return fused_ops.rms_norm(x, self.weight, self.eps)
        x32 = x.float()
        y = x32 * torch.rsqrt(x32.square().mean(dim=-1, keepdim=True) + self.eps)
        return (y * self.weight.float()).to(dtype=x.dtype)


class SwiGLU(nn.Module):
    def __init__(self, d_model, hidden_dim, bias=False):
        super().__init__()
        self.gate_proj = nn.Linear(d_model, hidden_dim, bias=bias)
        self.up_proj = nn.Linear(d_model, hidden_dim, bias=bias)
        self.down_proj = nn.Linear(hidden_dim, d_model, bias=bias)

        self._gate_up = fused_ops.FusedRows(self.gate_proj, self.up_proj)

    def forward(self, x):
        if x.is_cuda:
            w, b = self._gate_up.get()
            h = fused_ops.linear_swiglu(x, w, b)
            return fused_ops.linear(h, self.down_proj.weight, self.down_proj.bias)
        return self.down_proj(F.silu(self.gate_proj(x)) * self.up_proj(x))

    def forward_residual_(self, x, norm):
        """x += forward(norm(x)) in place on a ROCm device, the norm taken in
        the gate/up projection's prologue and the add in down_proj's
        epilogue (the same rounded values as the separate ops). Returns x."""
        w, b = self._gate_up.get()
        h = fused_ops.linear_swiglu_rmsnorm(x, norm.weight, norm.eps, w, b)
        return fused_ops.linear_residual_(x, h, self.down_proj.weight, self.down_proj.bias)


class TokenEmbedding(nn.Module):
    def __init__(self, vocab_size, embed_dim):
        super().__init__()
        self.embedding = nn.Embedding(vocab_size, embed_dim)

    def forward(self, x):
        return self.embedding(x)


@dataclass
class ModelConfig:
    vocab_size: int = 50257
    d_model: int = 512
    num_layers: int = 34
    num_heads: int = 8
    num_kv_heads: int = 1
    max_seq_len: int = 512
    causal: bool = True
    dropout: float = 0.0
    bias: bool = False
    dtype: torch.dtype = torch.float32
    eos_token_id: int = 50256
    rope_theta: float = 10000.0
    rms_norm_eps: float = 1e-5

    def __post_init__(self):
        assert self.d_model % self.num_heads == 0
        assert self.num_heads % self.num_kv_heads == 0

    @property
    def head_dim(self) -> int:
        return self.d_model // self.num_heads

    @property
    def hidden_size(self) -> int:
        # the reference's MLP width equals d_model (model_config.py:32-34)
        return self.d_model


@dataclass
class CacheConfig:
    """KV cache settings (reference: models/model_config.py:45-51). kv_dtype
    None means the model's dtype; torch.float8_e4m3fn gives fp8 pools (new
    rows rounded on append, widened exactly by the attention kernels)."""
    block_size: int = 16
    num_gpu_blocks: int | None = None
    kv_budget_bytes: int = 2 * 1024**3
    kv_dtype: torch.dtype | None = None
    enable_prefix_caching: bool = False


@dataclass
class EngineConfig:
    """Model + cache + scheduler settings with the derived pool geometry
    (reference: models/model_config.py:73-100)."""
    model: ModelConfig = field(default_factory=ModelConfig)
    cache: CacheConfig = field(default_factory=CacheConfig)
    sched: "SchedulerConfig" = field(default_factory=lambda: SchedulerConfig())

    @property
    def kv_dtype(self) -> torch.dtype:
        return self.cache.kv_dtype or self.model.dtype

    @property
    def max_blocks_per_seq(self) -> int:
        return -(-self.model.max_seq_len // self.cache.block_size)

    @property
    def bytes_per_block(self) -> int:
        m, c = self.model, self.cache
        elem = torch.empty((), dtype=self.kv_dtype).element_size()
        return 2 * m.num_layers * c.block_size * m.num_kv_heads * m.head_dim * elem

    @property
    def num_blocks(self) -> int:
        n = self.cache.num_gpu_blocks
        return n if n is not None else self.cache.kv_budget_bytes // self.bytes_per_block

    def __post_init__(self):
        bs = self.cache.block_size
        assert bs & (bs - 1) == 0, "block_size must be a power of two"
        if not self.sched.enable_chunked_prefill:
            assert self.sched.max_num_batched_tokens >= self.model.max_seq_len, \
                "without chunked prefill, a full-length prompt must fit in one step"


@dataclass
class SchedulerConfig:
    """Scheduler limits (reference: models/model_config.py:56-70, where the
    fields exist but the reference scheduler does not read them; here
    serving.scheduler.Scheduler honours them when given one).
    cudagraph_batch_sizes is kept for the API; decode graphs are captured per
    batch by serving.graph_step.DecodeStepGraph instead."""
    max_num_seqs: int = 32
    max_num_batched_tokens: int = 512
    enable_chunked_prefill: bool = False
    preemption: str = "recompute"
    policy: str = "fcfs"
    cudagraph_batch_sizes: list = field(default_factory=lambda: [1, 2, 4, 8, 16, 32])

    def __post_init__(self):
        assert self.max_num_batched_tokens >= self.max_num_seqs, \
            "every decode takes 1 token, so the budget must cover all seqs"
        assert self.preemption == "recompute"
        assert self.policy == "fcfs"
        assert max(self.cudagraph_batch_sizes) <= self.max_num_seqs
