"""Paged decoder-only transformer — drop-in for serving/paged_model.py.

Same module tree and parameter names as the reference (embedding, layers[i]
{attn_norm, attn, mlp_norm, mlp}, final_norm, lm_head), built in the same
order, so reference checkpoints load and random init under one seed draws
the same weights. `forward_batch` packs the step's metadata once and shares
it across layers instead of rebuilding it per layer.
"""
from __future__ import annotations

import torch
import torch.nn as nn

from . import fused_ops
from .layers import ModelConfig, RMSNorm, SwiGLU, TokenEmbedding
from .paged_meta import pack_batch_meta
from .paged_mqa import MQA_Paged


class PagedBlock(nn.Module):
    def __init__(self, config, layer_idx, backend="pytorch"):
        super().__init__()
        self.layer_idx = layer_idx
        self.attn_norm = RMSNorm(config.d_model)
        self.attn = MQA_Paged(config, backend=backend)
        self.mlp_norm = RMSNorm(config.d_model)
        self.mlp = SwiGLU(config.d_model, config.hidden_size, config.bias)

    def forward(self, x, pool, block_table, start):
        x = x + self.attn.forward_paged(self.attn_norm(x), pool, self.layer_idx, block_table, start)
        return x + self.mlp(self.mlp_norm(x))

    def forward_meta(self, x, pool, meta):
        x = x + self.attn.forward_meta(self.attn_norm(x), pool, self.layer_idx, meta)
        return x + self.mlp(self.mlp_norm(x))


class PagedTransformer(nn.Module):
    def __init__(self, config, backend="pytorch"):
        super().__init__()
        self.embedding = TokenEmbedding(config.vocab_size, config.d_model)
        self.layers = nn.ModuleList(
            [PagedBlock(config, i, backend) for i in range(config.num_layers)])
        self.final_norm = RMSNorm(config.d_model)
        self.lm_head = nn.Linear(config.d_model, config.vocab_size, bias=False)

    def forward(self, input_ids, pool, block_table, start):
        """Single sequence (reference: paged_model.py:42-47): logits of the
        last token, [1, 1, vocab]."""
        x = self.embedding(input_ids)
        for layer in self.layers:
            x = layer(x, pool, block_table, start)
        x = x[:, -1:, :]
        return self.lm_head(self.final_norm(x))

    @torch.no_grad()
    def forward_batch(self, batch, pool):
        """Ragged batch step (reference: paged_model.py:50-67): logits of each
        sequence's last new token, [num_seqs, vocab]."""
        T = batch.input_ids.numel()
        meta = pack_batch_meta(batch.block_tables, batch.query_start_loc, batch.positions,
                               T, batch.input_ids.device, pool.block_size)
        return self.forward_step(batch.input_ids, pool, meta)

    @torch.no_grad()
    def forward_step(self, input_ids, pool, meta):
        """forward_batch with pre-packed metadata (PagedBatchMeta).

        On a ROCm device every norm runs in the prologue of the projection
        that consumes it and every residual add in the epilogue of the
        projection that produces it, so a layer is four projection kernels
        and one attention call: norm + qkv GEMM + RoPE, append + attention,
        out GEMM + add, norm + gate/up GEMM + SwiGLU gate, down GEMM + add.
        The arithmetic is that of PagedBlock.forward_meta: each sum is
        rounded to the model dtype before it is normalised or carried on."""
        x = self.embedding(input_ids)
        last = meta.query_start_loc[1:].long() - 1
        if not x.is_cuda:
            for layer in self.layers:
                x = layer.forward_meta(x, pool, meta)
            return self.lm_head(self.final_norm(x.index_select(0, last)))
        x = x.contiguous()
        for layer in self.layers:
            layer.attn.forward_meta_residual_(x, layer.attn_norm, pool, layer.layer_idx, meta)
            layer.mlp.forward_residual_(x, layer.mlp_norm)
        if not meta.is_decode:
            x = x.index_select(0, last)
        return self.lm_head(self.final_norm(x))


def load_paged_model(ckpt_path, device):
    """Checkpoint {model, model_config, ...} -> (PagedTransformer, ModelConfig)
    (reference: paged_model.py:70-80). Loaded with weights_only=True."""
    ckpt = torch.load(ckpt_path, map_location="cpu", weights_only=True)
    raw = ckpt.get("model_config")
    if raw is None:
        raise ValueError("checkpoint is missing model_config")
    values = dict(raw) if isinstance(raw, dict) else vars(raw)
    cfg = ModelConfig(**{k: v for k, v in values.items() if k in ModelConfig.__dataclass_fields__})
    attn_type = ckpt.get("train_config", {}).get("attn_type", "mqa")
    if attn_type != "mqa":
        raise ValueError(f"paged serving supports MQA checkpoints, got {attn_type!r}")
    model = PagedTransformer(cfg, backend="pytorch")
    sd = {k.replace("_orig_mod.", ""): v for k, v in ckpt["model"].items()}
    model.load_state_dict(sd)
    return model.to(device).eval(), cfg
