"""A greedy decode step of a PagedTransformer captured as one HIP graph.

The eager step (paged_model.PagedTransformer.forward_step) launches some
hundred kernels per token of the batch from Python: for every layer the
norms, the projections, RoPE, the slot-mapped append and the paged
attention. For a fixed batch whose metadata lives on the device
(paged_meta.PagedBatchMeta) none of those launches needs the host, so the
whole step - all layers, the greedy argmax, and the advance of every
sequence by one token (positions, start_pos and seq_lens + 1) - is captured
once and replayed. Every replay runs the same kernels on the same buffers as
the eager step.

The block tables are read from meta.block_tables at replay time, so a caller
that grows a sequence past a block boundary writes the new entry into that
tensor in place (same shape) before the replay. The attention plan (split-K
partition count) is fixed at capture for meta.max_kv_len; the kernels stay
exact for longer contexts (a longer partition per workgroup), so capture
with the bound the batch will reach.

The graph owns its scratch: the split-K partials and arrival counters of
the attention live in a workspace created for this graph, sized by the eager
warm-up steps and kept for the graph's lifetime. Eager attention calls made
between replays use the process-wide workspace, so when they grow (and free)
it, the buffer the graph captured is unaffected.
"""
from __future__ import annotations

import torch

from . import _native, fused_ops


class DecodeStepGraph:
    """Greedy decode step over a fixed batch, replayed from a HIP graph.

    ids: int64 [N] device tensor, the tokens fed to the first replay. After
    each replay, `ids` holds the argmax tokens (the next step's input) and
    `logits` the step's logits [N, vocab]. `meta` is advanced by one token
    per sequence on the device by every replay (its Python-side max_kv_len is
    not touched).
    """

    def __init__(self, model, pool, meta, ids: torch.Tensor, warmup: int = 0):
        if not ids.is_cuda or ids.dtype != torch.long or ids.dim() != 1:
            raise ValueError("ids must be a 1-D int64 device tensor")
        if ids.shape[0] != meta.num_tokens or not meta.is_decode:
            raise ValueError("DecodeStepGraph needs a decode batch: one token per sequence")
        if getattr(pool, "debug", False):
            raise ValueError("KVPool debug checks synchronise the host; disable them to capture")
        self.model, self.pool, self.meta = model, pool, meta
        self.ids = ids.clone()
        self.logits = None
        self.workspace = _native.Workspace()
        # eager steps on a side stream before capture (library handles, this
        # graph's workspace and caching-allocator pools are created here)
        side = torch.cuda.Stream(device=ids.device)
        side.wait_stream(torch.cuda.current_stream(ids.device))
        with _native.workspace_scope(self.workspace):
            with torch.cuda.stream(side), torch.no_grad():
                for _ in range(max(warmup, 1)):
                    self._step()
            torch.cuda.current_stream(ids.device).wait_stream(side)
            torch.cuda.synchronize(ids.device)
            self.graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(self.graph), torch.no_grad():
                self.logits = self._step()

    def _step(self):
        logits = self.model.forward_step(self.ids, self.pool, self.meta)
        fused_ops.argmax_rows(logits, out=self.ids)
        self.meta.advance_()
        return logits

    def replay(self) -> torch.Tensor:
        """One decode step; returns the tokens it produced (the `ids` buffer,
        overwritten by the next replay)."""
        self.graph.replay()
        return self.ids
