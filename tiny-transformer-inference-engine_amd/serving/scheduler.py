"""Continuous-batching scheduler — drop-in for serving/scheduler.py.

Admission (reference: scheduler.py:28-44): the head of the waiting queue is
admitted while, after giving it its prompt's blocks, at least one free block
per running sequence (itself included) remains as growth headroom. Each step
(scheduler.py:46-79) runs prefills (whole prompt) and decodes (last token)
in one ragged batch, samples one token per sequence, and releases finished
sequences' blocks.

Given a SchedulerConfig (the reference defines one, models/model_config.py:
56-70, but never reads it), a step is planned within its limits instead:
  - at most max_num_batched_tokens new tokens per step: decodes first (one
    token each), then prefills in admission order;
  - at most max_num_seqs running sequences;
  - enable_chunked_prefill: a prompt longer than the budget left is computed
    in chunks over several steps (the paged kernels attend each chunk to the
    blocks already written, bottom-right causal); a token is sampled only
    after its last chunk. Without it a prompt runs whole or waits;
  - preemption="recompute": when a decode needs a block and none is free,
    the most recently admitted running sequence is preempted (its blocks
    released, the request requeued at the head of the waiting queue with
    every token so far as its prompt, keeping its seq_id and generated count)
    and recomputed when it is admitted again.
Without a SchedulerConfig the behaviour is the reference's.
"""
from __future__ import annotations

from .batch import BatchStep, build_batch_step
from .sampling import sample
from .sequence import Sequence, blocks_for


class Scheduler:
    def __init__(self, model, pool, alloc, cfg, block_size=16,
                 temperature=1.0, top_k=32, top_p=0.9, sched_cfg=None):
        self.model = model
        self.pool = pool
        self.alloc = alloc
        self.cfg = cfg
        self.block_size = block_size
        self.temperature = temperature
        self.top_k = top_k
        self.top_p = top_p
        self.device = next(model.parameters()).device
        self.waiting = []
        self.running = []
        self.next_seq_id = 0
        self.sched_cfg = sched_cfg
        self.num_preemptions = 0
        self.last_batch_tokens = 0

    def add_request(self, prompt_ids, max_new_tokens):
        if self.sched_cfg is not None:
            sc = self.sched_cfg
            # without chunking a recomputed (preempted) request is prefilled whole,
            # prompt and generated tokens, so all of it must fit one step's budget
            longest = len(prompt_ids) + max_new_tokens
            if not sc.enable_chunked_prefill and longest > sc.max_num_batched_tokens:
                raise ValueError(
                    f"prompt + max_new_tokens = {longest} tokens exceeds "
                    f"max_num_batched_tokens={sc.max_num_batched_tokens} and chunked "
                    "prefill is disabled (a preempted request is recomputed in one step)")
            need = blocks_for(len(prompt_ids) + max_new_tokens, self.block_size)
            if need + 1 > self.alloc.num_usable:
                raise ValueError(f"request needs {need} blocks; the pool has "
                                 f"{self.alloc.num_usable} usable")
        self.waiting.append({"prompt_ids": prompt_ids, "max_new_tokens": max_new_tokens,
                             "generated": 0})

    def _try_admit(self):
        while self.waiting:
            req = self.waiting[0]
            seq = Sequence(self.next_seq_id, list(req["prompt_ids"]), self.block_size)
            headroom = len(self.running) + 1
            if self.alloc.num_free - seq.num_blocks_needed() < headroom:
                break
            seq.ensure_blocks(self.alloc)
            seq._meta = req
            seq._is_prefill = True
            self.running.append(seq)
            self.waiting.pop(0)
            self.next_seq_id += 1

    def _pick(self, row):
        return int(sample(row.unsqueeze(0), self.temperature, self.top_k, self.top_p))

    def step(self):
        """Returns [(seq_id, token, done)] for every sequence that sampled a
        token (with a SchedulerConfig, a prefill chunk that does not finish
        its prompt samples nothing)."""
        if self.sched_cfg is not None:
            return self._step_budgeted()
        self._try_admit()
        if not self.running:
            return []
        entries = [(seq, seq.token_ids if seq._is_prefill else [seq.token_ids[-1]])
                   for seq in self.running]
        logits = self.model.forward_batch(build_batch_step(entries, self.device), self.pool)

        results, still_running = [], []
        for i, seq in enumerate(self.running):
            tok = self._pick(logits[i])
            seq._is_prefill = False
            seq._meta["generated"] += 1
            done = (tok == self.cfg.eos_token_id
                    or seq._meta["generated"] >= seq._meta["max_new_tokens"])
            results.append((seq.seq_id, tok, done))
            if done:
                seq.release(self.alloc)
            else:
                seq.append_token(tok)
                seq.ensure_blocks(self.alloc)
                still_running.append(seq)
        self.running = still_running
        return results

    # ---- SchedulerConfig-driven steps ------------------------------------

    def _preempt(self, seq):
        """Recompute preemption: release the blocks, requeue every token so far."""
        seq.release(self.alloc)
        self.running.remove(seq)
        req = seq._meta
        req["prompt_ids"] = list(seq.token_ids)
        req["seq_id"] = seq.seq_id
        self.waiting.insert(0, req)
        self.num_preemptions += 1

    def _admit_one(self, req):
        seq_id = req.get("seq_id")
        if seq_id is None:
            seq_id = self.next_seq_id
            self.next_seq_id += 1
        seq = Sequence(seq_id, list(req["prompt_ids"]), self.block_size)
        seq.ensure_blocks(self.alloc)
        seq._meta = req
        seq._computed = 0
        self.running.append(seq)
        return seq

    def _step_budgeted(self):
        sc = self.sched_cfg
        budget = sc.max_num_batched_tokens
        plan = []  # (seq, first, end): tokens [first, end) computed this step
        # running sequences, in admission order: decodes and unfinished prefills
        for seq in list(self.running):
            if seq not in self.running:
                continue  # preempted earlier in this loop
            remaining = seq.num_tokens - seq._computed
            if remaining <= 0:
                continue
            if remaining > 1 and not sc.enable_chunked_prefill and remaining > budget:
                continue
            n = min(remaining, budget)
            if n <= 0:
                continue
            # blocks for the tokens this step computes (decodes grow by one)
            while seq.num_new_blocks_needed() > self.alloc.num_free:
                victim = self.running[-1]
                self._preempt(victim)
                if victim is seq:
                    break
            if seq not in self.running:
                continue
            seq.ensure_blocks(self.alloc)
            plan.append((seq, seq._computed, seq._computed + n))
            budget -= n
        # admission (FCFS) within the sequence cap, the block headroom and the budget
        while self.waiting and budget > 0 and len(self.running) < sc.max_num_seqs:
            req = self.waiting[0]
            ntok = len(req["prompt_ids"])
            need = blocks_for(ntok, self.block_size)
            if self.alloc.num_free - need < len(self.running) + 1:
                break
            if ntok > budget and not sc.enable_chunked_prefill:
                break
            self.waiting.pop(0)
            seq = self._admit_one(req)
            n = min(ntok, budget)
            plan.append((seq, 0, n))
            budget -= n
        if not plan:
            self.last_batch_tokens = 0
            return []
        ids, positions, qsl, tables, lens = [], [], [0], [], []
        for seq, a, b in plan:
            ids.extend(seq.token_ids[a:b])
            positions.extend(range(a, b))
            qsl.append(qsl[-1] + (b - a))
            tables.append(seq.block_table)
            lens.append(b)
        import torch
        batch = BatchStep(input_ids=torch.tensor(ids, dtype=torch.long, device=self.device),
                          positions=positions, query_start_loc=qsl, block_tables=tables,
                          seq_lens=lens)
        self.last_batch_tokens = len(ids)
        logits = self.model.forward_batch(batch, self.pool)

        results = []
        for i, (seq, a, b) in enumerate(plan):
            seq._computed = b
            if b < seq.num_tokens:
                continue  # prefill chunk: the prompt is not finished yet
            tok = self._pick(logits[i])
            req = seq._meta
            req["generated"] += 1
            done = tok == self.cfg.eos_token_id or req["generated"] >= req["max_new_tokens"]
            results.append((seq.seq_id, tok, done))
            if done:
                seq.release(self.alloc)
                self.running.remove(seq)
            else:
                seq.append_token(tok)
        return results
