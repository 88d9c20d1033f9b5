"""Continuous-batching scheduler — drop-in for serving/scheduler.py.

Behaviour without a SchedulerConfig is the reference's (scheduler.py:8-79):
  - admission (:28-44): the head of the waiting queue is admitted while,
    after giving it its prompt's blocks, at least one free block per running
    sequence (itself included) stays free as growth headroom;
  - a step (:46-79) computes, in one ragged batch, every running sequence's
    tokens whose K/V are not in the pool yet (the whole prompt on the step
    after admission, then the last sampled token), samples one token per
    sequence in running order, and releases finished sequences' blocks
    (a sequence is finished on EOS or at max_new_tokens).

Given a SchedulerConfig (the reference defines one, models/model_config.py:
56-70, but never reads it), a step is planned within its limits instead:
  - at most max_num_batched_tokens new tokens per step: running sequences
    first (one token each for decodes), then admissions in arrival order;
  - at most max_num_seqs running sequences;
  - enable_chunked_prefill: a prompt longer than the budget left is computed
    in chunks over several steps (the paged kernels attend each chunk to the
    blocks already written, bottom-right causal); a token is sampled only
    after its last chunk. Without it a prompt runs whole or waits;
  - preemption="recompute": when a running sequence needs a block and none
    is free, the most recently admitted running sequence is preempted (its
    blocks released, its request put back at the head of the queue with
    every token so far as its prompt, keeping its seq_id and its count of
    generated tokens) and computed again once it is readmitted.

State: `waiting` holds _Request records; `running` holds Sequence objects in
admission order; per running sequence the scheduler keeps its _Request and
`computed`, the number of its tokens whose K/V are in the pool. The tokens a
step feeds for a sequence are always token_ids[computed:] (capped by the
budget), which covers prompts, chunks, decodes and recomputes alike.
"""
from __future__ import annotations

from dataclasses import dataclass

from .batch import BatchStep, build_batch_step
from .sampling import sample
from .sequence import Sequence, blocks_for


@dataclass
class _Request:
    """A request waiting to run: the tokens to compute as its prompt, its
    budget of new tokens, how many it has produced, and (once preempted) the
    seq_id it keeps."""
    prompt_ids: list
    max_new_tokens: int
    generated: int = 0
    seq_id: int | None = None


@dataclass
class _Running:
    req: _Request
    computed: int = 0  # tokens of the sequence whose K/V are in the pool


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
        self.sched_cfg = sched_cfg
        self.waiting: list[_Request] = []
        self.running: list[Sequence] = []
        self._state: dict[int, _Running] = {}  # seq_id -> state of a running sequence
        self.next_seq_id = 0
        self.num_preemptions = 0
        self.last_batch_tokens = 0

    # ---- requests ---------------------------------------------------------

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
        self.waiting.append(_Request(list(prompt_ids), max_new_tokens))

    def computed_tokens(self, seq: Sequence) -> int:
        """Tokens of a running sequence whose K/V are in the pool."""
        return self._state[seq.seq_id].computed

    # ---- shared pieces ----------------------------------------------------

    def _fits(self, req: _Request) -> bool:
        """The reference's admission rule: the prompt's blocks, plus one free
        block per running sequence and the newcomer."""
        need = blocks_for(len(req.prompt_ids), self.block_size)
        return self.alloc.num_free - need >= len(self.running) + 1

    def _start(self, req: _Request) -> Sequence:
        if req.seq_id is None:
            req.seq_id = self.next_seq_id
            self.next_seq_id += 1
        seq = Sequence(req.seq_id, req.prompt_ids, self.block_size)
        seq.ensure_blocks(self.alloc)
        self.running.append(seq)
        self._state[seq.seq_id] = _Running(req)
        return seq

    def _finish(self, seq: Sequence) -> None:
        seq.release(self.alloc)
        del self._state[seq.seq_id]

    def _pick(self, row):
        return int(sample(row.unsqueeze(0), self.temperature, self.top_k, self.top_p))

    def _sampled(self, seq: Sequence, row):
        """Sample the next token of a sequence whose tokens are all computed;
        returns (token, done)."""
        tok = self._pick(row)
        req = self._state[seq.seq_id].req
        req.generated += 1
        return tok, tok == self.cfg.eos_token_id or req.generated >= req.max_new_tokens

    # ---- a step -----------------------------------------------------------

    def step(self):
        """Returns [(seq_id, token, done)] for every sequence that sampled a
        token (with a SchedulerConfig, a prefill chunk that does not finish
        its prompt samples nothing)."""
        if self.sched_cfg is not None:
            return self._step_budgeted()
        while self.waiting and self._fits(self.waiting[0]):
            self._start(self.waiting.pop(0))
        if not self.running:
            return []
        batch = [(seq, seq.token_ids[self._state[seq.seq_id].computed:]) for seq in self.running]
        logits = self.model.forward_batch(build_batch_step(batch, self.device), self.pool)

        results, kept = [], []
        for i, seq in enumerate(self.running):
            self._state[seq.seq_id].computed = seq.num_tokens
            tok, done = self._sampled(seq, logits[i])
            results.append((seq.seq_id, tok, done))
            if done:
                self._finish(seq)
            else:
                seq.append_token(tok)
                seq.ensure_blocks(self.alloc)
                kept.append(seq)
        self.running = kept
        return results

    # ---- SchedulerConfig-driven steps ------------------------------------

    def _preempt(self, seq: Sequence) -> None:
        """Recompute preemption: release the blocks, requeue every token so far."""
        req = self._state[seq.seq_id].req
        self._finish(seq)
        self.running.remove(seq)
        req.prompt_ids = list(seq.token_ids)
        self.waiting.insert(0, req)
        self.num_preemptions += 1

    def _step_budgeted(self):
        sc = self.sched_cfg
        budget = sc.max_num_batched_tokens
        plan = []  # (seq, first, end): tokens [first, end) computed this step
        # running sequences, in admission order: decodes and unfinished prefills
        for seq in list(self.running):
            if seq.seq_id not in self._state:
                continue  # preempted earlier in this loop
            st = self._state[seq.seq_id]
            todo = seq.num_tokens - st.computed
            if todo <= 0 or budget <= 0:
                continue
            if todo > 1 and todo > budget and not sc.enable_chunked_prefill:
                continue  # a whole prompt that does not fit what is left
            n = min(todo, budget)
            # the blocks of the tokens computed now, freeing the newest sequences'
            while seq.num_new_blocks_needed() > self.alloc.num_free:
                victim = self.running[-1]
                self._preempt(victim)
                if victim is seq:
                    break
            if seq.seq_id not in self._state:
                continue
            seq.ensure_blocks(self.alloc)
            plan.append((seq, st.computed, st.computed + n))
            budget -= n
        # admission (FCFS) within the sequence cap, the block headroom and the budget
        while self.waiting and budget > 0 and len(self.running) < sc.max_num_seqs:
            req = self.waiting[0]
            if not self._fits(req):
                break
            if len(req.prompt_ids) > budget and not sc.enable_chunked_prefill:
                break
            seq = self._start(self.waiting.pop(0))
            n = min(seq.num_tokens, budget)
            plan.append((seq, 0, n))
            budget -= n
        if not plan:
            self.last_batch_tokens = 0
            return []
        import torch
        ids = [t for seq, a, b in plan for t in seq.token_ids[a:b]]
        qsl = [0]
        for _, a, b in plan:
            qsl.append(qsl[-1] + (b - a))
        batch = BatchStep(input_ids=torch.tensor(ids, dtype=torch.long, device=self.device),
                          positions=[p for _, a, b in plan for p in range(a, b)],
                          query_start_loc=qsl, block_tables=[seq.block_table for seq, _, _ in plan],
                          seq_lens=[b for _, _, b in plan])
        self.last_batch_tokens = len(ids)
        logits = self.model.forward_batch(batch, self.pool)

        results = []
        for i, (seq, _, b) in enumerate(plan):
            self._state[seq.seq_id].computed = b
            if b < seq.num_tokens:
                continue  # prefill chunk: the prompt is not finished yet
            tok, done = self._sampled(seq, logits[i])
            results.append((seq.seq_id, tok, done))
            if done:
                self._finish(seq)
                self.running.remove(seq)
            else:
                seq.append_token(tok)
        return results
