"""Continuous-batching admission and step planning (behaviour of nv/scheduler.py:11-116).

The policy is the reference's, because it fixes the batch composition and so
every block the pool hands out (the packing metadata must be bit-exact):

  * at admission a request reserves ceil((runtime prompt + max_new_tokens) /
    block_size) blocks for its whole life; admission is first-come
    first-served and stops at the first waiting request that does not fit
    (``max_num_seqs`` or the block budget); there is no preemption;
  * a step retires first (pending token == EOS, or the output budget spent),
    then admits, then takes every running request that holds a sampled token,
    in admission order.  A request admitted in this step is prefilled and
    joins the decode batch from the next step on.

The plan is this module's own: it also separates the requests whose pending
token is their last (committed without a forward, so a request runs
max_new_tokens - 1 decode forwards) from those that need a forward, and the
engine only executes it.  If nothing runs and the head of the queue needs more
blocks than the whole pool holds, that request is aborted.
"""
from __future__ import annotations

import math
from collections import deque
from dataclasses import dataclass, field

from .sequence import Sequence, SequenceStatus


@dataclass
class StepPlan:
    retired: list[Sequence] = field(default_factory=list)     # finished while planning
    admitted: list[Sequence] = field(default_factory=list)    # to prefill
    last_token: list[Sequence] = field(default_factory=list)  # commit the pending token, then finish
    forward: list[Sequence] = field(default_factory=list)     # to decode, admission order


class _BlockBudget:
    """Whole-life block reservations of the running requests against the pool size."""

    def __init__(self, total: int):
        self.total = total
        self.reserved = 0

    def fits(self, n: int) -> bool:
        return self.reserved + n <= self.total

    def take(self, n: int) -> None:
        self.reserved += n

    def give(self, n: int) -> None:
        self.reserved -= n


class MiniScheduler:
    def __init__(self, max_num_seqs: int, block_size: int, total_num_blocks: int):
        self.max_num_seqs = max_num_seqs
        self.block_size = block_size
        self.total_num_blocks = total_num_blocks
        self.budget = _BlockBudget(total_num_blocks)
        self.waiting: deque[Sequence] = deque()
        self.running: dict[int, Sequence] = {}   # admission order
        self.finished: dict[int, Sequence] = {}
        self.seqs: dict[int, Sequence] = {}
        self._ids = 0

    @property
    def reserved_blocks_total(self) -> int:
        return self.budget.reserved

    def reset(self) -> None:
        self.__init__(self.max_num_seqs, self.block_size, self.total_num_blocks)

    def next_seq_id(self) -> int:
        seq_id, self._ids = self._ids, self._ids + 1
        return seq_id

    def compute_required_blocks(self, runtime_prompt_len: int, max_new_tokens: int) -> int:
        return max(0, math.ceil((runtime_prompt_len + max_new_tokens) / self.block_size))

    def add_request(self, seq: Sequence) -> Sequence:
        self.seqs[seq.seq_id] = seq
        self.waiting.append(seq)
        return seq

    def has_unfinished(self) -> bool:
        return len(self.waiting) + len(self.running) > 0

    def head_fits(self) -> bool:
        """Whether the next plan admits the head of the queue even if nothing retires first."""
        return (len(self.waiting) > 0 and len(self.running) < self.max_num_seqs
                and self.budget.fits(self.waiting[0].reserved_blocks))

    def retire(self, seq: Sequence, reason: str) -> None:
        """Move a running request to ``finished`` and return its reservation."""
        self.running.pop(seq.seq_id)
        self.budget.give(seq.reserved_blocks)
        seq.finish(reason)
        self.finished[seq.seq_id] = seq

    @staticmethod
    def _finish_reason(seq: Sequence, eos_token_id: int) -> str | None:
        pending = seq.next_token_id
        if pending is not None and pending == eos_token_id:
            return "eos"
        return "max_new_tokens" if seq.reach_max_tokens() else None

    def plan_next_step(self, eos_token_id: int) -> StepPlan:
        plan = StepPlan()
        verdicts = [(seq, self._finish_reason(seq, eos_token_id)) for seq in self.running.values()]
        for seq, reason in verdicts:
            if reason is not None:
                self.retire(seq, reason)
                plan.retired.append(seq)

        while self.waiting:
            head = self.waiting[0]
            if len(self.running) >= self.max_num_seqs or not self.budget.fits(head.reserved_blocks):
                break
            self.waiting.popleft()
            head.status = SequenceStatus.RUNNING
            self.budget.take(head.reserved_blocks)
            self.running[head.seq_id] = head
            plan.admitted.append(head)

        if not self.running and self.waiting and self.waiting[0].reserved_blocks > self.total_num_blocks:
            head = self.waiting.popleft()  # could never fit, even alone
            head.finish("aborted_no_capacity")
            self.finished[head.seq_id] = head
            plan.retired.append(head)

        for seq in self.running.values():
            if seq.next_token_id is None:
                continue  # admitted in this step: prefilled now, decoded from the next step
            (plan.last_token if seq.pending_is_last() else plan.forward).append(seq)
        return plan
