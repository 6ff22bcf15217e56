"""Continuous-batching admission (nv/scheduler.py:11-116).

FIFO admission under ``max_num_seqs`` and a whole-request block reservation of
ceil((runtime_prompt_len + max_new_tokens) / block_size).  No preemption.
A step first finishes sequences whose pending token is EOS or that reached
their token budget, then admits waiting requests in order, then lists every
running sequence that has a pending token for decode, in admission order
(``running`` is an insertion-ordered dict).  That order fixes the decode batch
composition and the order in which blocks are allocated.
"""
from __future__ import annotations

import math
from collections import deque
from dataclasses import dataclass, field

from .sequence import Sequence, SequenceStatus


@dataclass
class SchedulerStep:
    prefill_seqs: list[Sequence] = field(default_factory=list)
    decode_seqs: list[Sequence] = field(default_factory=list)
    finish_seqs: list[Sequence] = field(default_factory=list)


class MiniScheduler:
    def __init__(self, max_num_seqs: int, block_size: int, total_num_blocks: int):
        self.max_num_seqs = max_num_seqs
        self.block_size = block_size
        self.total_num_blocks = total_num_blocks
        self.waiting: deque[Sequence] = deque()
        self.running: dict[int, Sequence] = {}
        self.finished: dict[int, Sequence] = {}
        self.seqs: dict[int, Sequence] = {}
        self.reserved_blocks_total = 0
        self._next_seq_id = 0

    def reset(self) -> None:
        for container in (self.waiting, self.running, self.finished, self.seqs):
            container.clear()
        self.reserved_blocks_total = 0
        self._next_seq_id = 0

    def next_seq_id(self) -> int:
        self._next_seq_id += 1
        return self._next_seq_id - 1

    def add_request(self, seq: Sequence) -> Sequence:
        self.seqs[seq.seq_id] = seq
        self.waiting.append(seq)
        return seq

    def compute_required_blocks(self, runtime_prompt_len: int, max_new_tokens: int) -> int:
        tokens = runtime_prompt_len + max_new_tokens
        return math.ceil(tokens / self.block_size) if tokens > 0 else 0

    def has_unfinished(self) -> bool:
        return bool(self.waiting) or bool(self.running)

    def _can_admit(self, seq: Sequence) -> bool:
        return (len(self.running) < self.max_num_seqs
                and self.reserved_blocks_total + seq.reserved_blocks <= self.total_num_blocks)

    def _finish_sequence(self, seq: Sequence, reason: str) -> None:
        del self.running[seq.seq_id]
        self.reserved_blocks_total -= seq.reserved_blocks
        seq.finish(reason)
        self.finished[seq.seq_id] = seq

    def finish_sequences(self, seqs: list[Sequence], reason: str) -> list[Sequence]:
        """Finish those of `seqs` that are still running; return them."""
        done = [seq for seq in seqs if seq.seq_id in self.running]
        for seq in done:
            self._finish_sequence(seq, reason)
        return done

    def _should_finish(self, seq: Sequence, eos_token_id: int) -> str | None:
        if seq.next_token_id is not None and seq.next_token_id == eos_token_id:
            return "eos"
        return "max_new_tokens" if seq.reach_max_tokens() else None

    def plan_next_step(self, eos_token_id: int) -> SchedulerStep:
        step = SchedulerStep()
        for seq in list(self.running.values()):
            reason = self._should_finish(seq, eos_token_id)
            if reason is not None:
                self._finish_sequence(seq, reason)
                step.finish_seqs.append(seq)

        while self.waiting and self._can_admit(self.waiting[0]):
            seq = self.waiting.popleft()
            seq.status = SequenceStatus.RUNNING
            self.running[seq.seq_id] = seq
            self.reserved_blocks_total += seq.reserved_blocks
            step.prefill_seqs.append(seq)

        # A request that could never fit is dropped once nothing else is running.
        if self.waiting and not self.running and self.waiting[0].reserved_blocks > self.total_num_blocks:
            seq = self.waiting.popleft()
            seq.finish("aborted_no_capacity")
            self.finished[seq.seq_id] = seq
            step.finish_seqs.append(seq)

        step.decode_seqs = [seq for seq in self.running.values() if seq.next_token_id is not None]
        return step
