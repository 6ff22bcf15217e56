"""Plain restatement of the reference's request state, scheduler and engine step (test infrastructure only).

Follows nv/sequence.py:20-67, nv/scheduler.py:20-116 and nv/engine.py:8-56
step by step, so that with ``BlockManagerRef`` it reproduces the reference's
block allocation order for any submission schedule and token stream:

  * a step finishes running requests whose pending token is EOS or whose
    output budget is spent (nv/scheduler.py:88-96), admits waiting requests
    FIFO under max_num_seqs and the block reservation (98-103), aborts an
    unfittable head when nothing runs (105-111), and lists running requests
    that hold a token for decode in admission order (113-115);
  * the engine frees the finished, prefills the admitted, commits the final
    token of requests on their last one without a forward, frees them, and
    decodes the rest (nv/engine.py:26-51).

Only tests/ import this module; the product's scheduler, engine and sequence
are separate code.  Pins (tests/test_oracle.py): every golden trace written
from the reference's own classes (tests/golden/block_traces.json) is
reproduced event for event when these classes drive ``BlockManagerRef``.
"""
from __future__ import annotations

import math
from collections import deque


class SequenceRef:
    """nv/sequence.py:20-67: the fields the runner and the scheduler read."""

    def __init__(self, seq_id, prompt, max_new_tokens, prompt_token_ids, sampling_params):
        self.seq_id = seq_id
        self.prompt = prompt
        self.max_new_tokens = max_new_tokens
        self.prompt_token_ids = prompt_token_ids
        self.sampling_params = sampling_params
        self.status = "waiting"
        self.estimated_prompt_len = 0
        self.reserved_blocks = 0
        self.finish_reason = None
        self.cached_prefix_len = 0
        self.cached_block_ids = []
        self.runtime_prompt_token_ids = None
        self.runtime_prompt_len = 0
        self.prompt_len = 0
        self.cache_position = 0
        self.next_token_id = None
        self.generated_token_ids = []

    def set_prefill_result(self, next_token_id, prompt_len):  # nv/sequence.py:45-48
        self.next_token_id = next_token_id
        self.prompt_len = prompt_len
        self.cache_position = prompt_len

    def append_next_token(self):  # nv/sequence.py:50-56
        if self.next_token_id is None:
            raise RuntimeError("no next token")
        self.generated_token_ids.append(self.next_token_id)
        return self.next_token_id

    def set_decode_result(self, next_token_id):  # nv/sequence.py:58-60
        self.next_token_id = next_token_id
        self.cache_position += 1


class _Plan:
    def __init__(self):
        self.prefill_seqs, self.decode_seqs, self.finish_seqs = [], [], []


class SchedulerRef:
    """nv/scheduler.py:17-116."""

    def __init__(self, max_num_seqs, block_size, total_num_blocks):
        self.max_num_seqs = max_num_seqs
        self.block_size = block_size
        self.total_num_blocks = total_num_blocks
        self.waiting = deque()
        self.running = {}
        self.finished = {}
        self.seqs = {}
        self.reserved = 0
        self.counter = 0

    def next_seq_id(self):  # :40-43
        self.counter += 1
        return self.counter - 1

    def add_request(self, seq):  # :45-48
        self.seqs[seq.seq_id] = seq
        self.waiting.append(seq)
        return seq

    def compute_required_blocks(self, runtime_prompt_len, max_new_tokens):  # :50-54
        n = runtime_prompt_len + max_new_tokens
        return 0 if n <= 0 else math.ceil(n / self.block_size)

    def has_unfinished(self):  # :56-57
        return len(self.waiting) > 0 or len(self.running) > 0

    def _finish(self, seq, reason):  # :64-68
        self.running.pop(seq.seq_id, None)
        self.reserved -= seq.reserved_blocks
        seq.status = "finished"
        seq.finish_reason = reason
        self.finished[seq.seq_id] = seq

    def finish_sequences(self, seqs, reason):  # :70-81
        out = []
        for seq in seqs:
            if seq.seq_id in self.running:
                self._finish(seq, reason)
                out.append(seq)
        return out

    def plan_next_step(self, eos):  # :88-116
        plan = _Plan()
        for seq in list(self.running.values()):
            if seq.next_token_id is not None and seq.next_token_id == eos:
                reason = "eos"
            elif len(seq.generated_token_ids) >= seq.max_new_tokens:
                reason = "max_new_tokens"
            else:
                continue
            self._finish(seq, reason)
            plan.finish_seqs.append(seq)
        while self.waiting:
            seq = self.waiting[0]
            if len(self.running) >= self.max_num_seqs or self.reserved + seq.reserved_blocks > self.total_num_blocks:
                break
            self.waiting.popleft()
            seq.status = "running"
            self.running[seq.seq_id] = seq
            self.reserved += seq.reserved_blocks
            plan.prefill_seqs.append(seq)
        if self.waiting and not self.running and self.waiting[0].reserved_blocks > self.total_num_blocks:
            seq = self.waiting.popleft()
            seq.status = "finished"
            seq.finish_reason = "aborted_no_capacity"
            self.finished[seq.seq_id] = seq
            plan.finish_seqs.append(seq)
        plan.decode_seqs = [seq for seq in self.running.values() if seq.next_token_id is not None]
        return plan


class EngineRef:
    """nv/engine.py:8-51."""

    def __init__(self, runner, scheduler):
        self.runner = runner
        self.scheduler = scheduler

    def step(self, eos):
        plan = self.scheduler.plan_next_step(eos)
        for seq in plan.finish_seqs:
            self.runner.free_seq(seq)
        done = list(plan.finish_seqs)
        if plan.prefill_seqs:
            self.runner.prefill(plan.prefill_seqs)
        if plan.decode_seqs:
            last = [s for s in plan.decode_seqs if len(s.generated_token_ids) + 1 >= s.max_new_tokens]
            rest = [s for s in plan.decode_seqs if len(s.generated_token_ids) + 1 < s.max_new_tokens]
            for seq in last:
                seq.append_next_token()
            ended = self.scheduler.finish_sequences(last, "max_new_tokens")
            for seq in ended:
                self.runner.free_seq(seq)
            done.extend(ended)
            if rest:
                self.runner.decode(rest)
        return done
