"""Per-request state (nv/sequence.py:14-67).

Packing reads ``cached_prefix_len``, ``cached_block_ids``,
``runtime_prompt_token_ids/len``, ``cache_position`` and ``next_token_id``.
The position of the token fed to a decode step is ``cache_position`` =
prompt_len + number of decode steps already run.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from enum import Enum
from typing import Any


class SequenceStatus(str, Enum):
    WAITING = "waiting"
    RUNNING = "running"
    FINISHED = "finished"


@dataclass
class Sequence:
    seq_id: int
    prompt: str
    max_new_tokens: int
    prompt_token_ids: Any  # 1-D int tensor or list of token ids
    sampling_params: Any

    status: SequenceStatus = SequenceStatus.WAITING
    estimated_prompt_len: int = 0
    reserved_blocks: int = 0
    finish_reason: str | None = None
    cached_prefix_len: int = 0
    cached_block_ids: list[int] = field(default_factory=list)
    runtime_prompt_token_ids: Any = None
    runtime_prompt_len: int = 0

    # set by prefill
    prompt_len: int = 0
    cache_position: int = 0
    next_token_id: int | None = None

    # generated tokens only (no prompt tokens)
    generated_token_ids: list[int] = field(default_factory=list)

    def set_prefill_result(self, next_token_id: int, prompt_len: int) -> None:
        self.next_token_id = next_token_id
        self.prompt_len = prompt_len
        self.cache_position = prompt_len

    def append_next_token(self) -> int:
        """Commit the pending sampled token to the output and return it."""
        if self.next_token_id is None:
            raise RuntimeError(f"seq {self.seq_id} has no next_token_id")
        self.generated_token_ids.append(self.next_token_id)
        return self.next_token_id

    def set_decode_result(self, next_token_id: int) -> None:
        self.next_token_id = next_token_id
        self.cache_position += 1

    def reach_max_tokens(self) -> bool:
        return len(self.generated_token_ids) >= self.max_new_tokens

    def finish(self, reason: str | None = None) -> None:
        self.status = SequenceStatus.FINISHED
        self.finish_reason = reason
