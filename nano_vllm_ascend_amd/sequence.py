"""Per-request state of the continuous-batching engine.

The model runner talks to a request through the attribute and method names of
nv/sequence.py:20-67 (the prefix-cache plan fields, ``set_prefill_result``,
``append_next_token``, ``set_decode_result``, ``cache_position``,
``next_token_id``, ``generated_token_ids``); those names are the interface.
The representation is this module's own:

  * a request moves WAITING -> RUNNING -> FINISHED (``status``);
  * after its prefill it always holds exactly one sampled token that is not
    yet part of its output (``next_token_id``, ``None`` before the prefill);
  * a decode step commits that token to the output, feeds it to the model at
    ``cache_position`` and receives the next one, so ``cache_position`` is
    derived, not stored: prompt_len + decode steps taken.
"""
from __future__ import annotations

from enum import Enum
from typing import Any


class SequenceStatus(str, Enum):
    WAITING = "waiting"
    RUNNING = "running"
    FINISHED = "finished"


class Sequence:
    __slots__ = (
        "seq_id", "prompt", "max_new_tokens", "prompt_token_ids", "sampling_params",
        "status", "finish_reason", "reserved_blocks",
        # prefix-cache plan, filled at submit time by the runner
        "estimated_prompt_len", "cached_prefix_len", "cached_block_ids", "runtime_prompt_token_ids",
        "runtime_prompt_len",
        # generation state
        "prompt_len", "generated_token_ids", "_pending", "_decode_steps",
    )

    def __init__(self, seq_id: int, prompt: str, max_new_tokens: int, prompt_token_ids: Any, sampling_params: Any):
        self.seq_id = seq_id
        self.prompt = prompt
        self.max_new_tokens = max_new_tokens
        self.prompt_token_ids = prompt_token_ids
        self.sampling_params = sampling_params
        self.status = SequenceStatus.WAITING
        self.finish_reason: str | None = None
        self.reserved_blocks = 0
        self.estimated_prompt_len = 0
        self.cached_prefix_len = 0
        self.cached_block_ids: list[int] = []
        self.runtime_prompt_token_ids = None
        self.runtime_prompt_len = 0
        self.prompt_len = 0
        self.generated_token_ids: list[int] = []
        self._pending: int | None = None
        self._decode_steps = 0

    def __repr__(self) -> str:
        return (f"Sequence(id={self.seq_id}, {self.status.value}, out={len(self.generated_token_ids)}"
                f"/{self.max_new_tokens}, pending={self._pending})")

    # ------------------------------------------------------------ derived
    @property
    def next_token_id(self) -> int | None:
        """The sampled token not yet committed to the output (None before the prefill)."""
        return self._pending

    @property
    def cache_position(self) -> int:
        """Position of the token the next decode step feeds: prompt_len + decode steps taken."""
        return self.prompt_len + self._decode_steps

    @property
    def tokens_left(self) -> int:
        """Output tokens still to commit, counting the pending one."""
        return self.max_new_tokens - len(self.generated_token_ids)

    def pending_is_last(self) -> bool:
        """Committing the pending token fills the output budget, so it needs no forward."""
        return self.tokens_left <= 1

    def reach_max_tokens(self) -> bool:
        return self.tokens_left <= 0

    # ------------------------------------------------------------ transitions
    def set_prefill_result(self, next_token_id: int, prompt_len: int) -> None:
        self.prompt_len = prompt_len
        self._decode_steps = 0
        self._pending = next_token_id

    def append_next_token(self) -> int:
        """Move the pending token into the output; return it."""
        token = self._pending
        if token is None:
            raise RuntimeError(f"seq {self.seq_id} has no next_token_id")
        self.generated_token_ids.append(token)
        return token

    def set_decode_result(self, next_token_id: int) -> None:
        self._decode_steps += 1
        self._pending = next_token_id

    def finish(self, reason: str | None = None) -> None:
        self.status = SequenceStatus.FINISHED
        self.finish_reason = reason
