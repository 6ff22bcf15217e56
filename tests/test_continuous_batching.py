"""Engine and scheduler behaviour on the CPU with a scripted runner.

The expected values are the reference's known answers for admission, output
order, final-token commits and EOS (tests/test_continuous_batching.py:74-148
of the reference): a prefill samples 10 * seq_id and every decode step
samples the token it was fed plus one.
"""
from __future__ import annotations

from types import SimpleNamespace

import torch

from nano_vllm_ascend_amd.engine import LLM, EngineCore
from nano_vllm_ascend_amd.scheduler import MiniScheduler


class ScriptedRunner:
    """Records every runner call as (kind, seq_id); tokens follow the rule in the module docstring."""

    def __init__(self):
        self.tokenizer = SimpleNamespace(eos_token_id=-1,
                                         decode=lambda ids, skip_special_tokens=True: ",".join(map(str, ids)))
        self.calls: list[tuple[str, int]] = []

    def ids(self, kind: str) -> list[int]:
        return [seq_id for k, seq_id in self.calls if k == kind]

    def tokenize_prompts(self, prompts):
        return [torch.arange(1, len(p) + 1) for p in prompts]

    def prepare_sequences(self, seqs):
        for seq in seqs:
            seq.estimated_prompt_len = seq.runtime_prompt_len = int(seq.prompt_token_ids.numel())

    def prefill(self, seqs):
        for seq in seqs:
            self.calls.append(("prefill", seq.seq_id))
            seq.set_prefill_result(10 * seq.seq_id, seq.estimated_prompt_len)

    def decode(self, seqs):
        for seq in seqs:
            self.calls.append(("decode", seq.seq_id))
            seq.set_decode_result(seq.append_next_token() + 1)

    def free_seq(self, seq):
        self.calls.append(("free", seq.seq_id))


def engine(max_num_seqs=2, total_blocks=16) -> LLM:
    llm = object.__new__(LLM)  # the public API over a scripted runner; no device
    llm.runner = ScriptedRunner()
    llm.scheduler = MiniScheduler(max_num_seqs=max_num_seqs, block_size=4, total_num_blocks=total_blocks)
    llm.engine_core = EngineCore(llm.runner, llm.scheduler)
    return llm


def waiting(llm):
    return [seq.seq_id for seq in llm.scheduler.waiting]


def test_submit_queues_the_request():
    llm = engine()
    assert llm.submit("hello", max_new_tokens=1) == 0
    assert waiting(llm) == [0] and llm.has_unfinished()


def test_request_admitted_once_a_slot_frees():
    llm = engine(max_num_seqs=1)
    a = llm.submit("first", max_new_tokens=2)
    assert llm.step() == []
    b = llm.submit("second", max_new_tokens=1)
    assert llm.runner.ids("prefill") == [a] and waiting(llm) == [b]
    assert llm.step() == []
    assert [o["request_id"] for o in llm.step()] == [a]
    assert llm.runner.ids("prefill") == [a]
    assert llm.step() == []
    assert [o["request_id"] for o in llm.step()] == [b]
    assert llm.runner.ids("prefill") == [a, b]


def test_request_joins_while_capacity_remains():
    llm = engine(max_num_seqs=2)
    a = llm.submit("first", max_new_tokens=3)
    assert llm.step() == []
    b = llm.submit("second", max_new_tokens=2)
    assert list(llm.scheduler.running) == [a] and waiting(llm) == [b]
    assert llm.step() == []
    assert list(llm.scheduler.running) == [a, b] and waiting(llm) == []
    assert llm.runner.ids("prefill") == [a, b]


def test_admission_after_several_decode_steps():
    llm = engine(max_num_seqs=2)
    a = llm.submit("first", max_new_tokens=5)
    for _ in range(3):
        assert llm.step() == []
    b = llm.submit("second", max_new_tokens=2)
    assert list(llm.scheduler.running) == [a]
    assert len(llm.scheduler.seqs[a].generated_token_ids) == 2
    assert llm.step() == []
    assert list(llm.scheduler.running) == [a, b]
    assert llm.runner.ids("prefill") == [a, b]


def test_generate_returns_outputs_in_prompt_order():
    assert engine().generate(["a", "bb"], max_new_tokens=1) == [
        {"texts": "0", "token_ids": [0]},
        {"texts": "10", "token_ids": [10]},
    ]


def test_last_token_is_committed_without_a_forward():
    """A request runs max_new_tokens - 1 decode forwards (nv/engine.py:35-48)."""
    llm = engine()
    assert llm.generate(["abc"], max_new_tokens=4)[0]["token_ids"] == [0, 1, 2, 3]
    assert llm.runner.ids("decode") == [0, 0, 0]


def test_one_step_frees_then_prefills_then_commits_then_decodes():
    llm = engine(max_num_seqs=3)
    llm.submit("aa", max_new_tokens=1)   # 0: prefill, then its last token at the second step
    llm.submit("bb", max_new_tokens=5)   # 1: decodes at the second step
    llm.step()
    llm.submit("cc", max_new_tokens=3)   # 2: admitted at the second step
    llm.runner.calls.clear()
    assert [o["request_id"] for o in llm.step()] == [0]
    assert llm.runner.calls == [("prefill", 2), ("free", 0), ("decode", 1)]


def test_request_larger_than_the_pool_is_aborted():
    llm = engine(max_num_seqs=2, total_blocks=2)
    rid = llm.submit("x" * 20, max_new_tokens=4)  # needs ceil(24 / 4) = 6 blocks
    assert [o["request_id"] for o in llm.step()] == [rid]
    assert llm.scheduler.finished[rid].finish_reason == "aborted_no_capacity"
    assert not llm.has_unfinished()


def test_eos_finishes_a_request():
    llm = engine()
    llm.runner.tokenizer.eos_token_id = 11
    a = llm.submit("ab", max_new_tokens=10)
    b = llm.submit("cd", max_new_tokens=3)
    while llm.has_unfinished():
        llm.step()
    assert llm.scheduler.finished[a].finish_reason == "max_new_tokens"
    assert llm.scheduler.finished[b].finish_reason == "eos"  # 10 -> 11 == eos
    assert llm.scheduler.finished[b].generated_token_ids == [10]


def test_reservations_bound_admission_and_return_on_finish():
    llm = engine(max_num_seqs=4, total_blocks=5)
    a = llm.submit("abcdef", max_new_tokens=6)  # 3 blocks
    b = llm.submit("ab", max_new_tokens=6)      # 2 blocks
    c = llm.submit("a", max_new_tokens=3)       # 1 block: waits, 3 + 2 + 1 > 5
    llm.step()
    assert list(llm.scheduler.running) == [a, b] and waiting(llm) == [c]
    assert llm.scheduler.reserved_blocks_total == 5
    while c not in llm.scheduler.running:
        llm.step()
    assert a not in llm.scheduler.running or b not in llm.scheduler.running
