"""Step-by-step admission traces of the engine (behaviour of tests/test_continuous_batching.py:74-148)."""
from __future__ import annotations

from nano_vllm_ascend_amd.engine import EngineCore, LLM
from nano_vllm_ascend_amd.scheduler import MiniScheduler


class FakeTokenIds:
    def __init__(self, values):
        self.values = values

    def numel(self):
        return len(self.values)


class FakeTokenizer:
    eos_token_id = -1

    def decode(self, token_ids, skip_special_tokens=True):
        return ",".join(str(t) for t in token_ids)


class FakeRunner:
    def __init__(self):
        self.tokenizer = FakeTokenizer()
        self.prefilled, self.decoded, self.freed = [], [], []

    def tokenize_prompts(self, prompts):
        return [FakeTokenIds(list(range(1, len(p) + 1))) for p in prompts]

    def prepare_sequences(self, seqs):
        for seq in seqs:
            seq.estimated_prompt_len = seq.prompt_token_ids.numel()
            seq.runtime_prompt_len = seq.estimated_prompt_len

    def prefill(self, seqs):
        for seq in seqs:
            self.prefilled.append(seq.seq_id)
            seq.set_prefill_result(seq.seq_id * 10, seq.estimated_prompt_len)

    def decode(self, seqs):
        for seq in seqs:
            self.decoded.append(seq.seq_id)
            seq.set_decode_result(seq.append_next_token() + 1)

    def free_seq(self, seq):
        self.freed.append(seq.seq_id)


def make_llm(max_num_seqs=2, total_blocks=16):
    llm = object.__new__(LLM)
    llm.runner = FakeRunner()
    llm.scheduler = MiniScheduler(max_num_seqs=max_num_seqs, block_size=4, total_num_blocks=total_blocks)
    llm.engine_core = EngineCore(llm.runner, llm.scheduler)
    return llm


def test_submit_adds_request_to_waiting_queue():
    llm = make_llm()
    assert llm.submit("hello", max_new_tokens=1) == 0
    assert [s.seq_id for s in llm.scheduler.waiting] == [0]
    assert llm.has_unfinished()


def test_later_request_admitted_after_capacity_frees():
    llm = make_llm(max_num_seqs=1)
    first = llm.submit("first", max_new_tokens=2)
    assert llm.step() == []
    second = llm.submit("second", max_new_tokens=1)
    assert llm.runner.prefilled == [first]
    assert [s.seq_id for s in llm.scheduler.waiting] == [second]
    assert llm.step() == []
    assert [o["request_id"] for o in llm.step()] == [first]
    assert llm.runner.prefilled == [first]
    assert llm.step() == []
    assert [o["request_id"] for o in llm.step()] == [second]
    assert llm.runner.prefilled == [first, second]


def test_later_request_runs_with_available_capacity():
    llm = make_llm(max_num_seqs=2)
    first = llm.submit("first", max_new_tokens=3)
    assert llm.step() == []
    second = llm.submit("second", max_new_tokens=2)
    assert list(llm.scheduler.running) == [first]
    assert [s.seq_id for s in llm.scheduler.waiting] == [second]
    assert llm.step() == []
    assert list(llm.scheduler.running) == [first, second]
    assert list(llm.scheduler.waiting) == []
    assert llm.runner.prefilled == [first, second]


def test_admission_after_several_decode_steps():
    llm = make_llm(max_num_seqs=2)
    first = llm.submit("first", max_new_tokens=5)
    for _ in range(3):
        assert llm.step() == []
    second = llm.submit("second", max_new_tokens=2)
    assert list(llm.scheduler.running) == [first]
    assert len(llm.scheduler.seqs[first].generated_token_ids) == 2
    assert llm.step() == []
    assert list(llm.scheduler.running) == [first, second]
    assert llm.runner.prefilled == [first, second]


def test_generate_keeps_output_shape_and_order():
    llm = make_llm()
    assert llm.generate(["a", "bb"], max_new_tokens=1) == [
        {"texts": "0", "token_ids": [0]},
        {"texts": "10", "token_ids": [10]},
    ]


def test_final_token_committed_without_forward():
    """A request runs max_new_tokens - 1 decode forwards (nv/engine.py:35-48)."""
    llm = make_llm()
    out = llm.generate(["abc"], max_new_tokens=4)
    assert out[0]["token_ids"] == [0, 1, 2, 3]
    assert llm.runner.decoded == [0, 0, 0]  # 3 = max_new_tokens - 1 decode forwards


def test_request_larger_than_pool_is_aborted():
    llm = make_llm(max_num_seqs=2, total_blocks=2)
    rid = llm.submit("x" * 20, max_new_tokens=4)  # needs ceil(24/4) = 6 blocks
    outs = llm.step()
    assert [o["request_id"] for o in outs] == [rid]
    assert llm.scheduler.finished[rid].finish_reason == "aborted_no_capacity"
    assert not llm.has_unfinished()


def test_eos_finishes_sequence():
    llm = make_llm()
    llm.runner.tokenizer.eos_token_id = 11
    rid = llm.submit("ab", max_new_tokens=10)
    llm.submit("cd", max_new_tokens=3)
    while llm.has_unfinished():
        llm.step()
    assert llm.scheduler.finished[rid].finish_reason == "max_new_tokens"
    assert llm.scheduler.finished[1].finish_reason == "eos"  # 10 -> 11 == eos
    assert llm.scheduler.finished[1].generated_token_ids == [10]
