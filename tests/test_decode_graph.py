"""Decode graph runner state machine on the CPU with fake graph primitives (nv/npu/acl_graph.py behaviour)."""
from __future__ import annotations

import contextlib
import sys
import types
from types import SimpleNamespace

import pytest
import torch

from nano_vllm_ascend_amd.block_manager import PagedKVCacheMetadata
from nano_vllm_ascend_amd.graph import DecodeGraphRunner
from nano_vllm_ascend_amd.qwen3 import CausalLMOutput


class FakeGraph:
    def __init__(self):
        self.replays = 0

    def replay(self):
        self.replays += 1


class FakeModel:
    config = SimpleNamespace(num_attention_heads=2, num_key_value_heads=1)

    def __init__(self):
        self.calls = 0

    def __call__(self, **kw):
        self.calls += 1
        return CausalLMOutput(logits=torch.full((kw["input_ids_flat"].numel(), 8), float(self.calls)))


def make_runner(model, sizes):
    r = DecodeGraphRunner(model, kv_cache=SimpleNamespace(block_size=4), batch_sizes=sizes, max_model_len=16,
                          block_size=4)
    r.make_graph = FakeGraph
    r.graph_context = lambda g, pool: contextlib.nullcontext()
    r.synchronize = lambda: None
    return r


def metadata(b, width=2):
    return PagedKVCacheMetadata(block_tables=torch.zeros(b, width, dtype=torch.int32),
                                context_lens=torch.ones(b, dtype=torch.int32),
                                slot_mapping=torch.zeros(b, dtype=torch.int64))


def test_captures_once_then_replays():
    model = FakeModel()
    runner = make_runner(model, [1])
    first = runner.forward(torch.tensor([1]), torch.tensor([2]), metadata(1))
    second = runner.forward(torch.tensor([3]), torch.tensor([4]), metadata(1))
    assert first is second  # the static logits buffer
    assert model.calls == 2  # one eager warm-up run, one captured run
    stats = runner.stats_dict()
    assert (stats["captures"], stats["replays"], stats["updates"]) == (1, 2, 2)
    assert runner.entries[1].graph.replays == 2
    assert runner.entries[1].buffers["input_ids"].tolist() == [3]


def test_failed_capture_disables_only_that_batch_size():
    class FailingModel(FakeModel):
        def __call__(self, **kw):
            raise RuntimeError("capture failed")

    runner = make_runner(FailingModel(), [1, 2])
    assert runner.forward(torch.tensor([1]), torch.tensor([2]), metadata(1)) is None
    assert 1 in runner.disabled_batch_sizes and runner.supports(2) and not runner.supports(1)
    stats = runner.stats_dict()
    assert stats["capture_failures"] == 1 and stats["fallbacks"] == 1


def test_unsupported_size_falls_back_and_wide_tables_raise():
    runner = make_runner(FakeModel(), [1, 2])
    assert runner.forward(torch.tensor([1, 2, 3]), torch.tensor([1, 2, 3]), metadata(3)) is None
    assert runner.stats_dict()["fallbacks"] == 1
    with pytest.raises(RuntimeError):  # static width ceil(16 / 4) = 4 < 5
        runner.forward(torch.tensor([1, 2]), torch.tensor([1, 2]), metadata(2, width=5))


def test_default_graph_sizes_and_llm_passes_none(monkeypatch):
    from nano_vllm_ascend_amd import model_runner
    from nano_vllm_ascend_amd.engine import LLM

    assert model_runner.DEFAULT_DECODE_GRAPH_BATCH_SIZES == [1, 2, 4, 8, 16, 32]
    captured = {}

    class FakeModelRunner:
        def __init__(self, **kw):
            captured.update(kw)
            self.num_blocks = 16

    fake = types.ModuleType("nano_vllm_ascend_amd.model_runner")
    fake.ModelRunner = FakeModelRunner
    monkeypatch.setitem(sys.modules, "nano_vllm_ascend_amd.model_runner", fake)
    LLM("model", max_num_seqs=3, enable_decode_graph=True)
    assert captured["enable_decode_graph"] is True and captured["decode_graph_batch_sizes"] is None
