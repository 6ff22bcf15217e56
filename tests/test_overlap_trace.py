"""Overlapped decode keeps the reference's block allocation order (CPU).

1. The oracle engine (oracle/engine_ref.py) with the oracle block manager
   reproduces every golden trace written from the reference's own classes,
   including the 128-token-block scenarios with mid-run admissions and EOS;
   a planted ordering mistake is caught.
2. The block manager's decode-ahead API: packing a step ahead leaves the pool
   untouched, a confirmed step allocates exactly the blocks it packed, and the
   advisor's scenario (a boundary crossing while another request is admitted)
   gives the reference's blocks.
3. The product ModelRunner with overlap on, driven by the product engine over
   a fake model that stores every fed token in a fake KV cache at its slot and
   samples from the whole cached context read back through the block table:
   its metadata equals the oracle engine's replay of the same run, its tokens
   equal the synchronous loop's, and a continuation request after an EOS
   cannot pick up a stale step launched ahead.
"""
from __future__ import annotations

import json
import random
import sys
from pathlib import Path
from types import SimpleNamespace

import pytest
import torch

from nano_vllm_ascend_amd import _C
from nano_vllm_ascend_amd.engine import LLM, EngineCore
from nano_vllm_ascend_amd.graph import DecodeGraphRunner
from nano_vllm_ascend_amd.model_runner import ModelRunner
from nano_vllm_ascend_amd.qwen3 import CausalLMOutput
from nano_vllm_ascend_amd.scheduler import MiniScheduler
from oracle.block_manager_ref import BlockManagerRef
from oracle.engine_ref import EngineRef

GOLDEN = Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(GOLDEN))
import trace_driver  # noqa: E402
from host_pack import HostPackedBlockManager  # noqa: E402
from trace_check import ORACLE, assert_same_metadata, make_schedule, oracle_replay, run_product  # noqa: E402


# ---------------------------------------------------------------- 1. oracle engine vs golden traces
@pytest.mark.parametrize("name", sorted(trace_driver.SCENARIOS))
def test_oracle_engine_reproduces_golden_trace(name):
    golden = json.loads((GOLDEN / "block_traces.json").read_text())[name]
    got = json.loads(json.dumps(trace_driver.run_scenario(name, **ORACLE)))
    assert len(got) == len(golden)
    for i, (g, r) in enumerate(zip(got, golden)):
        assert g == r, f"{name}: event {i} differs\n got {g}\n ref {r}"


def test_golden_scenarios_cover_eos_admissions_and_boundaries():
    golden = json.loads((GOLDEN / "block_traces.json").read_text())
    for name in ("bs128_prefix_eos", "bs128_tight_eos"):
        ev = golden[name]
        assert "eos" in ev[-1]["finish_reasons"].values()
        decodes = [e for e in ev if e["event"] == "decode"]
        assert any(p % 128 == 0 for e in decodes for p in e["start_positions"])  # a step opens a new block
        prefills = [e for e in ev if e["event"] == "prefill"]
        first_decode = next(i for i, e in enumerate(ev) if e["event"] == "decode")
        assert any(ev.index(p) > first_decode for p in prefills)  # admissions while others decode


class _DecodeFirstEngine(EngineRef):
    """Planted mistake: allocates the decode batch's blocks before the admitted requests'
    prefill (the order a step launched ahead used to impose)."""

    def step(self, eos):
        plan = self.scheduler.plan_next_step(eos)
        for seq in plan.finish_seqs:
            self.runner.free_seq(seq)
        last = [s for s in plan.decode_seqs if len(s.generated_token_ids) + 1 >= s.max_new_tokens]
        rest = [s for s in plan.decode_seqs if len(s.generated_token_ids) + 1 < s.max_new_tokens]
        if rest:
            self.runner.decode(rest)
        if plan.prefill_seqs:
            self.runner.prefill(plan.prefill_seqs)
        for seq in last:
            seq.append_next_token()
        ended = self.scheduler.finish_sequences(last, "max_new_tokens")
        for seq in ended:
            self.runner.free_seq(seq)
        return list(plan.finish_seqs) + ended


def test_planted_engine_order_mistake_is_caught():
    golden = json.loads((GOLDEN / "block_traces.json").read_text())
    differs = []
    for name in sorted(trace_driver.SCENARIOS):
        got = json.loads(json.dumps(trace_driver.run_scenario(name, **{**ORACLE, "EngineCore": _DecodeFirstEngine})))
        differs.append(got != golden[name])
    assert sum(differs) >= 3, differs


# ---------------------------------------------------------------- 2. decode-ahead API of the block manager
def _pool_state(bm):
    return (list(bm.free_block_ids), {s: list(t) for s, t in bm.block_tables.items()}, dict(bm.seq_lens),
            [b.ref_count for b in bm.blocks], [b.block_hash for b in bm.blocks])


def test_decode_ahead_leaves_pool_untouched_and_commit_takes_the_packed_blocks():
    bm = HostPackedBlockManager(num_blocks=12, block_size=4, device="cpu")
    bm.prepare_prefill_metadata(slots=[0, 1, 2], seq_lens=[4, 6, 8], start_positions=[0, 0, 0],
                                prefix_block_ids=[[], [], []])
    before = _pool_state(bm)
    md, taken = bm.prepare_decode_ahead([0, 1, 2], [4, 6, 8], token_ids=[7, 8, 9], width=6)
    assert _pool_state(bm) == before
    assert taken == [(0, 5), (2, 6)]  # slots 0 and 2 open a block, in batch order: the free-queue front
    assert md.block_tables.tolist() == [[0, 5, 0, 0, 0, 0], [1, 2, 0, 0, 0, 0], [3, 4, 6, 0, 0, 0]]
    assert md.slot_mapping.tolist() == [20, 10, 24] and md.context_lens.tolist() == [5, 7, 9]
    ref = HostPackedBlockManager(num_blocks=12, block_size=4, device="cpu")
    ref.prepare_prefill_metadata(slots=[0, 1, 2], seq_lens=[4, 6, 8], start_positions=[0, 0, 0],
                                 prefix_block_ids=[[], [], []])
    want = ref.prepare_decode_metadata([0, 1, 2], [4, 6, 8], 1)
    bm.commit_decode_ahead([0, 1, 2], [4, 6, 8], taken)
    assert _pool_state(bm) == _pool_state(ref)
    assert want.block_tables.tolist() == [r[:3] for r in md.block_tables.tolist()]


def test_decode_ahead_refuses_blocks_that_carry_a_prefix_key():
    bm = HostPackedBlockManager(num_blocks=4, block_size=4, device="cpu")
    toks = torch.arange(8)
    bm.prepare_prefill_metadata(slots=[0], seq_lens=[8], start_positions=[0], prefix_block_ids=[[]])
    bm.cache_full_blocks(slot=0, token_ids=toks)
    bm.free_slot(0)  # blocks 1, 0 go back to the queue with their keys: [2, 3, 1, 0]
    bm.prepare_prefill_metadata(slots=[1], seq_lens=[4], start_positions=[0], prefix_block_ids=[[]])
    bm.prepare_prefill_metadata(slots=[2], seq_lens=[4], start_positions=[0], prefix_block_ids=[[]])
    assert bm.free_block_ids == [1, 0]
    assert bm.peek_decode_blocks([1], [4]) is None  # block 1 holds cached content
    assert bm.prepare_decode_ahead([1], [4], token_ids=[5]) is None
    assert bm.peek_decode_blocks([1], [3]) == []  # no new block needed


def test_reference_order_when_an_admission_lands_between():
    """A crosses into a new block while C is admitted: the reference prefills C first."""
    def run(cls, ahead):
        bm = cls(num_blocks=8, block_size=4) if cls is BlockManagerRef else cls(num_blocks=8, block_size=4,
                                                                              device="cpu")
        bm.prepare_prefill_metadata(slots=[0, 1], seq_lens=[8, 3], start_positions=[0, 0], prefix_block_ids=[[], []])
        if ahead:  # the product packs A's and B's next step ahead ...
            assert bm.prepare_decode_ahead([0, 1], [8, 3], token_ids=[1, 2]) is not None
        # ... but the next engine step admits C: the launched step is dropped unapplied
        bm.prepare_prefill_metadata(slots=[2], seq_lens=[5], start_positions=[0], prefix_block_ids=[[]])
        md = bm.prepare_decode_metadata([0, 1], [8, 3], 1)
        return md.block_tables.tolist(), md.slot_mapping.tolist(), {s: list(t) for s, t in bm.block_tables.items()}

    ref = run(BlockManagerRef, False)
    assert run(HostPackedBlockManager, True) == ref
    assert ref[2][0] == [0, 1, 5] and ref[2][2] == [3, 4]


# ---------------------------------------------------------------- 3. product runner with overlap
VOCAB = 509


def _fold(tokens) -> int:
    h = 17
    for t in tokens:
        h = (h * 1000003 + int(t) + 1) % 2147483647
    return h % VOCAB


class FakeKVModel:
    """Stores each fed token at its slot; samples from the cached context read through the block table."""

    config = SimpleNamespace(num_attention_heads=2, num_key_value_heads=1)

    def __init__(self, block_size: int):
        self.bs = block_size
        self.cache: dict[int, int] = {}

    def __call__(self, input_ids_flat, position_ids_flat, kv_cache, attn_metadata, is_prefill, logits_indices=None):
        md = attn_metadata
        for tok, slot in zip(input_ids_flat.tolist(), md.slot_mapping.tolist()):
            self.cache[slot] = tok
        bt = md.block_tables.tolist()
        rows = []
        for i, ctx in enumerate(md.context_lens.tolist()):
            rows.append(_fold(self.cache[bt[i][p // self.bs] * self.bs + p % self.bs] for p in range(ctx)))
        logits = torch.zeros(len(rows), VOCAB)
        logits[torch.arange(len(rows)), torch.tensor(rows, dtype=torch.long)] = 1.0
        return CausalLMOutput(logits=logits)


class LiveGraphRunner(DecodeGraphRunner):
    """A graph whose replay reruns the fake model on the static buffers (argmax into greedy_ids)."""

    def _capture(self, entry):
        entry.graph = True
        entry.logits = torch.zeros(entry.batch_size, VOCAB)
        self.stats.captures += 1
        return True

    def replay(self, entry):
        if entry.graph is None:
            self._capture(entry)
        b = entry.buffers
        out = self.model(input_ids_flat=b["input_ids"], position_ids_flat=b["positions"], kv_cache=None,
                         attn_metadata=entry.metadata, is_prefill=False)
        entry.logits.copy_(out.logits)
        b["greedy_ids"].copy_(out.logits.argmax(-1))
        self.stats.updates += 1
        self.stats.replays += 1
        return entry.logits


class HostErrorWord:
    """Stands in for the device's index-error word: a host flag that a test can raise."""

    pending = 0  # bits the next fetch will find

    def __init__(self):
        self.bits = 0

    def fetch(self):
        self.bits, HostErrorWord.pending = HostErrorWord.pending, 0

    def raise_if_set(self):
        if self.bits:
            bits, self.bits = self.bits, 0
            raise IndexError(f"index out of range in the step's kernels: {_C.describe_index_errors(bits)}")


def make_llm(monkeypatch, *, block_size, num_blocks, max_num_seqs, prefix, overlap, max_model_len=1024,
             sizes=(1, 2, 4, 8)) -> LLM:
    monkeypatch.setattr(_C, "argmax_rows", lambda logits, out=None: logits.argmax(-1))
    monkeypatch.setattr(_C, "alloc_paged_decode_workspace", lambda *a, **k: None)
    runner = object.__new__(ModelRunner)
    runner._init_step_state(overlap)
    runner.error_word_factory = HostErrorWord
    runner.device = torch.device("cpu")
    runner.block_size, runner.max_model_len = block_size, max_model_len
    runner.enable_prefix_cache, runner.enable_decode_graph = prefix, True
    runner.tokenizer = SimpleNamespace(eos_token_id=-1, decode=lambda ids, skip_special_tokens=True: "")
    runner.model = FakeKVModel(block_size)
    runner.num_blocks, runner.kv_cache = num_blocks, None
    runner.block_manager = HostPackedBlockManager(num_blocks=num_blocks, block_size=block_size, device="cpu")
    runner.decode_graph_runner = LiveGraphRunner(runner.model, None, list(sizes), max_model_len, block_size)
    runner._fetch_tokens = lambda b, ids: SimpleNamespace(tokens=ids.clone().tolist)
    llm = object.__new__(LLM)
    llm.runner = runner
    llm.scheduler = MiniScheduler(max_num_seqs=max_num_seqs, block_size=block_size, total_num_blocks=num_blocks)
    llm.engine_core = EngineCore(runner, llm.scheduler)
    runner.next_step_admits = llm.scheduler.head_fits
    return llm


CASES = {
    # 16-token blocks: many boundary crossings; shared prefix with the cache on; tight pool
    "bs16_prefix": dict(block_size=16, num_blocks=40, max_num_seqs=3, prefix=True, seed=21, n=10, len_lo=5,
                        len_hi=60, new_lo=4, new_hi=70, shared_blocks=2),
    # the product's 128-token blocks, prefix cache off
    "bs128": dict(block_size=128, num_blocks=14, max_num_seqs=4, prefix=False, seed=22, n=9, len_lo=100,
                  len_hi=260, new_lo=10, new_hi=160, shared_blocks=0),
    # 128-token blocks, shared 2-block prefix, cache on
    "bs128_prefix": dict(block_size=128, num_blocks=30, max_num_seqs=4, prefix=True, seed=23, n=10, len_lo=60,
                         len_hi=200, new_lo=10, new_hi=150, shared_blocks=2),
}


@pytest.mark.parametrize("case", sorted(CASES))
def test_overlapped_runner_metadata_equals_oracle_replay(monkeypatch, case):
    c = CASES[case]
    cfg = dict(block_size=c["block_size"], num_blocks=c["num_blocks"], max_num_seqs=c["max_num_seqs"],
               prefix=c["prefix"])
    schedule = make_schedule(c["seed"], c["n"], c["block_size"], c["len_lo"], c["len_hi"], c["new_lo"], c["new_hi"],
                             c["shared_blocks"])
    # an EOS token that some requests sample mid-run: taken from a run without EOS
    _, plain, _ = run_product(make_llm(monkeypatch, overlap=False, **cfg), schedule, -1)
    eos = plain[1][len(plain[1]) // 2]
    sync_events, sync_out, sync_reasons = run_product(make_llm(monkeypatch, overlap=False, **cfg), schedule, eos)
    llm = make_llm(monkeypatch, overlap=True, **cfg)
    events, out, reasons = run_product(llm, schedule, eos)
    assert out == sync_out and reasons == sync_reasons
    assert "eos" in reasons.values()
    stats = llm.runner.overlap_stats
    assert stats["launched"] > 0 and stats["used"] > 0, stats
    if case == "bs128":  # EOS found while the next step was in flight: launches were discarded
        assert stats["discarded"] > 0, stats
    ref = oracle_replay(schedule, out, reasons, eos, **cfg)
    assert_same_metadata(sync_events, ref)
    assert_same_metadata(events, ref)


def _dry_pool_run(schedule, cfg, monkeypatch):
    """Run a schedule on which the reference's reservation over-commits the pool: the oracle and
    both product loops must raise the same error after the same packing metadata.

    The reference reserves blocks for the uncached prompt suffix plus the output budget only
    (src/nanovllm_ascend/engine.py:161-164), while a prefix hit takes its cached blocks off the
    free queue, so a tight pool can run dry in a later decode."""
    ref_events = []
    with pytest.raises(RuntimeError, match="out of free blocks"):
        trace_driver.run_schedule(schedule, lambda seq_id, n: 1, -1, block_size=cfg["block_size"],
                                  num_blocks=cfg["num_blocks"], max_num_seqs=cfg["max_num_seqs"],
                                  prefix_cache=cfg["prefix"], events=ref_events, **ORACLE)
    ref = [e for e in ref_events if e["event"] in ("prefill", "decode")]
    for overlap in (False, True):
        events = []
        with pytest.raises(RuntimeError, match="out of free blocks"):
            run_product(make_llm(monkeypatch, overlap=overlap, **cfg), schedule, -1, events=events)
        assert_same_metadata(events, ref)


@pytest.mark.parametrize("seed", range(16))
def test_overlapped_runner_random_schedules_equal_oracle_replay(monkeypatch, seed):
    """Seeded random configurations (block size, a tight pool, slots, prefix cache, arrivals,
    lengths, shared prefixes, an EOS token): the overlapped runner's tokens and every step's
    packing metadata equal the synchronous loop's and the oracle's replay of the same run.
    Where the reference's own accounting runs the pool dry (seed 10), all three raise alike."""
    rng = random.Random(1000 + seed)
    bs = rng.choice([16, 32, 128])
    n = rng.randint(5, 12)
    len_hi = rng.randint(bs // 2, 3 * bs)
    new_hi = rng.randint(4, 2 * bs)
    shared = rng.choice([0, 1, 2])
    per_req = -(-(shared * bs + len_hi + new_hi) // bs)  # blocks of the largest request
    cfg = dict(block_size=bs, num_blocks=per_req + rng.randint(0, 3 * per_req), max_num_seqs=rng.randint(2, 6),
               prefix=rng.random() < 0.5)
    schedule = make_schedule(seed, n, bs, 1, len_hi, 1, new_hi, shared)
    try:  # without EOS, scheduling does not depend on the tokens
        trace_driver.run_schedule(schedule, lambda seq_id, n: 1, -1, block_size=bs, num_blocks=cfg["num_blocks"],
                                  max_num_seqs=cfg["max_num_seqs"], prefix_cache=cfg["prefix"], **ORACLE)
    except RuntimeError as e:
        assert "out of free blocks" in str(e)
        _dry_pool_run(schedule, cfg, monkeypatch)
        return
    _, plain, _ = run_product(make_llm(monkeypatch, overlap=False, **cfg), schedule, -1)
    longest = max(plain.values(), key=len)
    eos = longest[len(longest) // 2] if len(longest) > 2 else -1
    sync_events, sync_out, sync_reasons = run_product(make_llm(monkeypatch, overlap=False, **cfg), schedule, eos)
    llm = make_llm(monkeypatch, overlap=True, **cfg)
    events, out, reasons = run_product(llm, schedule, eos)
    assert out == sync_out and reasons == sync_reasons
    ref = oracle_replay(schedule, out, reasons, eos, **cfg)
    assert_same_metadata(sync_events, ref)
    assert_same_metadata(events, ref)


def test_continuation_after_eos_does_not_take_a_stale_step(monkeypatch):
    """A request that stops on EOS while its next step is in flight, then a continuation request
    (prompt + response) in a new generate(): same tokens as the synchronous loop."""
    cfg = dict(block_size=16, num_blocks=32, max_num_seqs=2, prefix=False)
    prompt = list(range(3, 40))
    plain = make_llm(monkeypatch, overlap=False, **cfg)
    first = plain.generate([prompt], max_new_tokens=30)[0]["token_ids"]
    eos = first[12]
    results = {}
    for overlap in (False, True):
        llm = make_llm(monkeypatch, overlap=overlap, **cfg)
        llm.runner.tokenizer.eos_token_id = eos
        a = llm.generate([prompt], max_new_tokens=30)[0]["token_ids"]
        b = llm.generate([prompt + a], max_new_tokens=12)[0]["token_ids"]
        results[overlap] = (a, b, dict(llm.runner.overlap_stats))
    assert results[True][:2] == results[False][:2]
    assert results[True][2]["discarded"] > 0 and results[True][2]["launched"] > 0


def test_index_error_reported_by_the_kernels_raises_after_the_step(monkeypatch):
    """Where the reference's indexing raises, the kernels set a bit in the device's error word; the
    runner reads the word with the step's tokens and raises IndexError from that step, before its
    tokens are applied (eager sampling path: prefill and uncaptured decode)."""
    cfg = dict(block_size=16, num_blocks=40, max_num_seqs=2, prefix=False)
    llm = make_llm(monkeypatch, overlap=False, sizes=(), **cfg)
    ids = [llm.submit(list(range(20)), max_new_tokens=6), llm.submit(list(range(5, 40)), max_new_tokens=6)]
    llm.step()  # prefill: clean
    llm.step()  # decode: clean
    seqs = [llm.scheduler.seqs[i] for i in ids]
    # a decode step first commits each sequence's pending token, then runs the forward that samples
    # the next one
    committed = [list(s.generated_token_ids) + [s.next_token_id] for s in seqs]
    HostErrorWord.pending = _C.ERR_SLOT  # the next step's kernels skip an out-of-range slot
    with pytest.raises(IndexError, match="slot_mapping entry outside the KV cache"):
        llm.step()
    # the failed forward's tokens were not taken
    assert [list(s.generated_token_ids) for s in seqs] == committed
    assert all(s.next_token_id is None or s.next_token_id == c[-1] for s, c in zip(seqs, committed))


def test_index_error_bits_are_described():
    assert "RoPE table" in _C.describe_index_errors(_C.ERR_POSITION)
    text = _C.describe_index_errors(_C.ERR_CONTEXT | _C.ERR_BLOCK | 64)
    assert "block-table row" in text and "block pool" in text and "unknown bits 0x40" in text
