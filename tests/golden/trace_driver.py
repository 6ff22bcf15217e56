"""Deterministic continuous-batching traces of the block manager + scheduler.

Drives an engine (EngineCore + MiniScheduler + Sequence) with a fake model
runner whose bookkeeping restates nv/model_runner.py:146-167 (prefix lookup at
submit time), :199-238 (prefill: metadata, sampled token, cache_full_blocks)
and :240-286 (decode: append token, metadata at cache_position, new token).
Sampled tokens are a fixed function of (seq_id, tokens generated); in the
scenarios with EOS, a seeded subset of requests samples EOS_TOKEN after a
seeded number of tokens.  A scenario is fully deterministic.

``run_schedule`` drives the same engine from a submission schedule and a
recorded token stream instead (it replays a run of the product on the GPU).

Every metadata call is recorded (slots, lengths, block tables, context lens,
slot mapping, cumulative lengths, paged-prefill flag), with the prefix lookup
of each submit and the final free queue.  The same driver runs the reference's
classes (tests/golden/make_block_traces.py, in the development container
only) and this repository's classes (tests/test_block_trace.py).
"""
from __future__ import annotations

import random


EOS_TOKEN = 1000  # outside next_token's range [0, 997)


def next_token(seq_id: int, n_generated: int) -> int:
    return (seq_id * 7919 + n_generated * 104729) % 997


def eos_token_fn(eos_at: dict[int, int]):
    """next_token, except that request ``s`` samples EOS_TOKEN as its token number eos_at[s]."""

    def fn(seq_id: int, n_generated: int) -> int:
        if eos_at.get(seq_id) == n_generated:
            return EOS_TOKEN
        return next_token(seq_id, n_generated)

    return fn


class FakeTokenizer:
    eos_token_id = -1

    def decode(self, token_ids, skip_special_tokens=True):
        return ",".join(str(t) for t in token_ids)


def _as_list(x):
    if x is None:
        return None
    if hasattr(x, "tolist"):
        return x.tolist()
    return list(x)


class TraceRunner:
    """Fake runner over a real BlockManager; `metadata_hook` sees every metadata object."""

    def __init__(self, block_manager, block_size: int, enable_prefix_cache: bool, torch_mod, record,
                 token_fn=next_token):
        self.token_fn = token_fn
        self.block_manager = block_manager
        self.block_size = block_size
        self.enable_prefix_cache = enable_prefix_cache
        self.torch = torch_mod
        self.tokenizer = FakeTokenizer()
        self.record = record

    def tokenize_prompts(self, prompts):
        return [self.torch.tensor(p, dtype=self.torch.long) for p in prompts]

    def prepare_sequences(self, seqs):
        bs = self.block_size
        for seq in seqs:
            seq.estimated_prompt_len = int(seq.prompt_token_ids.numel())
            seq.cached_block_ids = []
            seq.cached_prefix_len = 0
            if self.enable_prefix_cache:
                max_blocks = seq.estimated_prompt_len // bs
                if seq.estimated_prompt_len % bs == 0 and max_blocks > 0:
                    max_blocks -= 1
                if max_blocks > 0:
                    seq.cached_block_ids = self.block_manager.find_longest_prefix_blocks(
                        seq.prompt_token_ids, max_cache_blocks=max_blocks)
                    seq.cached_prefix_len = len(seq.cached_block_ids) * bs
            seq.runtime_prompt_token_ids = seq.prompt_token_ids[seq.cached_prefix_len:]
            seq.runtime_prompt_len = int(seq.runtime_prompt_token_ids.numel())
            if seq.runtime_prompt_len <= 0:
                raise ValueError(f"seq {seq.seq_id} has empty runtime prompt suffix")
            self.record({"event": "submit", "seq": seq.seq_id, "cached_block_ids": list(seq.cached_block_ids)})

    def _log(self, kind, slots, md, extra):
        self.record({
            "event": kind,
            "slots": list(slots),
            **extra,
            "block_tables": _as_list(md.block_tables),
            "context_lens": _as_list(md.context_lens),
            "slot_mapping": _as_list(md.slot_mapping),
            "actual_seq_lengths_q": md.actual_seq_lengths_q,
            "actual_seq_lengths_kv": md.actual_seq_lengths_kv,
            "use_paged_prefill": bool(md.use_paged_prefill),
        })

    def prefill(self, seqs):
        if not seqs:
            return
        slots = [s.seq_id for s in seqs]
        lens = [s.runtime_prompt_len for s in seqs]
        starts = [s.cached_prefix_len for s in seqs]
        md = self.block_manager.prepare_prefill_metadata(
            slots=slots, seq_lens=lens, start_positions=starts, prefix_block_ids=[s.cached_block_ids for s in seqs])
        self._log("prefill", slots, md, {"seq_lens": lens, "start_positions": starts})
        for seq in seqs:
            seq.set_prefill_result(next_token_id=self.token_fn(seq.seq_id, 0), prompt_len=seq.estimated_prompt_len)
            if self.enable_prefix_cache:
                self.block_manager.cache_full_blocks(
                    slot=seq.seq_id, token_ids=seq.prompt_token_ids, num_cached_blocks=len(seq.cached_block_ids),
                    num_full_blocks=seq.estimated_prompt_len // self.block_size)

    def decode(self, seqs):
        if not seqs:
            return
        for seq in seqs:
            seq.append_next_token()
        positions = [s.cache_position for s in seqs]
        slots = [s.seq_id for s in seqs]
        md = self.block_manager.prepare_decode_metadata(slots=slots, start_positions=positions, q_len=1)
        self._log("decode", slots, md, {"start_positions": positions})
        for seq in seqs:
            seq.set_decode_result(self.token_fn(seq.seq_id, len(seq.generated_token_ids)))

    def free_seq(self, seq):
        self.block_manager.free_slot(seq.seq_id)


SCENARIOS = {
    # small pages, shared prefixes, prefix cache on, requests arriving mid-run,
    # then a second wave that hits blocks cached by the first
    "prefix_small": dict(block_size=4, num_blocks=48, max_num_seqs=5, prefix_cache=True, seed=1, n_first=10,
                         n_second=8, len_lo=3, len_hi=22, new_lo=1, new_hi=9, shared=8),
    # tight pool: admission waits on reservations; lazy eviction recycles cached blocks
    "prefix_tight": dict(block_size=16, num_blocks=24, max_num_seqs=4, prefix_cache=True, seed=2, n_first=9,
                         n_second=6, len_lo=10, len_hi=70, new_lo=2, new_hi=30, shared=32),
    # prefix cache off
    "no_cache": dict(block_size=8, num_blocks=40, max_num_seqs=3, prefix_cache=False, seed=3, n_first=8,
                     n_second=0, len_lo=1, len_hi=40, new_lo=1, new_hi=20, shared=0),
    # the product's page size: 128-token blocks, a shared 2-block prefix, requests admitted
    # mid-run, and a third of the requests stopping on EOS (decode steps cross block
    # boundaries while others are admitted or finish)
    "bs128_prefix_eos": dict(block_size=128, num_blocks=36, max_num_seqs=4, prefix_cache=True, seed=4, n_first=8,
                             n_second=4, len_lo=90, len_hi=330, new_lo=8, new_hi=140, shared=256, eos_frac=0.34),
    # 128-token blocks, prefix cache off, a pool tight enough that admission waits on reservations
    "bs128_tight_eos": dict(block_size=128, num_blocks=12, max_num_seqs=3, prefix_cache=False, seed=9, n_first=9,
                            n_second=0, len_lo=100, len_hi=300, new_lo=20, new_hi=150, shared=0, eos_frac=0.34),
}


def make_eos_at(cfg, prompts) -> dict[int, int]:
    """Seeded EOS schedule of a scenario: request i samples EOS as token number eos_at[i]."""
    frac = cfg.get("eos_frac", 0.0)
    if not frac:
        return {}
    rng = random.Random(cfg["seed"] + 1000)
    eos_at = {}
    for i, (_, max_new) in enumerate(prompts):
        if max_new >= 3 and rng.random() < frac:
            eos_at[i] = rng.randint(1, max_new - 2)
    return eos_at


def make_prompts(cfg):
    rng = random.Random(cfg["seed"])
    shared = [rng.randint(0, 500) for _ in range(cfg["shared"])]
    prompts = []
    for i in range(cfg["n_first"] + cfg["n_second"]):
        n = rng.randint(cfg["len_lo"], cfg["len_hi"])
        body = [rng.randint(0, 500) for _ in range(n)]
        p = shared + body if (shared and i % 2 == 0) else body
        prompts.append((p, rng.randint(cfg["new_lo"], cfg["new_hi"])))
    return prompts


def run_scenario(name, *, BlockManager, MiniScheduler, EngineCore, Sequence, SamplingParams, torch_mod,
                 device="cpu", metadata_hook=None):
    """Run one scenario with the given classes; return the list of recorded events."""
    cfg = SCENARIOS[name]
    events = []

    def record(ev):
        events.append(ev)

    prompts = make_prompts(cfg)
    eos_at = make_eos_at(cfg, prompts)
    eos = EOS_TOKEN if eos_at else -1
    bm = BlockManager(num_blocks=cfg["num_blocks"], block_size=cfg["block_size"], device=device)
    runner = TraceRunner(bm, cfg["block_size"], cfg["prefix_cache"], torch_mod, record,
                         token_fn=eos_token_fn(eos_at))
    if metadata_hook is not None:
        base_log = runner._log

        def log(kind, slots, md, extra):
            metadata_hook(kind, slots, md, extra)
            base_log(kind, slots, md, extra)

        runner._log = log
    sched = MiniScheduler(max_num_seqs=cfg["max_num_seqs"], block_size=cfg["block_size"],
                          total_num_blocks=cfg["num_blocks"])
    core = EngineCore(runner, sched)
    params = SamplingParams()

    def submit(tokens, max_new):
        seq = Sequence(seq_id=sched.next_seq_id(), prompt="", max_new_tokens=max_new,
                       prompt_token_ids=runner.tokenize_prompts([tokens])[0], sampling_params=params)
        runner.prepare_sequences([seq])
        seq.reserved_blocks = sched.compute_required_blocks(runtime_prompt_len=seq.runtime_prompt_len,
                                                            max_new_tokens=max_new)
        sched.add_request(seq)

    first = prompts[: cfg["n_first"]]
    second = prompts[cfg["n_first"]:]
    # first wave: half up front, the rest one per step while the engine runs
    for tokens, max_new in first[: len(first) // 2]:
        submit(tokens, max_new)
    pending = list(first[len(first) // 2:])
    step = 0
    while sched.has_unfinished() or pending:
        if pending and step % 2 == 1:
            submit(*pending.pop(0))
        finished = core.step(eos)
        events.append({"event": "step", "finished": [s.seq_id for s in finished],
                       "running": list(sched.running), "waiting": [s.seq_id for s in sched.waiting]})
        step += 1
        if step > 10000:
            raise RuntimeError("scenario did not terminate")
    # second wave: submitted together, after the first finished (prefix hits)
    for tokens, max_new in second:
        submit(tokens, max_new)
    while sched.has_unfinished():
        finished = core.step(eos)
        events.append({"event": "step", "finished": [s.seq_id for s in finished],
                       "running": list(sched.running), "waiting": [s.seq_id for s in sched.waiting]})
    events.append({"event": "end", "free_block_ids": list(bm.free_block_ids),
                   "outputs": {str(k): list(v.generated_token_ids) for k, v in sched.finished.items()},
                   "finish_reasons": {str(k): v.finish_reason for k, v in sched.finished.items()}})
    return events


def run_schedule(schedule, token_fn, eos_token_id, *, block_size, num_blocks, max_num_seqs, prefix_cache,
                 BlockManager, MiniScheduler, EngineCore, Sequence, SamplingParams, torch_mod, device="cpu",
                 events=None):
    """Drive an engine from a submission schedule and a token stream; return the recorded events.

    ``schedule`` maps an engine step index to the (prompt token ids, max_new_tokens) submitted
    just before that step runs; ``token_fn(seq_id, n)`` is the token request ``seq_id`` samples
    as its token number n (EOS included).  Steps run until nothing is left and no submission
    is pending.  Events go to ``events`` when given, so a caller keeps those recorded before
    an exception.
    """
    events = [] if events is None else events
    bm = BlockManager(num_blocks=num_blocks, block_size=block_size, device=device)
    runner = TraceRunner(bm, block_size, prefix_cache, torch_mod, events.append, token_fn=token_fn)
    sched = MiniScheduler(max_num_seqs=max_num_seqs, block_size=block_size, total_num_blocks=num_blocks)
    core = EngineCore(runner, sched)
    params = SamplingParams()
    last = max(schedule) if schedule else 0
    step = 0
    while sched.has_unfinished() or step <= last:
        for tokens, max_new in schedule.get(step, []):
            seq = Sequence(seq_id=sched.next_seq_id(), prompt="", max_new_tokens=max_new,
                           prompt_token_ids=runner.tokenize_prompts([tokens])[0], sampling_params=params)
            runner.prepare_sequences([seq])
            seq.reserved_blocks = sched.compute_required_blocks(runtime_prompt_len=seq.runtime_prompt_len,
                                                                max_new_tokens=max_new)
            sched.add_request(seq)
        finished = core.step(eos_token_id)
        events.append({"event": "step", "finished": [s.seq_id for s in finished]})
        step += 1
        if step > 100000:
            raise RuntimeError("schedule did not terminate")
    return events
