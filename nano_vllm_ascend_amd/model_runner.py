"""Model runner: packing, graph/eager dispatch and sampling (nv/model_runner.py:15-297).

Differences from the reference, all on the hot path:
  - prefill and decode inputs (token ids, positions, slot_mapping, block
    tables, context lengths, cu_seqlens, last-token indices) are packed on the
    GPU from one host-to-device transfer per step (BlockManager._pack);
  - decode at a captured batch size packs straight into the graph's static
    buffers, so a replay needs no device-to-device input copies;
  - greedy sampling of a batch is one argmax and ONE device-to-host read per
    step (the reference synchronised once per sequence);
  - overlapped decode: when step N+1's batch is predictable before step N's
    tokens reach the host (every sequence continues unless it samples EOS,
    nothing was prefilled in between, greedy sampling, a captured batch
    size), step N+1 is launched right behind step N with step N's argmax as
    its input ids (the graph writes the argmax over its input-id buffer), and
    the host reads step N's tokens and plans the next engine step while the
    GPU runs.  ``last_logits`` of such a step is None unless ``retain_logits``
    asks for a copy (the static logits buffer belongs to the step launched).  Step N+1 is packed ahead
    WITHOUT touching the block pool: a sequence that crosses into a new block
    uses the block the pool would hand out next (the front of the free queue
    in batch order), which is the block the synchronous loop allocates if
    nothing else touches the pool first.  The next ``decode`` call confirms
    the step only for the same Sequence objects at the same positions, and
    only then allocates (checking it gets those blocks); any ``prefill`` or
    ``free_seq`` in between discards it first.  So block allocation, and with
    it every block table and slot mapping, follows the synchronous order.  A
    discarded step wrote K/V only into rows no live sequence has reached and
    into free blocks that carry no prefix-cache key (others are never packed
    ahead), and every later write to those rows is ordered after it on the
    stream.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import torch

from . import _C
from .block_manager import BlockManager, PagedKVCacheMetadata
from .config import load_config
from .graph import DecodeGraphRunner
from .layers import RotaryEmbedding, Sampler
from .paged_kv_cache import PagedKVCache
from .qwen3 import Qwen3ForCausalLM, load_safetensors_dir
from .sequence import Sequence

DEFAULT_DECODE_GRAPH_BATCH_SIZES = [1, 2, 4, 8, 16, 32]


class _TokenFetch:
    """A pinned host copy of one step's greedy ids and of the device's index-error word, and the
    event that says both have landed."""

    def __init__(self, n: int, errors):
        self.buf = torch.empty(n, dtype=torch.int64, pin_memory=True)
        self.errors = errors
        self.event = torch.cuda.Event()

    def start(self, ids: torch.Tensor) -> "_TokenFetch":
        self.buf.copy_(ids, non_blocking=True)
        self.errors.fetch()
        self.event.record()
        return self

    def tokens(self) -> list[int]:
        self.event.synchronize()
        self.errors.raise_if_set()  # an index the reference would have refused: IndexError
        return self.buf.tolist()


class _InFlightStep:
    """A decode step launched ahead of the call that asks for it (not yet applied to the pool)."""

    def __init__(self, seqs, positions, taken, entry, fetch: _TokenFetch, logits: torch.Tensor, snapshot=None):
        self.seqs = list(seqs)
        self.slots = [seq.seq_id for seq in seqs]
        self.positions = positions
        self.taken = taken          # (slot, block) the step packed before the pool handed them out
        self.entry = entry
        self.fetch = fetch
        self.logits = logits
        self.snapshot = snapshot    # host copy of its metadata, kept only for a metadata hook

    def matches(self, seqs, positions) -> bool:
        return (len(seqs) == len(self.seqs) and all(a is b for a, b in zip(seqs, self.seqs))
                and positions == self.positions)


class TokenIdTokenizer:
    """Stand-in when the model directory has no tokenizer: prompts must be token ids; decode gives ''."""

    def __init__(self, eos_token_id: int):
        self.eos_token_id = eos_token_id

    def decode(self, token_ids, skip_special_tokens=True) -> str:
        return ""


def _load_tokenizer(model_path, eos_token_id: int):
    if isinstance(model_path, (str, Path)) and Path(model_path).is_dir():
        path = Path(model_path)
        if (path / "tokenizer.json").exists() or (path / "tokenizer_config.json").exists():
            from transformers import AutoTokenizer

            return AutoTokenizer.from_pretrained(str(path), trust_remote_code=True, local_files_only=True)
    return TokenIdTokenizer(eos_token_id)


class ModelRunner:
    def __init__(self, model_path, max_model_len: int, num_blocks: int | None, block_size: int, device_id: int,
                 npu_memory_utilization: float, enable_prefix_cache: bool = False, enable_decode_graph: bool = False,
                 decode_graph_batch_sizes: list[int] | None = None, seed: int = 0, max_num_seqs: int = 64,
                 enable_overlap: bool = True, retain_logits: bool = False):
        torch.cuda.set_device(device_id)
        self.device = torch.device("cuda", device_id)
        self.model_path = model_path
        self.max_model_len = max_model_len
        self.block_size = block_size
        self.dtype = torch.bfloat16
        self.sampler = Sampler()
        self.enable_prefix_cache = enable_prefix_cache
        self.enable_decode_graph = enable_decode_graph
        self._init_step_state(enable_overlap, retain_logits)
        self.config = load_config(model_path)
        self.tokenizer = _load_tokenizer(model_path, self.config.eos_token_id)

        self.model = self._load_model(seed)
        self.num_blocks = num_blocks or self._num_blocks_from_memory(npu_memory_utilization)
        self.block_manager = BlockManager(num_blocks=self.num_blocks, block_size=block_size, device=self.device,
                                          max_seqs=max(max_num_seqs, 8),
                                          max_blocks_per_seq=max(1, -(-max_model_len // block_size)))
        cfg = self.config
        self.kv_cache = PagedKVCache(cfg.num_hidden_layers, self.num_blocks, block_size, cfg.num_key_value_heads,
                                     cfg.head_dim, self.dtype, self.device)
        self.decode_graph_runner = None
        if enable_decode_graph:
            self.decode_graph_runner = DecodeGraphRunner(
                model=self.model, kv_cache=self.kv_cache,
                batch_sizes=decode_graph_batch_sizes or DEFAULT_DECODE_GRAPH_BATCH_SIZES,
                max_model_len=max_model_len, block_size=block_size)

    def _init_step_state(self, enable_overlap: bool, retain_logits: bool = False) -> None:
        """Per-step bookkeeping: last logits, the step launched ahead, token fetch buffers."""
        self.last_logits: torch.Tensor | None = None
        self.retain_logits = retain_logits  # keep overlapped steps' logits readable (a copy per step)
        self.enable_overlap = enable_overlap
        self._in_flight: _InFlightStep | None = None
        self._prefilled_since_decode = False
        self._fetch: dict[int, list] = {}      # batch size -> [two _TokenFetch, next index]
        self._logits_keep: dict[int, torch.Tensor] = {}
        # the device's index-error word, read with every step's tokens (a factory so a test can
        # stand in for the device)
        self.error_word_factory = _C.IndexErrorWord
        self._eager_errors = None
        self.overlap_stats = {"launched": 0, "used": 0, "discarded": 0}
        # prefill batches, those on the paged (prefix-hit) route, and the prompt tokens whose K/V
        # came from the prefix cache instead of being computed
        self.prefill_stats = {"batches": 0, "paged_batches": 0, "cached_tokens": 0, "computed_tokens": 0}
        # test hook: called as hook(kind, slots, metadata) with a host copy of the metadata of
        # every prefill and every decode step that is actually taken
        self.metadata_hook = None
        # set by the engine's owner: whether the next engine step admits a waiting request (its
        # batch then differs, so no step is launched ahead)
        self.next_step_admits = None

    @torch.inference_mode()
    def _load_model(self, seed: int) -> Qwen3ForCausalLM:
        cfg = self.config
        with torch.device(self.device):
            model = Qwen3ForCausalLM(cfg, self.block_size, self.max_model_len)
        model = model.to(dtype=self.dtype)
        # the cast above rounded the RoPE table; rebuild it in fp32
        model.model.rotary_emb = RotaryEmbedding(cfg.head_dim, cfg.max_position_embeddings,
                                                 cfg.rope_theta).to(self.device)
        sd = load_safetensors_dir(self.model_path) if isinstance(self.model_path, (str, Path)) else None
        if sd is None:
            model.init_random(seed)
        else:
            missing = model.load_hf_state_dict(sd)
            if missing:
                print(f"[load] missing={missing}")
        model.eval()
        return model

    def _num_blocks_from_memory(self, utilization: float) -> int:
        free, total = torch.cuda.mem_get_info(self.device)
        budget = int(total * utilization) - (total - free)
        cfg = self.config
        per_block = PagedKVCache.bytes_per_block(cfg.num_hidden_layers, self.block_size, cfg.num_key_value_heads,
                                                 cfg.head_dim)
        return max(1, budget // per_block)

    # -------------------------------------------------------------- prompts
    def _tokenize_prompt(self, prompt) -> torch.Tensor:
        if isinstance(prompt, str):
            if isinstance(self.tokenizer, TokenIdTokenizer):
                raise ValueError("this model directory has no tokenizer: submit prompts as token ids")
            enc = self.tokenizer.apply_chat_template([{"role": "user", "content": prompt}],
                                                     add_generation_prompt=True, enable_thinking=False,
                                                     tokenize=True, return_dict=True, return_tensors="pt")
            return enc["input_ids"][0]
        return torch.as_tensor(prompt, dtype=torch.long).reshape(-1)

    def tokenize_prompts(self, prompts) -> list[torch.Tensor]:
        ids = [self._tokenize_prompt(p) for p in prompts]
        longest = max(int(t.numel()) for t in ids)
        if longest > self.max_model_len:
            raise ValueError(f"prompt length {longest} exceeds max_model_len {self.max_model_len}")
        return ids

    def prepare_sequences(self, seqs: list[Sequence]) -> None:
        """Prefix lookup at submit time (nv/model_runner.py:146-167)."""
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

    # ------------------------------------------------------------ sampling
    def _sample(self, logits: torch.Tensor, seqs: list[Sequence], greedy_ids: torch.Tensor | None = None) -> list[int]:
        if self._eager_errors is None:
            self._eager_errors = self.error_word_factory()
        self._eager_errors.fetch()  # queued behind the step's kernels, read with its tokens
        if all(seq.sampling_params.is_greedy() for seq in seqs):
            ids = greedy_ids if greedy_ids is not None else _C.argmax_rows(logits)
            tokens = ids.tolist()  # one device-to-host read for the batch
        else:
            tokens = [int(self.sampler.sample(logits[i : i + 1], seq.sampling_params).item())
                      for i, seq in enumerate(seqs)]
        self._eager_errors.raise_if_set()
        return tokens

    # ------------------------------------------------------------- forward
    def _drop_in_flight(self) -> None:
        """Forget a step launched ahead: the batch it assumed is not the next one."""
        if self._in_flight is not None:
            self._in_flight = None
            self.overlap_stats["discarded"] += 1

    @staticmethod
    def _host_metadata(md) -> PagedKVCacheMetadata:
        """A host copy (never a view: static graph buffers are overwritten by the next step)."""
        def host(t):
            return t.to("cpu", copy=True)

        return PagedKVCacheMetadata(block_tables=host(md.block_tables), context_lens=host(md.context_lens),
                                    slot_mapping=host(md.slot_mapping),
                                    actual_seq_lengths_q=md.actual_seq_lengths_q,
                                    actual_seq_lengths_kv=md.actual_seq_lengths_kv,
                                    use_paged_prefill=md.use_paged_prefill)

    def _report(self, kind: str, slots, md, is_host_copy: bool = False) -> None:
        if self.metadata_hook is not None:
            self.metadata_hook(kind, list(slots), md if is_host_copy else self._host_metadata(md))

    @torch.inference_mode()
    def prefill(self, seqs: list[Sequence]) -> None:
        if not seqs:
            return
        self._drop_in_flight()
        self._prefilled_since_decode = True
        md = self.block_manager.prepare_prefill_metadata(
            slots=[s.seq_id for s in seqs], seq_lens=[s.runtime_prompt_len for s in seqs],
            start_positions=[s.cached_prefix_len for s in seqs], prefix_block_ids=[s.cached_block_ids for s in seqs],
            token_ids=[np.asarray(s.runtime_prompt_token_ids) for s in seqs])
        self._report("prefill", [s.seq_id for s in seqs], md)
        st = self.prefill_stats
        st["batches"] += 1
        st["paged_batches"] += int(md.use_paged_prefill)
        st["cached_tokens"] += sum(s.cached_prefix_len for s in seqs)
        st["computed_tokens"] += sum(s.runtime_prompt_len for s in seqs)
        out = self.model(input_ids_flat=md.input_ids, position_ids_flat=md.positions, kv_cache=self.kv_cache,
                         attn_metadata=md, is_prefill=True, logits_indices=md.last_token_indices)
        self.last_logits = out.logits  # rows in `seqs` order; a graph replay reuses this buffer
        for seq, token in zip(seqs, self._sample(out.logits, seqs)):
            seq.set_prefill_result(next_token_id=token, prompt_len=seq.estimated_prompt_len)
            if self.enable_prefix_cache:
                self.block_manager.cache_full_blocks(slot=seq.seq_id, token_ids=seq.prompt_token_ids,
                                                     num_cached_blocks=len(seq.cached_block_ids),
                                                     num_full_blocks=seq.estimated_prompt_len // self.block_size)

    def _fetch_tokens(self, b: int, ids: torch.Tensor) -> _TokenFetch:
        slot = self._fetch.get(b)
        if slot is None:
            slot = self._fetch[b] = [_TokenFetch(b, self.error_word_factory()),
                                     _TokenFetch(b, self.error_word_factory()), 0]
        f = slot[slot[2]]
        slot[2] ^= 1  # ping-pong: the step launched ahead uses the other buffer
        return f.start(ids)

    def _keep_logits(self, b: int, logits: torch.Tensor) -> torch.Tensor:
        """Copy a graph step's logits out of the static buffer the next replay overwrites."""
        keep = self._logits_keep.get(b)
        if keep is None or keep.shape != logits.shape:
            keep = self._logits_keep[b] = torch.empty_like(logits)
        keep.copy_(logits)
        return keep

    def _can_launch_ahead(self, seqs: list[Sequence]) -> bool:
        # the next engine step decodes exactly these sequences when none samples EOS (unknown
        # until the tokens are read: the next call then discards the launch), none takes its
        # final-token commit (engine.py) and nothing is admitted or prefilled in between
        return self.enable_overlap and all(
            seq.sampling_params.is_greedy() and not seq.pending_is_last() for seq in seqs)

    @torch.inference_mode()
    def decode(self, seqs: list[Sequence]) -> None:
        if not seqs:
            return
        tokens = np.fromiter((seq.append_next_token() for seq in seqs), dtype=np.int64, count=len(seqs))
        positions = [seq.cache_position for seq in seqs]
        slots = [seq.seq_id for seq in seqs]
        b = len(seqs)
        graph = self.decode_graph_runner
        ahead, self._in_flight = self._in_flight, None
        entry = fetch = logits = None
        reported = False
        if ahead is not None and ahead.matches(seqs, positions):
            # launched by the previous call: apply it to the pool now that the batch is confirmed
            self.block_manager.commit_decode_ahead(ahead.slots, ahead.positions, ahead.taken)
            entry, fetch, logits = ahead.entry, ahead.fetch, ahead.logits
            self.overlap_stats["used"] += 1
            if ahead.snapshot is not None:
                self._report("decode", slots, ahead.snapshot, is_host_copy=True)
        else:
            if ahead is not None:
                self.overlap_stats["discarded"] += 1
            if graph is not None and graph.supports(b):
                entry = graph.entry_for(b, 1, self.device, self.block_size)
                md = self.block_manager.prepare_decode_metadata(slots, positions, 1, token_ids=tokens,
                                                                width=entry.width, out=entry.buffers)
                self._report("decode", slots, md)
                reported = True
                logits = graph.replay(entry)  # the static buffers now hold this step's inputs
                if logits is None:
                    entry = None
            else:
                if graph is not None:
                    graph.stats.fallbacks += 1
            if entry is None:
                md = self.block_manager.prepare_decode_metadata(slots, positions, 1, token_ids=tokens)
                if not reported:
                    self._report("decode", slots, md)
                logits = self.model(input_ids_flat=md.input_ids, position_ids_flat=md.positions,
                                    kv_cache=self.kv_cache, attn_metadata=md, is_prefill=False).logits
            elif all(seq.sampling_params.is_greedy() for seq in seqs):
                fetch = self._fetch_tokens(b, entry.buffers["greedy_ids"])
        self._prefilled_since_decode, prefilled = False, self._prefilled_since_decode
        admits = self.next_step_admits is not None and self.next_step_admits()
        if entry is not None and fetch is not None and not prefilled and not admits and self._can_launch_ahead(seqs):
            logits = self._launch_ahead(seqs, positions, entry, logits)
        self.last_logits = logits
        ids = fetch.tokens() if fetch is not None else self._sample(logits, seqs)
        for seq, token in zip(seqs, ids):
            seq.set_decode_result(token)

    def _launch_ahead(self, seqs, positions, entry, logits) -> torch.Tensor | None:
        """Launch step N+1 behind step N: same sequences, next positions, input ids = step N's
        argmax (the graph writes it over its input ids).  Returns step N's logits: unchanged when
        nothing is launched, else copied out of the static buffer the launched replay overwrites
        when ``retain_logits`` is set, and None otherwise (only greedy steps launch ahead, so
        nothing else reads them)."""
        b = len(seqs)
        nxt = [p + 1 for p in positions]
        packed = self.block_manager.prepare_decode_ahead([seq.seq_id for seq in seqs], nxt, token_ids=None,
                                                         width=entry.width, out=entry.buffers)
        if packed is None:
            return logits
        md, taken = packed
        kept = self._keep_logits(b, logits) if self.retain_logits else None
        snapshot = self._host_metadata(md) if self.metadata_hook is not None else None
        nxt_logits = self.decode_graph_runner.replay(entry)  # its input ids: step N's argmax, in place
        self._in_flight = _InFlightStep(seqs, nxt, taken, entry, self._fetch_tokens(b, entry.buffers["greedy_ids"]),
                                        nxt_logits, snapshot)
        self.overlap_stats["launched"] += 1
        return kept

    def decode_graph_stats(self) -> dict[str, int]:
        return {} if self.decode_graph_runner is None else self.decode_graph_runner.stats_dict()

    def free_seq(self, seq: Sequence) -> None:
        self._drop_in_flight()  # a finishing sequence was in the launched batch
        self.block_manager.free_slot(seq.seq_id)

    def clear_prefix_cache(self) -> None:
        self.block_manager.clear_prefix_cache()
