"""Engine step loop and the public ``LLM`` API (nv/engine.py:8-199).

``EngineCore.step`` runs one ``SchedulerStep``: free finished sequences,
prefill the admitted ones, commit the final token of sequences that reach
their budget without a forward (so a request runs max_new_tokens - 1 decode
forwards), then decode the rest as one batch.
"""
from __future__ import annotations

from .sampling_params import SamplingParams
from .scheduler import MiniScheduler
from .sequence import Sequence


class EngineCore:
    def __init__(self, runner, scheduler: MiniScheduler):
        self.runner = runner
        self.scheduler = scheduler

    def _free_finished(self, seqs) -> None:
        for seq in seqs:
            self.runner.free_seq(seq)

    def _commit_final_tokens(self, seqs):
        for seq in seqs:
            seq.append_next_token()
        finished = self.scheduler.finish_sequences(list(seqs), "max_new_tokens")
        self._free_finished(finished)
        return finished

    def step(self, eos_token_id: int):
        plan = self.scheduler.plan_next_step(eos_token_id)
        self._free_finished(plan.finish_seqs)
        finished = list(plan.finish_seqs)

        if plan.prefill_seqs:
            self.runner.prefill(plan.prefill_seqs)

        if plan.decode_seqs:
            last, rest = [], []
            for seq in plan.decode_seqs:
                (last if len(seq.generated_token_ids) + 1 >= seq.max_new_tokens else rest).append(seq)
            if last:
                finished.extend(self._commit_final_tokens(last))
            if rest:
                self.runner.decode(rest)
        return finished

    def run(self, eos_token_id: int) -> None:
        while self.scheduler.has_unfinished():
            self.step(eos_token_id)


class LLM:
    """Offline engine: ``generate`` / ``submit`` + ``step`` over continuous batching.

    ``model_path`` is a local directory holding a Qwen3 ``config.json`` (and,
    optionally, safetensors weights and tokenizer files); weights that are not
    found are initialised from N(0, 0.02) with a fixed seed.  The remaining
    arguments keep the reference's names and defaults (nv/engine.py:59-71);
    ``npu_memory_utilization`` is the fraction of device memory the KV pool
    may grow to when ``num_blocks`` is not given.  ``enable_overlap`` (not in
    the reference) lets the runner launch a decode step while the host still
    processes the previous one's tokens; outputs are unchanged.
    """

    def __init__(
        self,
        model_path,
        max_model_len: int = 2048,
        block_size: int = 128,
        num_blocks: int | None = None,
        max_num_seqs: int = 4,
        device_id: int = 0,
        npu_memory_utilization: float = 0.8,
        enable_prefix_cache: bool = False,
        enable_decode_graph: bool = True,
        decode_graph_batch_sizes: list[int] | None = None,
        seed: int = 0,
        enable_overlap: bool = True,
    ):
        from .model_runner import ModelRunner

        self.runner = ModelRunner(
            model_path=model_path,
            max_model_len=max_model_len,
            num_blocks=num_blocks,
            block_size=block_size,
            device_id=device_id,
            npu_memory_utilization=npu_memory_utilization,
            enable_prefix_cache=enable_prefix_cache,
            enable_decode_graph=enable_decode_graph,
            decode_graph_batch_sizes=decode_graph_batch_sizes,
            seed=seed,
            max_num_seqs=max_num_seqs,
            enable_overlap=enable_overlap,
        )
        self.scheduler = MiniScheduler(
            max_num_seqs=max_num_seqs,
            block_size=block_size,
            total_num_blocks=self.runner.num_blocks,
        )
        self.engine_core = EngineCore(self.runner, self.scheduler)

    def _resolve_sampling_params(self, sampling_params: SamplingParams | None, **overrides) -> SamplingParams:
        return (sampling_params or SamplingParams()).with_overrides(**overrides)

    def generate(self, prompts: list, max_new_tokens: int = 128, sampling_params: SamplingParams | None = None, *,
                 temperature: float | None = None, top_k: int | None = None, top_p: float | None = None):
        """Run prompts (strings, or lists of token ids) to completion; outputs keep the prompt order."""
        if not prompts:
            return []
        params = self._resolve_sampling_params(sampling_params, temperature=temperature, top_k=top_k, top_p=top_p)
        self.scheduler.reset()
        ids = [self.submit(p, max_new_tokens=max_new_tokens, sampling_params=params) for p in prompts]
        by_id = {}
        while self.has_unfinished():
            for output in self.step():
                by_id[output["request_id"]] = output
        return [{"texts": by_id[i]["texts"], "token_ids": by_id[i]["token_ids"]} for i in ids]

    def submit(self, prompt, max_new_tokens: int = 128, sampling_params: SamplingParams | None = None, *,
               temperature: float | None = None, top_k: int | None = None, top_p: float | None = None) -> int:
        """Queue one request; ``prompt`` is a string (tokenized with the chat template) or token ids."""
        params = self._resolve_sampling_params(sampling_params, temperature=temperature, top_k=top_k, top_p=top_p)
        token_ids = self.runner.tokenize_prompts([prompt])[0]
        seq = Sequence(
            seq_id=self.scheduler.next_seq_id(),
            prompt=prompt if isinstance(prompt, str) else "",
            max_new_tokens=max_new_tokens,
            prompt_token_ids=token_ids,
            sampling_params=params,
        )
        self.runner.prepare_sequences([seq])
        seq.reserved_blocks = self.scheduler.compute_required_blocks(
            runtime_prompt_len=seq.runtime_prompt_len, max_new_tokens=max_new_tokens)
        self.scheduler.add_request(seq)
        return seq.seq_id

    def step(self) -> list[dict[str, object]]:
        eos = int(self.runner.tokenizer.eos_token_id)
        finished = self.engine_core.step(eos)
        return [
            {
                "request_id": seq.seq_id,
                "texts": self.runner.tokenizer.decode(seq.generated_token_ids, skip_special_tokens=True),
                "token_ids": list(seq.generated_token_ids),
            }
            for seq in finished
        ]

    def has_unfinished(self) -> bool:
        return self.scheduler.has_unfinished()

    def clear_prefix_cache(self) -> None:
        self.runner.clear_prefix_cache()

    def warm(self, prompt="warm", max_new_tokens: int = 1, sampling_params: SamplingParams | None = None) -> None:
        self.generate([prompt], max_new_tokens=max_new_tokens, sampling_params=sampling_params)
