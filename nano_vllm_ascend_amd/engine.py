"""Engine step loop and the public ``LLM`` API (behaviour of nv/engine.py:8-199).

``EngineCore.step`` executes one ``StepPlan`` in the order that fixes block
allocation: release the retired requests' blocks, prefill the admitted ones,
commit the last token of requests whose budget it fills (no forward), then
decode the rest as one batch.

``LLM`` keeps the reference's constructor arguments and defaults
(nv/engine.py:59-71), ``generate`` / ``submit`` / ``step`` / ``has_unfinished`` /
``clear_prefix_cache`` / ``warm``, and the output dictionaries
(``{"texts", "token_ids"}`` from ``generate``, plus ``"request_id"`` from
``step``).
"""
from __future__ import annotations

from .sampling_params import SamplingParams
from .scheduler import MiniScheduler
from .sequence import Sequence


class EngineCore:
    def __init__(self, runner, scheduler: MiniScheduler):
        self.runner = runner
        self.scheduler = scheduler

    def step(self, eos_token_id: int) -> list[Sequence]:
        """Run one step; return the requests that finished in it."""
        plan = self.scheduler.plan_next_step(eos_token_id)
        for seq in plan.retired:
            self.runner.free_seq(seq)
        if plan.admitted:
            self.runner.prefill(plan.admitted)
        for seq in plan.last_token:
            seq.append_next_token()
            self.scheduler.retire(seq, "max_new_tokens")
            self.runner.free_seq(seq)
        if plan.forward:
            self.runner.decode(plan.forward)
        return plan.retired + plan.last_token

    def run(self, eos_token_id: int) -> None:
        while self.scheduler.has_unfinished():
            self.step(eos_token_id)


def _params(base: SamplingParams | None, temperature, top_k, top_p) -> SamplingParams:
    return (base or SamplingParams()).with_overrides(temperature=temperature, top_k=top_k, top_p=top_p)


class LLM:
    """Offline engine: ``generate``, or ``submit`` + ``step``, over continuous batching.

    ``model_path`` is a local directory with a Qwen3 ``config.json`` (optionally
    safetensors weights and tokenizer files) or a config object; weights that
    are not found are drawn from N(0, 0.02) with ``seed``.  Without
    ``num_blocks`` the KV pool takes ``npu_memory_utilization`` of device
    memory.  ``enable_overlap`` (not in the reference) lets the runner launch
    a decode step before the host has read the previous step's tokens; tokens
    and packing metadata are those of the synchronous loop.  ``retain_logits``
    (not in the reference, which exposes no logits) keeps every step's logits
    readable as ``runner.last_logits``, at one logits-sized copy per overlapped
    step.
    """

    def __init__(self, model_path, max_model_len: int = 2048, block_size: int = 128, num_blocks: int | None = None,
                 max_num_seqs: int = 4, device_id: int = 0, npu_memory_utilization: float = 0.8,
                 enable_prefix_cache: bool = False, enable_decode_graph: bool = True,
                 decode_graph_batch_sizes: list[int] | None = None, seed: int = 0, enable_overlap: bool = True,
                 retain_logits: bool = False):
        from .model_runner import ModelRunner

        self.runner = ModelRunner(
            model_path=model_path, max_model_len=max_model_len, num_blocks=num_blocks, block_size=block_size,
            device_id=device_id, npu_memory_utilization=npu_memory_utilization,
            enable_prefix_cache=enable_prefix_cache, enable_decode_graph=enable_decode_graph,
            decode_graph_batch_sizes=decode_graph_batch_sizes, seed=seed, max_num_seqs=max_num_seqs,
            enable_overlap=enable_overlap, retain_logits=retain_logits)
        self.scheduler = MiniScheduler(max_num_seqs=max_num_seqs, block_size=block_size,
                                       total_num_blocks=self.runner.num_blocks)
        self.engine_core = EngineCore(self.runner, self.scheduler)
        self.runner.next_step_admits = self.scheduler.head_fits

    def _new_request(self, prompt, max_new_tokens: int, params: SamplingParams) -> Sequence:
        seq = Sequence(seq_id=self.scheduler.next_seq_id(), prompt=prompt if isinstance(prompt, str) else "",
                       max_new_tokens=max_new_tokens, prompt_token_ids=self.runner.tokenize_prompts([prompt])[0],
                       sampling_params=params)
        self.runner.prepare_sequences([seq])  # prefix lookup happens here, at submit time
        seq.reserved_blocks = self.scheduler.compute_required_blocks(runtime_prompt_len=seq.runtime_prompt_len,
                                                                     max_new_tokens=max_new_tokens)
        return self.scheduler.add_request(seq)

    def submit(self, prompt, max_new_tokens: int = 128, sampling_params: SamplingParams | None = None, *,
               temperature: float | None = None, top_k: int | None = None, top_p: float | None = None) -> int:
        """Queue one request (a string, tokenized with the chat template, or token ids); return its id."""
        params = _params(sampling_params, temperature, top_k, top_p)
        return self._new_request(prompt, max_new_tokens, params).seq_id

    def _output(self, seq: Sequence) -> dict[str, object]:
        tokens = list(seq.generated_token_ids)
        return {"request_id": seq.seq_id,
                "texts": self.runner.tokenizer.decode(tokens, skip_special_tokens=True),
                "token_ids": tokens}

    def step(self) -> list[dict[str, object]]:
        """Advance every request by one engine step; return the outputs of those that finished."""
        finished = self.engine_core.step(int(self.runner.tokenizer.eos_token_id))
        return [self._output(seq) for seq in finished]

    def generate(self, prompts: list, max_new_tokens: int = 128, sampling_params: SamplingParams | None = None, *,
                 temperature: float | None = None, top_k: int | None = None, top_p: float | None = None):
        """Run prompts to completion; one ``{"texts", "token_ids"}`` per prompt, in prompt order."""
        if not prompts:
            return []
        params = _params(sampling_params, temperature, top_k, top_p)
        self.scheduler.reset()
        self.runner.next_step_admits = self.scheduler.head_fits
        order = [self._new_request(p, max_new_tokens, params).seq_id for p in prompts]
        done: dict[int, dict] = {}
        while self.has_unfinished():
            done.update((out["request_id"], out) for out in self.step())
        return [{"texts": done[i]["texts"], "token_ids": done[i]["token_ids"]} for i in order]

    def has_unfinished(self) -> bool:
        return self.scheduler.has_unfinished()

    def clear_prefix_cache(self) -> None:
        self.runner.clear_prefix_cache()

    def warm(self, prompt="warm", max_new_tokens: int = 1, sampling_params: SamplingParams | None = None) -> None:
        self.generate([prompt], max_new_tokens=max_new_tokens, sampling_params=sampling_params)
