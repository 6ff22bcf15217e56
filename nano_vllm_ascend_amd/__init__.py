"""MI355X-native continuous-batching attention path with nano_vllm_ascend's API.

Lazily exports the reference's public names (nv/__init__.py:1-13): LLM,
EngineCore and SamplingParams.
"""


def __getattr__(name: str):
    if name in {"LLM", "EngineCore"}:
        from .engine import EngineCore, LLM

        return {"LLM": LLM, "EngineCore": EngineCore}[name]
    if name == "SamplingParams":
        from .sampling_params import SamplingParams

        return SamplingParams
    raise AttributeError(name)


__all__ = ["LLM", "EngineCore", "SamplingParams"]
