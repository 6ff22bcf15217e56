"""Sampling parameters (same fields, defaults and validation as nv/sampling_params.py:6-35)."""
from __future__ import annotations

from dataclasses import dataclass, replace


@dataclass(frozen=True)
class SamplingParams:
    """temperature <= 0 means greedy argmax; top_k 0 and top_p 1.0 disable the filters."""

    temperature: float = 0.0
    top_k: int = 0
    top_p: float = 1.0

    def __post_init__(self) -> None:
        checks = (
            (self.temperature >= 0, "temperature must be >= 0"),
            (self.top_k >= 0, "top_k must be >= 0"),
            (0 < self.top_p <= 1, "top_p must be in (0, 1]"),
        )
        for ok, message in checks:
            if not ok:
                raise ValueError(message)

    def is_greedy(self) -> bool:
        return self.temperature <= 0

    def with_overrides(self, *, temperature: float | None = None, top_k: int | None = None,
                       top_p: float | None = None) -> "SamplingParams":
        """Copy with every non-None argument replacing the matching field."""
        changes = {name: value for name, value in (("temperature", temperature), ("top_k", top_k), ("top_p", top_p))
                   if value is not None}
        return replace(self, **changes)
