"""``SamplingParams`` with the fields, defaults and validation of
``rwkvtune/sampling_params.py:11-79`` (vLLM-style)."""

from __future__ import annotations

from dataclasses import dataclass, fields
from typing import List, Optional


@dataclass
class SamplingParams:
    max_tokens: int = 256
    temperature: float = 1.0
    top_p: float = 1.0
    top_k: int = 0
    stop: Optional[List[str]] = None
    stop_token_ids: Optional[List[int]] = None
    skip_special_tokens: bool = True
    repetition_penalty: float = 1.0
    logit_bias: Optional[dict] = None

    def __post_init__(self):
        if self.temperature < 0:
            raise ValueError(f"temperature must be >= 0, got: {self.temperature}")
        if not 0 <= self.top_p <= 1:
            raise ValueError(f"top_p must be in [0, 1] range, got: {self.top_p}")
        if self.top_k < 0:
            raise ValueError(f"top_k must be >= 0, got: {self.top_k}")
        if self.max_tokens < 1:
            raise ValueError(f"max_tokens must be >= 1, got: {self.max_tokens}")
        self.stop = [] if self.stop is None else self.stop
        self.stop_token_ids = [] if self.stop_token_ids is None else self.stop_token_ids

    @classmethod
    def from_dict(cls, d: dict) -> "SamplingParams":
        names = {f.name for f in fields(cls)}
        return cls(**{k: v for k, v in d.items() if k in names})

    def to_dict(self) -> dict:
        return {f.name: getattr(self, f.name) for f in fields(self)}
