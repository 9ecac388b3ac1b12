"""Result records with the fields of ``rwkvtune/outputs.py:12-67``."""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import List, Optional


@dataclass
class CompletionOutput:
    index: int
    text: str
    token_ids: List[int] = field(default_factory=list)
    cumulative_logprob: Optional[float] = None
    finish_reason: Optional[str] = None  # "stop", "length" or None


@dataclass
class RequestOutput:
    request_id: str
    prompt: str
    prompt_token_ids: List[int] = field(default_factory=list)
    outputs: List[CompletionOutput] = field(default_factory=list)
    finished: bool = True
