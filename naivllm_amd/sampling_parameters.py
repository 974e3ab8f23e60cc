"""Per-request sampling settings, as src/myvllm/sampling_parameters.py:4-13
(same fields, defaults and check): temperature 0 selects greedy decoding,
which the acceptance step treats as temperature <= 1e-6."""

from __future__ import annotations

from dataclasses import dataclass


@dataclass
class SamplingParams:
    temperature: float = 1.0
    max_tokens: int = 64                  # completion tokens at most
    ignore_eos: bool = False
    max_model_length: int | None = None   # prompt + completion tokens at most

    def __post_init__(self):
        assert self.temperature == 0 or self.temperature >= 1e-6, "temperature must be 0 (greedy) or >= 1e-6"
