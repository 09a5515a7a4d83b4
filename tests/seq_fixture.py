"""Test fixture: the per-sequence host state the verify drop-in reads.

The tests build run_verify inputs from it, as the reference engine builds them
from its own Sequence objects; the product package does not import it.

Mirror of mini_vllm/engine/sequence.py:14-132 and mini_vllm/sampling_params.py:4-15
(the fields run_verify and the spec block read: token_ids, last_token,
num_tokens, num_prompt_tokens, num_computed_tokens, block_table, temperature,
top_k, top_p, max_tokens, ignore_eos). The one difference: a temperature of 0
is accepted and selects greedy acceptance (sampling_params.py:13 rejects it).
"""
from __future__ import annotations

from dataclasses import dataclass
from enum import Enum, auto
from itertools import count


@dataclass
class SamplingParams:
    temperature: float = 1.0
    max_tokens: int = 64
    ignore_eos: bool = False
    top_k: int = -1
    top_p: float = 1.0

    def __post_init__(self):
        if self.temperature < 0:
            raise ValueError("temperature must be >= 0 (0 selects greedy)")
        if not (self.top_k == -1 or self.top_k > 0):
            raise ValueError("top_k must be -1 or > 0")
        if not (0.0 < self.top_p <= 1.0):
            raise ValueError("top_p must be in (0, 1]")


class SequenceStatus(Enum):
    WAITING = auto()
    RUNNING = auto()
    FINISHED = auto()


class Sequence:
    block_size = 256
    counter = count()

    def __init__(self, token_ids: list[int], sampling_params: SamplingParams | None = None):
        sp = sampling_params or SamplingParams()
        self.seq_id = next(Sequence.counter)
        self.status = SequenceStatus.WAITING
        self.token_ids = list(token_ids)
        self.last_token = self.token_ids[-1]
        self.num_tokens = len(self.token_ids)
        self.num_prompt_tokens = len(self.token_ids)
        self.num_cached_tokens = 0
        self.num_computed_tokens = 0
        self.block_table: list[int] = []
        self.temperature = sp.temperature
        self.max_tokens = sp.max_tokens
        self.ignore_eos = sp.ignore_eos
        self.top_k = sp.top_k
        self.top_p = sp.top_p

    def __len__(self):
        return self.num_tokens

    def __getitem__(self, key):
        return self.token_ids[key]

    @property
    def is_finished(self):
        return self.status == SequenceStatus.FINISHED

    @property
    def num_completion_tokens(self):
        return self.num_tokens - self.num_prompt_tokens

    @property
    def num_blocks(self):
        return (self.num_tokens + self.block_size - 1) // self.block_size

    def append_token(self, token_id: int):
        self.token_ids.append(token_id)
        self.last_token = token_id
        self.num_tokens += 1
