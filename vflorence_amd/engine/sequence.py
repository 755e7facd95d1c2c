"""Request / sequence bookkeeping (vflorence/engine/sequence.py:8-86 semantics).

A Sequence is one decoder hypothesis: its tokens, its block table in the paged
self-attention pool and how many of its tokens already have K/V there.  Beams are
ordinary sequences of one request; ``fork`` makes a child that the block manager
then points at the parent's blocks.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

from ..sampling_params import SamplingParams


@dataclass
class Request:
    input_ids: list[int]
    pixel_values: torch.Tensor | None = None


@dataclass
class RequestOut:
    input_ids: list[int]
    completion_token_ids: list[int]
    pixel_values: torch.Tensor | None = None


@dataclass(eq=False)
class Sequence:
    request_id: int
    decoder_token_ids: list[int]
    encoder_token_ids: list[int]
    sampling_params: SamplingParams
    pixel_values: torch.Tensor | None = None
    mm_hash: str | None = None
    token_ids: list[int] = field(init=False)
    block_table: list[int] = field(default_factory=list)
    num_cached_tokens: int = 0
    cum_logprob: float = 0.0

    def __post_init__(self) -> None:
        self.decoder_token_ids = list(self.decoder_token_ids)
        self.encoder_token_ids = list(self.encoder_token_ids)
        self.token_ids = list(self.decoder_token_ids)

    def append_token(self, token_id: int) -> None:
        self.token_ids.append(token_id)

    def fork(self, token_id: int, cum_logprob: float = 0.0) -> "Sequence":
        """A child hypothesis extending this one by ``token_id`` (blocks not yet shared).

        A shallow copy of every field (what ``copy.copy`` gives, without its generic
        reduce protocol: beam search forks every running row each step)."""
        child = Sequence.__new__(Sequence)
        child.__dict__.update(self.__dict__)
        child.token_ids = [*self.token_ids, token_id]
        child.block_table = []
        child.cum_logprob = cum_logprob
        return child

    @property
    def num_generated(self) -> int:
        return len(self.token_ids) - len(self.decoder_token_ids)

    @property
    def completion_token_ids(self) -> list[int]:
        return self.token_ids[len(self.decoder_token_ids):]

    @property
    def is_finished(self) -> bool:
        sp = self.sampling_params
        return self.token_ids[-1] in sp.eos_ids() or self.num_generated >= sp.max_tokens

    @property
    def score(self) -> float:
        """Length-penalised beam score."""
        return self.cum_logprob / (max(self.num_generated, 1) ** self.sampling_params.length_penalty)

    def to_output(self) -> RequestOut:
        return RequestOut(self.encoder_token_ids, self.completion_token_ids, self.pixel_values)
