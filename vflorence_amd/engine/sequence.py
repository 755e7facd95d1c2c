"""Requests, their outputs, and the per-hypothesis record of the block-manager API.

``Request`` / ``RequestOut`` are the reference's request and result types
(vflorence/engine/sequence.py:10-21).  ``Sequence`` is the hypothesis record that the
reference's block-manager API works on (vflorence/engine/sequence.py:24-86): a token
list, a block table into the self-attention pool and a count of tokens whose K/V are
cached.  The engine itself keeps its running hypotheses in the native host core
(``engine/core.py``); a ``Sequence`` there is the record of a submitted request.
"""

from __future__ import annotations

from dataclasses import dataclass

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


class Sequence:
    """One decoder hypothesis of a request.

    ``token_ids`` starts as the decoder prompt; ``block_table`` lists the pool blocks
    holding its K/V, ``num_cached_tokens`` how many of its tokens are there;
    ``cum_logprob`` is its beam-search score before the length penalty.
    """

    __slots__ = ("request_id", "decoder_token_ids", "encoder_token_ids", "sampling_params",
                 "pixel_values", "mm_hash", "token_ids", "block_table", "num_cached_tokens",
                 "cum_logprob")

    def __init__(self, request_id: int, decoder_token_ids, encoder_token_ids,
                 sampling_params: SamplingParams, pixel_values: torch.Tensor | None = None,
                 mm_hash: str | None = None):
        self.request_id = request_id
        self.decoder_token_ids = list(decoder_token_ids)
        self.encoder_token_ids = list(encoder_token_ids)
        self.sampling_params = sampling_params
        self.pixel_values = pixel_values
        self.mm_hash = mm_hash
        self.token_ids = list(self.decoder_token_ids)
        self.block_table: list[int] = []
        self.num_cached_tokens = 0
        self.cum_logprob = 0.0

    def __repr__(self) -> str:
        return (f"Sequence(request_id={self.request_id}, tokens={self.token_ids}, "
                f"table={self.block_table}, cached={self.num_cached_tokens})")

    def append_token(self, token_id: int) -> None:
        self.token_ids.append(token_id)

    def fork(self, token_id: int, cum_logprob: float = 0.0) -> "Sequence":
        """A child that extends this hypothesis by ``token_id``; it holds no blocks until
        a block manager shares this one's with it."""
        child = Sequence.__new__(Sequence)
        for name in Sequence.__slots__:
            setattr(child, name, getattr(self, name))
        child.token_ids = self.token_ids + [token_id]
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
        """Ended by one of the stop tokens or by the token budget."""
        params = self.sampling_params
        return (self.num_generated >= params.max_tokens
                or self.token_ids[-1] in params.eos_ids())

    @property
    def score(self) -> float:
        """``cum_logprob`` divided by (tokens generated) ** length_penalty."""
        steps = max(self.num_generated, 1)
        return self.cum_logprob / steps ** self.sampling_params.length_penalty

    def to_output(self) -> RequestOut:
        return RequestOut(self.encoder_token_ids, self.completion_token_ids, self.pixel_values)
