"""Decoding parameters, with the reference's validation and defaulting rules
(vflorence/sampling_params.py:8-129): every field None means "take the checkpoint's
generation config", num_beams == 1 is greedy, > 1 is beam search."""

from __future__ import annotations

from dataclasses import dataclass, fields, replace
from math import isfinite
from numbers import Real


def _finite_number(v) -> bool:
    return not isinstance(v, bool) and isinstance(v, Real) and isfinite(v)


def _token_id(v) -> bool:
    return type(v) is int and v >= 0


def _token_ids(v) -> bool:
    return isinstance(v, list) and all(_token_id(t) for t in v)


@dataclass(slots=True)
class SamplingParams:
    max_tokens: int | None = None
    num_beams: int | None = None
    repetition_penalty: float | None = None
    eos_token_id: int | list[int] | None = None  # []: never stop
    length_penalty: float | None = None
    no_repeat_ngram_size: int | None = None
    min_length: int | None = None
    forced_bos_token_id: int | None = None
    forced_eos_token_id: int | list[int] | None = None
    suppress_tokens: list[int] | None = None
    begin_suppress_tokens: list[int] | None = None
    early_stopping: bool | None = None

    def __post_init__(self) -> None:
        self.validate()

    def validate(self) -> None:
        for name, lowest in (("max_tokens", 1), ("num_beams", 1), ("no_repeat_ngram_size", 0),
                             ("min_length", 0)):
            v = getattr(self, name)
            if v is not None and (type(v) is not int or v < lowest):
                raise ValueError(f"{name} must be an integer >= {lowest}")
        rp = self.repetition_penalty
        if rp is not None and (not _finite_number(rp) or rp <= 0):
            raise ValueError("repetition_penalty must be a positive finite number")
        if self.length_penalty is not None and not _finite_number(self.length_penalty):
            raise ValueError("length_penalty must be a finite number")
        if self.early_stopping is not None and type(self.early_stopping) is not bool:
            raise ValueError("early_stopping must be True or False")
        if self.forced_bos_token_id is not None and not _token_id(self.forced_bos_token_id):
            raise ValueError("forced_bos_token_id must be a single token ID")
        for name in ("eos_token_id", "forced_eos_token_id"):
            v = getattr(self, name)
            if v is not None and not (_token_id(v) or _token_ids(v)):
                raise ValueError(f"{name} must be a token ID or a list of token IDs")
        for name in ("suppress_tokens", "begin_suppress_tokens"):
            v = getattr(self, name)
            if v is not None and not _token_ids(v):
                raise ValueError(f"{name} must be a list of token IDs")

    def with_defaults(self, default: "SamplingParams") -> "SamplingParams":
        """A copy whose None fields take ``default``'s values (transformers' generate())."""
        return replace(self, **{f.name: getattr(default, f.name) for f in fields(self)
                                if getattr(self, f.name) is None})

    def eos_ids(self) -> set[int]:
        eos = self.eos_token_id
        if eos is None:
            return set()
        return {eos} if isinstance(eos, int) else set(eos)

    @classmethod
    def from_generation_config(cls, config, eos_token_id=None, decoder_prompt_len: int = 1):
        """Fill every field from a transformers GenerationConfig."""

        def pick(value, fallback):
            return fallback if value is None else value

        if config.max_new_tokens is not None:
            max_tokens = config.max_new_tokens
        elif config.max_length is not None:
            max_tokens = config.max_length - decoder_prompt_len
        else:
            max_tokens = 64
        return cls(
            max_tokens=max_tokens,
            num_beams=pick(config.num_beams, 1),
            repetition_penalty=pick(config.repetition_penalty, 1.0),
            length_penalty=pick(config.length_penalty, 1.0),
            no_repeat_ngram_size=pick(config.no_repeat_ngram_size, 0),
            min_length=pick(config.min_length, 0),
            eos_token_id=pick(config.eos_token_id, eos_token_id),
            forced_bos_token_id=config.forced_bos_token_id,
            forced_eos_token_id=config.forced_eos_token_id,
            suppress_tokens=None if config.suppress_tokens is None else list(config.suppress_tokens),
            begin_suppress_tokens=None if config.begin_suppress_tokens is None
            else list(config.begin_suppress_tokens),
            # transformers' "never" counts as False (the length heuristic)
            early_stopping=config.early_stopping is True,
        )
