"""Decoding parameters (the reference's SamplingParams, vflorence/sampling_params.py).

Every field left None means "take the checkpoint's generation config"; num_beams 1
decodes greedily, more runs beam search.  Field names, the defaulting rule
(``with_defaults``, as transformers' generate() fills a GenerationConfig) and the
validation messages are the reference's interface; the checks are expressed here as
one rule per field.
"""

from __future__ import annotations

from dataclasses import dataclass, fields, replace
from math import isfinite
from numbers import Real


def _real(v) -> bool:
    return isinstance(v, Real) and not isinstance(v, bool) and isfinite(v)


def _token(v) -> bool:
    return type(v) is int and v >= 0


def _tokens(v) -> bool:
    return isinstance(v, list) and all(map(_token, v))


# field -> (accepts a value, message when it does not); None is always accepted
_RULES = {
    "max_tokens": (lambda v: type(v) is int and v >= 1, "max_tokens must be an integer >= 1"),
    "num_beams": (lambda v: type(v) is int and v >= 1, "num_beams must be an integer >= 1"),
    "no_repeat_ngram_size": (lambda v: type(v) is int and v >= 0,
                             "no_repeat_ngram_size must be an integer >= 0"),
    "min_length": (lambda v: type(v) is int and v >= 0, "min_length must be an integer >= 0"),
    "repetition_penalty": (lambda v: _real(v) and v > 0,
                           "repetition_penalty must be a positive finite number"),
    "length_penalty": (_real, "length_penalty must be a finite number"),
    "early_stopping": (lambda v: type(v) is bool, "early_stopping must be True or False"),
    "forced_bos_token_id": (_token, "forced_bos_token_id must be a single token ID"),
    "eos_token_id": (lambda v: _token(v) or _tokens(v),
                     "eos_token_id must be a token ID or a list of token IDs"),
    "forced_eos_token_id": (lambda v: _token(v) or _tokens(v),
                            "forced_eos_token_id must be a token ID or a list of token IDs"),
    "suppress_tokens": (_tokens, "suppress_tokens must be a list of token IDs"),
    "begin_suppress_tokens": (_tokens, "begin_suppress_tokens must be a list of token IDs"),
}


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
        """ValueError naming the first field (in declaration order of the checks) whose
        value is out of range."""
        for name, (ok, message) in _RULES.items():
            value = getattr(self, name)
            if value is not None and not ok(value):
                raise ValueError(message)

    def with_defaults(self, default: "SamplingParams") -> "SamplingParams":
        """A copy whose None fields take ``default``'s values."""
        unset = {f.name: getattr(default, f.name) for f in fields(self)
                 if getattr(self, f.name) is None}
        return replace(self, **unset)

    def eos_ids(self) -> set[int]:
        eos = self.eos_token_id
        if eos is None:
            return set()
        return set(eos) if isinstance(eos, list) else {eos}

    @classmethod
    def from_generation_config(cls, config, eos_token_id=None, decoder_prompt_len: int = 1):
        """Every field from a transformers GenerationConfig (unset fields get
        transformers' defaults; max_tokens from max_new_tokens, else max_length minus
        the decoder prompt, else 64)."""
        if config.max_new_tokens is not None:
            max_tokens = config.max_new_tokens
        elif config.max_length is not None:
            max_tokens = config.max_length - decoder_prompt_len
        else:
            max_tokens = 64

        def given(value, fallback):
            return fallback if value is None else value

        def as_list(value):
            return None if value is None else list(value)

        return cls(
            max_tokens=max_tokens,
            num_beams=given(config.num_beams, 1),
            repetition_penalty=given(config.repetition_penalty, 1.0),
            length_penalty=given(config.length_penalty, 1.0),
            no_repeat_ngram_size=given(config.no_repeat_ngram_size, 0),
            min_length=given(config.min_length, 0),
            eos_token_id=given(config.eos_token_id, eos_token_id),
            forced_bos_token_id=config.forced_bos_token_id,
            forced_eos_token_id=config.forced_eos_token_id,
            suppress_tokens=as_list(config.suppress_tokens),
            begin_suppress_tokens=as_list(config.begin_suppress_tokens),
            # transformers' "never" counts as False (the length heuristic)
            early_stopping=config.early_stopping is True,
        )
