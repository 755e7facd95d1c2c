"""transformers' logits rules for one SamplingParams, applied to a whole batch on the GPU.

Same rules, order and meaning as vflorence/layers/logits_processor.py:6-51 (which
follows transformers' generate): repetition penalty, no-repeat n-gram, min length,
forced BOS, forced EOS, suppressed tokens, suppressed-at-begin tokens.  Everything is
written as masks over the ``[rows, vocab]`` score matrix so a step runs without a
device->host synchronisation: token histories arrive as a ``[rows, width]`` int64
device tensor left-padded with -1, lengths as an int64 device vector.
"""

from __future__ import annotations

import torch

_NEG_INF = float("-inf")


def _in_vocab(tokens, vocab_size: int) -> list[int]:
    if tokens is None:
        return []
    if isinstance(tokens, int):
        tokens = [tokens]
    return [t for t in tokens if 0 <= t < vocab_size]


class LogitsProcessor:
    def __init__(self, sampling_params, *, vocab_size: int, max_length: int, begin_index: int,
                 device="cuda"):
        sp = self.sampling_params = sampling_params
        self.vocab_size = vocab_size
        self.max_length = max_length
        self.begin_index = begin_index
        self.needs_history = sp.repetition_penalty != 1.0 or sp.no_repeat_ngram_size > 0

        def ids(tokens):
            kept = _in_vocab(tokens, vocab_size)
            return torch.tensor(kept, dtype=torch.long, device=device) if kept else None

        self.eos = ids(sorted(sp.eos_ids()))
        self.suppress = ids(sp.suppress_tokens)
        self.begin_suppress = ids(sp.begin_suppress_tokens)
        self.forced_bos = ids(sp.forced_bos_token_id)
        self.forced_eos = ids(sp.forced_eos_token_id)

    def __call__(self, history: torch.Tensor | None, scores: torch.Tensor,
                 lengths: torch.Tensor) -> torch.Tensor:
        """Apply every enabled rule to ``scores`` ([rows, vocab] float32) in place."""
        sp = self.sampling_params
        if sp.repetition_penalty != 1.0:
            seen = self._token_mask(history, history >= 0, history)
            penalised = torch.where(scores < 0, scores * sp.repetition_penalty,
                                    scores / sp.repetition_penalty)
            scores.copy_(torch.where(seen, penalised, scores))
        if sp.no_repeat_ngram_size > 0:
            self._no_repeat_ngram(scores, history, sp.no_repeat_ngram_size)
        if sp.min_length > 0 and self.eos is not None:
            self._set(scores, lengths < sp.min_length, self.eos, _NEG_INF)
        if self.forced_bos is not None:
            self._force(scores, lengths == 1, self.forced_bos)
        if self.forced_eos is not None:
            self._force(scores, lengths == self.max_length - 1, self.forced_eos)
        if self.suppress is not None:
            scores.index_fill_(1, self.suppress, _NEG_INF)
        if self.begin_suppress is not None:
            self._set(scores, lengths == self.begin_index, self.begin_suppress, _NEG_INF)
        return scores

    def topk_rules(self):
        """These rules packed for the fused log-softmax + rules + top-k kernel, or None
        when a rule reads the token history (repetition penalty, n-gram bans)."""
        if self.needs_history:
            return None
        if not hasattr(self, "_topk_rules"):
            from ..decoder_ops import TopkRules

            def ids(t):
                return [] if t is None else t.tolist()

            device = next((t.device for t in (self.eos, self.suppress, self.begin_suppress,
                                              self.forced_bos, self.forced_eos) if t is not None),
                          None)
            self._topk_rules = TopkRules(
                eos=ids(self.eos), suppress=ids(self.suppress),
                begin_suppress=ids(self.begin_suppress), forced_bos=ids(self.forced_bos),
                forced_eos=ids(self.forced_eos), min_length=self.sampling_params.min_length,
                max_length=self.max_length, begin_index=self.begin_index, device=device)
        return self._topk_rules

    def _token_mask(self, history, valid, tokens) -> torch.Tensor:
        """[rows, vocab] bool: True where ``tokens[r, j]`` is a token and ``valid[r, j]``."""
        rows = history.shape[0]
        mask = torch.zeros(rows, self.vocab_size + 1, dtype=torch.bool, device=history.device)
        # invalid entries land in the spare last column
        index = torch.where(valid & (tokens < self.vocab_size), tokens, self.vocab_size)
        mask.scatter_(1, index, True)
        return mask[:, : self.vocab_size]

    def _no_repeat_ngram(self, scores, history, n: int) -> None:
        """Ban each token that would repeat an n-gram already in the row's history."""
        width = history.shape[1]
        if width < n:
            return
        grams = history.unfold(1, n, 1)  # [rows, width - n + 1, n]
        tail = history[:, width - n + 1:].unsqueeze(1)  # the row's last n - 1 tokens
        hit = (grams[..., :-1] == tail).all(-1) & (grams[..., -1] >= 0)
        banned = self._token_mask(history, hit, grams[..., -1])
        scores.masked_fill_(banned, _NEG_INF)

    @staticmethod
    def _set(scores, rows: torch.Tensor, tokens: torch.Tensor, value: float) -> None:
        cols = scores.index_select(1, tokens)
        scores.index_copy_(1, tokens, cols.masked_fill(rows.unsqueeze(1), value))

    def _force(self, scores, rows: torch.Tensor, tokens: torch.Tensor) -> None:
        """Rows where ``rows`` holds may only choose ``tokens`` (score 0, others -inf)."""
        scores.masked_fill_(rows.unsqueeze(1), _NEG_INF)
        self._set(scores, rows, tokens, 0.0)
