"""Engine configuration (vflorence/config.py:15-91 semantics), for one GPU.

The reference reads the checkpoint's config from the hub; here ``model`` is a local
checkpoint directory (``config.json`` + weights, what ``save_pretrained`` writes) or an
in-memory ``transformers`` config (random-init weights, synthetic workloads).  Pool
sizing follows the reference: ``num_blocks = max_num_seqs * ceil(max_decoder_len / bs)``
(:83-86) and ``num_cross_blocks = max_num_seqs * ceil(max_encoder_len / bs)`` (:87-89),
with lengths rounded up to whole blocks (:53-57).  The block size is 16, the paged
kernels' block.
"""

from __future__ import annotations

import os
from dataclasses import dataclass, field

import torch

from .sampling_params import SamplingParams

BLOCK_SIZE = 16


@dataclass
class Config:
    model: object  # checkpoint directory or a transformers PretrainedConfig
    max_num_seqs: int = 32
    dtype: torch.dtype = torch.float32
    max_decoder_len: int | None = None
    max_encoder_len: int | None = None
    num_blocks: int | None = None
    device: str = "cuda"
    # decode steps replayed from HIP graphs, one per batch size (eager when False)
    cuda_graphs: bool = False
    # the decoder step under torch.compile(dynamic=True), as the reference compiles it
    # (vflorence/engine/model_runner.py:102-124); the attention, KV-write, LayerNorm and
    # projection custom ops stay opaque.  An alternative to cuda_graphs, not combined.
    compile: bool = False
    block_size: int = field(init=False)
    num_cross_blocks: int = field(init=False)
    hf_config: object = field(init=False)
    text_config: object = field(init=False)
    generation_config: object = field(init=False)

    def __post_init__(self) -> None:
        self.block_size = BLOCK_SIZE
        self._check_options()
        self.hf_config, self.generation_config = _model_configs(self.model)
        self.text_config = self.hf_config.get_text_config()
        limit = self.text_config.max_position_embeddings
        if self.max_decoder_len is None:
            # the generation config's token budget, padded to the block it ends in
            budget = SamplingParams.from_generation_config(self.generation_config).max_tokens
            self.max_decoder_len = min(_blocks(min(budget, limit)) * BLOCK_SIZE, limit)
        if self.max_encoder_len is None:
            self.max_encoder_len = limit
        for name, value in (("max_decoder_len", self.max_decoder_len),
                            ("max_encoder_len", self.max_encoder_len)):
            if value < 1 or value > limit:
                raise ValueError(f"{name}={value} is outside 1..{limit}, the model's "
                                 "max_position_embeddings")
        # one pool of decoder blocks and one of encoder blocks, each for max_num_seqs
        # requests at their longest
        if self.num_blocks is None:
            self.num_blocks = self.max_num_seqs * _blocks(self.max_decoder_len)
        self.num_cross_blocks = self.max_num_seqs * _blocks(self.max_encoder_len)
        if self.num_blocks <= 0:
            raise ValueError(f"num_blocks={self.num_blocks}: the decoder pool needs a block")

    def _check_options(self) -> None:
        if self.max_num_seqs < 1:
            raise ValueError(f"max_num_seqs={self.max_num_seqs}: at least one request "
                             "must fit a step")
        if self.compile and self.cuda_graphs:
            raise ValueError("compile and cuda_graphs are alternatives; choose one")
        if self.dtype not in _DTYPES:
            raise ValueError(f"dtype {self.dtype} is not one of the caches' types "
                             "(torch.float32, torch.bfloat16, torch.float16)")


_DTYPES = (torch.float32, torch.bfloat16, torch.float16)


def _blocks(tokens: int) -> int:
    """Blocks of BLOCK_SIZE tokens that hold ``tokens`` tokens."""
    return -(-tokens // BLOCK_SIZE)


def _model_configs(model):
    """(model config, generation config) of an in-memory transformers config or of a
    local checkpoint directory; a directory without generation_config.json gets the
    library's defaults."""
    from transformers import AutoConfig, GenerationConfig, PretrainedConfig

    if isinstance(model, PretrainedConfig):
        return model, GenerationConfig()
    path = os.fspath(model)
    if not os.path.isdir(path):
        raise ValueError(f"model must be a local checkpoint directory, got {path!r}")
    hf = AutoConfig.from_pretrained(path, local_files_only=True)
    try:
        gen = GenerationConfig.from_pretrained(path, local_files_only=True)
    except OSError:
        gen = GenerationConfig()
    return hf, gen
