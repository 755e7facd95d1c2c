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

import math
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
        from transformers import AutoConfig, GenerationConfig, PretrainedConfig

        self.block_size = BLOCK_SIZE
        if self.max_num_seqs <= 0:
            raise ValueError("max_num_seqs must be positive")
        if self.compile and self.cuda_graphs:
            raise ValueError("compile and cuda_graphs are alternatives; choose one")
        if self.dtype not in (torch.float32, torch.bfloat16, torch.float16):
            raise ValueError("dtype must be torch.float32, torch.bfloat16 or torch.float16")
        if isinstance(self.model, PretrainedConfig):
            self.hf_config = self.model
            self.generation_config = GenerationConfig()
        else:
            path = os.fspath(self.model)
            if not os.path.isdir(path):
                raise ValueError(f"model must be a local checkpoint directory, got {path!r}")
            self.hf_config = AutoConfig.from_pretrained(path, local_files_only=True)
            try:
                self.generation_config = GenerationConfig.from_pretrained(
                    path, local_files_only=True)
            except OSError:
                self.generation_config = GenerationConfig()
        self.text_config = self.hf_config.get_text_config()
        max_positions = self.text_config.max_position_embeddings
        bs = self.block_size

        def whole_blocks(n):
            return min(math.ceil(min(n, max_positions) / bs) * bs, max_positions)

        if self.max_decoder_len is None:
            self.max_decoder_len = whole_blocks(
                SamplingParams.from_generation_config(self.generation_config).max_tokens)
        if self.max_encoder_len is None:
            self.max_encoder_len = whole_blocks(math.inf)
        for name in ("max_decoder_len", "max_encoder_len"):
            if not 0 < getattr(self, name) <= max_positions:
                raise ValueError(
                    f"{name} must be in [1, max_position_embeddings={max_positions}]")
        if self.num_blocks is None:
            self.num_blocks = self.max_num_seqs * math.ceil(self.max_decoder_len / bs)
        self.num_cross_blocks = self.max_num_seqs * math.ceil(self.max_encoder_len / bs)
        if self.num_blocks <= 0:
            raise ValueError("num_blocks must be positive")
