"""The five BASELINE workloads as seeded synthetic inputs.

cfg0  0.6B text layer 0, f32 cache pre-filled with 156 rows N(0, 1), one decode step at position 156.
cfg1  0.6B, 28 layers, f16 cache, prefill 156 (143 audio rows + 13 prompt ids), 64 greedy tokens.
cfg2  1.7B, same prompt shape, 128 greedy tokens.
cfg3  1.7B, prefill 3913 (3900 audio rows + 13 prompt ids), 256 greedy tokens.
cfg4  1.7B, 32 streams, lengths U[156, 3913] pre-filled with K/V N(0, 1), 64 lock-step decode steps.

Greedy generation follows the reference loop (text-decoder.cpp:2209-2311): N tokens take one
prefill and N - 1 decode forwards.  Config 4 has no reference counterpart (the reference is batch
1); stream s starts from token first_ids[s] at cur_len = len_s, each step appends one token and the
next input is the step's greedy pick; stop ids are not applied, every stream runs all steps.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import (QA_CACHE_F16, QA_CACHE_F32, QWEN3_ASR_0_6B, QWEN3_ASR_1_7B, SEED_IDS, SEED_INPUTS, SEED_KV,
               SEED_LENGTHS, ModelSize, synth_ids, synth_normal)


@dataclass(frozen=True)
class Workload:
    index: int
    size: ModelSize
    cache_type: int
    n_layers: int = 28
    audio_tokens: int = 143
    prompt_tokens: int = 13
    new_tokens: int = 0
    streams: int = 1
    steps: int = 0

    @property
    def prompt(self) -> int:
        return self.audio_tokens + self.prompt_tokens

    @property
    def max_seq(self) -> int:
        if self.index == 0:
            return 157
        if self.index == 4:
            return 3913 + self.steps
        return self.prompt + self.new_tokens


CONFIGS = {
    0: Workload(0, QWEN3_ASR_0_6B, QA_CACHE_F32, n_layers=1, new_tokens=1),
    1: Workload(1, QWEN3_ASR_0_6B, QA_CACHE_F16, new_tokens=64),
    2: Workload(2, QWEN3_ASR_1_7B, QA_CACHE_F16, new_tokens=128),
    3: Workload(3, QWEN3_ASR_1_7B, QA_CACHE_F16, audio_tokens=3900, new_tokens=256),
    4: Workload(4, QWEN3_ASR_1_7B, QA_CACHE_F16, streams=32, steps=64),
}


def cfg0_inputs(hidden: int, n_kv: int = 8, head_dim: int = 128, length: int = 156):
    """x [1][hidden] N(0, 1) and the layer-0 cache rows K, V [1][n_kv][length][head_dim] N(0, 1)."""
    x = synth_normal(hidden, SEED_INPUTS, "cfg0.hidden_input").reshape(1, hidden)
    k = synth_normal(n_kv * length * head_dim, SEED_KV, "cfg0.layer0.k").reshape(1, n_kv, length, head_dim)
    v = synth_normal(n_kv * length * head_dim, SEED_KV, "cfg0.layer0.v").reshape(1, n_kv, length, head_dim)
    return x, k, v


def cfg4_lengths(streams: int = 32) -> np.ndarray:
    return synth_ids(streams, SEED_LENGTHS, "cfg4.lengths", 156, 3913)


def cfg4_first_ids(streams: int = 32, vocab: int = 151936) -> np.ndarray:
    return synth_ids(streams, SEED_IDS, "cfg4.first_ids", 0, vocab - 1)


def cfg4_stream_kv(stream: int, length: int, n_layers: int = 28, n_kv: int = 8, head_dim: int = 128):
    """K, V of one stream: [n_layers][n_kv][length][head_dim] N(0, 1)."""
    n = n_layers * n_kv * length * head_dim
    k = synth_normal(n, SEED_KV, f"cfg4.stream{stream}.k").reshape(n_layers, n_kv, length, head_dim)
    v = synth_normal(n, SEED_KV, f"cfg4.stream{stream}.v").reshape(n_layers, n_kv, length, head_dim)
    return k, v
