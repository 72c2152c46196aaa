"""Token sampling on the HIP path -- the engine's Sampler (src/sampler.rs:6-43)
and Qwen2Model::sample_token (src/models.rs:385-432).

  temperature == 0     greedy: luc_argmax (sampling.cu)
  top_p < 1            GPU top-k / top-p: luc_sort_and_sample (32-partition
                       top-k filter, bitonic sort, softmax, nucleus cut, draw)
  otherwise            the reference samples on the host (Sampler::sample over
                       the logits copied back); that CPU sampler is not part of
                       this library, and such a call raises.

top_k is normalised as Sampler::new does (sampler.rs:19-23): 0 -> 1024, else
the next power of two, clamped to [32, 1024].  The reference draws rand_val
from an unseeded thread RNG (models.rs:413); here it comes from the sampler's
own seeded generator, a float32 uniform in [0, 1), so a run can be repeated.
"""
from __future__ import annotations

import numpy as np
import torch

SORT_BUFFER_BYTES = 1024 * 8  # the engine's sort_buffer (models.rs:171-174)


def normalize_top_k(top_k: int) -> int:
    """Sampler::new's top_k rule (sampler.rs:19-23)."""
    if top_k == 0:
        return 1024
    p = 1
    while p < top_k:
        p *= 2
    return min(max(p, 32), 1024)


class Sampler:
    """Sampling settings and the random stream of one generation."""

    def __init__(self, seed=None, temperature: float = 0.0, top_p: float = 1.0, top_k: int = 0):
        self.rng = np.random.default_rng(seed)
        self.temperature = float(temperature)
        self.top_p = float(top_p)
        self.top_k = normalize_top_k(int(top_k))

    def is_greedy(self) -> bool:
        return self.temperature == 0.0

    def next_rand(self) -> float:
        return float(self.rng.random(dtype=np.float32))


class DeviceSampler:
    """The device buffers sample_token uses (models.rs:45-46, 168-174) and the
    dispatch between greedy and top-p sampling."""

    def __init__(self, lib, device):
        self.lib = lib
        self.idx = torch.zeros(1, dtype=torch.int32, device=device)
        self.sort_buffer = torch.zeros(SORT_BUFFER_BYTES // 4, dtype=torch.int32, device=device)

    def sample(self, logits: torch.Tensor, sampler: Sampler) -> int:
        """Token id drawn from one bf16 logits row."""
        if sampler.is_greedy():
            self.lib.argmax(logits, self.idx)
        elif sampler.top_p < 1.0:
            self.lib.sort_and_sample(logits, sampler.top_p, sampler.top_k, sampler.next_rand(),
                                     self.sort_buffer, self.idx)
        else:
            raise NotImplementedError(
                "temperature sampling without top_p < 1 runs on the host in the reference "
                "(Sampler::sample); this library provides the GPU paths only")
        return int(self.idx.cpu().item())
