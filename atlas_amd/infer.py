"""Host mirror of the reference's `atlas-infer` facade.

``StigmergicHook`` (crates/atlas-infer/src/hook.rs:58-72), ``PheromoneDeposit``
(crates/atlas-infer/src/engine.rs:51-59) and ``InferEngine``
(engine.rs:77-218): without a hook, ``generate`` runs the GPU-resident greedy /
sampled decode; with a hook it runs the hooked path, whose per-token deposit
is the sum of max(delta, 0) over the layers that returned Some and the count
of those layers.  Unlike the reference (which routes hooked generation to its
CPU forward), the hooked path here is the HIP engine with a per-layer
download of the hidden state.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Callable, List, Optional, Sequence, Tuple

import numpy as np

from .model import OlmoModel, SamplingConfig


class StigmergicHook:
    """hook.rs:58-72: on_layer(layer_idx, hidden) -> Optional[float]."""

    def on_layer(self, layer_idx: int, hidden: np.ndarray) -> Optional[float]:
        raise NotImplementedError


@dataclass
class PheromoneDeposit:
    token_id: int
    total_delta: float
    layers_fired: int


class InferEngine:
    def __init__(self, model: OlmoModel):
        self.model = model
        self.hook: Optional[StigmergicHook] = None

    def with_hook(self, hook: StigmergicHook) -> "InferEngine":
        self.hook = hook
        return self

    def set_hook(self, hook: Optional[StigmergicHook]) -> None:
        self.hook = hook

    def has_hook(self) -> bool:
        return self.hook is not None

    def reset(self) -> None:
        self.model.reset()

    def generate(self, prompt: Sequence[int], max_new: int,
                 cfg: SamplingConfig) -> Tuple[List[int], List[PheromoneDeposit]]:
        """engine.rs:132-163."""
        if self.hook is None:
            return self.model.generate_with_sampling(prompt, max_new, cfg), []
        toks, raw = self.model.generate_with_sampling_hooked(prompt, max_new, cfg,
                                                             self.hook.on_layer)
        return toks, [PheromoneDeposit(t, d, f) for (t, d, f) in raw]

    def generate_streaming(self, prompt: Sequence[int], max_new: int, cfg: SamplingConfig,
                           on_token: Callable[[int, Optional[PheromoneDeposit]], bool]) -> int:
        """engine.rs:171-218."""
        if self.hook is None:
            count = [0]

            def cb(t):
                count[0] += 1
                return on_token(t, None)

            self.model.generate_streaming(prompt, max_new, cfg, cb)
            return count[0]
        toks, raw = self.model.generate_with_sampling_hooked(prompt, max_new, cfg,
                                                             self.hook.on_layer)
        count = 0
        for (t, d, f) in raw:
            count += 1
            if not on_token(t, PheromoneDeposit(t, d, f)):
                break
        return count
