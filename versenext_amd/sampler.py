"""Sampler / GreedySampler with the reference's interface
(packages/verse_infra/verse_infra/verse_inference/sampler.py:28-158) on the
"rocm" backend.

Same constructor arguments, defaults and ValueErrors; sample(logits) returns
the int token id.  The draw runs on the GPU (vnx_sampler_sample: temperature,
top-k, softmax, top-p and the inverse-CDF draw in one launch); the one uniform
it needs per call comes from numpy's default_rng(seed) when a seed is given,
else from numpy's global legacy stream, as the reference draws its choice
from either (sampler.py:64, :135-137), and reaches the kernel as the float64
value numpy's choice would compare against the CDF.
"""
from __future__ import annotations

from typing import Optional

import numpy as np


class Sampler:
    def __init__(self, temperature: float = 1.0, top_k: int = 0, top_p: float = 1.0, seed: Optional[int] = None,
                 device: str = "rocm"):
        if temperature < 0.0:
            raise ValueError(f"temperature must be >= 0, got {temperature}")
        if top_k < 0:
            raise ValueError(f"top_k must be >= 0, got {top_k}")
        if not 0.0 < top_p <= 1.0:
            raise ValueError(f"top_p must be in (0, 1], got {top_p}")
        self.temperature = float(temperature)
        self.top_k = int(top_k)
        self.top_p = float(top_p)
        self.seed = seed
        self._rng = np.random.default_rng(seed) if seed is not None else None
        self._device = device
        self._backend = None

    def _hip(self):
        if self._backend is None:
            from .device import get_backend
            self._backend = get_backend(self._device)
        return self._backend

    def _uniform(self) -> float:
        rng = self._rng if self._rng is not None else np.random
        return float(rng.random())

    def sample(self, logits) -> int:
        """One token id from logits (vocab_size,) (any array-like or tensor)."""
        hip = self._hip()
        x = np.asarray(logits, dtype=np.float32).reshape(-1) if not hasattr(logits, "device") else logits
        if getattr(x, "size", None) == 0 or (hasattr(x, "numel") and x.numel() == 0):
            raise ValueError("logits is empty")
        # the float64 uniform numpy's choice compares against the CDF, unrounded
        u = np.array([self._uniform() if self.temperature != 0.0 else 0.0], np.float64)
        ids = hip.sampler_sample(x.reshape(1, -1), u, self.temperature, self.top_k, self.top_p)
        return int(ids.cpu()[0])

    def greedy(self, logits) -> int:
        """argmax of the logits (numpy.argmax order), on the device."""
        x = np.asarray(logits, dtype=np.float32).reshape(1, -1) if not hasattr(logits, "device") else logits
        ids = self._hip().sampler_sample(x.reshape(1, -1), np.zeros(1, np.float32), 0.0)
        return int(ids.cpu()[0])

    def __repr__(self) -> str:
        return (f"Sampler(temperature={self.temperature}, top_k={self.top_k}, "
                f"top_p={self.top_p}, seed={self.seed!r})")


class GreedySampler(Sampler):
    """Always the argmax (temperature 0)."""

    def __init__(self, device: str = "rocm"):
        super().__init__(temperature=1.0, top_k=0, top_p=1.0, device=device)

    def sample(self, logits) -> int:
        return self.greedy(logits)


def cometspark_sample(hip, logits, temperature: float, top_k: Optional[int] = None, calib_factor=None,
                      uniforms=None, rng=None):
    """The per-step sampling of CometSparkNexLM._generate_with_logits
    (packages/verse_nex/verse_nex/cometspark.py:886-910) for logits (B, V), in
    one vnx_sampler_sample launch: the logit calibration when calib_factor is
    not None (a VMPC-compressed model, :922-948), temperature <= 0 -> argmax,
    else logits / max(temperature, 1e-8), top_k > 0 -> exactly min(top_k, V)
    tokens (argpartition, ties by lower id), softmax, one draw per row with
    uniforms[b] (drawn from rng, default numpy.random.default_rng(), when
    None).  Returns the (B,) int64 token ids on the device."""
    x = logits
    B = x.shape[0]
    T = float(temperature)
    k = int(top_k) if top_k else 0
    if T <= 0:
        u = np.zeros(B, np.float32)
        return hip.sampler_sample(x, u, 0.0, calib_factor=calib_factor)
    if uniforms is None:
        uniforms = (rng if rng is not None else np.random.default_rng()).random(B)   # float64, as choice uses it
    return hip.sampler_sample(x, uniforms, max(T, 1e-8), k, 1.0, exact_k=True, calib_factor=calib_factor)


__all__ = ["Sampler", "GreedySampler", "cometspark_sample"]
