"""Temperature / top-p sampling of the next token from the step's logits.

The reference samples on the host from the logits it reads back
(`sampleToken`, Sources/M1MoE/InferenceEngine.swift:550-575); so does this
mirror, from the f32 logits the GPU step returns.  Arithmetic is f32 and in
the reference's order: probabilities exp((l - max) / T) with a sequential
sum, the nucleus taken in descending probability until its running sum
reaches top_p, then r uniform in [0, nucleus sum) walked down the nucleus.
Equal probabilities are ordered by the lower index (Swift's sort is not
stable, so the reference leaves that order unspecified).  temperature <= 0
is the greedy argmax (:552-556).
"""
from __future__ import annotations

from typing import Optional

import numpy as np


def greedy(logits: np.ndarray) -> int:
    """:552-556: a scan from index 0 with a strict >."""
    x = np.asarray(logits, dtype=np.float32)
    if np.isnan(x[0]):
        return 0
    finite = np.where(np.isnan(x), -np.inf, x)
    return int(np.argmax(finite))  # first index of the maximum


def sample_token(logits: np.ndarray, temperature: float, top_p: float,
                 u: Optional[float] = None, rng: Optional[np.random.Generator] = None) -> int:
    """:557-574.  u in [0, 1) is the uniform draw (from rng when None)."""
    if temperature <= 0:
        return greedy(logits)
    x = np.asarray(logits, dtype=np.float32)
    mx = np.float32(x.max())
    probs = np.exp((x - mx) / np.float32(temperature)).astype(np.float32)
    total = np.add.accumulate(probs, dtype=np.float32)[-1]  # sequential f32 sum
    probs = probs * (np.float32(1.0) / total)
    order = np.argsort(-probs, kind="stable")
    cumul = np.add.accumulate(probs[order], dtype=np.float32)
    k = int(np.argmax(cumul >= np.float32(top_p))) if bool((cumul >= np.float32(top_p)).any()) \
        else order.size - 1
    nucleus = order[:k + 1]
    ns = cumul[k]  # the nucleus' own sequential sum
    if u is None:
        u = (rng or np.random.default_rng()).random(dtype=np.float32)
    r = np.float32(u) * ns
    for idx in nucleus:
        r = np.float32(r - probs[idx])
        if r <= 0:
            return int(idx)
    return int(nucleus[-1])
