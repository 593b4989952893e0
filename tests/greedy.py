"""Greedy-token comparison with a near-tie certificate (test helper).

Two greedy streams computed in different floating-point orders may part at
a step whose top two candidates are closer than the logit tolerance. The
streams must be identical up to the first divergence, and there the oracle's
scores (its logits after the repetition penalty over the tokens generated so
far, the rule the choice was made under) must hold a second candidate within
`rel` * max|logit| of the best, with the GPU's token among those candidates.
After a certified divergence the streams are free to differ.
"""
from __future__ import annotations

import numpy as np

from oracle import oracle as O


def penalised(logits, context, penalty: float) -> np.ndarray:
    """The scores the greedy rule compares: the repetition penalty over
    `context` (sampler.rs:599-613) unless |penalty - 1| < 0.01."""
    l = np.array(logits, dtype=np.float32, copy=True)
    if abs(np.float32(penalty) - np.float32(1.0)) >= np.float32(0.01):
        ctx = np.ascontiguousarray(np.asarray(context, dtype=np.uint32))
        O.lib().jo_repetition_penalty(l, l.size, ctx, ctx.size, np.float32(penalty))
    return l


def first_divergence(got, want) -> int:
    return next((i for i, (a, b) in enumerate(zip(got, want)) if a != b), min(len(got), len(want)))


def assert_same_or_near_tie(got, want, oracle_logits, penalty: float, rel: float = 2e-3, prompt=()):
    """got/want: token lists; oracle_logits[i]: the oracle's raw logits at
    decode step i. Returns the index of the first divergence (len(want) when
    the streams are identical)."""
    i = first_divergence(got, want)
    if i == len(want) and len(got) == len(want):
        return i
    assert i < len(oracle_logits), (i, got, want)
    s = penalised(oracle_logits[i], want[:i], penalty)
    tol = rel * float(np.max(np.abs(s)))
    best = float(np.max(s))
    near = np.flatnonzero(s >= best - tol)
    assert near.size >= 2 and got[i] in near, (
        f"streams part at step {i} (GPU {got[i]}, oracle {want[i]}) without a near tie: "
        f"oracle top-2 gap {best - float(np.sort(s)[-2]):.3e} against {tol:.3e}")
    return i
