"""Pure-Python restatement of the engine's token sampling (the oracle for
heliopause_amd/csrc/sample.hip).

TEST INFRASTRUCTURE ONLY: only tests/ may import this module.

Follows packages/engine/src/generation.ts:
  resolve_options             resolveGenerationSamplingOptions  40-76
  DeterministicRng            createDeterministicRng            78-87
  sample_next_token           sampleNextToken                   89-108
  token_sampling_distribution tokenSamplingDistribution         110-133
  _apply_top_p                applyTopP                         135-155
  _softmax                    softmax                           157-165
JS numbers are IEEE doubles, as Python floats are; Math.exp is the oracle's
restatement of the JS engine's exp (hpo_exp, pinned to Math.exp outputs);
Math.imul and the >>> 0 conversions are 32-bit wrapping integer operations.
"""
from __future__ import annotations

import math

from . import oracle as O

DEFAULT_SAMPLING_SEED = 0x48454C49
DEFAULT = {"doSample": True, "temperature": 1.0, "topP": 0.95, "topK": 64}
_M = 0xFFFFFFFF


def resolve_options(doSample=None, temperature=None, topP=None, topK=None, seed=None) -> dict:
    d = DEFAULT["doSample"] if doSample is None else doSample
    t = DEFAULT["temperature"] if temperature is None else temperature
    p = DEFAULT["topP"] if topP is None else topP
    k = DEFAULT["topK"] if topK is None else topK
    s = DEFAULT_SAMPLING_SEED if seed is None else seed
    if not math.isfinite(t) or t < 0:
        raise ValueError("temperature must be a finite number greater than or equal to 0.")
    if not math.isfinite(p) or p <= 0 or p > 1:
        raise ValueError("topP must be a finite number in the range (0, 1].")
    if not math.isfinite(k) or k < 1:
        raise ValueError("topK must be a positive finite number.")
    if not math.isfinite(s):
        raise ValueError("seed must be a finite number.")
    k = max(1, math.floor(k))
    greedy = d is False or t == 0
    return {"doSample": d, "temperature": t, "topP": p, "topK": k, "seed": math.floor(s) & _M,
            "logitsTopK": 1 if greedy else k}


def _imul(a: int, b: int) -> int:
    return (a * b) & _M


class DeterministicRng:
    """createDeterministicRng: a 32-bit state advanced by 0x6d2b79f5 per draw."""

    def __init__(self, seed):
        self.state = math.floor(seed) & _M

    def __call__(self) -> float:
        self.state = (self.state + 0x6D2B79F5) & _M
        v = self.state
        v = _imul(v ^ (v >> 15), v | 1)
        v = v ^ ((v + _imul(v ^ (v >> 7), v | 61)) & _M)
        return ((v ^ (v >> 14)) & _M) / 4294967296.0


def _softmax(values):
    m = -math.inf
    for v in values:   # Math.max: NaN if any argument is NaN
        m = math.nan if (math.isnan(m) or math.isnan(v)) else max(m, v)
    e = [O.exp(v - m) for v in values]
    total = 0.0
    for x in e:
        total = total + x
    if total <= 0 or not math.isfinite(total):
        return [1.0 if i == 0 else 0.0 for i in range(len(values))]
    return [x / total for x in e]


def _apply_top_p(candidates, top_p):
    if top_p >= 1 or len(candidates) <= 1:
        return candidates
    probs = _softmax([c["value"] for c in candidates])
    kept, cumulative = [], 0.0
    for c, p in zip(candidates, probs):
        kept.append(c)
        cumulative += p
        if cumulative >= top_p:
            break
    return kept if kept else candidates[:1]


def _greedy(opts) -> bool:
    return opts["doSample"] is False or opts["temperature"] == 0


def token_sampling_distribution(candidates, opts):
    """[{id, value, probability}]; candidates are {id, value} with f64 values."""
    if not candidates:
        raise ValueError("Cannot sample from an empty candidate list.")
    ordered = sorted(candidates, key=lambda c: (-c["value"], c["id"]))   # finite values
    if _greedy(opts):
        return [dict(ordered[0], probability=1.0)]
    top = ordered[: max(1, math.floor(opts["topK"]))]
    nucleus = _apply_top_p(top, opts["topP"])
    probs = _softmax([c["value"] / opts["temperature"] for c in nucleus])
    return [dict(c, probability=p) for c, p in zip(nucleus, probs)]


def sample_next_token(candidates, opts, rng) -> int:
    dist = token_sampling_distribution(candidates, opts)
    if _greedy(opts):
        return dist[0]["id"]
    draw = rng()
    cumulative = 0.0
    for c in dist:
        cumulative += c["probability"]
        if draw < cumulative:
            return c["id"]
    return dist[-1]["id"]
