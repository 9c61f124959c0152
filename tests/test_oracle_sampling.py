"""The sampling oracle (oracle/sampling.py, generation.ts:40-165) and the
exp it uses (hpo_exp), pinned by the reference's own known answers and by
the JS engine's Math.exp outputs.

Known answers: packages/engine/test/generation.test.ts -- defaults and
validation (12-42), the first draw of the default-seeded generator and the
non-greedy pick of id 11 (44-64), the top-p boundary token and greedy top-1
(66-81).  exp: tests/golden/v8_exp.json, Math.exp of 23,194 inputs written by
tests/golden/make_v8_exp.js under this container's Node.
"""
import base64
import json
import math
from pathlib import Path

import numpy as np
import pytest

from heliopause_amd import hip_kernels as H
from oracle import oracle as O
from oracle import sampling as SM

GOLDEN = Path(__file__).resolve().parent / "golden"


def test_exp_matches_js_engine():
    data = json.loads((GOLDEN / "v8_exp.json").read_text())
    xs = np.frombuffer(base64.b64decode(data["x_f64le_base64"]), dtype=np.float64)
    ys = np.frombuffer(base64.b64decode(data["exp_f64le_base64"]), dtype=np.float64)
    assert xs.size == data["count"] > 20000
    got = np.array([O.exp(float(x)) for x in xs])
    same = (got.view(np.uint64) == ys.view(np.uint64)) | (np.isnan(got) & np.isnan(ys))
    assert same.all(), xs[~same][:5]
    assert O.exp(1.0) == 2.718281828459045   # the JS engine's exact answer for e


def test_reference_known_answers():
    rng = SM.DeterministicRng(SM.DEFAULT_SAMPLING_SEED)
    assert rng() == 0.9744378970935941                               # generation.test.ts:46
    four = [{"id": 10, "value": 3.0}, {"id": 11, "value": 2.0}, {"id": 12, "value": 1.0}, {"id": 13, "value": 0.0}]
    opts = {"doSample": True, "temperature": 1.0, "topP": 0.8, "topK": 4}
    assert SM.sample_next_token(four, opts, SM.DeterministicRng(SM.DEFAULT_SAMPLING_SEED)) == 11   # 48-63
    three = four[:3]
    greedy = {"doSample": False, "temperature": 1.0, "topP": 0.1, "topK": 3}
    assert SM.sample_next_token(three, greedy, lambda: 0.99) == 10    # 73-76
    boundary = {"doSample": True, "temperature": 1.0, "topP": 0.8, "topK": 3}
    assert SM.sample_next_token(three, boundary, lambda: 0.99) == 11  # 77-80


@pytest.mark.parametrize("resolve", [SM.resolve_options, H.resolveGenerationSamplingOptions],
                         ids=["oracle", "product"])
def test_resolve_options(resolve):
    r = resolve()                                                     # generation.test.ts:12-30
    assert (r["doSample"], r["temperature"], r["topP"], r["topK"], r["logitsTopK"], r["seed"]) == \
        (True, 1.0, 0.95, 64, 64, 0x48454C49)
    assert resolve(doSample=False, topK=64)["logitsTopK"] == 1       # 32-42
    assert resolve(temperature=0, topK=64)["logitsTopK"] == 1
    assert resolve(topK=64.9)["topK"] == 64
    for kw, word in (({"temperature": -1}, "temperature"), ({"topP": 0}, "topP"), ({"topP": 1.1}, "topP"),
                     ({"topK": 0}, "topK")):
        with pytest.raises(ValueError, match=word):
            resolve(**kw)
    assert resolve(seed=-1)["seed"] == 0xFFFFFFFF                     # floor(seed) >>> 0


def test_rng_is_the_stated_32_bit_mix():
    """An independent statement of the generator in signed 32-bit JS terms
    (ToInt32 after each operation), against the oracle's unsigned one."""
    def to_i32(v):
        v &= 0xFFFFFFFF
        return v - (1 << 32) if v >= 1 << 31 else v

    def js_rng(seed):
        state = seed & 0xFFFFFFFF
        while True:
            state = (state + 0x6D2B79F5) & 0xFFFFFFFF
            value = to_i32(state)
            value = to_i32((to_i32(value ^ ((value & 0xFFFFFFFF) >> 15)) * to_i32(value | 1)))
            value = to_i32(value ^ (value + to_i32(to_i32(value ^ ((value & 0xFFFFFFFF) >> 7)) * to_i32(value | 61))))
            yield ((value ^ ((value & 0xFFFFFFFF) >> 14)) & 0xFFFFFFFF) / 4294967296

    for seed in (0, 1, SM.DEFAULT_SAMPLING_SEED, 0xFFFFFFFF, 123456789):
        a, b = SM.DeterministicRng(seed), js_rng(seed)
        draws = [a() for _ in range(200)]
        assert draws == [next(b) for _ in range(200)]
        assert all(0 <= d < 1 for d in draws)


def _candidates(rng, n, spread=4.0):
    vals = np.sort((rng.standard_normal(n) * spread).astype(np.float32))[::-1]
    if n > 6:
        vals[3:6] = vals[3]                                            # ties, broken by id
    ids = rng.permutation(100000)[:n]
    cands = [{"id": int(i), "value": float(v)} for i, v in zip(ids, vals)]
    return sorted(cands, key=lambda c: (-c["value"], c["id"]))


@pytest.mark.parametrize("seed", range(20))
def test_distribution_properties(seed):
    """Closed-form properties of the oracle's distribution: the nucleus is the
    shortest prefix whose softmax mass reaches topP, the probabilities are
    exp((v - max)/T) normalised, and they sum to 1."""
    rng = np.random.default_rng(seed)
    cands = _candidates(rng, int(rng.integers(1, 65)))
    opts = {"doSample": True, "temperature": float(rng.choice([0.3, 0.7, 1.0, 1.7])),
            "topP": float(rng.choice([0.5, 0.9, 0.95, 1.0])), "topK": int(rng.integers(1, 70))}
    dist = SM.token_sampling_distribution(cands, opts)
    top = cands[:min(len(cands), opts["topK"])]
    assert [d["id"] for d in dist] == [c["id"] for c in top[:len(dist)]]
    if opts["topP"] < 1 and len(top) > 1:
        vals = np.array([c["value"] for c in top])
        mass = np.exp(vals - vals.max())
        mass /= mass.sum()
        cum = np.cumsum(mass)
        n = len(dist)
        assert n == len(top) or cum[n - 1] >= opts["topP"] - 1e-12
        assert n == 1 or cum[n - 2] < opts["topP"] + 1e-12
    p = np.array([d["probability"] for d in dist])
    v = np.array([d["value"] for d in dist]) / opts["temperature"]
    ref = np.exp(v - v.max())
    assert np.allclose(p, ref / ref.sum(), rtol=1e-13, atol=1e-300)
    assert abs(p.sum() - 1) < 1e-12


def test_degenerate_softmax():
    """All -inf logits: the softmax total is NaN, so the first candidate gets
    probability 1 (generation.ts:161-163)."""
    cands = [{"id": 5, "value": -math.inf}, {"id": 7, "value": -math.inf}]
    dist = SM.token_sampling_distribution(cands, {"doSample": True, "temperature": 1.0, "topP": 1.0, "topK": 2})
    assert [d["probability"] for d in dist] == [1.0, 0.0]
