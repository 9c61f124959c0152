"""GPU parity: next-token sampling (hp_hip_sample_device and the fused
head + top-k + sample entry point) against the oracle's restatement of
generation.ts:78-165.  Bar: tokens, nucleus sizes and the generator state
identical; probabilities bit-identical doubles.
"""
import math

import numpy as np
import pytest

from heliopause_amd import hip_kernels as H
from heliopause_amd import synthetic as S
from oracle import sampling as SM

pytestmark = pytest.mark.gpu

OPTION_SETS = [
    {"doSample": True, "temperature": 1.0, "topP": 0.95, "topK": 64},     # the defaults
    {"doSample": True, "temperature": 0.7, "topP": 0.5, "topK": 40},
    {"doSample": True, "temperature": 2.0, "topP": 1.0, "topK": 5},
    {"doSample": True, "temperature": 1e-3, "topP": 0.9, "topK": 64},
    {"doSample": True, "temperature": 1.0, "topP": 1e-6, "topK": 64},
    {"doSample": True, "temperature": 1.3, "topP": 0.99, "topK": 1},
    {"doSample": True, "temperature": 1.0, "topP": 0.8, "topK": 100},
    {"doSample": False, "temperature": 1.0, "topP": 0.95, "topK": 64},     # greedy: no draw
    {"doSample": True, "temperature": 0.0, "topP": 0.95, "topK": 64},      # greedy: no draw
]


def _columns(rng, cols, k, count, spread):
    ids = np.zeros((cols, k), np.uint32)
    vals = np.zeros((cols, k), np.float32)
    for c in range(cols):
        v = np.sort((rng.standard_normal(count) * spread).astype(np.float32))[::-1].copy()
        if count > 8:
            v[2:5] = v[2]                                   # ties, ordered by id
        if c % 3 == 2:
            v[count // 2:] = -np.inf                         # masked tail
        i = rng.permutation(262144)[:count].astype(np.uint32)
        order = sorted(range(count), key=lambda j: (-float(v[j]), int(i[j])))
        ids[c, :count] = i[order]
        vals[c, :count] = v[order]
    return ids, vals


@pytest.mark.parametrize("opts", OPTION_SETS, ids=[f"opt{i}" for i in range(len(OPTION_SETS))])
@pytest.mark.parametrize("k,count", [(64, 64), (40, 40), (64, 17), (1, 1)])
def test_sample_device_matches_oracle(opts, k, count):
    import torch

    rng = np.random.default_rng(k * 100 + count)
    cols = 6
    spread = 3.0 if opts["temperature"] != 1e-3 else 0.01
    ids, vals = _columns(rng, cols, k, count, spread)
    seed = 0x48454C49 + k
    dev = torch.device("cuda:0")
    d_ids = torch.from_numpy(ids.view(np.int32)).to(dev)
    d_vals = torch.from_numpy(vals).to(dev)
    state = torch.from_numpy(np.array([seed], np.uint32).view(np.int32)).to(dev)
    tokens = torch.zeros(cols, dtype=torch.int32, device=dev)
    kept = torch.zeros(cols, dtype=torch.int32, device=dev)
    probs = torch.zeros(cols * k, dtype=torch.float64, device=dev)
    print(f"sample k={k} count={count} opts={opts}", flush=True)
    for call in range(2):                                   # the state carries over between calls
        H.sample_device(d_ids.data_ptr(), d_vals.data_ptr(), cols, k, count, opts, state.data_ptr(),
                        tokens.data_ptr(), probs.data_ptr(), kept.data_ptr())
        torch.cuda.synchronize()
        if call == 0:
            first = (tokens.cpu().numpy().copy(), kept.cpu().numpy().copy(), probs.cpu().numpy().copy())
    ref_rng = SM.DeterministicRng(seed)
    for call in range(2):
        got_tokens, got_kept, got_probs = first if call == 0 else \
            (tokens.cpu().numpy(), kept.cpu().numpy(), probs.cpu().numpy())
        got_probs = got_probs.reshape(cols, k)
        for c in range(cols):
            cands = [{"id": int(ids[c, j]), "value": float(vals[c, j])} for j in range(count)]
            dist = SM.token_sampling_distribution(cands, opts)
            tok = SM.sample_next_token(cands, opts, ref_rng)
            assert got_tokens[c] == tok, (call, c)
            assert got_kept[c] == len(dist), (call, c)
            want = np.array([d["probability"] for d in dist], np.float64)
            assert np.array_equal(got_probs[c, :len(dist)].view(np.uint64), want.view(np.uint64)), (call, c)
    assert int(state.cpu().numpy().view(np.uint32)[0]) == ref_rng.state


@pytest.mark.parametrize("m,softcap", [(1, 0.0), (4, 30.0)])
def test_head_topk_sample_matches_oracle(hip, oracle, m, softcap):
    """forwardOutput + sampleNextToken per column in one call."""
    rows, k_in = 20000, 2560
    seed = S.derive(S.config_seed(4), "sample-head", m)
    w = S.q6_k_blocks(seed, rows, k_in)
    x = S.activations(seed, m, k_in) * 3.0
    opts = H.resolveGenerationSamplingOptions(temperature=0.8, topP=0.9, topK=40, seed=777)
    state = H.HipSamplingState(opts["seed"])
    h = hip.createHipQuantizedWeightHandle("Q6_K", w, k_in, rows)
    print(f"head sample m={m}", flush=True)
    try:
        got = H.matMulQuantizedHipResidentTopKSample(h, x, k_in, m, opts, state, softcap=softcap)
    finally:
        hip.releaseHipQuantizedWeightHandle(h)
    logits = oracle.matmul(3, w, x, rows, threads=8).reshape(m, rows)
    ref_rng = SM.DeterministicRng(777)
    for c in range(m):
        row = logits[c] if softcap == 0 else np.array([oracle.softcap(float(v), softcap) for v in logits[c]],
                                                      np.float32)
        ids, vals = oracle.topk(row, 40)
        cands = [{"id": int(i), "value": float(v)} for i, v in zip(ids, vals)]
        dist = SM.token_sampling_distribution(cands, opts)
        assert got[c]["token"] == SM.sample_next_token(cands, opts, ref_rng)
        assert [d["id"] for d in got[c]["distribution"]] == [d["id"] for d in dist]
        gp = np.array([d["probability"] for d in got[c]["distribution"]])
        wp = np.array([d["probability"] for d in dist])
        assert np.array_equal(gp.view(np.uint64), wp.view(np.uint64))
    assert state.state.value == ref_rng.state
    assert not math.isnan(got[0]["distribution"][0]["probability"])
