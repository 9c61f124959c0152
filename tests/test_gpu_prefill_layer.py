"""GPU parity: a prefill chunk (more than 8 tokens) through the decoder layers
on the device, against the oracle's restatement of forwardAttentionLayer /
forwardFfn (layers.ts:161-473) over the same tokens.

- The prefill attention (attn_prefill.hip, matrix cores) through
  hp_hip_gqa_attention_device at 9..512 tokens: every token attends
  causally within the window of the chunk's last position, over a ring that
  already holds the chunk (hp_gqa_attention_f32, lib.rs:538-654, with
  causalMask, layers.ts:913-925).  Bars as for the decode attention: per
  head max relative error 2^-8 (relative to max(|ref|, 0.01 rms)), at most
  2 % of the f16 outputs one step or more away.
- The attention prologue (norms, RoPE, cache append) of 300 tokens: q within
  1 f32 ulp, cache rows within one f16 step.
- A whole layer of the 42-layer model over a 128- and a 512-token chunk
  (positions up to 4095 in a 4096-slot ring) and a two-layer chunked run
  (a 64-slot sliding ring, 150 tokens, so the call runs chunks of 64, 64 and
  22 tokens, slidingRingChunkTokenCount, wasm/segment-runner.ts:181-207):
  per token err = max |got - ref| / rms(ref row).  Two effects move a row:
  the attention's order of summation moves about 1 % of its f16 outputs by
  one step, and the projections of a chunk of 64 or more tokens run on the
  fast prefill kernel (1e-4 relative).  Each feeds the next projection's
  Q8_K quantisation, which is discontinuous: a change at a block's largest
  element rescales the block and re-rounds its quants, which can move that
  token's O output by a few percent and its residual by up to ~2e-2 of the
  row rms (2.4e-2 the largest measured).  So the bars are: every row within
  LAYER_TOL, the median row within ROW_TYPICAL, and at least ROWS_CLOSE of
  the rows within 1e-3 (measured values printed).
"""
import numpy as np
import pytest

from heliopause_amd import decode as DM
from heliopause_amd import synthetic as S

pytestmark = pytest.mark.gpu

LAYER_TOL = 5e-2    # every row
ROW_TYPICAL = 1e-4  # the median row
ROWS_CLOSE = 0.75   # the fraction of rows within 1e-3
FLOOR = 0.01


@pytest.fixture(scope="module")
def D(oracle):
    from oracle import decode_layer

    return decode_layer


def _dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(torch.device("cuda:0"))


def _f16_steps(got, ref):
    g = np.asarray(got).astype(np.float16).view(np.int16).astype(np.int64)
    r = np.asarray(ref).astype(np.float16).view(np.int16).astype(np.int64)
    g = np.where(g < 0, -(g & 0x7FFF), g)
    r = np.where(r < 0, -(r & 0x7FFF), r)
    return np.abs(g - r)


def _ulps(got, ref):
    g = np.ascontiguousarray(got, np.float32).view(np.int32).astype(np.int64)
    r = np.ascontiguousarray(ref, np.float32).view(np.int32).astype(np.int64)
    g = np.where(g < 0, -(g & 0x7FFFFFFF), g)
    r = np.where(r < 0, -(r & 0x7FFFFFFF), r)
    return np.abs(g - r)


def _rel(got, ref):
    got = np.asarray(got, np.float64).reshape(-1)
    ref = np.asarray(ref, np.float64).reshape(-1)
    den = np.maximum(np.abs(ref), FLOOR * np.sqrt(np.mean(ref * ref)))
    return float(np.max(np.abs(got - ref) / den))


def _row_errs(got, ref):
    """max |got - ref| / rms(ref row) of every row."""
    g = np.asarray(got, np.float64)
    r = np.asarray(ref, np.float64)
    g, r = g.reshape(-1, g.shape[-1]), r.reshape(-1, r.shape[-1])
    return np.array([np.max(np.abs(gr - rr)) / np.sqrt(np.mean(rr * rr)) for gr, rr in zip(g, r)])


def _check_rows(got, ref, what):
    e = _row_errs(got, ref)
    worst, median, close = float(e.max()), float(np.median(e)), float(np.mean(e <= 1e-3))
    print(f"{what}: max row err {worst:.3e}, median {median:.3e}, rows within 1e-3 {close:.3f}, identical rows "
          f"{np.mean(e == 0):.3f}", flush=True)
    assert worst <= LAYER_TOL
    assert median <= ROW_TYPICAL
    assert close >= ROWS_CLOSE


ATTN_CASES = [  # tokens, nq, nkv, capacity, first position, window, query scale
    (9, 8, 2, 4096, 4087, 0, 0.25),
    (64, 8, 2, 4096, 4032, 0, 0.25),
    (100, 8, 2, 300, 1000, 0, 0.25),
    (512, 8, 2, 4096, 3584, 0, 0.0625),
    (200, 8, 2, 4096, 0, 0, 0.25),
    (130, 8, 2, 4096, 2000, 160, 0.25),
    (48, 8, 1, 128, 70, 0, 0.25),
    (33, 6, 2, 64, 40, 0, 0.25),
    (40, 2, 2, 64, 10, 0, 1.0),
]


@pytest.mark.parametrize("tokens,nq,nkv,cap,pos,window,qscale", ATTN_CASES)
def test_prefill_attention(hip, D, tokens, nq, nkv, cap, pos, window, qscale):
    import torch

    rng = np.random.default_rng(tokens * 7919 + cap + pos + nq)
    q = (rng.standard_normal((tokens, nq, 256)) * qscale).astype(np.float32)
    kc = rng.standard_normal((nkv, cap, 256)).astype(np.float16)
    vc = rng.standard_normal((nkv, cap, 256)).astype(np.float16)
    dq, dkc, dvc = _dev(q), _dev(kc.view(np.int16)), _dev(vc.view(np.int16))
    dpos = _dev(np.array([pos], np.int32))
    out = torch.empty(tokens * nq * 256, dtype=torch.float32, device="cuda:0")
    cfg = hip.attention_config(nq, nkv, cap, sliding_window=window)
    print(f"prefill attention tokens={tokens} nq={nq} nkv={nkv} cap={cap} pos={pos} window={window}", flush=True)
    hip.gqa_attention_device(cfg, dq.data_ptr(), dkc.data_ptr(), dvc.data_ptr(), dpos.data_ptr(), out.data_ptr(),
                             token_count=tokens)
    torch.cuda.synchronize()
    ref = D.decode_attention(q, kc, vc, pos, window)
    got = out.cpu().numpy().reshape(tokens, nq, 256)
    assert np.array_equal(got.astype(np.float16).astype(np.float32), got)    # castF16Rows output
    errs = [_rel(got[t, h], ref[t, h]) for t in range(tokens) for h in range(nq)]
    steps = _f16_steps(got, ref)
    print(f"max rel err {max(errs):.2e}, elements off {np.count_nonzero(steps)} of {steps.size}, "
          f"max steps {steps.max()}", flush=True)
    assert max(errs) <= 2.0 ** -8
    assert np.count_nonzero(steps) <= 0.02 * steps.size


def test_prefill_attention_prep(hip, D):
    """Norms, RoPE and the cache append of 300 tokens (one launch)."""
    import torch

    tokens, nq, nkv, cap, pos = 300, 8, 2, 512, 400
    rng = np.random.default_rng(300)
    q = (rng.standard_normal((tokens, nq, 256)) * 2).astype(np.float32)
    k = (rng.standard_normal((tokens, nkv, 256)) * 2).astype(np.float32)
    v = (rng.standard_normal((tokens, nkv, 256)) * 2).astype(np.float32)
    wq = (1 + 0.1 * rng.standard_normal(256)).astype(np.float32)
    wk = (1 + 0.1 * rng.standard_normal(256)).astype(np.float32)
    kc = rng.standard_normal((nkv, cap, 256)).astype(np.float16)
    vc = rng.standard_normal((nkv, cap, 256)).astype(np.float16)
    dkc, dvc = _dev(kc.view(np.int16)), _dev(vc.view(np.int16))
    dq, dk, dv, dwq, dwk = _dev(q), _dev(k), _dev(v), _dev(wq), _dev(wk)
    dpos = _dev(np.array([pos], np.int32))
    qo = torch.empty(tokens * nq * 256, dtype=torch.float32, device="cuda:0")
    cfg = hip.attention_config(nq, nkv, cap)
    print("prefill attention prep tokens=300", flush=True)
    hip.attention_prep_device(cfg, dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), dwq.data_ptr(), dwk.data_ptr(),
                              dpos.data_ptr(), qo.data_ptr(), dkc.data_ptr(), dvc.data_ptr(), token_count=tokens)
    torch.cuda.synchronize()
    positions = np.arange(pos, pos + tokens)
    qr = D.rope_neox(D.rms_norm_rows(q, wq, 1e-6), positions, 256, 10000.0)
    kr = D.rope_neox(D.rms_norm_rows(k, wk, 1e-6), positions, 256, 10000.0)
    vn = D.rms_norm_rows(v, None, 1e-6)
    rk, rv = kc.copy(), vc.copy()
    for t, p_ in enumerate(positions):
        rk[:, p_ % cap] = kr[t].astype(np.float16)
        rv[:, p_ % cap] = vn[t].astype(np.float16)
    assert _ulps(qo.cpu().numpy().reshape(tokens, nq, 256), qr).max() <= 1
    assert _f16_steps(dkc.cpu().numpy().view(np.float16), rk).max() <= 1
    assert _f16_steps(dvc.cpu().numpy().view(np.float16), rv).max() <= 1


def _oracle_layer(D, shape, data):
    tids = {"Q4_K": 1, "Q6_K": 3}
    w = {n: (tids[t], blocks, rows) for n, (t, blocks, rows, _) in data["weights"].items()}
    return D.Layer(weights=w, norms=dict(data["norms"]), key_cache=data["key_cache"].copy(),
                   value_cache=data["value_cache"].copy(), head_count=shape.head_count,
                   head_count_kv=shape.head_count_kv, rope_dims=shape.rope_dims,
                   rope_freq_base=shape.rope_freq_base, sliding_window=shape.sliding_window,
                   epsilon=shape.epsilon, output_scale=float(data["output_scale"]))


@pytest.mark.parametrize("tokens,kernel", [(128, 4), (128, 0), (100, 0), (512, 0)],
                         ids=["chunk128-exact", "chunk128-auto", "chunk100-auto", "chunk512-auto"])
def test_prefill_layer_matches_oracle(hip, D, tokens, kernel):
    """One layer of the model over a chunk ending at position 4095 (kernel 4:
    the bit-exact prefill projections; 0: the automatic policy, the fast
    prefill kernel from 64 tokens, whose activation tiles the norm kernel
    writes; 100 tokens leave 28 padding columns in the last tile)."""
    import torch

    hip.setMatvecKernel(kernel)
    shape = DM.ModelShape()
    seed = S.derive(S.BASE_SEED, "prefill-layer", tokens)
    data = DM.layer_host_data(shape, seed, 0)
    model = DM.HipDecodeModel(shape)
    model.add_layer(data)
    pos = shape.capacity - tokens
    x = S.activations(S.derive(seed, "x"), tokens, shape.hidden) * 4
    dx = _dev(x.reshape(-1))
    dpos = _dev(np.array([pos], np.int32))
    print(f"prefill layer tokens={tokens} kernel={kernel}", flush=True)
    try:
        model.run_layers(dx.data_ptr(), dpos.data_ptr(), tokens=tokens)
        torch.cuda.synchronize()
        got = dx.cpu().numpy().reshape(tokens, shape.hidden)
        gk = model.caches[0][0].cpu().numpy().view(np.float16)
    finally:
        model.release()
        hip.setMatvecKernel(0)
    ol = _oracle_layer(D, shape, data)
    ref = D.forward_layer(ol, x, pos)
    _check_rows(got, ref, f"prefill layer tokens={tokens} kernel={kernel}")
    slots = [(pos + t) % shape.capacity for t in range(tokens)]
    if kernel == 4:   # bit-exact K projection: cache rows within one f16 step
        assert _f16_steps(gk[:, slots], ol.key_cache[:, slots]).max() <= 1
    else:             # K within 1e-4: cache rows within two f16 steps at their scale
        cache_err = float(_row_errs(gk[:, slots].astype(np.float32), ol.key_cache[:, slots].astype(np.float32)).max())
        print(f"cache rows: max err {cache_err:.3e} of the row rms", flush=True)
        assert cache_err <= 4e-3


def test_prefill_chunks_through_layers(hip, D):
    """150 tokens through two small layers with a 64-slot ring: the call
    runs chunks of 64, 64 and 22 tokens, each through both layers in turn, as
    the WASM runner's chunked path does; then the output norm."""
    import torch

    hip.setMatvecKernel(4)
    shape = DM.ModelShape(hidden=512, head_count=2, head_count_kv=1, ffn=1024, capacity=64, sliding_window=48)
    seed = S.derive(S.BASE_SEED, "prefill-chunks")
    datas = [DM.layer_host_data(shape, seed, i) for i in range(2)]
    onorm = (1 + 0.1 * S.normal(S.derive(seed, "onorm"), shape.hidden)).astype(np.float32)
    model = DM.HipDecodeModel(shape)
    for d in datas:
        model.add_layer(d)
    model.output_norm = _dev(onorm)
    tokens, pos = 150, 5
    x = S.activations(S.derive(seed, "x"), tokens, shape.hidden) * 4
    dx = _dev(x.reshape(-1))
    dpos = _dev(np.array([pos], np.int32))
    out = torch.empty(tokens * shape.hidden, dtype=torch.float32, device="cuda:0")
    print("prefill chunks 150 tokens, ring 64", flush=True)
    try:
        model.run_layers(dx.data_ptr(), dpos.data_ptr(), out.data_ptr(), tokens=tokens)
        torch.cuda.synchronize()
        got = dx.cpu().numpy().reshape(tokens, shape.hidden)
        got_out = out.cpu().numpy().reshape(tokens, shape.hidden)
    finally:
        model.release()
        hip.setMatvecKernel(0)
    ols = [_oracle_layer(D, shape, d) for d in datas]
    ref = np.empty_like(x)
    for c0 in range(0, tokens, shape.capacity):
        h = x[c0:c0 + shape.capacity].copy()
        for ol in ols:
            h = D.forward_layer(ol, h, pos + c0)
        ref[c0:c0 + len(h)] = h
    ref_out = D.rms_norm_rows(ref, onorm, shape.epsilon)
    _check_rows(got, ref, "chunked hidden")
    _check_rows(got_out, ref_out, "chunked output norm")
