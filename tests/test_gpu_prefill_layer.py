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
- Three layers of the model over a 512-token chunk on the automatic policy
  (fast prefill kernel, activation tiles written by the norm kernel,
  block-range sums handed from each layer's down launch to the next
  layer's norm) against the oracle's forward_layer chain, to the same row
  bars, then the last token through the output norm and the Q6_K
  262144 x 2560 head: its top-40 ids equal the oracle's end to end.
"""
import numpy as np
import pytest

from heliopause_amd import decode as DM
from heliopause_amd import synthetic as S

pytestmark = pytest.mark.gpu

LAYER_TOL = 3e-2    # every row
ROW_TYPICAL = 1e-4  # the median row
ROWS_CLOSE = 0.75   # the fraction of rows within 1e-3
TILE_OFF = 0.5      # the largest fraction of a 64-row tile beyond 1e-3
CHAIN_TOL = 6e-2    # every row after two layers on the fast prefill kernel
# Every row of a 512-token layer on a seed where one attention output lands
# an f16 step away at the largest element of one of O's Q8_K input blocks:
# the block re-rounds and that token's residual moves by up to 0.199 of its
# rms (0.174 with the bit-exact projections, so the projections are not the
# cause; test_prefill_stages_512_auto pins them stage by stage).
ATTN_STEP_TOL = 0.25
STAGE_TOL = 1e-4    # projections on the automatic policy, relative (FLOOR)
DOWN_TOL = 2e-4     # down on the GeGLU output: outputs near the floor carry the
                    # fast kernel's f32 accumulation order (1.29e-4 measured)
SWAP_TOL = 1e-2     # any row, one GPU stage output swapped into the oracle chain
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


def _check_rows(got, ref, what, tol=None):
    """The row bars, and that the rows beyond 1e-3 are spread over the
    chunk: no 64-token tile (the projections' column tile) has more than
    TILE_OFF of its rows beyond 1e-3, which a fault confined to one tile
    would break."""
    e = _row_errs(got, ref)
    worst, median, close = float(e.max()), float(np.median(e)), float(np.mean(e <= 1e-3))
    tiles = [np.mean(e[t:t + 64] > 1e-3) for t in range(0, len(e) - 15, 64)]
    tile_off = float(max(tiles)) if tiles else 0.0
    print(f"{what}: max row err {worst:.3e}, median {median:.3e}, rows within 1e-3 {close:.3f}, identical rows "
          f"{np.mean(e == 0):.3f}, worst tile off {tile_off:.3f}", flush=True)
    assert worst <= (LAYER_TOL if tol is None else tol)
    assert median <= ROW_TYPICAL
    assert close >= ROWS_CLOSE
    assert tile_off <= TILE_OFF


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


@pytest.mark.parametrize("kernel", [4, 0], ids=["exact", "auto"])
def test_prefill_chunks_through_layers(hip, D, kernel):
    """150 tokens through two small layers with a 64-slot ring: the call
    runs chunks of 64, 64 and 22 tokens, each through both layers in turn, as
    the WASM runner's chunked path does; then the output norm.  Kernel 4:
    the bit-exact prefill projections; 0: the automatic policy (the
    64-token chunks on the fast prefill kernel)."""
    import torch

    hip.setMatvecKernel(kernel)
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
    print(f"prefill chunks 150 tokens, ring 64, kernel {kernel}", flush=True)
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
    # the automatic policy's 1e-4 projections re-round Q8_K blocks in both
    # layers: the second layer carries the first one's moved rows (5.6e-2 of
    # the row rms the largest measured)
    tol = None if kernel == 4 else CHAIN_TOL
    _check_rows(got, ref, "chunked hidden", tol)
    _check_rows(got_out, ref_out, "chunked output norm", tol)


@pytest.mark.parametrize("tokens", [512, 100])
def test_prefill_folds_bit_identical(hip, tokens):
    """The launch folds of a prefill chunk (activation tiles written by the
    norm launches and by the attention's slice merge, block-range sums added
    by the next launch, f16 queries from the attention prologue) against the
    plain launches (hp_hip_set_prefill_folds(0)): two layers of the model's
    shape at 512 and 100 tokens (the last 64-column tile padded), hidden
    states, output norm and both layers' caches bit-identical."""
    import torch

    shape = DM.ModelShape()
    seed = S.derive(S.BASE_SEED, "prefill-folds", tokens)
    datas = [DM.layer_host_data(shape, seed, i) for i in range(2)]
    onorm = (1 + 0.1 * S.normal(S.derive(seed, "onorm"), shape.hidden)).astype(np.float32)
    x = S.activations(S.derive(seed, "x"), tokens, shape.hidden) * 4
    pos = shape.capacity - tokens
    results = []
    for folds in (True, False):
        hip.setPrefillFolds(folds)
        model = DM.HipDecodeModel(shape)
        try:
            for d in datas:
                model.add_layer(d)
            model.output_norm = _dev(onorm)
            dx = _dev(x.reshape(-1))
            dpos = _dev(np.array([pos], np.int32))
            out = torch.empty(tokens * shape.hidden, dtype=torch.float32, device="cuda:0")
            launches0 = hip.hipResidentWeightStats()["kernelLaunches"]
            print(f"prefill folds {folds}, {tokens} tokens", flush=True)
            model.run_layers(dx.data_ptr(), dpos.data_ptr(), out.data_ptr(), tokens=tokens)
            torch.cuda.synchronize()
            launches = hip.hipResidentWeightStats()["kernelLaunches"] - launches0
            caches = [c.cpu().numpy().copy() for layer in model.caches for c in layer]
            results.append((dx.cpu().numpy(), out.cpu().numpy(), caches, launches))
        finally:
            model.release()
            hip.setPrefillFolds(True)
    (h1, o1, c1, n1), (h0, o0, c0, n0) = results
    print(f"launches with folds {n1}, without {n0}", flush=True)
    assert n1 < n0
    assert np.array_equal(h1, h0)
    assert np.array_equal(o1, o0)
    assert len(c1) == len(c0) and all(np.array_equal(a, b) for a, b in zip(c1, c0))


def _topk_near_ties(g_ids, g_logits, ref_logits, k, what):
    """Top-k ids of logits that carry an end-to-end perturbation: with D the
    largest |g - ref| over the row, an id can sit in one top-k and not the
    other only if its reference logit is within 2D of the reference's k-th
    largest (a larger margin keeps it on the same side in both)."""
    ids = np.argsort(-ref_logits, kind="stable")[:k]
    kth = float(ref_logits[ids[-1]])
    d = float(np.max(np.abs(np.asarray(g_logits, np.float64) - ref_logits)))
    moved = set(int(i) for i in g_ids) ^ set(int(i) for i in ids)
    shared = len(set(int(i) for i in g_ids) & set(int(i) for i in ids))
    print(f"{what}: top-{k} shared {shared}, logits max diff {d:.3e}, k-th logit {kth:.4f}, "
          f"moved ids {sorted(moved)[:8]}", flush=True)
    for i in moved:
        assert abs(float(ref_logits[i]) - kth) <= 2 * d, (what, i, float(ref_logits[i]), kth, d)
    return shared


def test_prefill_three_layers_512_auto_with_head(hip, D, oracle):
    """Three layers of the 42-layer model over one 512-token chunk ending at
    position 4095, on the automatic policy.

    - The three layers in one call (block-range sums of each down launch
      added by the next layer's norm launch) bit-identical to three calls
      of one layer each (whose sums are reduced at the call's end).
    - Each layer against the oracle's forward_layer on that layer's own
      input, to the single-layer row bars except the every-row bar, which is
      ATTN_STEP_TOL on this seed.
    - The output norm of the last token through the Q6_K 262144 x 2560 head:
      the oracle's head on the GPU's normed row gives the same logits and
      top-40; end to end (the oracle's own three layers, whose moved Q8_K
      blocks the next layers amplify), the top-40 ids agree up to near-ties
      of the measured logit difference."""
    import torch

    shape = DM.ModelShape()
    tokens, n_layers, head_rows = 512, 3, 262144
    seed = S.derive(S.BASE_SEED, "prefill-3-layers")
    datas = [DM.layer_host_data(shape, seed, i) for i in range(n_layers)]
    onorm = (1 + 0.1 * S.normal(S.derive(seed, "onorm"), shape.hidden)).astype(np.float32)
    head_blocks = S.q6_k_blocks(S.derive(seed, "head"), head_rows, shape.hidden)
    models = [DM.HipDecodeModel(shape), DM.HipDecodeModel(shape)]
    for m in models:
        for d in datas:
            m.add_layer(d)
        m.output_norm = _dev(onorm)
    head = hip.createHipQuantizedWeightHandle("Q6_K", head_blocks, shape.hidden, head_rows)
    pos = shape.capacity - tokens
    x = S.activations(S.derive(seed, "x"), tokens, shape.hidden) * 4
    dpos = _dev(np.array([pos], np.int32))
    print("prefill 3 layers 512 tokens, automatic policy", flush=True)
    try:
        hip.setMatvecKernel(0)
        dx = _dev(x.reshape(-1))
        out = torch.empty(tokens * shape.hidden, dtype=torch.float32, device="cuda:0")
        models[0].run_layers(dx.data_ptr(), dpos.data_ptr(), out.data_ptr(), tokens=tokens)
        # the same layers one call each, on the second copy of the caches
        lx = _dev(x.reshape(-1))
        lout = torch.empty_like(out)
        inputs = [x.copy()]
        twin = models[1]
        for i in range(n_layers):
            one = (type(twin.layers[0]) * 1)(twin.layers[i])
            last = i == n_layers - 1
            hip.assertHipOk(hip.lib().hp_hip_decode_layers_device(
                one, 1, tokens, lx.data_ptr(), dpos.data_ptr(), twin.output_norm.data_ptr() if last else None,
                lout.data_ptr() if last else None, None), "decode_layers")
            torch.cuda.synchronize()
            inputs.append(lx.cpu().numpy().reshape(tokens, shape.hidden))
        logits = torch.empty(head_rows, dtype=torch.float32, device="cuda:0")
        hip.matmul_multi_device([head.handle], out[(tokens - 1) * shape.hidden:].data_ptr(), shape.hidden, 1,
                                [logits.data_ptr()], [head_rows])
        torch.cuda.synchronize()
        got = dx.cpu().numpy().reshape(tokens, shape.hidden)
        got_out = out.cpu().numpy().reshape(tokens, shape.hidden)
        got_lout = lout.cpu().numpy().reshape(tokens, shape.hidden)
        got_logits = logits.cpu().numpy()
        got_top = hip.topKHip(got_logits.reshape(1, head_rows), 40)
    finally:
        for m in models:
            m.release()
        hip.releaseHipQuantizedWeightHandle(head)
        hip.setMatvecKernel(0)
    assert np.array_equal(got.view(np.uint32), inputs[-1].view(np.uint32)), "one call != one layer per call"
    assert np.array_equal(got_out.view(np.uint32), got_lout.view(np.uint32)), "output norm differs"
    for i, d in enumerate(datas):
        ref = D.forward_layer(_oracle_layer(D, shape, d), inputs[i], pos)
        _check_rows(inputs[i + 1], ref, f"layer {i} on its own input", ATTN_STEP_TOL)
    # the head and top-40 on the GPU's normed last row
    ref_logits = oracle.matmul(3, head_blocks, got_out[-1:], head_rows, threads=8)[0]
    assert np.array_equal(got_logits.view(np.uint32), ref_logits.view(np.uint32))
    ids, _ = oracle.topk(ref_logits, 40)
    g_ids = np.array([c["id"] for c in got_top[0]], np.uint32)
    assert np.array_equal(g_ids, ids)
    # end to end
    h = x.copy()
    for d in datas:
        h = D.forward_layer(_oracle_layer(D, shape, d), h, pos)
    ref_out = D.rms_norm_rows(h, onorm, shape.epsilon)
    e2e = oracle.matmul(3, head_blocks, ref_out[-1:], head_rows, threads=8)[0].astype(np.float64)
    shared = _topk_near_ties(g_ids, got_logits, e2e, 40, "last token end to end")
    assert shared >= 36


def _rel(got, ref, floor=FLOOR):
    got = np.asarray(got, np.float64).reshape(-1)
    ref = np.asarray(ref, np.float64).reshape(-1)
    den = np.maximum(np.abs(ref), floor * np.sqrt(np.mean(ref * ref)))
    return float(np.max(np.abs(got - ref) / den))


def test_prefill_stages_512_auto(hip, D, oracle):
    """The projections of one 512-token layer on the automatic policy (the
    fast prefill kernel), each on the oracle's own input to that stage:
    Q/K/V on attn_norm, O on the attention output, gate/up on ffn_norm, down
    on the GeGLU output, each within its relative bar.  Then each stage's
    GPU output swapped into the oracle's chain in place of the oracle's: no
    row of the layer output moves by more than SWAP_TOL of its rms, so the
    projections stay well inside the whole-layer bars."""
    import torch

    shape = DM.ModelShape()
    tokens = 512
    seed = S.derive(S.BASE_SEED, "prefill-3-layers")
    data = DM.layer_host_data(shape, seed, 0)
    pos = shape.capacity - tokens
    x = S.activations(S.derive(seed, "x"), tokens, shape.hidden) * 4
    L = _oracle_layer(D, shape, data)
    ref = D.forward_layer(L, x, pos)
    tr = L.trace
    w = {n: data["weights"][n] for n in DM.PROJ_NAMES}
    tid = {"Q4_K": 1, "Q6_K": 3}
    hs = {n: hip.createHipQuantizedWeightHandle(t, b, k, r) for n, (t, b, r, k) in w.items()}

    def gpu(names, inp):
        inp = np.ascontiguousarray(inp, np.float32).reshape(tokens, -1)
        di = _dev(inp.reshape(-1))
        outs = [torch.empty(tokens * w[n][2], dtype=torch.float32, device="cuda:0") for n in names]
        hip.matmul_multi_device([hs[n].handle for n in names], di.data_ptr(), inp.shape[1], tokens,
                                [o.data_ptr() for o in outs], [o.numel() for o in outs])
        torch.cuda.synchronize()
        return [o.cpu().numpy().reshape(tokens, -1) for o in outs]

    print("prefill stages 512 tokens, automatic policy", flush=True)
    try:
        hip.setMatvecKernel(0)
        gq, gk, gv = gpu(["attn_q", "attn_k", "attn_v"], tr["attn_norm"])
        go, = gpu(["attn_output"], tr["attention"])
        gg, gu = gpu(["ffn_gate", "ffn_up"], tr["ffn_norm"])
        gd, = gpu(["ffn_down"], tr["ffn_hidden"])
    finally:
        for h in hs.values():
            hip.releaseHipQuantizedWeightHandle(h)
    og, ou = oracle.matmul_multi([tid[w["ffn_gate"][0]], tid[w["ffn_up"][0]]], [w["ffn_gate"][1], w["ffn_up"][1]],
                                 tr["ffn_norm"], [w["ffn_gate"][2], w["ffn_up"][2]], threads=8)
    errs = {"q": _rel(gq, tr["q"]), "k": _rel(gk, tr["k"]), "v": _rel(gv, tr["v"]), "o": _rel(go, tr["o"]),
            "gate": _rel(gg, og), "up": _rel(gu, ou), "down": _rel(gd, tr["down"])}
    print("stage rel err " + ", ".join(f"{k} {v:.2e}" for k, v in errs.items()), flush=True)
    for k, v in errs.items():
        assert v <= (DOWN_TOL if k == "down" else STAGE_TOL), (k, v)

    eps = shape.epsilon
    nrm = data["norms"]

    def chain(o=None, gate=None, up=None, down=None):
        o = tr["o"] if o is None else o
        x1 = D.residual_add(x, D.rms_norm_rows(o, nrm["post_attention_norm"], eps))
        xn2 = D.rms_norm_rows(x1, nrm["ffn_norm"], eps)
        g0, u0 = oracle.matmul_multi([1, 1], [w["ffn_gate"][1], w["ffn_up"][1]], xn2,
                                     [w["ffn_gate"][2], w["ffn_up"][2]], threads=8)
        h = oracle.geglu(g0 if gate is None else gate, u0 if up is None else up)
        y = oracle.matmul_multi([3], [w["ffn_down"][1]], h, [w["ffn_down"][2]], threads=8)[0] if down is None else down
        x2 = D.residual_add(x1, D.rms_norm_rows(y, nrm["post_ffw_norm"], eps))
        return (x2.astype(np.float64) * np.float64(np.float32(data["output_scale"]))).astype(np.float32)

    assert np.array_equal(chain(), ref)   # the replayed chain is forward_layer's
    for what, out in (("o", chain(o=go)), ("gate/up", chain(gate=gg, up=gu)), ("down", chain(down=gd))):
        e = float(_row_errs(out, ref).max())
        print(f"{what} swapped in: max row err {e:.3e}", flush=True)
        assert e <= SWAP_TOL, (what, e)
