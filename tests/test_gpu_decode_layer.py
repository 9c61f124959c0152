"""GPU parity: the decoder-layer steps and a whole layer for one decode token
against the oracle's restatement of forwardAttentionLayer / forwardFfn
(layers.ts:161-473) and hp_gqa_attention_f32 (lib.rs:538-654).

The reference sums in index order (norm sums of squares in f64, attention
dot products and softmax sums in f32); the GPU sums in trees, so the bars
are tolerances stated per step:
- norms: every element within 1 f32 ulp of the oracle (an f64 sum in
  another order moves the scale by ~1e-16 relative, which can move an f32
  rounding by one step);
- attention prologue: q within 1 f32 ulp; cache entries (f16) within one
  f16 step;
- attention output (f16-rounded by castF16Rows): per head, max relative
  error 2^-8 (four f16 steps; 2.7e-3 is the largest measured), relative to
  max(|ref|, 0.01 rms(ref)): with unscaled N(0,1) queries and keys the
  scores reach |s| ~ 50, their f32 sums differ by ~1e-5 between summation
  orders, and outputs that cancel to a few percent of the head's scale carry
  that absolute error; at most 2 % of elements off at all (1.6 % measured
  with unscaled queries, where each output is dominated by a few keys);
- a whole layer: per token, max |got - ref| <= LAYER_TOL * rms(ref row) of
  the new residual stream.  An f16 step of the attention output feeds the O
  projection's Q8_K input, where it can move a block's rounding and shift O
  by ~1 %, which the post-attention norm carries into the residual (3.0e-3
  of the row rms the largest measured, over 42 layers of a 4-token draft).
  The one-token layer cases here come out bit-identical to the oracle, and
  the tests assert it.
Projections inside the layer are the bit-exact matvec kernels.
"""
import numpy as np
import pytest

from heliopause_amd import decode as DM
from heliopause_amd import hip_kernels as H
from heliopause_amd import synthetic as S

pytestmark = pytest.mark.gpu

LAYER_TOL = 3.5e-3
FLOOR = 0.01


@pytest.fixture(scope="module")
def D(oracle):
    from oracle import decode_layer

    return decode_layer


def _dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(torch.device("cuda:0"))


def _ulps(got, ref):
    g = np.ascontiguousarray(got, np.float32).view(np.int32).astype(np.int64)
    r = np.ascontiguousarray(ref, np.float32).view(np.int32).astype(np.int64)
    g = np.where(g < 0, -(g & 0x7FFFFFFF), g)
    r = np.where(r < 0, -(r & 0x7FFFFFFF), r)
    return np.abs(g - r)


def _f16_steps(got, ref):
    """Distance in f16 steps between two arrays of f16 values."""
    g = np.asarray(got).astype(np.float16).view(np.int16).astype(np.int64)
    r = np.asarray(ref).astype(np.float16).view(np.int16).astype(np.int64)
    g = np.where(g < 0, -(g & 0x7FFF), g)
    r = np.where(r < 0, -(r & 0x7FFF), r)
    return np.abs(g - r)


def _row_err(got, ref):
    """max over token rows of max |got - ref| / rms(ref row)."""
    g = np.asarray(got, np.float64)
    r = np.asarray(ref, np.float64)
    g, r = g.reshape(-1, g.shape[-1]), r.reshape(-1, r.shape[-1])
    return float(max(np.max(np.abs(gr - rr)) / np.sqrt(np.mean(rr * rr)) for gr, rr in zip(g, r)))


def _rel(got, ref):
    got = np.asarray(got, np.float64).reshape(-1)
    ref = np.asarray(ref, np.float64).reshape(-1)
    den = np.maximum(np.abs(ref), FLOOR * np.sqrt(np.mean(ref * ref)))
    return float(np.max(np.abs(got - ref) / den))


@pytest.mark.parametrize("rows,n,weighted", [(1, 2560, True), (3, 2560, False), (2, 4096, True), (1, 1, True),
                                             (4, 256, True), (1, 10240 // 4, True)])
def test_rms_norm(hip, D, rows, n, weighted):
    import torch

    rng = np.random.default_rng(rows * 7 + n)
    x = (rng.standard_normal((rows, n)) * 3).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32) if weighted else None
    dx, out = _dev(x), torch.empty(rows * n, dtype=torch.float32, device="cuda:0")
    dw = _dev(w) if weighted else None
    print(f"rms_norm rows={rows} n={n} weighted={weighted}", flush=True)
    H.rms_norm_device(dx.data_ptr(), rows, n, dw.data_ptr() if weighted else 0, 1e-6, out.data_ptr())
    torch.cuda.synchronize()
    ref = D.rms_norm_rows(x, w, 1e-6)
    u = _ulps(out.cpu().numpy().reshape(rows, n), ref)
    assert u.max() <= 1, u.max()


def test_residual_norm(hip, D):
    import torch

    rng = np.random.default_rng(11)
    n = 2560
    y = rng.standard_normal(n).astype(np.float32) * 5
    res = rng.standard_normal(n).astype(np.float32) * 20
    wp = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    wn = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    dy, dres, dwp, dwn = _dev(y), _dev(res), _dev(wp), _dev(wn)
    xo = torch.empty(n, dtype=torch.float32, device="cuda:0")
    nx = torch.empty(n, dtype=torch.float32, device="cuda:0")
    print("residual_norm", flush=True)
    H.residual_norm_device(dy.data_ptr(), 1, n, dwp.data_ptr(), dres.data_ptr(), 0.8, xo.data_ptr(), dwn.data_ptr(),
                           nx.data_ptr(), 1e-6)
    torch.cuda.synchronize()
    post = D.rms_norm_rows(y, wp, 1e-6)
    ref_x = (D.residual_add(res, post).astype(np.float64) * np.float64(np.float32(0.8))).astype(np.float32)
    got_x = xo.cpu().numpy()
    assert _ulps(got_x, ref_x).max() <= 1
    # the next norm of the GPU's own residual (isolates the norm's order of summation)
    assert _ulps(nx.cpu().numpy(), D.rms_norm_rows(got_x, wn, 1e-6)).max() <= 1
    # in place (residual_out == residual), no next norm
    H.residual_norm_device(dy.data_ptr(), 1, n, dwp.data_ptr(), dres.data_ptr(), 1.0, dres.data_ptr(), 0, 0, 1e-6)
    torch.cuda.synchronize()
    assert _ulps(dres.cpu().numpy(), D.residual_add(res, post)).max() <= 1


PREP_CASES = [  # nq, nkv, capacity, position, rope_dims, freq factors, shared value
    (8, 2, 4096, 4096, 256, False, False),
    (8, 2, 4096, 0, 256, False, False),
    (8, 2, 64, 130000, 128, True, False),
    (4, 1, 32, 7, 256, False, True),
    (2, 2, 16, 3, 0, False, False),
]


@pytest.mark.parametrize("nq,nkv,cap,pos,rdims,use_ff,shared", PREP_CASES)
def test_attention_prep(hip, D, nq, nkv, cap, pos, rdims, use_ff, shared):
    import torch

    rng = np.random.default_rng(nq + 10 * cap + pos)
    q = (rng.standard_normal(nq * 256) * 2).astype(np.float32)
    k = (rng.standard_normal(nkv * 256) * 2).astype(np.float32)
    v = (rng.standard_normal(nkv * 256) * 2).astype(np.float32)
    wq = (1 + 0.1 * rng.standard_normal(256)).astype(np.float32)
    wk = (1 + 0.1 * rng.standard_normal(256)).astype(np.float32)
    ff = (1.0 + rng.random(max(rdims // 2, 1))).astype(np.float32) if use_ff else None
    kc = rng.standard_normal((nkv, cap, 256)).astype(np.float16)
    vc = rng.standard_normal((nkv, cap, 256)).astype(np.float16)
    dkc, dvc = _dev(kc.view(np.int16)), _dev(vc.view(np.int16))
    dq, dk, dv, dwq, dwk = _dev(q), _dev(k), _dev(v), _dev(wq), _dev(wk)
    dff = _dev(ff) if use_ff else None
    dpos = _dev(np.array([pos], np.int32))
    qo = torch.empty(nq * 256, dtype=torch.float32, device="cuda:0")
    cfg = H.attention_config(nq, nkv, cap, rope_dims=rdims, d_rope_freq_factors=dff.data_ptr() if use_ff else 0)
    print(f"attention_prep nq={nq} nkv={nkv} cap={cap} pos={pos} rope={rdims} ff={use_ff} shared={shared}",
          flush=True)
    H.attention_prep_device(cfg, dq.data_ptr(), dk.data_ptr(), 0 if shared else dv.data_ptr(), dwq.data_ptr(),
                            dwk.data_ptr(), dpos.data_ptr(), qo.data_ptr(), dkc.data_ptr(), dvc.data_ptr())
    torch.cuda.synchronize()
    qr = D.rope_neox(D.rms_norm_rows(q.reshape(nq, 256), wq, 1e-6), [pos], rdims, 10000.0, ff)
    kr = D.rope_neox(D.rms_norm_rows(k.reshape(nkv, 256), wk, 1e-6), [pos], rdims, 10000.0, ff)
    vn = D.rms_norm_rows((k if shared else v).reshape(nkv, 256), None, 1e-6)
    assert _ulps(qo.cpu().numpy().reshape(nq, 256), qr).max() <= 1
    gk = dkc.cpu().numpy().view(np.float16)
    gv = dvc.cpu().numpy().view(np.float16)
    slot = pos % cap
    assert _f16_steps(gk[:, slot], kr.astype(np.float16)).max() <= 1
    assert _f16_steps(gv[:, slot], vn.astype(np.float16)).max() <= 1
    others = np.arange(cap) != slot
    assert np.array_equal(gk[:, others].view(np.int16), kc[:, others].view(np.int16))
    assert np.array_equal(gv[:, others].view(np.int16), vc[:, others].view(np.int16))


ATTN_CASES = [  # nq, nkv, capacity, position, window, query scale
    (8, 2, 4096, 4096, 0, 1.0),
    (8, 2, 4096, 4096, 0, 0.0625),
    (8, 2, 4096, 10, 0, 0.0625),
    (8, 2, 300, 1000, 0, 0.0625),
    (8, 2, 4096, 2000, 512, 0.25),
    (2, 2, 64, 63, 0, 0.0625),
    (8, 1, 128, 127, 0, 0.0625),
    (4, 2, 100, 0, 0, 1.0),
    (8, 2, 65, 64, 0, 0.0625),
]


@pytest.mark.parametrize("nq,nkv,cap,pos,window,qscale", ATTN_CASES)
def test_gqa_attention(hip, D, nq, nkv, cap, pos, window, qscale):
    import torch

    rng = np.random.default_rng(nq * 1000 + cap + pos)
    q = (rng.standard_normal((nq, 256)) * qscale).astype(np.float32)
    kc = rng.standard_normal((nkv, cap, 256)).astype(np.float16)
    vc = rng.standard_normal((nkv, cap, 256)).astype(np.float16)
    dq, dkc, dvc = _dev(q), _dev(kc.view(np.int16)), _dev(vc.view(np.int16))
    dpos = _dev(np.array([pos], np.int32))
    out = torch.empty(nq * 256, dtype=torch.float32, device="cuda:0")
    cfg = H.attention_config(nq, nkv, cap, sliding_window=window)
    print(f"gqa_attention nq={nq} nkv={nkv} cap={cap} pos={pos} window={window} qscale={qscale}", flush=True)
    H.gqa_attention_device(cfg, dq.data_ptr(), dkc.data_ptr(), dvc.data_ptr(), dpos.data_ptr(), out.data_ptr())
    torch.cuda.synchronize()
    ref = D.decode_attention(q, kc, vc, pos, window)
    got = out.cpu().numpy().reshape(nq, 256)
    steps = _f16_steps(got, ref)
    assert np.array_equal(got.astype(np.float16).astype(np.float32), got)   # castF16Rows output
    errs = [_rel(got[h], ref[h]) for h in range(nq)]
    print(f"max rel err per head {max(errs):.2e}, elements off {np.count_nonzero(steps)}, max steps {steps.max()}",
          flush=True)
    assert max(errs) <= 2.0 ** -8
    assert np.count_nonzero(steps) <= 0.02 * steps.size, np.count_nonzero(steps)


def _small_shape(**kw):
    base = dict(hidden=512, head_count=2, head_count_kv=1, ffn=1024, capacity=64)
    base.update(kw)
    return DM.ModelShape(**base)


def _oracle_layer(D, shape, data):
    tids = {"Q4_K": 1, "Q6_K": 3}
    w = {n: (tids[t], blocks, rows) for n, (t, blocks, rows, _) in data["weights"].items()}
    return D.Layer(weights=w, norms=dict(data["norms"]), key_cache=data["key_cache"].copy(),
                   value_cache=data["value_cache"].copy(), head_count=shape.head_count,
                   head_count_kv=shape.head_count_kv, rope_dims=shape.rope_dims,
                   rope_freq_base=shape.rope_freq_base, sliding_window=shape.sliding_window,
                   epsilon=shape.epsilon, output_scale=float(data["output_scale"]))


@pytest.mark.parametrize("full,pos,kernel", [(True, 4096, 0), (False, 70, 0), (False, 5, 0), (False, 70, 2)],
                         ids=["model-4096", "small-wrap", "small-short", "small-matrix-cores"])
def test_decode_layer_matches_oracle(hip, D, full, pos, kernel):
    """kernel 2 forces the matrix-core matvec, whose launches cannot form
    their input in the prologue: the norms then run as their own launches."""
    import torch

    hip.setMatvecKernel(kernel)
    shape = DM.ModelShape() if full else _small_shape()
    seed = S.derive(S.BASE_SEED, "decode-layer", full, pos)
    data = DM.layer_host_data(shape, seed, 0)
    model = DM.HipDecodeModel(shape)
    model.add_layer(data)
    x = S.activations(S.derive(seed, "x"), 1, shape.hidden).reshape(-1) * 4
    dx = _dev(x)
    dpos = _dev(np.array([pos], np.int32))
    print(f"decode layer hidden={shape.hidden} pos={pos}", flush=True)
    try:
        model.run_layers(dx.data_ptr(), dpos.data_ptr())
        torch.cuda.synchronize()
        got = dx.cpu().numpy()
        gk = model.caches[0][0].cpu().numpy().view(np.float16)
        gv = model.caches[0][1].cpu().numpy().view(np.float16)
    finally:
        model.release()
        hip.setMatvecKernel(0)
    ol = _oracle_layer(D, shape, data)
    ref = D.forward_layer(ol, x, pos)
    err = _row_err(got, ref)
    print(f"layer err {err:.3e} of the row rms; identical {np.mean(got == ref):.4f}", flush=True)
    assert err <= LAYER_TOL
    assert np.array_equal(np.asarray(got, np.float32).view(np.uint32), np.asarray(ref, np.float32).view(np.uint32))
    slot = pos % shape.capacity
    assert _f16_steps(gk[:, slot], ol.key_cache[:, slot]).max() <= 1
    assert _f16_steps(gv[:, slot], ol.value_cache[:, slot]).max() <= 1


@pytest.mark.parametrize("full", [True, False], ids=["model", "small"])
def test_decode_layer_kernels_bit_identical(hip, full):
    """One decode layer of the 42-layer model (hidden 2560, FFN 10240) and of
    a small model (hidden 512, FFN 1024) with the automatic kernel choice (the wide gate/up + GeGLU launch with its
    residual-norm prologue, the wide down projection), the vector-ALU
    kernels and the half-split kernels: every projection is the oracle's
    bits and every norm prologue sums in one order, so the layer's output and
    cache entries agree bit for bit."""
    import torch

    shape = DM.ModelShape() if full else _small_shape()
    seed = S.derive(S.BASE_SEED, "decode-layer-kernels", full)
    data = DM.layer_host_data(shape, seed, 0)
    x = S.activations(S.derive(seed, "x"), 1, shape.hidden).reshape(-1) * 4
    outs = {}
    for kernel in (0, 1, 3, 6, 7, 8):
        hip.setMatvecKernel(kernel)
        model = DM.HipDecodeModel(shape)
        model.add_layer(data)
        dx = _dev(x)
        dpos = _dev(np.array([1000 if full else 40], np.int32))
        print(f"decode layer kernel={kernel}", flush=True)
        try:
            model.run_layers(dx.data_ptr(), dpos.data_ptr())
            torch.cuda.synchronize()
            outs[kernel] = (dx.cpu().numpy(), model.caches[0][0].cpu().numpy(), model.caches[0][1].cpu().numpy())
        finally:
            model.release()
            hip.setMatvecKernel(0)
    for kernel in (1, 3, 6, 7, 8):
        for got, ref in zip(outs[kernel], outs[0]):
            assert np.array_equal(got.view(np.uint8), ref.view(np.uint8)), kernel


def test_decode_layers_chain_output_norm_and_graph(hip, D):
    """Three small layers + output norm: eager vs the oracle, then the same
    step captured in a HIP graph and replayed at three positions (the
    position tensor changes between replays) against eager runs on a twin
    model: bit-identical hidden states, outputs and caches."""
    import torch

    shape = _small_shape(capacity=32, sliding_window=0)
    seed = S.derive(S.BASE_SEED, "decode-chain")
    datas = [DM.layer_host_data(shape, seed, i) for i in range(3)]
    onorm = (1 + 0.1 * S.normal(S.derive(seed, "onorm"), shape.hidden)).astype(np.float32)
    twins = []
    for _ in range(2):
        m = DM.HipDecodeModel(shape)
        for d in datas:
            m.add_layer(d)
        m.output_norm = _dev(onorm)
        twins.append(m)
    eager, graphed = twins
    x = S.activations(S.derive(seed, "x"), 1, shape.hidden).reshape(-1) * 4
    try:
        # eager vs oracle at position 40 (ring of 32: wraps)
        dx = _dev(x)
        dpos = _dev(np.array([40], np.int32))
        out = torch.empty(shape.hidden, dtype=torch.float32, device="cuda:0")
        print("decode chain eager", flush=True)
        eager.run_layers(dx.data_ptr(), dpos.data_ptr(), out.data_ptr())
        torch.cuda.synchronize()
        ols = [_oracle_layer(D, shape, d) for d in datas]
        h = x.copy()
        for ol in ols:
            h = D.forward_layer(ol, h, 40)
        ref_out = D.rms_norm_rows(h, onorm, shape.epsilon)
        print(f"chain hidden err {_row_err(dx.cpu().numpy(), h):.3e} out err "
              f"{_row_err(out.cpu().numpy(), ref_out):.3e}", flush=True)
        assert _row_err(dx.cpu().numpy(), h) <= 3 * LAYER_TOL
        assert _row_err(out.cpu().numpy(), ref_out) <= 3 * LAYER_TOL
        # graph replay vs eager at positions 41..43 (the eager twin continues).
        # Scratch belongs to the stream a call is queued on and is sized by an
        # uncaptured call: one warm-up step on the capture stream, whose
        # results are then overwritten with the eager twin's state.
        gx = _dev(dx.cpu().numpy())
        gpos = _dev(np.array([41], np.int32))
        gout = torch.empty(shape.hidden, dtype=torch.float32, device="cuda:0")
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            graphed.run_layers(gx.data_ptr(), gpos.data_ptr(), gout.data_ptr(), side.cuda_stream)
        torch.cuda.synchronize()
        gx.copy_(dx)
        for (kc, vc), (ek, ev) in zip(graphed.caches, eager.caches):
            kc.copy_(ek)
            vc.copy_(ev)
        torch.cuda.synchronize()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=side):
                graphed.run_layers(gx.data_ptr(), gpos.data_ptr(), gout.data_ptr(),
                                   torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        for p in (41, 42, 43):
            print(f"decode chain replay position {p}", flush=True)
            gpos.copy_(torch.tensor([p], dtype=torch.int32))
            torch.cuda.synchronize()
            graph.replay()
            dpos.copy_(torch.tensor([p], dtype=torch.int32))
            eager.run_layers(dx.data_ptr(), dpos.data_ptr(), out.data_ptr())
            torch.cuda.synchronize()
            assert torch.equal(gx, dx) and torch.equal(gout, out), p
            for (kc, vc), (ek, ev) in zip(graphed.caches, eager.caches):
                assert torch.equal(kc, ek) and torch.equal(vc, ev), p
    finally:
        for m in twins:
            m.release()


def test_decode_layer_rejects_bad_shapes(hip):
    import torch

    shape = _small_shape()
    data = DM.layer_host_data(shape, S.derive(S.BASE_SEED, "decode-bad"), 0, cache_fill=False)
    model = DM.HipDecodeModel(shape)
    model.add_layer(data)
    dx = torch.zeros(shape.hidden, dtype=torch.float32, device="cuda:0")
    dpos = torch.zeros(1, dtype=torch.int32, device="cuda:0")
    try:
        L = model.layers[0]
        L.attention.head_count = 3                       # 3 % 1 == 0 but Q rows are 2 * 256
        with pytest.raises(ValueError):
            model.run_layers(dx.data_ptr(), dpos.data_ptr())
        L.attention.head_count = 2
        L.attention.head_dim = 128
        with pytest.raises(ValueError):
            model.run_layers(dx.data_ptr(), dpos.data_ptr())
        L.attention.head_dim = 256
        L.ffn_down = L.ffn_up                            # down must map ffn -> hidden
        with pytest.raises(ValueError):
            model.run_layers(dx.data_ptr(), dpos.data_ptr())
    finally:
        model.release()


@pytest.mark.parametrize("nq,nkv,cap,pos,window", [(8, 2, 4096, 4000, 0), (8, 1, 300, 1000, 0),
                                                   (6, 2, 4096, 3000, 512)])
def test_one_token_attention_matches_draft_row(hip, nq, nkv, cap, pos, window):
    """A one-token call splits each KV head's query heads over two workgroups
    per chunk (when the group is even); a three-token call does not.  The
    third token's row of the three-token call attends over the same window
    and keys as a one-token call at its position: the rows must be
    bit-identical."""
    import torch

    rng = np.random.default_rng(nq * 100 + nkv * 10 + cap + pos)
    q = (rng.standard_normal((3, nq, 256)) * 0.25).astype(np.float32)
    kc = rng.standard_normal((nkv, cap, 256)).astype(np.float16)
    vc = rng.standard_normal((nkv, cap, 256)).astype(np.float16)
    dkc, dvc = _dev(kc.view(np.int16)), _dev(vc.view(np.int16))
    cfg = H.attention_config(nq, nkv, cap, sliding_window=window)
    print(f"one-token vs draft row nq={nq} nkv={nkv} cap={cap} pos={pos} window={window}", flush=True)
    out3 = torch.empty(3 * nq * 256, dtype=torch.float32, device="cuda:0")
    dq3, dpos3 = _dev(q), _dev(np.array([pos], np.int32))
    H.gqa_attention_device(cfg, dq3.data_ptr(), dkc.data_ptr(), dvc.data_ptr(), dpos3.data_ptr(), out3.data_ptr(),
                           token_count=3)
    out1 = torch.empty(nq * 256, dtype=torch.float32, device="cuda:0")
    dq1, dpos1 = _dev(np.ascontiguousarray(q[2])), _dev(np.array([pos + 2], np.int32))
    H.gqa_attention_device(cfg, dq1.data_ptr(), dkc.data_ptr(), dvc.data_ptr(), dpos1.data_ptr(), out1.data_ptr())
    torch.cuda.synchronize()
    row = out3.cpu().numpy().reshape(3, nq * 256)[2]
    assert np.array_equal(out1.cpu().numpy().view(np.uint32), row.view(np.uint32))


@pytest.mark.parametrize("tokens,cap,pos,window,qscale", [(3, 4096, 4094, 0, 0.25), (4, 64, 70, 0, 1.0),
                                                          (8, 4096, 100, 0, 0.0625), (2, 4096, 3000, 512, 0.25),
                                                          (5, 40, 2, 0, 0.25)])
def test_draft_attention_prep_and_attention(hip, D, tokens, cap, pos, window, qscale):
    """Several tokens (a draft): every token's key and value appended at its
    own slot, then each token attends causally within the shared window."""
    import torch

    nq, nkv = 8, 2
    rng = np.random.default_rng(tokens * 1000 + cap + pos)
    q = (rng.standard_normal((tokens, nq, 256)) * 2).astype(np.float32)
    k = (rng.standard_normal((tokens, nkv, 256)) * 2).astype(np.float32)
    v = (rng.standard_normal((tokens, nkv, 256)) * 2).astype(np.float32)
    wq = (qscale * (1 + 0.1 * rng.standard_normal(256))).astype(np.float32)
    wk = (1 + 0.1 * rng.standard_normal(256)).astype(np.float32)
    kc = rng.standard_normal((nkv, cap, 256)).astype(np.float16)
    vc = rng.standard_normal((nkv, cap, 256)).astype(np.float16)
    dkc, dvc = _dev(kc.view(np.int16)), _dev(vc.view(np.int16))
    dq, dk, dv, dwq, dwk = _dev(q), _dev(k), _dev(v), _dev(wq), _dev(wk)
    dpos = _dev(np.array([pos], np.int32))
    qo = torch.empty(tokens * nq * 256, dtype=torch.float32, device="cuda:0")
    out = torch.empty(tokens * nq * 256, dtype=torch.float32, device="cuda:0")
    cfg = H.attention_config(nq, nkv, cap, sliding_window=window)
    print(f"draft attention tokens={tokens} cap={cap} pos={pos} window={window}", flush=True)
    H.attention_prep_device(cfg, dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), dwq.data_ptr(), dwk.data_ptr(),
                            dpos.data_ptr(), qo.data_ptr(), dkc.data_ptr(), dvc.data_ptr(), token_count=tokens)
    H.gqa_attention_device(cfg, qo.data_ptr(), dkc.data_ptr(), dvc.data_ptr(), dpos.data_ptr(), out.data_ptr(),
                           token_count=tokens)
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
    gk = dkc.cpu().numpy().view(np.float16)
    gv = dvc.cpu().numpy().view(np.float16)
    assert _f16_steps(gk, rk).max() <= 1 and _f16_steps(gv, rv).max() <= 1
    ref = D.decode_attention(qo.cpu().numpy().reshape(tokens, nq, 256), gk, gv, pos, window)
    got = out.cpu().numpy().reshape(tokens, nq, 256)
    errs = [_rel(got[t, h], ref[t, h]) for t in range(tokens) for h in range(nq)]
    steps = _f16_steps(got, ref)
    print(f"max rel err {max(errs):.2e}, elements off {np.count_nonzero(steps)}", flush=True)
    assert max(errs) <= 2.0 ** -8
    assert np.count_nonzero(steps) <= 0.02 * steps.size


@pytest.mark.parametrize("full,tokens,pos", [(True, 4, 4093), (True, 2, 4095), (False, 3, 62), (False, 8, 0)],
                         ids=["model-draft4", "model-draft2", "small-wrap-draft3", "small-start-draft8"])
def test_decode_draft_matches_oracle(hip, D, full, tokens, pos):
    """A draft of several tokens through one layer (every row kept)."""
    import torch

    shape = DM.ModelShape() if full else _small_shape()
    seed = S.derive(S.BASE_SEED, "decode-draft", full, tokens, pos)
    data = DM.layer_host_data(shape, seed, 0)
    model = DM.HipDecodeModel(shape)
    model.add_layer(data)
    x = S.activations(S.derive(seed, "x"), tokens, shape.hidden) * 4
    dx = _dev(x)
    dpos = _dev(np.array([pos], np.int32))
    print(f"decode draft hidden={shape.hidden} tokens={tokens} pos={pos}", flush=True)
    try:
        model.run_layers(dx.data_ptr(), dpos.data_ptr(), tokens=tokens)
        torch.cuda.synchronize()
        got = dx.cpu().numpy().reshape(tokens, shape.hidden)
        gk = model.caches[0][0].cpu().numpy().view(np.float16)
    finally:
        model.release()
    ol = _oracle_layer(D, shape, data)
    ref = D.forward_layer(ol, x, pos)
    errs = [_row_err(got[t], ref[t]) for t in range(tokens)]
    print(f"draft err {max(errs):.3e} of the row rms; identical {np.mean(got == ref):.4f}", flush=True)
    assert max(errs) <= LAYER_TOL
    assert _f16_steps(gk, ol.key_cache).max() <= 1


def test_layers_reject_token_counts(hip):
    """0 tokens and more than one call takes (65536, in chunks) fail before
    any memory is touched."""
    import torch

    shape = _small_shape()
    data = DM.layer_host_data(shape, S.derive(S.BASE_SEED, "decode-bad9"), 0, cache_fill=False)
    model = DM.HipDecodeModel(shape)
    model.add_layer(data)
    dx = torch.zeros(9 * shape.hidden, dtype=torch.float32, device="cuda:0")
    dpos = torch.zeros(1, dtype=torch.int32, device="cuda:0")
    try:
        for bad in (0, 65537):
            with pytest.raises(ValueError):
                model.run_layers(dx.data_ptr(), dpos.data_ptr(), tokens=bad)
    finally:
        model.release()


def _oracle_layer_ple(D, shape, data):
    """_oracle_layer plus the per-layer input step's weights and post_norm."""
    ol = _oracle_layer(D, shape, data)
    tids = {"Q4_K": 1, "Q6_K": 3}
    for name in ("inp_gate", "proj"):
        t, blocks, rows, _ = data["per_layer"][name]
        ol.weights[name] = (tids[t], blocks, rows)
    ol.norms["post_norm"] = data["per_layer"]["post_norm"]
    return ol


@pytest.mark.parametrize("full,tokens,pos", [(False, 1, 70), (False, 4, 61), (True, 1, 4096), (True, 4, 4093),
                                             (True, 128, 3968)],
                         ids=["small-decode", "small-draft4", "model-decode", "model-draft4", "model-prefill128"])
def test_decode_layer_with_per_layer_input(hip, D, full, tokens, pos):
    """A layer with the per-layer input step (applyPerLayerInput,
    layers.ts:475-521; P = 256): inp_gate, the gelu product with the
    layer's input rows, proj and post_norm between the FFN residual and the
    layer scale, against the oracle's layer on the same rows.  Decode and
    draft rows within LAYER_TOL; the 128-token chunk on the bit-exact
    prefill projections (selector 4) to the prefill bars (every row 3e-2,
    median 1e-4)."""
    import torch

    hip.setMatvecKernel(4 if tokens > 8 else 0)

    shape = DM.ModelShape() if full else _small_shape()
    P = 256
    seed = S.derive(S.BASE_SEED, "decode-ple", full, tokens)
    data = DM.layer_host_data(shape, seed, 0, per_layer_length=P)
    model = DM.HipDecodeModel(shape)
    model.add_layer(data)
    x = S.activations(S.derive(seed, "x"), tokens, shape.hidden) * 4
    pli = S.activations(S.derive(seed, "pli"), tokens, P)
    dx = _dev(x.reshape(-1))
    dp = _dev(pli.reshape(-1))
    dpos = _dev(np.array([pos], np.int32))
    print(f"decode layer with per-layer input hidden={shape.hidden} tokens={tokens} pos={pos}", flush=True)
    try:
        model.set_per_layer_input(0, dp.data_ptr())
        model.run_layers(dx.data_ptr(), dpos.data_ptr(), tokens=tokens)
        torch.cuda.synchronize()
        got = dx.cpu().numpy().reshape(tokens, shape.hidden)
    finally:
        model.release()
        hip.setMatvecKernel(0)
    ol = _oracle_layer_ple(D, shape, data)
    ref = D.forward_layer(ol, x, pos, pli)
    plain = D.forward_layer(_oracle_layer(D, shape, data), x, pos)
    errs = np.array([_row_err(got[t], ref[t]) for t in range(tokens)])
    moved = min(_row_err(ref[t], plain[t]) for t in range(tokens))
    print(f"per-layer input: max row err {errs.max():.3e}, median {np.median(errs):.2e}, identical "
          f"{np.mean(got == ref):.4f}; the step moves every row by at least {moved:.2e} of its rms", flush=True)
    assert moved > 1e-2                        # the step is not a no-op on these rows
    if tokens <= 8:
        assert errs.max() <= LAYER_TOL
    else:
        assert errs.max() <= 3e-2 and np.median(errs) <= 1e-4


def test_stream_scratch_release(hip):
    """A decode step on a side stream allocates that stream's scratch; after
    hp_hip_release_stream_scratch the library holds what it held before, a
    later step on the stream allocates anew and gives the same bits, and the
    library stream's own scratch cannot be released this way."""
    import torch

    shape = _small_shape()
    seed = S.derive(S.BASE_SEED, "stream-scratch")
    data = DM.layer_host_data(shape, seed, 0)
    model = DM.HipDecodeModel(shape)
    model.add_layer(data)
    x = S.activations(S.derive(seed, "x"), 1, shape.hidden).reshape(-1) * 4
    dpos = _dev(np.array([5], np.int32))
    side = torch.cuda.Stream()
    try:
        # a pooled stream may carry an earlier test's scratch: start from none
        torch.cuda.synchronize()
        hip.releaseStreamScratch(side.cuda_stream)
        base = hip.hipResidentWeightStats()["scratchBytes"]
        outs = []
        for _ in range(2):
            dx = _dev(x)
            k0 = model.caches[0][0].clone()
            with torch.cuda.stream(side):
                model.run_layers(dx.data_ptr(), dpos.data_ptr(), 0, side.cuda_stream)
            side.synchronize()
            held = hip.hipResidentWeightStats()["scratchBytes"]
            outs.append(dx.cpu().numpy())
            model.caches[0][0].copy_(k0)
            hip.releaseStreamScratch(side.cuda_stream)
            after = hip.hipResidentWeightStats()["scratchBytes"]
            print(f"scratch bytes: before {base}, after the step {held}, after release {after}", flush=True)
            assert held > base and after == base
        assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
        assert hip.lib().hp_hip_release_stream_scratch(None) == hip.HP_ERR_ARG
    finally:
        model.release()
