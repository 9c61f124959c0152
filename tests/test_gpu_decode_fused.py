"""GPU: the persistent one-token decode step (decode_fused.hip) against the
launch sequence of hp_hip_decode_layers_device, which test_gpu_decode_layer
and test_gpu_fullsize check against the oracle's restatement of
forwardAttentionLayer / forwardFfn (layers.ts:161-473).

Both paths compute every value in the same order (the same Q8_K input
images, integer dots, f32 block chains and tails, f64 norm sums, attention
chunk partials and merge), so the bar is bit-identity: the residual stream,
the output norm and every KV-cache entry.  Each case also checks which path
ran, from the runner's launch counter: one launch for the persistent step,
several for the sequence.

Cases: the 42-layer model at full size (wrapped ring position and an
unwrapped one), small models for each query-group size the step has a
kernel for (1, 2, 4, 8) with ring wrap, a sliding window, RoPE over 128 and
0 dims, RoPE frequency factors and a value shared with the key; shapes the
step does not cover (they must take the launch sequence); graph capture
with replays at advancing positions; and the bounded waits, forced from the
host with a one-tick limit.
"""
import hashlib

import numpy as np
import pytest

from heliopause_amd import decode as DM
from heliopause_amd import hip_kernels as H
from heliopause_amd import synthetic as S

pytestmark = pytest.mark.gpu


def _dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(torch.device("cuda:0"))


class _Model:
    """n_layers decoder layers cycling over `distinct` sets of weights, each
    layer with its own KV ring, plus the output norm."""

    def __init__(self, shape, n_layers, seed, distinct=3, shared_v=False, freq_factors=False):
        import torch

        self.shape = shape
        self.model = DM.HipDecodeModel(shape)
        datas = [DM.layer_host_data(shape, seed, i) for i in range(min(distinct, n_layers))]
        shared = [None] * len(datas)
        self.freq = None
        if freq_factors:
            ff = (1.0 + np.abs(S.normal(S.derive(seed, "ff"), shape.rope_dims // 2))).astype(np.float32)
            self.freq = _dev(ff)
        for i in range(n_layers):
            j = i % len(datas)
            self.model.add_layer(datas[j], shared_weights=shared[j])
            if shared[j] is None:
                shared[j] = {n: h for n, h in zip(DM.PROJ_NAMES, self.model.handles[-len(DM.PROJ_NAMES):])}
            L = self.model.layers[-1]
            if shared_v:
                L.attn_v = 0  # the value rows are the key rows
            if self.freq is not None:
                L.attention.d_rope_freq_factors = self.freq.data_ptr()
        onorm = (1.0 + 0.1 * S.normal(S.derive(seed, "on"), shape.hidden)).astype(np.float32)
        self.model.output_norm = _dev(onorm)
        self.x = _dev((S.activations(S.derive(seed, "x"), 1, shape.hidden).reshape(-1) * 4).astype(np.float32))
        self.pos = torch.zeros(1, dtype=torch.int32, device=torch.device("cuda:0"))
        self.caches0 = [(k.clone(), v.clone()) for k, v in self.model.caches]

    def restore(self):
        for (k, v), (k0, v0) in zip(self.model.caches, self.caches0):
            k.copy_(k0)
            v.copy_(v0)

    def cache_digest(self):
        h = hashlib.sha1()
        for k, v in self.model.caches:
            h.update(k.cpu().numpy().tobytes())
            h.update(v.cpu().numpy().tobytes())
        return h.hexdigest()

    def steps(self, fused, positions):
        """From the saved caches and x, one decode step per position in turn
        (each on the previous step's residual stream); per step the bits of
        the residual stream and the output norm, then the caches' digest and
        the launches per step."""
        import torch

        H.setDecodeFused(fused)
        self.restore()
        hid = self.x.clone()
        out = torch.empty_like(hid)
        rows, launches = [], []
        for p in positions:
            self.pos.fill_(p)
            l0 = H.hipResidentWeightStats()["kernelLaunches"]
            self.model.run_layers(hid.data_ptr(), self.pos.data_ptr(), out.data_ptr())
            torch.cuda.synchronize()
            launches.append(H.hipResidentWeightStats()["kernelLaunches"] - l0)
            assert H.decodeFusedStatus() == 0
            rows.append((hid.cpu().numpy().view(np.uint32).copy(), out.cpu().numpy().view(np.uint32).copy()))
        return rows, self.cache_digest(), launches

    def release(self):
        self.model.release()


def _assert_same(a, b, what):
    for t, ((ha, oa), (hb, ob)) in enumerate(zip(a, b)):
        nd = int(np.count_nonzero(ha != hb))
        assert nd == 0, f"{what}: step {t}: {nd} residual values differ"
        assert np.array_equal(oa, ob), f"{what}: step {t}: output norm differs"


def _compare(m, positions, what):
    ref, ref_cache, ref_launch = m.steps(False, positions)
    got, got_cache, got_launch = m.steps(True, positions)
    try:
        assert all(n > 1 for n in ref_launch), f"{what}: the launch sequence ran as {ref_launch} launches"
        assert got_launch == [1] * len(positions), f"{what}: the persistent step ran as {got_launch} launches"
        _assert_same(ref, got, what)
        assert ref_cache == got_cache, f"{what}: KV caches differ"
    finally:
        H.setDecodeFused(False)
    print(f"{what}: {len(positions)} steps bit-identical, launches {ref_launch[0]} -> 1")


def test_full_size_42_layers(hip):
    """The model of the decode-step benchmark: 42 layers of 2560 hidden, 8/2
    heads of 256, FFN 10240, a 4096-slot ring: the step at the ring's wrap
    (slot 0 overwritten) and one well inside it."""
    shape = DM.ModelShape()
    m = _Model(shape, 42, S.derive(S.config_seed(5), "fused-42"))
    try:
        _compare(m, [shape.capacity, shape.capacity + 1], "42 layers, wrap")
        _compare(m, [1000], "42 layers, position 1000")
    finally:
        m.release()


SMALL = [
    # (name, shape kwargs, layers, model options, positions)
    ("G1 wrap rope128", dict(hidden=512, head_count=4, head_count_kv=4, ffn=1024, capacity=64, rope_dims=128),
     3, {}, [100, 101]),
    ("G2 rope256 freq factors", dict(hidden=1024, head_count=4, head_count_kv=2, ffn=2048, capacity=256),
     3, dict(freq_factors=True), [37, 38]),
    ("G4 rope0 shared value", dict(hidden=768, head_count=8, head_count_kv=2, ffn=1536, capacity=300, rope_dims=0),
     4, dict(shared_v=True), [299, 300]),
    ("G8 window 32 wrap", dict(hidden=2048, head_count=8, head_count_kv=1, ffn=4096, capacity=128,
                                rope_dims=128, sliding_window=32), 5, {}, [500, 501, 502]),
    ("G2 one layer", dict(hidden=256, head_count=2, head_count_kv=1, ffn=512, capacity=32), 1, {}, [0, 1]),
]


@pytest.mark.parametrize("name,kw,n_layers,opts,positions", SMALL, ids=[c[0] for c in SMALL])
def test_small_models(hip, name, kw, n_layers, opts, positions):
    shape = DM.ModelShape(**kw)
    m = _Model(shape, n_layers, S.derive(S.config_seed(5), "fused-small", name), **opts)
    try:
        _compare(m, positions, name)
    finally:
        m.release()


FALLBACK = [
    ("G3", dict(hidden=768, head_count=6, head_count_kv=2, ffn=1536, capacity=64)),
    ("rope 64 dims", dict(hidden=512, head_count=2, head_count_kv=1, ffn=1024, capacity=64, rope_dims=64)),
    ("ring of 4608 slots", dict(hidden=512, head_count=2, head_count_kv=1, ffn=1024, capacity=4608)),
]


@pytest.mark.parametrize("name,kw", FALLBACK, ids=[c[0] for c in FALLBACK])
def test_uncovered_shapes_take_the_sequence(hip, name, kw):
    """Shapes outside the persistent step's cover run the launch sequence
    with the switch on, with its results."""
    shape = DM.ModelShape(**kw)
    m = _Model(shape, 2, S.derive(S.config_seed(5), "fused-fallback", name))
    try:
        ref, ref_cache, ref_launch = m.steps(False, [70, 71])
        got, got_cache, got_launch = m.steps(True, [70, 71])
        assert got_launch == ref_launch and min(ref_launch) > 1, (ref_launch, got_launch)
        _assert_same(ref, got, name)
        assert ref_cache == got_cache
    finally:
        H.setDecodeFused(False)
        m.release()


def test_graph_replays_at_advancing_positions(hip):
    """One persistent step captured in a HIP graph and replayed for three
    consecutive positions (the position read from device memory, host work
    between the replays): every replay equals the eager launch sequence."""
    import torch

    shape = DM.ModelShape(hidden=1024, head_count=8, head_count_kv=2, ffn=2048, capacity=96, rope_dims=256)
    m = _Model(shape, 4, S.derive(S.config_seed(5), "fused-graph"))
    positions = [95, 96, 97]
    try:
        ref, ref_cache, _ = m.steps(False, positions)
        H.setDecodeFused(True)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        hid = m.x.clone()
        out = torch.empty_like(hid)
        with torch.cuda.stream(side):
            # an eager step on the capture stream first: the descriptor table
            # and the exchange arena exist before the capture
            m.pos.fill_(positions[0])
            m.model.run_layers(hid.data_ptr(), m.pos.data_ptr(), out.data_ptr(), side.cuda_stream)
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=side):
                m.model.run_layers(hid.data_ptr(), m.pos.data_ptr(), out.data_ptr(),
                                   torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        assert H.decodeFusedStatus(side.cuda_stream) == 0
        m.restore()
        hid.copy_(m.x)
        got = []
        for p in positions:
            m.pos.fill_(p)
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            got.append((hid.cpu().numpy().view(np.uint32).copy(), out.cpu().numpy().view(np.uint32).copy()))
        assert H.decodeFusedStatus(side.cuda_stream) == 0
        _assert_same(ref, got, "graph replays")
        assert m.cache_digest() == ref_cache, "graph replays: KV caches differ"
        del g
    finally:
        H.setDecodeFused(False)
        m.release()


def test_wait_limit_reports_and_recovers(hip):
    """A one-tick bound on every stage wait: the launch stops at its first
    wait that is not already satisfied, the status reports HP_ERR_HIP once
    (reading clears it), and with the default bound the next step is exact."""
    import torch

    shape = DM.ModelShape(hidden=1024, head_count=4, head_count_kv=2, ffn=2048, capacity=64)
    m = _Model(shape, 8, S.derive(S.config_seed(5), "fused-timeout"))
    try:
        ref, ref_cache, _ = m.steps(False, [10])
        H.setDecodeFused(True)
        H.setFusedWaitLimit(1)
        m.restore()
        hid = m.x.clone()
        out = torch.empty_like(hid)
        m.pos.fill_(10)
        m.model.run_layers(hid.data_ptr(), m.pos.data_ptr(), out.data_ptr())
        torch.cuda.synchronize()
        assert H.decodeFusedStatus() == H.HP_ERR_HIP
        assert H.decodeFusedStatus() == 0
        H.setFusedWaitLimit(0)
        got, got_cache, got_launch = m.steps(True, [10])
        assert got_launch == [1]
        _assert_same(ref, got, "after a stopped step")
        assert got_cache == ref_cache
    finally:
        H.setFusedWaitLimit(0)
        H.setDecodeFused(False)
        m.release()
