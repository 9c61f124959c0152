"""GPU: weights kept in one resident layout (hp_hip_set_weight_layouts(0)).

Such a weight keeps only the vector-ALU tiles -- hp_hip_stats.resident_bytes
grows by exactly its GGUF bytes -- and the matrix-core kernels gather their
operands from the tiles instead of the segment copy.  Every matrix-core
kernel must give the same bits either way: the decode matrix-core kernel
(selector 2) and the bit-exact prefill kernel (selector 4) against the
oracle, the fast prefill kernel (selector 5, and the automatic policy's
gate/up + GeGLU tiles) against the same launch on weights kept in both
layouts.  Shapes: one- and two-iteration tile geometries (K = 2560: 6-row
tiles of 10 blocks; K = 10240: 3-row tiles, two iterations of 20 blocks),
ragged rows (partial last tile and last 16-row segment), Q4_K and Q6_K, and
a mixed-type Q/K/V launch.  Through whole layers too: two layers of the
model's shape over a 100-token prefill chunk (fast kernel), a 40-token chunk
(bit-exact kernel) and a 4-token draft (matrix-core decode kernel), hidden
states, output norm and caches bit-identical either way.
"""
import numpy as np
import pytest

from heliopause_amd import decode as DM
from heliopause_amd import synthetic as S

pytestmark = pytest.mark.gpu

TYPES = {"Q4_K": 1, "Q6_K": 3}


def _bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).reshape(-1).view(np.uint32)


def _dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(torch.device("cuda:0"))


def _device_matmul(hip, handles, x, k, m):
    import torch

    dx = _dev(np.asarray(x, np.float32).reshape(-1))
    outs = [torch.empty(h.rowCount * m, dtype=torch.float32, device="cuda:0") for h in handles]
    hip.matmul_multi_device([h.handle for h in handles], dx.data_ptr(), k, m, [o.data_ptr() for o in outs],
                            [o.numel() for o in outs])
    torch.cuda.synchronize()
    return [o.cpu().numpy() for o in outs]


def _upload(hip, both, specs, ws, k):
    hip.setWeightLayouts(both)
    try:
        return [hip.createHipQuantizedWeightHandle(t, w, k, r) for (t, r), w in zip(specs, ws)]
    finally:
        hip.setWeightLayouts(True)


@pytest.fixture
def selector(request, hip):
    hip.setMatvecKernel(request.param)
    yield request.param
    hip.setMatvecKernel(0)


def test_resident_bytes(hip):
    k, rows = 2560, 37
    w = S.q4_k_blocks(S.derive(S.BASE_SEED, "one-layout-bytes"), rows, k)
    base = hip.hipResidentWeightStats()["residentBytes"]
    (h1,) = _upload(hip, False, [("Q4_K", rows)], [w], k)
    one = hip.hipResidentWeightStats()["residentBytes"] - base
    (h2,) = _upload(hip, True, [("Q4_K", rows)], [w], k)
    both = hip.hipResidentWeightStats()["residentBytes"] - base - one
    hip.releaseHipQuantizedWeightHandle(h1)
    hip.releaseHipQuantizedWeightHandle(h2)
    assert one == np.asarray(w).nbytes
    assert both == np.asarray(w).nbytes + ((rows + 15) // 16) * (k // 256) * 2304
    assert hip.hipResidentWeightStats()["residentBytes"] == base


CASES = [(2, "Q4_K", 37, 2560, 3), (2, "Q6_K", 19, 10240, 8), (2, "Q4_K", 300, 10240, 5),
         (4, "Q4_K", 37, 2560, 40), (4, "Q6_K", 100, 10240, 33), (4, "Q6_K", 7, 2560, 64),
         (5, "Q4_K", 300, 2560, 70), (5, "Q6_K", 40, 10240, 130), (5, "Q4_K", 2560, 10240, 64),
         (5, "Q6_K", 512, 2560, 200)]


@pytest.mark.parametrize("selector,type_name,rows,k,m", CASES, indirect=["selector"])
def test_matrix_core_kernels_same_bits(hip, oracle, selector, type_name, rows, k, m):
    print(f"one layout selector={selector} {type_name} rows={rows} k={k} m={m}", flush=True)
    seed = S.derive(S.BASE_SEED, "one-layout", type_name, rows, k, m)
    w = S.weight_blocks(type_name, seed, rows, k)
    x = S.activations(S.derive(seed, "x"), m, k)
    (h1,) = _upload(hip, False, [(type_name, rows)], [w], k)
    (h2,) = _upload(hip, True, [(type_name, rows)], [w], k)
    try:
        one = _device_matmul(hip, [h1], x, k, m)[0]
        both = _device_matmul(hip, [h2], x, k, m)[0]
    finally:
        hip.releaseHipQuantizedWeightHandle(h1)
        hip.releaseHipQuantizedWeightHandle(h2)
    assert np.array_equal(_bits(one), _bits(both))
    if selector in (2, 4):
        ref = oracle.matmul(TYPES[type_name], w, x, rows, threads=8)
        assert np.array_equal(_bits(one), _bits(ref))


@pytest.mark.parametrize("selector", [4, 0], ids=["exact", "auto"], indirect=True)
def test_mixed_qkv_launch_same_bits(hip, oracle, selector):
    k, m = 2560, 96
    specs = [("Q4_K", 2048), ("Q4_K", 512), ("Q6_K", 512)]
    seed = S.derive(S.BASE_SEED, "one-layout-qkv")
    ws = [S.weight_blocks(t, S.derive(seed, i), r, k) for i, (t, r) in enumerate(specs)]
    x = S.activations(S.derive(seed, "x"), m, k)
    print(f"one layout qkv m={m} selector={selector}", flush=True)
    h1 = _upload(hip, False, specs, ws, k)
    h2 = _upload(hip, True, specs, ws, k)
    try:
        one = _device_matmul(hip, h1, x, k, m)
        both = _device_matmul(hip, h2, x, k, m)
    finally:
        for h in h1 + h2:
            hip.releaseHipQuantizedWeightHandle(h)
    for a, b in zip(one, both):
        assert np.array_equal(_bits(a), _bits(b))
    if selector == 4:
        refs = oracle.matmul_multi([TYPES[t] for t, _ in specs], ws, x, [r for _, r in specs], threads=8)
        for a, ref in zip(one, refs):
            assert np.array_equal(_bits(a), _bits(ref))


@pytest.mark.parametrize("selector,m", [(2, 3), (4, 40), (5, 70)], indirect=["selector"])
def test_mixed_layouts_in_one_launch(hip, selector, m):
    """Q kept in both layouts, K and V in one: the launch reads every weight
    from its tiles and gives the bits of the all-both launch."""
    k = 2560
    specs = [("Q4_K", 2048), ("Q4_K", 512), ("Q6_K", 512)]
    seed = S.derive(S.BASE_SEED, "mixed-layouts")
    ws = [S.weight_blocks(t, S.derive(seed, i), r, k) for i, (t, r) in enumerate(specs)]
    x = S.activations(S.derive(seed, "x", m), m, k)
    print(f"mixed layouts selector={selector} m={m}", flush=True)
    mixed = _upload(hip, True, specs[:1], ws[:1], k) + _upload(hip, False, specs[1:], ws[1:], k)
    both = _upload(hip, True, specs, ws, k)
    try:
        a = _device_matmul(hip, mixed, x, k, m)
        b = _device_matmul(hip, both, x, k, m)
    finally:
        for h in mixed + both:
            hip.releaseHipQuantizedWeightHandle(h)
    for u, v in zip(a, b):
        assert np.array_equal(_bits(u), _bits(v))


@pytest.mark.parametrize("rows,m", [(160, 96), (1000, 130)])
def test_geglu_tiles_same_bits(hip, rows, m):
    """gate/up + GeGLU on the fast prefill kernel's paired tiles (automatic
    policy from 64 columns on the device entry point)."""
    import torch

    k = 2560
    seed = S.derive(S.BASE_SEED, "one-layout-geglu", rows, m)
    wg = S.q4_k_blocks(S.derive(seed, "g"), rows, k)
    wu = S.q4_k_blocks(S.derive(seed, "u"), rows, k)
    x = S.activations(seed, m, k)
    print(f"one layout geglu rows={rows} m={m}", flush=True)
    outs = []
    for both in (False, True):
        hg, hu = _upload(hip, both, [("Q4_K", rows), ("Q4_K", rows)], [wg, wu], k)
        try:
            dx = _dev(x.reshape(-1))
            dout = torch.empty(rows * m, dtype=torch.float32, device="cuda:0")
            hip.matmul_geglu_device(hg.handle, hu.handle, dx.data_ptr(), k, m, dout.data_ptr(), rows)
            torch.cuda.synchronize()
            outs.append(dout.cpu().numpy())
        finally:
            hip.releaseHipQuantizedWeightHandle(hg)
            hip.releaseHipQuantizedWeightHandle(hu)
    assert np.array_equal(_bits(outs[0]), _bits(outs[1]))


@pytest.mark.parametrize("tokens", [100, 40, 4])
def test_layers_same_bits(hip, tokens):
    import torch

    shape = DM.ModelShape()
    seed = S.derive(S.BASE_SEED, "one-layout-layers", tokens)
    datas = [DM.layer_host_data(shape, seed, i) for i in range(2)]
    onorm = (1 + 0.1 * S.normal(S.derive(seed, "onorm"), shape.hidden)).astype(np.float32)
    x = S.activations(S.derive(seed, "x"), tokens, shape.hidden) * 4
    pos = shape.capacity - tokens
    results = []
    for both in (False, True):
        hip.setWeightLayouts(both)
        model = DM.HipDecodeModel(shape)
        try:
            for d in datas:
                model.add_layer(d)
            hip.setWeightLayouts(True)
            model.output_norm = _dev(onorm)
            dx = _dev(x.reshape(-1))
            dpos = _dev(np.array([pos], np.int32))
            out = torch.empty(tokens * shape.hidden, dtype=torch.float32, device="cuda:0")
            print(f"one layout layers both={both}, {tokens} tokens", flush=True)
            model.run_layers(dx.data_ptr(), dpos.data_ptr(), out.data_ptr(), tokens=tokens)
            torch.cuda.synchronize()
            caches = [c.cpu().numpy().copy() for layer in model.caches for c in layer]
            results.append((dx.cpu().numpy(), out.cpu().numpy(), caches))
        finally:
            model.release()
            hip.setWeightLayouts(True)
    (h1, o1, c1), (h2, o2, c2) = results
    assert np.array_equal(h1, h2)
    assert np.array_equal(o1, o2)
    assert len(c1) == len(c2) and all(np.array_equal(a, b) for a, b in zip(c1, c2))
