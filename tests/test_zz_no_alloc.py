"""GPU check of hp_hip_topk_device_noalloc, the allocation-free variant of
hp_hip_topk_device (its selection state in a static device array): through
the C ABI, against hp_hip_topk_device on the same logits, bit for bit, on
two calls in a row (the second with a smaller input), then captured in a HIP
graph on a stream no call has used and replayed over changed logits."""
import numpy as np
import pytest

from heliopause_amd import synthetic as S

pytestmark = pytest.mark.gpu


def _topk_pair(hip, L, logits, rows, n, k, softcap=0.0):
    import torch

    ids_a = torch.zeros(rows * k, dtype=torch.int32, device="cuda:0")
    vals_a = torch.zeros(rows * k, dtype=torch.float32, device="cuda:0")
    ids_b = torch.full((rows * k,), -1, dtype=torch.int32, device="cuda:0")
    vals_b = torch.full((rows * k,), -1.0, dtype=torch.float32, device="cuda:0")
    hip.assertHipOk(L.hp_hip_topk_device(logits.data_ptr(), rows, n, k, softcap, ids_a.data_ptr(),
                                         vals_a.data_ptr(), None), "topk_device")
    hip.assertHipOk(L.hp_hip_topk_device_noalloc(logits.data_ptr(), rows, n, k, softcap, ids_b.data_ptr(),
                                                 vals_b.data_ptr(), None), "topk_device_noalloc")
    torch.cuda.synchronize()
    return ids_a.cpu().numpy(), vals_a.cpu().numpy(), ids_b.cpu().numpy(), vals_b.cpu().numpy()


def test_noalloc_topk_matches_topk_device(hip, oracle):
    import torch

    L = hip.lib()
    hip.assertHipOk(L.hp_hip_init(0), "init")
    cases = [(20, 262144, 40, 0.0), (3, 5000, 17, 30.0)]   # the second call is smaller (and batches: 20 rows)
    for rows, n, k, cap in cases:
        print(f"noalloc topk rows={rows} n={n} k={k} softcap={cap}", flush=True)
        host = S.activations(S.derive(S.BASE_SEED, "noalloc", rows, n), rows, n) * 4.0
        host[0, 100:140] = host[0].max()                     # ties at the top, broken by the lower id
        logits = torch.from_numpy(host).to(torch.device("cuda:0"))
        ia, va, ib, vb = _topk_pair(hip, L, logits, rows, n, k, cap)
        assert np.array_equal(ia, ib)
        assert np.array_equal(va.view(np.uint32), vb.view(np.uint32))
        if cap == 0.0:
            for r in range(rows):
                ids, vals = oracle.topk(host[r], k)
                assert np.array_equal(ib.reshape(rows, k)[r].view(np.uint32), ids)
                assert np.array_equal(vb.reshape(rows, k)[r].view(np.uint32), vals.view(np.uint32))


def test_noalloc_topk_rejects_bad_shapes(hip):
    L = hip.lib()
    hip.assertHipOk(L.hp_hip_init(0), "init")
    assert L.hp_hip_topk_device_noalloc(1, 1, 524289, 40, 0.0, 1, 1, None) == 1     # n too large: HP_ERR_SHAPE
    assert L.hp_hip_topk_device_noalloc(1, 1, 1000, 65, 0.0, 1, 1, None) == 18      # k too large: HP_ERR_ARG
    assert L.hp_hip_topk_device_noalloc(None, 1, 1000, 40, 0.0, 1, 1, None) == 18   # null logits


def test_noalloc_topk_graph_on_fresh_stream(hip, oracle):
    """Captured on a stream no library call has used (the pooled entry point
    would refuse to size its scratch there), replayed three times over new
    logits with eager work in between; every replay matches the eager call."""
    import torch

    L = hip.lib()
    hip.assertHipOk(L.hp_hip_init(0), "init")
    rows, n, k = 2, 262144, 40
    logits = torch.zeros(rows * n, dtype=torch.float32, device="cuda:0")
    ids = torch.zeros(rows * k, dtype=torch.int32, device="cuda:0")
    vals = torch.zeros(rows * k, dtype=torch.float32, device="cuda:0")
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            hip.assertHipOk(L.hp_hip_topk_device_noalloc(logits.data_ptr(), rows, n, k, 0.0, ids.data_ptr(),
                                                         vals.data_ptr(), torch.cuda.current_stream().cuda_stream),
                            "topk_device_noalloc (captured)")
    torch.cuda.synchronize()
    for rep in range(3):
        host = S.activations(S.derive(S.BASE_SEED, "noalloc-graph", rep), rows, n) * 3.0
        logits.copy_(torch.from_numpy(host.reshape(-1)))
        torch.cuda.synchronize()
        print(f"noalloc topk graph replay {rep}", flush=True)
        graph.replay()
        torch.cuda.synchronize()
        ia, va, _, _ = _topk_pair(hip, L, logits, rows, n, k)   # eager calls between replays
        assert np.array_equal(ids.cpu().numpy(), ia), rep
        assert np.array_equal(vals.cpu().numpy().view(np.uint32), va.view(np.uint32)), rep
