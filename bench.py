"""Benchmark of the gfx950 quantized-projection path.

Default workload (the metric's configuration): the batched attention
projections of one decoder layer sharing one input -- Q = Q4_K 2048x2560,
K = Q4_K 512x2560, V = Q6_K 512x2560 -- as ONE multi-weight launch (shared
in-kernel Q8_K), M = 1 column.  A step is one such projection pass.

Other workloads (``--workload``): ``cfg1`` (one Q4_K 10240x2560 matvec),
``gate_up`` (two Q4_K 10240x2560 in one launch), ``down`` (Q6_K 2560x10240),
``ffn`` (gate/up launch -> GeGLU -> down), ``head`` (Q6_K 262144x2560 output
head + top-40 per column, candidates only), ``decode42`` (a full decode step
of a 42-layer model with a 4096-token KV cache, in one graph),
``decode42-proj`` (only that step's projection chain), ``prefill42`` (a
512-token chunk through that model's projections on the matrix cores) and
``gguf-load`` (a 3.02 GB GGUF file of that model streamed into HBM-resident
handles).

Weights are GGUF super-blocks generated from a fixed seed and uploaded once;
steps rotate over enough distinct weight copies (>= 640 MiB) that every step
streams its weights from HBM rather than from the 256 MB Infinity Cache.
Inputs and outputs stay in HBM.  Exactly ``--steps`` steps are timed: they
are captured in one HIP graph (step i on copy i % copies) and replayed once,
after a warm-up graph of the ``--warmup`` steps that also streams every other
copy.

Prints one JSON line.  ``value`` = algorithmic bytes per step (weights as
stored + f32 activations read and written) / wall time per step, in GB/s.
The default line also carries ``decode_step``: the 42-layer model's decode
step at M = 1 (``--workload decode42``), measured in the same run.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import platform
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "Q4_K/Q6_K matvec GB/s (% HBM peak); decode step ms at M=1 (1 GPU)"
HBM_PEAK_GBPS = 8000.0
TYPE_IDS = {"Q4_K": 1, "Q6_K": 3}
BLOCK = {"Q4_K": 144, "Q6_K": 210}

# name -> (config id, input size, weights of one launch, description)
WORKLOADS = {
    "qkv": (2, 2560, [("Q4_K", 2048), ("Q4_K", 512), ("Q6_K", 512)],
            "attention Q/K/V projections sharing one input: Q Q4_K 2048x2560, K Q4_K 512x2560, "
            "V Q6_K 512x2560, one multi-weight launch with in-kernel Q8_K"),
    "cfg1": (1, 2560, [("Q4_K", 10240)], "single Q4_K 10240x2560 matvec"),
    "gate_up": (3, 2560, [("Q4_K", 10240), ("Q4_K", 10240)], "FFN gate+up: two Q4_K 10240x2560 in one launch"),
    "down": (3, 10240, [("Q6_K", 2560)], "FFN down: Q6_K 2560x10240"),
    "ffn": (3, 2560, [("Q4_K", 10240), ("Q4_K", 10240)],
            "decoder FFN: gate/up Q4_K 10240x2560 + GeGLU -> down Q6_K 2560x10240"),
    "head": (4, 2560, [("Q6_K", 262144)], "output head Q6_K 262144x2560 + top-40 per column (candidates only)"),
}
FFN_DOWN = ("Q6_K", 2560, 10240)
TOPK = 40

# The 42-layer synthetic Gemma-like model: per layer (type, rows, input size)
LAYER = [("Q4_K", 2048, 2560), ("Q4_K", 512, 2560), ("Q6_K", 512, 2560),   # Q, K, V
         ("Q4_K", 2560, 2048),                                              # O
         ("Q4_K", 10240, 2560), ("Q4_K", 10240, 2560),                      # gate, up
         ("Q6_K", 2560, 10240)]                                             # down
N_LAYERS = 42
HEAD = ("Q6_K", 262144, 2560)


def row_bytes(t: str, k: int) -> int:
    return k // 256 * BLOCK[t]


def weight_bytes(workload: str) -> int:
    _, k, specs, _ = WORKLOADS[workload]
    b = sum(row_bytes(t, k) * r for t, r in specs)
    if workload == "ffn":
        b += row_bytes(FFN_DOWN[0], FFN_DOWN[2]) * FFN_DOWN[1]
    return b


def algorithmic_bytes(workload: str, m: int) -> int:
    """Weights as stored plus every f32 activation the step reads or writes."""
    _, k, specs, _ = WORKLOADS[workload]
    rows = sum(r for _, r in specs)
    b = weight_bytes(workload) + m * k * 4 + m * rows * 4
    if workload == "ffn":  # gate/up+GeGLU writes h (not gate, up); down reads h, writes y
        b += m * (10240 + 10240 + 2560) * 4 - m * sum(r for _, r in specs) * 4
    if workload == "head":  # logits read back by top-k, candidates written
        b += m * 262144 * 4 + m * TOPK * 8
    return b


def matvec_kernel_name(choice: str, k: int, m: int, specs: list) -> str:
    """The matvec kernel the runner picks for one launch of weights specs
    [(type, rows)] (its automatic policy restated: tile counts of the
    vector-ALU and matrix-core layouts; the weight-type template argument is
    the launch's common type id, 0 when the types differ)."""
    rows = [r for _, r in specs]
    types = {TYPE_IDS[t] for t, _ in specs}
    type_id = types.pop() if len(types) == 1 else 0
    nb = k // 256
    s = next(d for d in range(min(nb, 64), 0, -1) if nb % d == 0 and ((64 // d) * d >= 48 or d == 1))
    r6 = 64 // s
    tiles = sum((r + r6 - 1) // r6 for r in rows)
    tiles16 = sum((r + 15) // 16 for r in rows)
    wide = m <= 4 and type_id in (1, 3) and (choice.startswith("wide") or (choice == "auto" and nb >= 40))
    if wide:
        return f"kquant_wide_kernel<{m}, {type_id}>"
    half = s <= 32 and m <= 4 and (choice == "half" or
                                   (choice == "auto" and s <= 16 and tiles <= (2048 if m == 1 else 1024)))
    mfma = choice == "mfma" or (choice == "auto" and not half and k <= 2560 and
                                (m >= 5 or (m >= 2 and tiles16 >= 1024)))
    if half:
        return f"kquant_matvec_half_kernel<{m}, 0, {type_id}>"
    if mfma:
        return "kquant_mfma_kernel"
    return f"kquant_matvec_kernel<{m}, {'true' if m <= 3 else 'false'}, false, 0, {type_id if m <= 3 else 0}>"


def parse() -> argparse.Namespace:
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--m", type=int, default=1)
    p.add_argument("--workload", choices=sorted(WORKLOADS) + ["decode42", "decode42-proj", "prefill42", "prefill42-layers",
                                                            "gguf-load"], default="qkv")
    p.add_argument("--rotate-mib", type=int, default=640, help="distinct weight bytes cycled through")
    p.add_argument("--cpu-seconds", type=float, default=12.0)
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--no-decode", action="store_true",
                   help="leave the decode-step object out of the default line")
    p.add_argument("--kernel", choices=["auto", "valu", "mfma", "half", "wide", "wide-whole", "wide-half"],
                   default="auto",
                   help="matvec kernel: automatic choice, vector ALU, matrix cores, half-split vector ALU, "
                        "wide (one workgroup per block of rows), the wide kernel with whole or half "
                        "row-blocks per thread")
    p.add_argument("--weight-layouts", choices=["both", "one"], default="both",
                   help="resident weight layouts: both (vector-ALU tiles + matrix-core segments, the default) "
                        "or one (tiles only; the matrix-core kernels read them)")
    p.add_argument("--copy-probe", action="store_true",
                   help="only run a plain 256 MiB device copy (HBM counter calibration) and exit")
    return p.parse_args()


def copy_probe() -> int:
    """A plain device-to-device copy of a known size; its FETCH_SIZE/WRITE_SIZE
    per dispatch calibrate the HBM traffic counters of the projection kernel."""
    import torch

    n = 256 << 20
    a = torch.empty(n, dtype=torch.uint8, device="cuda:0").fill_(1)
    b = torch.empty_like(a)
    for _ in range(10):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_bytes": n, "dispatches": 10}))
    return 0


def host_cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), else what platform reports."""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def host_threads() -> int:
    """CPUs this process may run on (its affinity set), at most 16: the host
    share of one GPU on the benchmark machines."""
    try:
        n = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def time_calls(fn, min_seconds: float) -> tuple[float, int]:
    """prefill-kernels.bench.ts:90-121's loop: 8 warm-ups, then the iteration
    count doubles until one run lasts >= min_seconds; returns (seconds per
    call, calls in that run)."""
    for _ in range(8):
        fn()
    n = 1
    while True:
        t0 = time.perf_counter()
        for _ in range(n):
            fn()
        el = time.perf_counter() - t0
        if el >= min_seconds:
            return el / n, n
        n *= 2


def cpu_baseline(workload: str, ws, x, seconds: float) -> dict:
    """The oracle's threaded restatement of the reference's resident WASM path
    (hp_matmul_quantized_prepared_multi_f32 with splitRows sharding) on the
    same launch, bounded to about ``seconds`` of host time over four legs:
    the 128-bit SSE4.1 build (the width of wasm simd128) and a build for this
    host's own ISA (-march=native), each at the reference's default pool size
    and at every CPU the process may use.  ``value`` is the SSE4.1 leg at the
    default pool size, the reference's configuration."""
    import tempfile

    from oracle import oracle as O

    _, k, specs, _ = WORKLOADS[workload]
    tids = [TYPE_IDS[t] for t, _ in specs]
    rows = [r for _, r in specs]
    m = x.shape[0]
    launch_bytes = sum(row_bytes(t, k) * r for t, r in specs) + m * k * 4 + m * sum(rows) * 4
    t_default = O.default_threads()
    t_all = host_threads()
    libs = [("sse4.1 (wasm simd128 width)", None)]
    note = ""
    try:
        libs.append(("-march=native", O.native_lib(tempfile.mkdtemp(prefix="hp_oracle_"))))
    except (OSError, Exception) as exc:  # no compiler on the host: the leg is reported missing
        note = f"; native leg not built ({type(exc).__name__})"
    legs = []
    per_leg = max(0.75, seconds / (2 * len(libs)))
    for isa, library in libs:
        for threads in sorted({t_default, t_all}):
            sec, n = time_calls(lambda: O.matmul_multi(tids, ws, x, rows, threads=threads, library=library), per_leg)
            legs.append({"isa": isa, "threads": threads, "ms_per_call": round(sec * 1e3, 4),
                         "GB/s": round(launch_bytes / sec / 1e9, 3), "calls": n})
    ref_leg = legs[0]
    return {
        "value": ref_leg["GB/s"],
        "unit": "GB/s",
        "cores": t_default,
        "kind": "port",
        "sample": f"the {workload} projection launch at M={m} ({launch_bytes} algorithmic bytes); C restatement of "
                  f"lib.rs resident kernels with splitRows sharding, timed as prefill-kernels.bench.ts does (8 "
                  f"warm-ups, doubling to >= {per_leg:.2f} s per leg); value: SSE4.1 build on the reference's "
                  f"default pool of {t_default} threads; excludes the reference's JS/worker overhead{note}",
        "cpu_model": host_cpu_model(),
        "logical_cpus": os.cpu_count(),
        "usable_cpus": t_all,
        "legs": legs,
    }


def decode_chain(args) -> int:
    """Projection chain of one decode step of the 42-layer model at M = 1:
    per layer Q/K/V (one launch) -> O (fed Q's 2048 outputs) -> gate/up +
    GeGLU (one launch) -> down, then the head, top-40 and the sampled next
    token (generator state kept in HBM); every layer's weights
    are distinct device copies (3.02 GB, so nothing is Infinity-Cache hot).
    Attention, norms, RoPE and residuals are not part of this path and are
    not run; each layer's Q/K/V and the head read one fixed input, which does
    not change the launch order (one stream)."""
    import numpy as np
    import torch

    from heliopause_amd import hip_kernels as H
    from heliopause_amd import synthetic as S

    if args.m != 1:
        raise SystemExit("decode42 runs at M = 1")
    H.setMatvecKernel(KERNEL_CHOICES[args.kernel](H))
    torch.cuda.init()
    dev = torch.device("cuda:0")
    seed = S.config_seed(5)
    host = {}
    for i, (t, r, k) in enumerate(LAYER + [HEAD]):
        if (t, r, k) not in host:
            host[(t, r, k)] = S.weight_blocks(t, S.derive(seed, "decode42", i), r, k)
    layers = []
    for _ in range(N_LAYERS):
        layers.append([H.createHipQuantizedWeightHandle(t, host[(t, r, k)], k, r).handle for t, r, k in LAYER])
    head = H.createHipQuantizedWeightHandle(HEAD[0], host[HEAD], HEAD[2], HEAD[1]).handle
    x = torch.from_numpy(S.activations(S.derive(seed, "x"), 1, 2560)).to(dev)
    buf = {n: torch.empty(c, dtype=torch.float32, device=dev)
           for n, c in (("q", 2048), ("k", 512), ("v", 512), ("o", 2560), ("g", 10240), ("u", 10240),
                        ("h", 10240), ("y", 2560), ("logits", 262144))}
    ids = torch.empty(TOPK, dtype=torch.int32, device=dev)
    vals = torch.empty(TOPK, dtype=torch.float32, device=dev)
    # next-token sampling on the device (top-40 slice, top-p 0.95, T = 1); the
    # generator state stays in HBM and advances every step
    sampling = H.resolveGenerationSamplingOptions(topK=TOPK)
    rng = torch.from_numpy(np.array([sampling["seed"]], np.uint32).view(np.int32)).to(dev)
    token = torch.zeros(1, dtype=torch.int32, device=dev)
    kept = torch.zeros(1, dtype=torch.int32, device=dev)
    probs = torch.zeros(TOPK, dtype=torch.float64, device=dev)
    L = H.lib()
    p = {n: t.data_ptr() for n, t in buf.items()}

    def step(stream: int) -> None:
        for hs in layers:
            H.matmul_multi_device(hs[0:3], x.data_ptr(), 2560, 1, [p["q"], p["k"], p["v"]], [2048, 512, 512], stream)
            H.matmul_multi_device(hs[3:4], p["q"], 2048, 1, [p["o"]], [2560], stream)
            H.matmul_geglu_device(hs[4], hs[5], p["o"], 2560, 1, p["h"], 10240, stream)
            H.matmul_multi_device(hs[6:7], p["h"], 10240, 1, [p["y"]], [2560], stream)
        H.matmul_multi_device([head], x.data_ptr(), 2560, 1, [p["logits"]], [262144], stream)
        H.assertHipOk(L.hp_hip_topk_device(p["logits"], 1, 262144, TOPK, 0.0, ids.data_ptr(), vals.data_ptr(),
                                           stream), "topk")
        H.sample_device(ids.data_ptr(), vals.data_ptr(), 1, TOPK, TOPK, sampling, rng.data_ptr(), token.data_ptr(),
                        probs.data_ptr(), kept.data_ptr(), stream)

    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        step(side.cuda_stream)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            step(torch.cuda.current_stream().cuda_stream)
    for _ in range(max(1, args.warmup // 10)):
        graph.replay()
    torch.cuda.synchronize()
    steps = max(1, args.steps // 10)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    for _ in range(steps):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) / steps * 1e3
    ms = start.elapsed_time(end) / steps
    wbytes = N_LAYERS * sum(row_bytes(t, k) * r for t, r, k in LAYER) + row_bytes(HEAD[0], HEAD[2]) * HEAD[1]
    launches = N_LAYERS * 4 + 1 + 3 + 1
    line = {
        "metric": "decode step projection chain ms at M=1 (1 GPU)",
        "value": round(ms, 4), "unit": "ms", "n_gpus": 1, "steps": steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 4), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8", "data": "synthetic",
        "config": {"workload": "42-layer synthetic Gemma-like model, projections + GeGLU + head + top-40 + "
                               "next-token sampling at M=1 (attention, norms, RoPE, residuals not included)",
                   "weight_bytes": wbytes, "launches_per_step": launches, "wall_ms_per_step": round(wall_ms, 4),
                   "timing": "one step captured in a HIP graph and replayed"},
        "roofline": {"bound": "hbm", "achieved": round(wbytes / (ms * 1e-3) / 1e9, 2), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(wbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
                     "weight_bytes_over_peak_ms": round(wbytes / HBM_PEAK_GBPS / 1e6, 4)},
    }
    print(json.dumps(_label(line)))
    return 0


def measure_decode_step(m: int, steps: int, warmup: int, cpu_seconds: float | None) -> dict:
    """One decode step of the 42-layer synthetic Gemma-like model at M = m
    (hidden 2560, 8 query / 2 KV heads of 256, FFN 10240; Q4_K_M mix) with a
    4096-token f16 KV cache filled with N(0,1): the last token at position
    4096 attends over the last 4096 positions of every layer.  Per layer:
    attn_norm -> Q/K/V -> q/k norms + RoPE + v norm + cache append -> GQA
    attention -> O -> post-attention norm + residual + ffn_norm -> gate/up +
    GeGLU -> down -> post-FFN norm + residual + layer scale + next attn_norm;
    then output_norm, the Q6_K 262144x2560 head, top-40 and (one token) the
    sampled next token.  Every layer's weights and cache are distinct device
    copies (3.02 GB of weights + 352 MB of cache).  The step starts by copying
    the input hidden state into the residual buffer (standing in for the
    embedding row), so every replay computes the same step.  One step is
    captured in a HIP graph; `warmup` replays, then `steps` replays timed.
    The per-kernel split comes from one eager step with HIP events around
    every launch (hp_hip_profile)."""
    import numpy as np
    import torch

    from heliopause_amd import decode as DM
    from heliopause_amd import hip_kernels as H
    from heliopause_amd import synthetic as S

    if not 1 <= m <= 8:
        raise SystemExit("decode42 runs 1..8 tokens per step")
    torch.cuda.init()
    dev = torch.device("cuda:0")
    shape = DM.ModelShape()
    seed = S.config_seed(5)
    data = DM.layer_host_data(shape, seed, 0)
    model = DM.HipDecodeModel(shape)
    for _ in range(N_LAYERS):
        model.add_layer(data)
    head_blocks = S.weight_blocks(HEAD[0], S.derive(seed, "head"), HEAD[1], HEAD[2])
    head = H.createHipQuantizedWeightHandle(HEAD[0], head_blocks, HEAD[2], HEAD[1])
    model.set_head((1.0 + 0.1 * S.normal(S.derive(seed, "output_norm"), shape.hidden)).astype(np.float32), head)
    x0 = torch.from_numpy(S.activations(S.derive(seed, "x"), m, shape.hidden).reshape(-1) * 4).to(dev)
    hidden = torch.empty_like(x0)
    normed = torch.empty_like(x0)
    pos = torch.tensor([shape.capacity + 1 - m], dtype=torch.int32, device=dev)  # last token at 4096
    logits = torch.empty(m * HEAD[1], dtype=torch.float32, device=dev)
    ids = torch.empty(m * TOPK, dtype=torch.int32, device=dev)
    vals = torch.empty(m * TOPK, dtype=torch.float32, device=dev)
    sampling = H.resolveGenerationSamplingOptions(topK=TOPK)
    rng = torch.from_numpy(np.array([sampling["seed"]], np.uint32).view(np.int32)).to(dev)
    token = torch.zeros(1, dtype=torch.int32, device=dev)
    kept = torch.zeros(1, dtype=torch.int32, device=dev)
    probs = torch.zeros(TOPK, dtype=torch.float64, device=dev)
    L = H.lib()

    def step(stream: int) -> None:
        hidden.copy_(x0)
        model.run_layers(hidden.data_ptr(), pos.data_ptr(), normed.data_ptr(), stream, tokens=m)
        H.matmul_multi_device([head.handle], normed.data_ptr(), shape.hidden, m, [logits.data_ptr()],
                              [m * HEAD[1]], stream)
        H.assertHipOk(L.hp_hip_topk_device(logits.data_ptr(), m, HEAD[1], TOPK, 0.0, ids.data_ptr(),
                                           vals.data_ptr(), stream), "topk")
        if m == 1:  # a draft's positions are compared with the draft on the host (acceptMtpDraft)
            H.sample_device(ids.data_ptr(), vals.data_ptr(), 1, TOPK, TOPK, sampling, rng.data_ptr(),
                            token.data_ptr(), probs.data_ptr(), kept.data_ptr(), stream)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        launches0 = H.hipResidentWeightStats()["kernelLaunches"]
        step(side.cuda_stream)
        launches = H.hipResidentWeightStats()["kernelLaunches"] - launches0 + 1  # + the input copy
        torch.cuda.synchronize()
        # per-kernel split: one eager step with events around every launch
        H.profile(True)
        step(side.cuda_stream)
        torch.cuda.synchronize()
        split = {}
        for kid, name in H.KERNEL_NAMES.items():
            ms, n = H.profile_read(kid)
            if n:
                split[name] = {"us": round(ms * 1e3, 1), "launches": n}
        H.profile(False)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            step(torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    for _ in range(max(1, warmup)):
        graph.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    for _ in range(steps):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) / steps * 1e3
    ms = start.elapsed_time(end) / steps
    wbytes = N_LAYERS * sum(row_bytes(t, k) * r for t, r, k in LAYER) + row_bytes(HEAD[0], HEAD[2]) * HEAD[1]
    kv_bytes = N_LAYERS * 2 * shape.head_count_kv * shape.capacity * 256 * 2
    cpu = None if (cpu_seconds is None or m != 1) else decode_cpu_baseline(shape, data, head_blocks, cpu_seconds)
    resident = H.hipResidentWeightStats()["residentBytes"]  # the model's handles (both layouts by default)
    model.release()
    H.releaseHipQuantizedWeightHandle(head)
    return {"m": m, "ms": ms, "wall_ms": wall_ms, "steps": steps, "launches": launches, "split": split,
            "weight_bytes": wbytes, "kv_bytes": kv_bytes, "cpu": cpu, "resident_bytes": resident,
            "positions": [int(shape.capacity) + 1 - m, int(shape.capacity)]}


def decode_summary(r: dict) -> dict:
    """The decode-step object of the JSON line (one token)."""
    total = r["weight_bytes"] + r["kv_bytes"]
    target = 1.3 * r["weight_bytes"] / HBM_PEAK_GBPS / 1e6
    return {
        "workload": "42-layer synthetic Gemma-like model, full decode step at M=1 with a 4096-token f16 KV cache "
                    "(token at position 4096): norms, Q/K/V, RoPE, cache append, GQA attention, O, GeGLU FFN, "
                    "residuals, output norm, Q6_K 262144x2560 head, top-40, next-token sampling; one HIP graph",
        "ms_per_step": round(r["ms"], 4),
        "wall_ms_per_step": round(r["wall_ms"], 4),
        "steps": r["steps"],
        "weight_bytes": r["weight_bytes"],
        "kv_cache_bytes": r["kv_bytes"],
        "GB/s": round(total / (r["ms"] * 1e-3) / 1e9, 1),
        "frac_of_peak": round(total / (r["ms"] * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
        "target_ms": round(target, 4),
        "vs_target": round(r["ms"] / target, 3),
        "launches_per_step": r["launches"],
        "kernel_split_us": r["split"],
        "kernel_split_note": "one eager step with HIP events around each launch (includes per-launch gaps)",
    }


def decode_step(args) -> int:
    """``--workload decode42``: the decode step (or a draft of --m tokens) as
    its own JSON line."""
    from heliopause_amd import hip_kernels as H

    m = args.m
    H.setMatvecKernel(KERNEL_CHOICES[args.kernel](H))
    r = measure_decode_step(m, max(1, args.steps // 10), max(1, args.warmup // 10),
                            None if args.no_cpu else args.cpu_seconds)
    ms = r["ms"]
    total = r["weight_bytes"] + r["kv_bytes"]
    line = {
        "metric": "decode step ms at M=1 (1 GPU)" if m == 1 else f"draft verification step ms at M={m} (1 GPU)",
        "value": round(ms, 4), "unit": "ms", "n_gpus": 1, "steps": r["steps"], "warmup": max(1, args.warmup // 10),
        "ms_per_step": round(ms, 4), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8", "data": "synthetic",
        "config": {"workload": decode_summary(r)["workload"] if m == 1 else
                               f"42-layer synthetic Gemma-like model, verification of a {m}-token draft (every "
                               "position through every layer with causal attention over a 4096-token f16 KV cache, "
                               "output norm, head, top-40 per position)",
                   "weight_bytes": r["weight_bytes"], "resident_weight_bytes": r["resident_bytes"],
                   "kv_cache_bytes_read": r["kv_bytes"],
                   "launches_per_step": r["launches"], "wall_ms_per_step": round(r["wall_ms"], 4), "tokens": m,
                   "positions": r["positions"], "kernel_split_us": r["split"],
                   "timing": "one step captured in a HIP graph and replayed"},
        "roofline": {"bound": "hbm", "achieved": round(total / (ms * 1e-3) / 1e9, 2), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(total / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
                     "traffic": None, "bytes_per_step": total,
                     "weight_bytes_over_peak_ms": round(r["weight_bytes"] / HBM_PEAK_GBPS / 1e6, 4),
                     "target_ms": round(1.3 * r["weight_bytes"] / HBM_PEAK_GBPS / 1e6, 4)},
        "cpu_baseline": r["cpu"],
    }
    print(json.dumps(_label(line)))
    return 0


def decode_cpu_baseline(shape, data, head_blocks, seconds: float) -> dict:
    """The oracle's restatement of the WASM decode step on the host: layers of
    the same model (4096-token cache) run until ``seconds`` pass, plus the head
    once; the step time is extrapolated to 42 layers + head."""
    import numpy as np

    from oracle import decode_layer as OD
    from oracle import oracle as O

    tids = {"Q4_K": 1, "Q6_K": 3}
    w = {n: (tids[t], blocks, rows) for n, (t, blocks, rows, _) in data["weights"].items()}
    layer = OD.Layer(weights=w, norms=dict(data["norms"]), key_cache=data["key_cache"].copy(),
                     value_cache=data["value_cache"].copy(), head_count=shape.head_count,
                     head_count_kv=shape.head_count_kv, epsilon=shape.epsilon,
                     output_scale=float(data["output_scale"]))
    x = np.zeros(shape.hidden, np.float32) + 0.5
    n, t0 = 0, time.perf_counter()
    while True:
        x = OD.forward_layer(layer, x, shape.capacity)
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    per_layer = el / n
    th = time.perf_counter()
    O.matmul(TYPE_IDS[HEAD[0]], head_blocks, x.reshape(1, -1), head_blocks.shape[0], threads=O.default_threads())
    head_s = time.perf_counter() - th
    step_ms = (N_LAYERS * per_layer + head_s) * 1e3
    return {"value": round(step_ms, 2), "unit": "ms", "cores": O.default_threads(), "kind": "port",
            "sample": f"{n} decoder layers ({per_layer * 1e3:.1f} ms each: projections on {O.default_threads()} "
                      f"threads, attention over 4096 cached tokens on one) + the head once ({head_s * 1e3:.0f} ms), "
                      f"extrapolated to 42 layers + head; host {host_cpu_model()}, {os.cpu_count()} logical CPUs"}


MFMA_F16_PEAK_TFLOPS = 2500.0  # dense f16 matrix-core peak, MI355X


def prefill_chain(args) -> int:
    """Projections of one 512-token prefill chunk through the 42-layer model:
    per layer Q/K/V (one launch over all 512 columns) -> O (fed Q's outputs)
    -> gate/up + GeGLU -> down, every layer's weights a distinct device copy;
    captured in one HIP graph.  FLOPs = 2 * 512 * (projection weights of the
    42 layers) = 3.946e12.  The head is not part of prefill (only the last
    token's logits are needed) and attention is not run."""
    import numpy as np
    import torch

    from heliopause_amd import hip_kernels as H
    from heliopause_amd import synthetic as S

    m = args.m if args.m > 1 else 512
    H.setMatvecKernel(KERNEL_CHOICES[args.kernel](H))
    torch.cuda.init()
    dev = torch.device("cuda:0")
    seed = S.config_seed(5)
    host = {}
    for i, (t, r, k) in enumerate(LAYER):
        if (t, r, k) not in host:
            host[(t, r, k)] = S.weight_blocks(t, S.derive(seed, "decode42", i), r, k)
    layers = [[H.createHipQuantizedWeightHandle(t, host[(t, r, k)], k, r).handle for t, r, k in LAYER]
              for _ in range(N_LAYERS)]
    x = torch.from_numpy(S.activations(S.derive(seed, "prefill-x"), m, 2560)).to(dev)
    buf = {n: torch.empty(m * c, dtype=torch.float32, device=dev)
           for n, c in (("q", 2048), ("k", 512), ("v", 512), ("o", 2560), ("h", 10240), ("y", 2560))}
    p = {n: t.data_ptr() for n, t in buf.items()}

    def step(stream: int) -> None:
        for hs in layers:
            H.matmul_multi_device(hs[0:3], x.data_ptr(), 2560, m, [p["q"], p["k"], p["v"]],
                                  [2048 * m, 512 * m, 512 * m], stream)
            H.matmul_multi_device(hs[3:4], p["q"], 2048, m, [p["o"]], [2560 * m], stream)
            H.matmul_geglu_device(hs[4], hs[5], p["o"], 2560, m, p["h"], 10240, stream)
            H.matmul_multi_device(hs[6:7], p["h"], 10240, m, [p["y"]], [2560 * m], stream)

    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        launches0 = H.hipResidentWeightStats()["kernelLaunches"]
        step(side.cuda_stream)
        launches = H.hipResidentWeightStats()["kernelLaunches"] - launches0
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            step(torch.cuda.current_stream().cuda_stream)
    warm = max(1, args.warmup // 40)
    for _ in range(warm):
        graph.replay()
    torch.cuda.synchronize()
    steps = max(1, args.steps // 80)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    for _ in range(steps):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) / steps * 1e3
    ms = start.elapsed_time(end) / steps
    weights = N_LAYERS * sum(r * k for _, r, k in LAYER)
    flops = 2.0 * m * weights
    tflops = flops / (ms * 1e-3) / 1e12
    line = {
        "metric": f"prefill chunk projections ms at M={m} (1 GPU)",
        "value": round(ms, 4), "unit": "ms", "n_gpus": 1, "steps": steps, "warmup": warm,
        "ms_per_step": round(ms, 4), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "f16 MFMA (exact integers) + f32 tail", "data": "synthetic",
        "config": {"workload": f"42-layer synthetic Gemma-like model, projections + GeGLU of a {m}-token prefill "
                               "chunk (head and attention not included)",
                   "columns": m, "weight_elements": weights, "flops": flops,
                   "launches_per_step": launches, "wall_ms_per_step": round(wall_ms, 4),
                   "timing": "one chunk captured in a HIP graph and replayed"},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tflops / MFMA_F16_PEAK_TFLOPS, 4), "traffic": None},
    }
    print(json.dumps(_label(line)))
    return 0


def prefill_layers(args) -> int:
    """A 512-token prefill chunk through the whole 42-layer model on the
    device: per layer attn_norm -> Q/K/V -> q/k norms + RoPE + v norm + the
    chunk's cache append -> causal GQA attention over the ring (prefill
    attention on the matrix cores + merge) -> O -> residual + ffn_norm ->
    gate/up + GeGLU -> down -> residual + layer scale; then output_norm.  The
    chunk sits at positions 3584..4095 of a 4096-slot f16 cache filled with
    N(0,1), so the last token attends over all 4096 positions.  One chunk is
    captured in a HIP graph and replayed (every replay rewrites the same
    cache slots with the same values)."""
    import numpy as np
    import torch

    from heliopause_amd import decode as DM
    from heliopause_amd import hip_kernels as H
    from heliopause_amd import synthetic as S

    m = args.m if args.m > 1 else 512
    torch.cuda.init()
    dev = torch.device("cuda:0")
    shape = DM.ModelShape()
    seed = S.config_seed(5)
    data = DM.layer_host_data(shape, seed, 0)
    model = DM.HipDecodeModel(shape)
    for _ in range(N_LAYERS):
        model.add_layer(data)
    model.output_norm = torch.from_numpy(
        (1.0 + 0.1 * S.normal(S.derive(seed, "output_norm"), shape.hidden)).astype(np.float32)).to(dev)
    x0 = torch.from_numpy(S.activations(S.derive(seed, "prefill-x"), m, shape.hidden).reshape(-1) * 4).to(dev)
    hidden, normed = torch.empty_like(x0), torch.empty_like(x0)
    p0 = shape.capacity - m
    pos = torch.tensor([p0], dtype=torch.int32, device=dev)

    def step(stream: int) -> None:
        hidden.copy_(x0)
        model.run_layers(hidden.data_ptr(), pos.data_ptr(), normed.data_ptr(), stream, tokens=m)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        launches0 = H.hipResidentWeightStats()["kernelLaunches"]
        step(side.cuda_stream)
        launches = H.hipResidentWeightStats()["kernelLaunches"] - launches0 + 1
        torch.cuda.synchronize()
        H.profile(True)
        step(side.cuda_stream)
        torch.cuda.synchronize()
        split = {}
        for kid, name in H.KERNEL_NAMES.items():
            t_ms, n = H.profile_read(kid)
            if n:
                split[name] = {"us": round(t_ms * 1e3, 1), "launches": n}
        H.profile(False)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            step(torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    warm = max(1, args.warmup // 40)
    for _ in range(warm):
        graph.replay()
    torch.cuda.synchronize()
    steps = max(1, args.steps // 80)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    for _ in range(steps):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) / steps * 1e3
    ms = start.elapsed_time(end) / steps
    weights = N_LAYERS * sum(r * k for _, r, k in LAYER)
    proj_flops = 2.0 * m * weights
    # attention: token t sees p0 + t + 1 keys; q.k and p.v, 256 dims, every query head
    visits = sum(min(p0 + t + 1, shape.capacity) for t in range(m))
    attn_flops = N_LAYERS * shape.head_count * visits * 256 * 2 * 2
    flops = proj_flops + attn_flops
    tflops = flops / (ms * 1e-3) / 1e12
    model.release()
    line = {
        "metric": f"prefill chunk ms at M={m}, all layers (1 GPU)",
        "value": round(ms, 4), "unit": "ms", "n_gpus": 1, "steps": steps, "warmup": warm,
        "ms_per_step": round(ms, 4), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "f16 MFMA (exact integers) + f32 tail; f16 attention MFMA", "data": "synthetic",
        "config": {"workload": f"42-layer synthetic Gemma-like model, a {m}-token prefill chunk at positions "
                               f"{p0}..{p0 + m - 1} of a 4096-slot f16 KV ring through every layer (norms, Q/K/V, "
                               "RoPE, cache append, causal attention, O, GeGLU FFN, residuals) and the output norm",
                   "columns": m, "projection_flops": proj_flops, "attention_flops": attn_flops,
                   "launches_per_step": launches, "wall_ms_per_step": round(wall_ms, 4), "kernel_split_us": split,
                   "timing": "one chunk captured in a HIP graph and replayed"},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tflops / MFMA_F16_PEAK_TFLOPS, 4), "traffic": None},
    }
    print(json.dumps(_label(line)))
    return 0


PCIE_PEAK_GBPS = 64.0  # PCIe 5.0 x16, one direction


def _model_tensors(host) -> list:
    names = ["attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down"]
    ggml = {"Q4_K": 12, "Q6_K": 14}
    out = []
    for layer in range(N_LAYERS):
        for name, (t, r, k) in zip(names, LAYER):
            out.append((f"blk.{layer}.{name}.weight", [k, r], ggml[t], host[(t, r, k)]))
    out.append(("output.weight", [HEAD[2], HEAD[1]], ggml[HEAD[0]], host[HEAD]))
    return out


def gguf_load(args) -> int:
    """Model load: a GGUF v3 file holding the 42-layer model's projections and
    head (3.02 GB of Q4_K/Q6_K blocks, 295 tensors) is parsed and every tensor
    streamed into an HBM-resident handle (file -> pinned chunks with parallel
    pread -> device staging -> repack into the resident layouts).  The file
    sits in the page cache (tmpfs), as on a warm restart; a step is one full
    load, and the handles are released between steps, untimed.  Also timed:
    the same tensors uploaded from bytes already in host memory (the
    one-tensor-at-a-time pageable path, hp_hip_weight_upload)."""
    import tempfile

    import torch

    from heliopause_amd import gguf as G
    from heliopause_amd import hip_kernels as H
    from heliopause_amd import synthetic as S

    support = H.checkHipSupport()
    if not support["available"]:
        raise SystemExit(f"HIP runner unavailable: {support}")
    torch.cuda.init()
    seed = S.config_seed(5)
    host = {}
    for i, (t, r, k) in enumerate(LAYER + [HEAD]):
        if (t, r, k) not in host:
            host[(t, r, k)] = S.weight_blocks(t, S.derive(seed, "decode42", i), r, k)
    tensors = _model_tensors(host)
    tmpdir = "/dev/shm" if os.path.isdir("/dev/shm") and os.access("/dev/shm", os.W_OK) else None
    fd, path = tempfile.mkstemp(suffix=".gguf", dir=tmpdir)
    os.close(fd)
    try:
        md = [("general.architecture", G.GGUF_STRING, "gemma4"), ("general.alignment", G.GGUF_UINT32, 32),
              ("gemma4.block_count", G.GGUF_UINT32, N_LAYERS)]
        G.write_gguf(path, md, tensors)
        tensor_bytes = sum(x.size for _, _, _, x in tensors)
        file_bytes = os.path.getsize(path)

        def load_once() -> float:
            with G.GgufFile(path) as f:
                w = G.GgufHipWeights(f)
                t0 = time.perf_counter()
                hs = w.upload_all()
                el = time.perf_counter() - t0
                assert all(h is not None for h in hs.values())
                w.release()
            return el

        for _ in range(max(1, args.warmup // 40)):
            load_once()
        steps = max(1, args.steps // 100)
        times = [load_once() for _ in range(steps)]
        sec = sum(times) / len(times)
        # the same tensors from bytes already in host memory, one call per tensor
        t0 = time.perf_counter()
        hs = [H.createHipQuantizedWeightHandle({12: "Q4_K", 14: "Q6_K"}[t], x, d[0], d[1]) for _, d, t, x in tensors]
        mem_sec = time.perf_counter() - t0
        for h in hs:
            H.releaseHipQuantizedWeightHandle(h)
        cpu = None if args.no_cpu else gguf_cpu_baseline(path, args.cpu_seconds)
    finally:
        os.unlink(path)
    gbps = tensor_bytes / sec / 1e9
    line = {
        "metric": "GGUF model load GB/s into HBM-resident handles (1 GPU)",
        "value": round(gbps, 3), "unit": "GB/s", "n_gpus": 1, "steps": steps, "warmup": max(1, args.warmup // 40),
        "ms_per_step": round(sec * 1e3, 3), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "u8", "data": "synthetic",
        "config": {"workload": "GGUF v3 file of the 42-layer synthetic Gemma-like model (295 Q4_K/Q6_K tensors) "
                               "in the page cache -> parse -> stream -> repack into resident handles",
                   "tensor_bytes": tensor_bytes, "file_bytes": file_bytes, "tensors": len(tensors),
                   "file_location": "tmpfs" if tmpdir else "default temp dir",
                   "host_bytes_upload_gbps": round(tensor_bytes / mem_sec / 1e9, 3),
                   "load_seconds": [round(t, 4) for t in times]},
        "roofline": {"bound": "pcie", "achieved": round(gbps, 3), "peak": PCIE_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(gbps / PCIE_PEAK_GBPS, 4), "traffic": None},
    }
    if cpu:
        line["cpu_baseline"] = cpu
    print(json.dumps(_label(line)))
    return 0


def gguf_cpu_baseline(path: str, seconds: float) -> dict:
    """The engine's own load path on the CPU, as far as it reaches before the
    WASM upload: parseGguf (the oracle's restatement) and readTensorBytes of
    every tensor into host memory, one thread."""
    import numpy as np

    from oracle import gguf as OG

    t0 = time.perf_counter()
    with open(path, "rb") as f:
        head = f.read(1 << 20)
    meta = OG.parse_gguf(head)
    done = 0
    with open(path, "rb") as f:
        for t in meta["tensors"]:
            n = OG.tensor_byte_length(t)
            f.seek(t["dataOffset"])
            buf = np.empty(n, dtype=np.uint8)
            f.readinto(memoryview(buf))
            done += n
            if time.perf_counter() - t0 > seconds:
                break
    el = time.perf_counter() - t0
    return {"value": round(done / el / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"parse + read of {done / 1e9:.2f} GB of tensor bytes into host memory in {el:.2f} s "
                      "(the engine's path up to the WASM upload; no scale preparation)"}


WEIGHT_LAYOUTS = "both"


def _label(line: dict) -> dict:
    """Names the resident-layout mode in a line measured with one layout."""
    if WEIGHT_LAYOUTS != "both" and isinstance(line.get("config"), dict):
        line["config"]["weight_layouts"] = WEIGHT_LAYOUTS
    return line


def main() -> int:
    global WEIGHT_LAYOUTS
    args = parse()
    WEIGHT_LAYOUTS = args.weight_layouts
    if args.copy_probe:
        return copy_probe()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1", "n_gpus": args.gpus}))
        return 2
    if args.weight_layouts == "one":
        from heliopause_amd import hip_kernels as H

        H.setWeightLayouts(False)
    if args.workload == "decode42":
        return decode_step(args)
    if args.workload == "decode42-proj":
        return decode_chain(args)
    if args.workload == "gguf-load":
        return gguf_load(args)
    if args.workload == "prefill42":
        return prefill_chain(args)
    if args.workload == "prefill42-layers":
        return prefill_layers(args)
    from heliopause_amd import hip_kernels as H

    support = H.checkHipSupport()
    if not support["available"]:
        raise SystemExit(f"HIP runner unavailable: {support}")
    H.setMatvecKernel(KERNEL_CHOICES[args.kernel](H))
    wl, m = args.workload, args.m
    r = measure_matvec(wl, m, args.kernel, max(1, args.steps), max(0, args.warmup), args.rotate_mib)

    extra = {}
    if wl == "qkv" and m == 1 and not args.no_decode:
        # the other matvec configurations with a budget of their own, timed
        # the same way in the same run: config 1 and the head with top-40
        for name in ("cfg1", "head"):
            e = measure_matvec(name, 1, args.kernel, 20 if name == "cfg1" else 10, 5, args.rotate_mib)
            extra[name] = matvec_summary(e)
        extra["decode_step"] = decode_summary(measure_decode_step(1, 20, 3, None))

    traffic = None
    tfile = ROOT / "profiles" / f"{wl}_m{m}_traffic.json"
    if tfile.exists():
        try:
            traffic = json.loads(tfile.read_text()).get("hbm_bytes_per_launch")
        except (ValueError, OSError):
            traffic = None

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(wl, r["ws"], r["x_host"], args.cpu_seconds)

    K = r["steps"]
    line = {
        "metric": METRIC,
        "value": round(r["value"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": round(r["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {
            "workload": r["desc"],
            "M": m,
            "weight_bytes": weight_bytes(wl),
            "algorithmic_bytes_per_step": r["step_bytes"],
            "weight_copies_rotated": r["copies"],
            "parallelism": "single GPU",
            "timing": f"exactly {K} steps (step i on weight copy i % {r['copies']}) captured in one HIP graph and "
                      f"replayed once, after a warm-up graph of {r['warm_count']} steps over the other copies",
            "eager_host_launch_ms_per_step": round(r["eager_ms"], 5),
            "graph_launch": graph_launch_summary(r),
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(r["achieved"], 2),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(r["achieved"] / HBM_PEAK_GBPS, 4),
            "traffic": traffic,
            "traffic_source": (f"profiles/{tfile.name}: rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE of this launch "
                               "in an earlier run, scaled by a plain copy kernel's counters; not measured by "
                               "this run") if traffic is not None else None,
            "kernel": r["kernel"],
            "kernel_avg_us": round(r["kern_us"], 3),
            "kernel_avg_us_mall_hot": round(r["hot_us"], 3),
        },
        "cpu_baseline": cpu,
    }
    line.update(extra)
    print(json.dumps(_label(line)))
    return 0


KERNEL_CHOICES = {"auto": lambda H: H.MATVEC_AUTO, "valu": lambda H: H.MATVEC_VALU, "mfma": lambda H: H.MATVEC_MFMA,
                  "half": lambda H: H.MATVEC_HALF, "wide": lambda H: H.MATVEC_WIDE,
                  "wide-whole": lambda H: H.MATVEC_WIDE_WHOLE, "wide-half": lambda H: H.MATVEC_WIDE_HALF}

# per-call budgets at 8 TB/s (weights plus activations)
BUDGET_US = {"cfg1": 2.642}


def measure_matvec(wl: str, m: int, kernel: str, K: int, W: int, rotate_mib: int) -> dict:
    """K steps of workload wl at M = m, each on its own weight copy, in one
    HIP graph after a warm-up graph over the other copies (so the timed
    steps start with cold weights); HIP events on the launch stream bracket
    the timed replay.  Also: eager host-submitted launches, the same K steps
    on one copy (Infinity-Cache hot), and an empty graph of as many kernel
    nodes as the timed one (what the graph launch itself costs)."""
    import numpy as np
    import torch

    from heliopause_amd import hip_kernels as H
    from heliopause_amd import synthetic as S

    torch.cuda.init()
    dev = torch.device("cuda:0")
    cfg, k, specs, desc = WORKLOADS[wl]
    seed = S.config_seed(cfg)
    ws = [S.weight_blocks(t, S.derive(seed, wl, i), r, k) for i, (t, r) in enumerate(specs)]
    w_down = S.weight_blocks(FFN_DOWN[0], S.derive(seed, wl, "down"), FFN_DOWN[1], FFN_DOWN[2]) if wl == "ffn" else None
    x_host = S.activations(S.derive(seed, wl), m, k)

    # distinct copies: >= rotate_mib in all, and enough that the steps just
    # before the timed ones (the warm-up graph) cover >= 320 MiB of other
    # copies, more than the 256 MB Infinity Cache holds
    wb = weight_bytes(wl)
    copies = max(1, math.ceil(rotate_mib * 2**20 / wb))
    if rotate_mib >= 320:
        copies = max(copies, min(K, 4096) + math.ceil(320 * 2**20 / wb))
    handles, down_handles = [], []
    for _ in range(copies):
        handles.append([H.createHipQuantizedWeightHandle(t, w, k, r).handle for (t, r), w in zip(specs, ws)])
        if wl == "ffn":
            down_handles.append(H.createHipQuantizedWeightHandle(FFN_DOWN[0], w_down, FFN_DOWN[2],
                                                                 FFN_DOWN[1]).handle)
    x = torch.from_numpy(x_host).to(dev)
    outs = [torch.empty(m * r, dtype=torch.float32, device=dev) for _, r in specs]
    out_ptrs = [o.data_ptr() for o in outs]
    out_lens = [o.numel() for o in outs]
    h_ffn = torch.empty(m * 10240, dtype=torch.float32, device=dev)
    y_ffn = torch.empty(m * 2560, dtype=torch.float32, device=dev)
    ids = torch.empty(m * TOPK, dtype=torch.int32, device=dev)
    vals = torch.empty(m * TOPK, dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream().cuda_stream
    L = H.lib()

    def step(i: int) -> None:
        if wl == "ffn":  # gate/up + GeGLU (one launch for one column), then down
            H.matmul_geglu_device(handles[i % copies][0], handles[i % copies][1], x.data_ptr(), k, m,
                                  h_ffn.data_ptr(), 10240, stream)
        else:
            H.matmul_multi_device(handles[i % copies], x.data_ptr(), k, m, out_ptrs, out_lens, stream)
        if wl == "ffn":
            H.matmul_multi_device([down_handles[i % copies]], h_ffn.data_ptr(), 10240, m, [y_ffn.data_ptr()],
                                  [m * 2560], stream)
        elif wl == "head":
            H.assertHipOk(L.hp_hip_topk_device(out_ptrs[0], m, 262144, TOPK, 0.0, ids.data_ptr(), vals.data_ptr(),
                                               stream), "topk")

    try:
        # correctness guard on the benchmarked path (first copy vs the host API)
        if wl != "ffn":
            step(0)
            torch.cuda.synchronize()
            host = [H.matMulQuantizedHipResident(H.HipQuantizedWeightHandle(h, t, 0, r, k), x_host, k, r, m)
                    for h, (t, r) in zip(handles[0], specs)]
            for a, b in zip(outs, host):
                if not np.array_equal(a.cpu().numpy().view(np.uint32), b.view(np.uint32)):
                    raise SystemExit("device-pointer path disagrees with the host path")

        step_bytes = algorithmic_bytes(wl, m)
        # eager: host-submitted launches (bounded by the host submission rate)
        for i in range(min(W, 8)):
            step(K + i)
        torch.cuda.synchronize()
        n_eager = min(K, 100)
        launches0 = H.hipResidentWeightStats()["kernelLaunches"]
        t0 = time.perf_counter()
        for i in range(n_eager):
            step(K + i)
        torch.cuda.synchronize()
        eager_ms = (time.perf_counter() - t0) / n_eager * 1e3
        nodes_per_step = (H.hipResidentWeightStats()["kernelLaunches"] - launches0) / n_eager

        # Graphs on one side stream (warmed by an uncaptured step first): the
        # timed graph holds exactly K steps, step i on copy i % copies; the
        # warm-up graph holds the W warm-up steps and at least every copy the
        # timed graph does not touch first, so the timed steps start with cold
        # weights.
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())

        def capture(first: int, count: int, same_copy: bool = False):
            nonlocal stream
            g = torch.cuda.CUDAGraph()
            with torch.cuda.stream(side):
                with torch.cuda.graph(g, stream=side):
                    stream = torch.cuda.current_stream().cuda_stream
                    for i in range(count):
                        step(0 if same_copy else first + i)
            return g

        with torch.cuda.stream(side):
            stream = side.cuda_stream
            step(0)
        torch.cuda.synchronize()
        warm_count = max(W, copies - K if K < copies else 0, 1)
        g_warm = capture(K, warm_count)
        g_timed = capture(0, K)
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(side):
            g_warm.replay()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            start.record()
            g_timed.replay()
            end.record()
            torch.cuda.synchronize()
            wall = time.perf_counter() - t0
        ms_per_step = wall / K * 1e3
        # HIP events bracketing the timed region on the launch stream: average
        # device time per step (for one-kernel steps, the launch duration)
        kern_us = start.elapsed_time(end) / K * 1e3

        # Infinity-Cache-hot reference: K steps on one resident copy
        hot = capture(0, K, same_copy=True)
        with torch.cuda.stream(side):
            hot.replay()
            torch.cuda.synchronize()
            start.record()
            hot.replay()
            end.record()
            torch.cuda.synchronize()
        hot_us = start.elapsed_time(end) / K * 1e3

        # an empty graph of as many kernel nodes, bracketed the same way
        nodes = max(1, round(nodes_per_step * K))
        g_empty = torch.cuda.CUDAGraph()
        with torch.cuda.stream(side):
            with torch.cuda.graph(g_empty, stream=side):
                H.emptyLaunches(nodes, torch.cuda.current_stream().cuda_stream)
            g_empty.replay()
            torch.cuda.synchronize()
            start.record()
            g_empty.replay()
            end.record()
            torch.cuda.synchronize()
        empty_us = start.elapsed_time(end) * 1e3
    finally:
        for hs in handles:
            for h in hs:
                L.hp_hip_weight_release(h)
        for h in down_handles:
            L.hp_hip_weight_release(h)
        handles.clear()
        down_handles.clear()
    kernels = {"ffn": "gate/up+GeGLU matvec + down matvec", "head": "matvec + top-k"}
    return {"wl": wl, "m": m, "desc": desc, "ws": ws, "x_host": x_host, "copies": copies, "warm_count": warm_count,
            "steps": K, "step_bytes": step_bytes, "ms_per_step": ms_per_step,
            "value": step_bytes / (ms_per_step * 1e-3) / 1e9, "kern_us": kern_us,
            "achieved": step_bytes / (kern_us * 1e-6) / 1e9, "hot_us": hot_us, "eager_ms": eager_ms,
            "kernel": kernels.get(wl, matvec_kernel_name(kernel, k, m, specs)),
            "nodes_per_step": nodes_per_step, "empty_graph_us": empty_us}


def graph_launch_summary(r: dict) -> dict:
    """What launching the graph costs inside the timed bracket: an empty graph
    of as many kernel nodes, timed with the same events."""
    timed_us = r["kern_us"] * r["steps"]
    return {"kernel_nodes": round(r["nodes_per_step"] * r["steps"]),
            "empty_graph_us": round(r["empty_graph_us"], 2),
            "timed_bracket_us": round(timed_us, 2),
            "share": round(r["empty_graph_us"] / timed_us, 4)}


def matvec_summary(r: dict) -> dict:
    """A matvec configuration's object of the JSON line (HIP-event timing)."""
    o = {"workload": r["desc"], "M": r["m"], "steps": r["steps"], "weight_copies_rotated": r["copies"],
         "algorithmic_bytes_per_step": r["step_bytes"], "kernel": r["kernel"],
         "us_per_step": round(r["kern_us"], 3), "us_per_step_wall": round(r["ms_per_step"] * 1e3, 3),
         "us_per_step_mall_hot": round(r["hot_us"], 3),
         "GB/s": round(r["achieved"], 2), "frac": round(r["achieved"] / HBM_PEAK_GBPS, 4),
         "graph_launch": graph_launch_summary(r)}
    if r["wl"] in BUDGET_US:
        o["budget_us"] = BUDGET_US[r["wl"]]
    return o


if __name__ == "__main__":
    sys.exit(main())
