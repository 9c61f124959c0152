"""Stage timeline of the persistent one-token decode step.

    python -m heliopause_amd.fused_timeline [--layers 42] [--reps 3]

Builds the synthetic 42-layer Gemma-like model (hidden 2560, 8/2 heads of
256, FFN 10240, Q4_K with Q6_K for V and down, a 4096-slot f16 ring at its
wrap position), times one step as the launch sequence and as the persistent
launch (both replayed from HIP graphs), then turns on the step's stage
trace (hp_hip_set_fused_trace) and prints, per stage, the median over
workgroups and layers 2.. of the time between the trace points:

    k1 loads issued, k2 input arrived, k3 prologue done, k4 weights in
    registers, k5 products done, k6 chains done, k7 end,

with "crit" the stage's span on the critical path (the last workgroup's
end of the previous stage to the last workgroup's end of this one).  All
times in microseconds from the 100 MHz s_memrealtime clock.
"""
from __future__ import annotations

import argparse

import numpy as np

from . import decode as DM
from . import hip_kernels as H
from . import synthetic as S

STAGES = ("Q/K/V", "attention", "merge", "O", "gate/up", "down")


def _graph_ms(model, hid, pos, out, steps=20):
    import torch

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        model.run_layers(hid.data_ptr(), pos.data_ptr(), out.data_ptr(), side.cuda_stream)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=side):
            model.run_layers(hid.data_ptr(), pos.data_ptr(), out.data_ptr(), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    if H.decodeFusedStatus(side.cuda_stream) != 0:
        raise RuntimeError("a persistent step stopped at a wait")
    return e0.elapsed_time(e1) / steps


def main(argv=None) -> None:
    import torch

    ap = argparse.ArgumentParser()
    ap.add_argument("--layers", type=int, default=42)
    ap.add_argument("--reps", type=int, default=3)
    args = ap.parse_args(argv)
    dev = torch.device("cuda:0")
    shape = DM.ModelShape()
    nl = args.layers
    seed = S.derive(S.config_seed(5), "fused-timeline")
    datas = [DM.layer_host_data(shape, seed, i) for i in range(min(3, nl))]
    model = DM.HipDecodeModel(shape)
    shared = [None] * len(datas)
    for i in range(nl):
        j = i % len(datas)
        model.add_layer(datas[j], shared_weights=shared[j])
        if shared[j] is None:
            shared[j] = {n: h for n, h in zip(DM.PROJ_NAMES, model.handles[-len(DM.PROJ_NAMES):])}
    model.output_norm = torch.from_numpy((1.0 + 0.1 * S.normal(S.derive(seed, "on"), shape.hidden))
                                         .astype(np.float32)).to(dev)
    x = torch.from_numpy((S.activations(S.derive(seed, "x"), 1, shape.hidden).reshape(-1) * 4)
                         .astype(np.float32)).to(dev)
    pos = torch.tensor([shape.capacity], dtype=torch.int32, device=dev)
    hid, out = x.clone(), torch.empty_like(x)
    try:
        for fused in (False, True):
            H.setDecodeFused(fused)
            ms = _graph_ms(model, hid, pos, out)
            print(f"{'persistent launch' if fused else 'launch sequence'}: {ms:.3f} ms per step "
                  f"({nl} layers + output norm, graph replay)", flush=True)
        H.setDecodeFused(True)
        W = H.hipResidentWeightStats()["computeUnits"]
        K = 8
        tr = torch.zeros(W * nl * 6 * K, dtype=torch.int64, device=dev)
        per_layer, rows = [], []
        for rep in range(args.reps):
            tr.zero_()
            H.setFusedTrace(tr.data_ptr(), tr.numel())
            hid.copy_(x)
            model.run_layers(hid.data_ptr(), pos.data_ptr(), out.data_ptr())
            torch.cuda.synchronize()
            H.setFusedTrace(0, 0)
            if H.decodeFusedStatus() != 0:
                raise RuntimeError("a traced step stopped at a wait")
            t = tr.cpu().numpy().reshape(W, nl, 6, K).astype(np.float64)
            t0 = t[t > 0].min()
            t = np.where(t > 0, (t - t0) * 0.01, np.nan)
            per_layer.append(np.nanmax(t) / nl)
            end_all = np.nanmax(t[:, :, :, 7], axis=0)
            prev_end = np.concatenate([[0.0], end_all.reshape(-1)[:-1]]).reshape(nl, 6)
            keep = slice(min(2, nl - 1), nl)
            rep_rows = []
            for s in range(6):
                crit = float(np.median((end_all[:, s] - prev_end[:, s])[keep]))
                deltas = []
                for k in range(1, 8):
                    d = t[:, keep, s, k] - t[:, keep, s, k - 1]
                    deltas.append(float(np.nanmedian(d)) if np.any(~np.isnan(d)) else None)
                arrive = float(np.nanmedian(t[:, keep, s, 2] - prev_end[keep, s][None, :]))
                rep_rows.append((crit, deltas, arrive))
            rows.append(rep_rows)
        print(f"traced steps: {', '.join(f'{v:.2f}' for v in per_layer)} us per layer", flush=True)
        print("| stage | crit | k1 issue | k2 input | k3 prologue | k4 regs | k5 products | k6 chains | k7 tails "
              "| input - prev end |")
        print("|---|---|---|---|---|---|---|---|---|---|")
        for s in range(6):
            crit = np.median([r[s][0] for r in rows])
            deltas = []
            for k in range(7):
                v = [r[s][1][k] for r in rows if r[s][1][k] is not None]
                deltas.append(f"{np.median(v):.2f}" if v else "-")
            arrive = np.median([r[s][2] for r in rows])
            print(f"| {STAGES[s]} | {crit:.2f} | " + " | ".join(deltas) + f" | {arrive:.2f} |")
    finally:
        H.setFusedTrace(0, 0)
        H.setDecodeFused(False)
        model.release()


if __name__ == "__main__":
    main()
