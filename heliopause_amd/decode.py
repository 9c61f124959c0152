"""Decode-step runner on the GPU: resident decoder layers and their KV rings.

Host side of forwardAttentionLayer / forwardFfn / forwardOutput
(packages/engine/src/runner/wasm/layers.ts:161-473, 381-416) for one decode
token.  A ``HipDecodeModel`` owns, per layer, the weight handles, the f32
norm weights and the f16 KV ring in HBM, and runs

    hp_hip_decode_layers_device  (every layer, then output_norm)
    hp_hip_matmul_multi_device   (output head -> logits)
    hp_hip_topk_device / hp_hip_sample_device

on one stream, so a whole step can be captured in one HIP graph; the
position lives in device memory and is read when the kernels run.

``layer_host_data`` makes one layer of the synthetic Gemma-like model with
the documented block distributions (Q4_K for Q, K, O, gate, up; Q6_K for V
and down), norm weights 1 + 0.1 N(0,1) and an N(0,1) f16 KV cache.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional

import numpy as np

from . import hip_kernels as H
from . import synthetic as S

NORM_NAMES = ("attn_norm", "attn_q_norm", "attn_k_norm", "post_attention_norm", "ffn_norm", "post_ffw_norm")
PROJ_NAMES = ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down")


@dataclass
class ModelShape:
    """Attention/FFN sizes of the Gemma-like decoder."""
    hidden: int = 2560
    head_count: int = 8
    head_count_kv: int = 2
    ffn: int = 10240
    vocab: int = 262144
    capacity: int = 4096
    rope_dims: int = 256
    rope_freq_base: float = 10000.0
    sliding_window: int = 0
    epsilon: float = 1e-6

    def projections(self):
        """(name, type, rows, input size) of one layer's projections."""
        q, kv = self.head_count * 256, self.head_count_kv * 256
        return [("attn_q", "Q4_K", q, self.hidden), ("attn_k", "Q4_K", kv, self.hidden),
                ("attn_v", "Q6_K", kv, self.hidden), ("attn_output", "Q4_K", self.hidden, q),
                ("ffn_gate", "Q4_K", self.ffn, self.hidden), ("ffn_up", "Q4_K", self.ffn, self.hidden),
                ("ffn_down", "Q6_K", self.hidden, self.ffn)]


def layer_host_data(shape: ModelShape, seed: int, layer: int, *, cache_fill: bool = True,
                    per_layer_length: int = 0) -> dict:
    """Deterministic synthetic data of one layer (host arrays); with
    per_layer_length > 0 also the per-layer input step's weights (inp_gate
    Q4_K [P][hidden], proj Q4_K [hidden][P], post_norm)."""
    ls = S.derive(seed, "layer", layer)
    data = {"weights": {}, "norms": {}}
    for name, t, rows, k in shape.projections():
        data["weights"][name] = (t, S.weight_blocks(t, S.derive(ls, name), rows, k), rows, k)
    for name in NORM_NAMES:
        n = 256 if name in ("attn_q_norm", "attn_k_norm") else shape.hidden
        data["norms"][name] = (1.0 + 0.1 * S.normal(S.derive(ls, name), n)).astype(np.float32)
    data["output_scale"] = np.float32(1.0 + 0.05 * S.normal(S.derive(ls, "scale"), 1)[0])
    if per_layer_length:
        P = per_layer_length
        # inp_gate as Q6_K (symmetric scales: zero-mean weights, so the
        # residual stream's offset does not push every gate below gelu's -10
        # cut) with d scaled by 2^-6 (exact in f16): gate values of a few
        # units, inside gelu's active range
        gate = S.weight_blocks("Q6_K", S.derive(ls, "inp_gate"), P, shape.hidden)
        g = gate.reshape(-1, 210)
        d = g[:, 208:210].copy().view(np.float16) * np.float16(2.0 ** -6)
        g[:, 208:210] = d.view(np.uint8).reshape(-1, 2)
        data["per_layer"] = {
            "inp_gate": ("Q6_K", gate, P, shape.hidden),
            "proj": ("Q4_K", S.weight_blocks("Q4_K", S.derive(ls, "proj"), shape.hidden, P), shape.hidden, P),
            "post_norm": (1.0 + 0.1 * S.normal(S.derive(ls, "post_norm"), shape.hidden)).astype(np.float32),
        }
    cshape = (shape.head_count_kv, shape.capacity, 256)
    n = int(np.prod(cshape))
    if cache_fill:
        data["key_cache"] = S.normal(S.derive(ls, "kcache"), n).astype(np.float16).reshape(cshape)
        data["value_cache"] = S.normal(S.derive(ls, "vcache"), n).astype(np.float16).reshape(cshape)
    else:
        data["key_cache"] = np.zeros(cshape, np.float16)
        data["value_cache"] = np.zeros(cshape, np.float16)
    return data


@dataclass
class HipDecodeModel:
    """Resident decoder layers (+ optional output norm and head) on cuda:0."""
    shape: ModelShape
    layers: list = field(default_factory=list)       # HipDecodeLayer structs
    handles: list = field(default_factory=list)      # HipQuantizedWeightHandle
    tensors: list = field(default_factory=list)      # device tensors kept alive
    caches: list = field(default_factory=list)       # (key, value) device tensors per layer
    output_norm: Optional[object] = None
    head: Optional[H.HipQuantizedWeightHandle] = None

    def add_layer(self, data: dict, shared_weights: Optional[dict] = None) -> None:
        """Uploads one layer (``shared_weights``: name -> handle to reuse)."""
        import torch

        dev = torch.device("cuda:0")
        hs = {}
        for name in PROJ_NAMES:
            if shared_weights and name in shared_weights:
                hs[name] = shared_weights[name]
                continue
            t, blocks, rows, k = data["weights"][name]
            h = H.createHipQuantizedWeightHandle(t, blocks, k, rows)
            self.handles.append(h)
            hs[name] = h
        norms = {n: torch.from_numpy(data["norms"][n]).to(dev) for n in NORM_NAMES}
        kc = torch.from_numpy(data["key_cache"].view(np.int16)).to(dev)
        vc = torch.from_numpy(data["value_cache"].view(np.int16)).to(dev)
        self.tensors.extend(norms.values())
        self.caches.append((kc, vc))
        sh = self.shape
        cfg = H.attention_config(sh.head_count, sh.head_count_kv, sh.capacity, rope_dims=sh.rope_dims,
                                 rope_freq_base=sh.rope_freq_base, sliding_window=sh.sliding_window,
                                 epsilon=sh.epsilon)
        L = H.HipDecodeLayer()
        for name in PROJ_NAMES:
            setattr(L, name, hs[name].handle)
        for n in NORM_NAMES:
            setattr(L, "d_" + n, norms[n].data_ptr())
        L.layer_output_scale = float(data["output_scale"])
        L.reserved = 0
        L.d_key_cache, L.d_value_cache = kc.data_ptr(), vc.data_ptr()
        L.attention = cfg
        if "per_layer" in data:
            # applyPerLayerInput: inp_gate / proj handles and post_norm; the
            # layer's per-layer input rows are set per call (set_per_layer_input)
            ple = data["per_layer"]
            for name in ("inp_gate", "proj"):
                t, blocks, rows, k = ple[name]
                h = H.createHipQuantizedWeightHandle(t, blocks, k, rows)
                self.handles.append(h)
                setattr(L, name, h.handle)
            pn = torch.from_numpy(ple["post_norm"]).to(dev)
            self.tensors.append(pn)
            L.d_post_norm = pn.data_ptr()
        self.layers.append(L)

    def set_per_layer_input(self, index: int, d_rows: int) -> None:
        """Layer `index`'s rows of the per-layer inputs ([tokens][P] f32 on
        the device) for the next run_layers call."""
        self.layers[index].d_per_layer_input = d_rows

    def set_head(self, output_norm: np.ndarray, head: H.HipQuantizedWeightHandle) -> None:
        import torch

        self.output_norm = torch.from_numpy(np.asarray(output_norm, np.float32)).to(torch.device("cuda:0"))
        self.head = head

    def layers_array(self):
        """The layer structs as one C array (read by the call, not kept)."""
        return (H.HipDecodeLayer * len(self.layers))(*self.layers)

    def run_layers(self, d_hidden: int, d_position: int, d_normed: int = 0, stream: int = 0,
                   tokens: int = 1) -> None:
        """Every layer on d_hidden ([tokens][hidden], in place) for the tokens
        at *d_position + t; the output norm into d_normed."""
        arr = self.layers_array()
        onorm = self.output_norm.data_ptr() if (d_normed and self.output_norm is not None) else 0
        H.assertHipOk(H.lib().hp_hip_decode_layers_device(arr, len(self.layers), tokens, d_hidden, d_position,
                                                          onorm or None, d_normed if onorm else None,
                                                          stream or None), "decode_layers")

    def release(self) -> None:
        for h in self.handles:
            H.releaseHipQuantizedWeightHandle(h)
        self.handles.clear()
        self.layers.clear()
        self.tensors.clear()
        self.caches.clear()
