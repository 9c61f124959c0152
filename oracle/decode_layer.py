"""CPU restatement of one decoder layer for the tokens of one decode call
(one token, or a draft of up to eight being verified).

TEST INFRASTRUCTURE ONLY: this module is the checker.  Only tests/,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may
import it; the HIP product path never does.

Follows forwardAttentionLayer (packages/engine/src/runner/wasm/layers.ts:
161-379) and forwardFfn (418-473) with causal attention, keeping every
token's row:
the element-wise steps are the C restatements in hp_oracle.c
(hpo_rms_norm_vector, hpo_rope_neox, hpo_gqa_attention_f32,
hpo_cast_f16_rows, hpo_residual_add) and the projections the oracle's
restatement of the WASM matmul (lib.rs:224-426).

KV cache: the GPU path keeps f16 entries ``[kv_heads][capacity][256]``; the
reference's WASM runner keeps f32 entries (runtime.ts FullAttentionCache) and
the WebGPU runner f16 ones.  Here the cache is an f16 array in the GPU
layout, entries rounded to nearest even when appended, and attention reads
it widened to f32 in the layouts hp_gqa_attention_f32 takes (key
token-major, value "dim-head-token"): lib.rs's attention over an f32 cache
whose entries are f16 values.
"""
from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass, field

import numpy as np

from . import oracle as O

HEAD_DIM = 256
_f32p = ctypes.POINTER(ctypes.c_float)
_i32p = ctypes.POINTER(ctypes.c_int32)
_sz = ctypes.c_size_t
_declared = False


def _lib():
    global _declared
    L = O.lib()
    if not _declared:
        L.hpo_rms_norm_vector.argtypes = [_f32p, _sz, _f32p, ctypes.c_double, _f32p]
        L.hpo_rms_norm_vector.restype = None
        L.hpo_residual_add.argtypes = [_f32p, _f32p, _sz, _f32p]
        L.hpo_residual_add.restype = None
        L.hpo_cast_f16_rows.argtypes = [_f32p, _sz, _f32p]
        L.hpo_cast_f16_rows.restype = None
        L.hpo_rope_neox.argtypes = [_f32p, _sz, _sz, _sz, _i32p, _sz, ctypes.c_double, _f32p, _f32p]
        L.hpo_rope_neox.restype = ctypes.c_int32
        L.hpo_gqa_attention_f32.argtypes = [_f32p, _sz, _f32p, _sz, _f32p, _sz, _f32p, _sz, _sz, _sz, _sz, _sz, _sz,
                                            _sz, _sz, ctypes.c_float, ctypes.c_int32, ctypes.c_int32, _f32p, _sz]
        L.hpo_gqa_attention_f32.restype = ctypes.c_int32
        _declared = True
    return L


def _f(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _p(a, t=_f32p):
    return a.ctypes.data_as(t) if a is not None else None


def rms_norm_rows(x, w, eps: float) -> np.ndarray:
    """rmsNormRows over rows of len(w) (w None: rmsNormRowsNoWeight of rows of n)."""
    x = _f(x)
    n = x.shape[-1]
    rows = x.reshape(-1, n)
    out = np.empty_like(rows)
    wf = _f(w) if w is not None else None
    for r in range(rows.shape[0]):
        _lib().hpo_rms_norm_vector(_p(rows[r]), n, _p(wf), eps, _p(out[r]))
    return out.reshape(x.shape)


def residual_add(a, b) -> np.ndarray:
    a, b = _f(a), _f(b)
    out = np.empty_like(a)
    _lib().hpo_residual_add(_p(a), _p(b), a.size, _p(out))
    return out


def cast_f16_rows(x) -> np.ndarray:
    x = _f(x)
    out = np.empty_like(x)
    _lib().hpo_cast_f16_rows(_p(x), x.size, _p(out))
    return out


def rope_neox(x, positions, n_dims: int, freq_base: float, freq_factors=None) -> np.ndarray:
    """x [tokens][heads][head_size] (or [heads][head_size] for one token)."""
    x = _f(x)
    one = x.ndim == 2
    xx = x[None] if one else x
    tokens, heads, hs = xx.shape
    pos = np.ascontiguousarray(np.atleast_1d(positions), dtype=np.int32)
    ff = _f(freq_factors) if freq_factors is not None else None
    out = np.empty_like(xx)
    rc = _lib().hpo_rope_neox(_p(xx), hs, heads, tokens, _p(pos, _i32p), n_dims, freq_base, _p(ff), _p(out))
    if rc != O.OK:
        raise ValueError(f"rope status {rc}")
    return out[0] if one else out


def attention_range(position: int, capacity: int, window: int = 0, context_length: int | None = None):
    """attentionRange (layers.ts:972-980) -> (start, count)."""
    ctx = context_length if context_length is not None else 1 << 30
    available = min(ctx, position + 1)
    count = min(capacity, window if window > 0 else capacity, available)
    return max(0, position + 1 - count), count


def gqa_attention_f32(query, key, value, *, head_size, query_heads, kv_heads, token_count, kv_count, kv_start,
                      capacity, scale=1.0, value_layout=1, quantize_query_f16=1, mask=None):
    """hp_gqa_attention_f32 (lib.rs:538-654) on f32 arrays in its layouts;
    returns (status, output)."""
    q, k, v = _f(query).reshape(-1), _f(key).reshape(-1), _f(value).reshape(-1)
    m = _f(mask).reshape(-1) if mask is not None else None
    out = np.zeros(token_count * query_heads * head_size, np.float32)
    rc = _lib().hpo_gqa_attention_f32(_p(q), q.size, _p(k), k.size, _p(v), v.size, _p(m), 0 if m is None else m.size,
                                      head_size, query_heads, kv_heads, token_count, kv_count, kv_start, capacity,
                                      scale, value_layout, quantize_query_f16, _p(out), out.size)
    return rc, out


def decode_attention(q, key_cache, value_cache, position: int, window: int = 0) -> np.ndarray:
    """Attention of tokens at position .. position + T - 1 (q [T][nq][256], or
    [nq][256] for one token, after RoPE) over f16 caches [nkv][capacity][256]
    that already hold every token, as forwardAttentionLayer runs it
    (layers.ts:270-335): one window, attentionRange of the largest position;
    causalMask per token; scale 1; f16 query; then castF16Rows."""
    q = _f(q)
    one = q.ndim == 2
    qq = q[None] if one else q
    tokens, nq, _ = qq.shape
    nkv, cap, hd = key_cache.shape
    start, count = attention_range(position + tokens - 1, cap, window)
    key = np.ascontiguousarray(key_cache.astype(np.float32).transpose(1, 0, 2))      # [slot][head][dim]
    value = np.ascontiguousarray(value_cache.astype(np.float32).transpose(2, 0, 1))  # [dim][head][slot]
    # causalMask (layers.ts:913-925): key position start + j <= the token's position
    kpos = start + np.arange(count)
    mask = np.stack([np.where(kpos <= position + t, 0.0, -np.inf) for t in range(tokens)]).astype(np.float32)
    rc, out = gqa_attention_f32(qq, key, value, head_size=hd, query_heads=nq, kv_heads=nkv, token_count=tokens,
                                kv_count=count, kv_start=start, capacity=cap, mask=mask)
    if rc != O.OK:
        raise ValueError(f"attention status {rc}")
    out = cast_f16_rows(out).reshape(tokens, nq, hd)
    return out[0] if one else out


@dataclass
class Layer:
    """One decoder layer: raw GGUF blocks per projection with their type ids,
    f32 norm weights, f16 caches [nkv][capacity][256] (updated in place)."""
    weights: dict            # name -> (type_id, blocks u8 [rows][row_bytes], rows)
    norms: dict              # attn_norm, attn_q_norm, attn_k_norm, post_attention_norm, ffn_norm, post_ffw_norm
    key_cache: np.ndarray
    value_cache: np.ndarray
    head_count: int
    head_count_kv: int
    rope_dims: int = HEAD_DIM
    rope_freq_base: float = 10000.0
    rope_freq_factors: np.ndarray | None = None
    sliding_window: int = 0
    epsilon: float = 1e-6
    output_scale: float = 1.0
    trace: dict = field(default_factory=dict)


def _proj(layer: Layer, names, x) -> list:
    """Projections of the columns x [T][k]: outputs [T][rows] each."""
    specs = [layer.weights[n] for n in names]
    xx = _f(x)
    xx = xx.reshape(-1, xx.shape[-1])
    return O.matmul_multi([t for t, _, _ in specs], [w for _, w, _ in specs], xx, [r for _, _, r in specs],
                          threads=8)


def apply_per_layer_input(layer: Layer, x: np.ndarray, per_layer_input: np.ndarray) -> np.ndarray:
    """applyPerLayerInput (layers.ts:475-521) on rows x [T][n] with this
    layer's per-layer input rows [T][P]: gate = gelu(inp_gate . x) (gelu
    1062-1076), mixed = f32(gate * input) (503-510), projected = proj .
    mixed, x + rmsNormRows(projected, post_norm).  f32(gelu(g) * u) is the
    GeGLU product (450-456), so hpo_geglu forms `mixed`."""
    eps = layer.epsilon
    t = layer.trace
    t["ple_gate"] = gate = _proj(layer, ["inp_gate"], x)[0]
    pli = _f(per_layer_input).reshape(gate.shape)
    t["ple_mixed"] = mixed = O.geglu(gate, pli)
    t["ple_proj"] = projected = _proj(layer, ["proj"], mixed)[0]
    return residual_add(x, rms_norm_rows(projected, layer.norms["post_norm"], eps))


def forward_layer(layer: Layer, hidden, position: int, per_layer_input=None) -> np.ndarray:
    """forwardAttentionLayer + forwardFfn (+ applyPerLayerInput when the
    layer has inp_gate / proj and per_layer_input [T][P] is given) + layer
    output scale for the tokens at position .. position + T - 1 (hidden
    [T][n], or [n] for one token); appends every token's key and value to the
    caches.  Every token's row is returned."""
    eps, hd = layer.epsilon, HEAD_DIM
    nq, nkv = layer.head_count, layer.head_count_kv
    x0 = _f(hidden)
    one = x0.ndim == 1
    x = x0.reshape(-1, x0.shape[-1])
    tokens = x.shape[0]
    positions = np.arange(position, position + tokens, dtype=np.int32)
    t = layer.trace
    t["attn_norm"] = xn = rms_norm_rows(x, layer.norms["attn_norm"], eps)
    shared = "attn_v" not in layer.weights
    outs = _proj(layer, ["attn_q", "attn_k"] + ([] if shared else ["attn_v"]), xn)
    q, k = outs[0], outs[1]
    v = k if shared else outs[2]
    t["q"], t["k"], t["v"] = q, k, v
    qn = rms_norm_rows(q.reshape(tokens, nq, hd), layer.norms["attn_q_norm"], eps)
    qr = rope_neox(qn, positions, layer.rope_dims, layer.rope_freq_base, layer.rope_freq_factors)
    kn = rms_norm_rows(k.reshape(tokens, nkv, hd), layer.norms["attn_k_norm"], eps)
    vn = rms_norm_rows(v.reshape(tokens, nkv, hd), None, eps)
    kr = rope_neox(kn, positions, layer.rope_dims, layer.rope_freq_base, layer.rope_freq_factors)
    for i, p in enumerate(positions):  # updateFullAttentionCache
        slot = int(p) % layer.key_cache.shape[1]
        layer.key_cache[:, slot, :] = kr[i].astype(np.float16)
        layer.value_cache[:, slot, :] = vn[i].astype(np.float16)
    t["q_rope"] = qr
    t["attention"] = att = decode_attention(qr, layer.key_cache, layer.value_cache, position, layer.sliding_window)
    t["o"] = o = _proj(layer, ["attn_output"], att.reshape(tokens, -1))[0]
    t["x1"] = x1 = residual_add(x, rms_norm_rows(o, layer.norms["post_attention_norm"], eps))
    t["ffn_norm"] = xn2 = rms_norm_rows(x1, layer.norms["ffn_norm"], eps)
    gate, up = _proj(layer, ["ffn_gate", "ffn_up"], xn2)
    t["ffn_hidden"] = h = O.geglu(gate, up)
    t["down"] = y = _proj(layer, ["ffn_down"], h)[0]
    x2 = residual_add(x1, rms_norm_rows(y, layer.norms["post_ffw_norm"], eps))
    if per_layer_input is not None and "inp_gate" in layer.weights:
        t["ffn_residual"] = x2
        x2 = apply_per_layer_input(layer, x2, per_layer_input)
    out = (x2.astype(np.float64) * np.float64(np.float32(layer.output_scale))).astype(np.float32)
    return out[0] if one else out


def rope_theta_table(position: int, n_dims: int, freq_base: float) -> np.ndarray:
    """The angles ropeNeox uses for one position (pairs 0 .. n_dims/2 - 1)."""
    scale = math.pow(freq_base, -2.0 / n_dims)
    theta = float(position)
    out = []
    for _ in range(n_dims // 2):
        out.append(theta)
        theta = float(np.float32(theta * scale))
    return np.array(out, np.float64)
