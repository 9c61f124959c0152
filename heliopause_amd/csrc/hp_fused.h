// hp_fused.h -- the persistent decode step (decode_fused.hip): one launch
// runs every decoder layer of a one-token step, one workgroup per CU, with
// the stage boundaries inside the kernel.
//
// Stages per layer (forwardAttentionLayer + forwardFfn, packages/engine/src/
// runner/wasm/layers.ts:161-473): Q/K/V (with the attn_norm prologue and the
// previous layer's post-FFN residual), attention partials (head norms, RoPE,
// cache append), their merge, O, gate/up + GeGLU (with the post-attention
// residual and ffn_norm), down.  Every stage computes what the launch
// sequence of hp_hip_decode_layers_device computes, in the same order, so
// the two give identical bits.
//
// Stage boundaries.  Values that cross workgroups travel as 8-byte words
// (f32 value, 32-bit round tag) written with agent-coherent stores and read
// with agent-coherent loads; a reader re-reads a word until its tag is the
// round it waits for.  No flag, counter or fence: a value and its readiness
// arrive together.  Tags are unique per (step, layer, boundary): epoch *
// kFusedTagStride + layer * 8 + boundary + 1, with the epoch a counter in
// device memory that the last workgroup to finish advances, so a word left
// by an earlier step or layer never matches and zeroed memory never does.
// Before a stage waits for its input, it issues the loads of its own weights
// (and the attention stage its cache rows), so those stream in while the
// previous stage finishes elsewhere.
//
// Every wait is bounded: a wait longer than the launch's limit (a
// s_memrealtime interval) sets a status bit in device memory, and every
// workgroup leaves at its next wait or stage boundary once any status bit
// is set, so the launch always ends.  The status stays set (later launches
// skip their work) until the host reads and clears it.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include "hp_common.h"

namespace hp {

// Threads per workgroup: four waves, one per SIMD, so each wave may use the
// whole register file (arch and accumulation registers); the stages' chains
// are latency-bound, not issue-bound.
constexpr int kFusedThreads = 256;
constexpr int kFusedTagStride = 4096;     // tags per step: 8 per layer
constexpr int kFusedMaxLayers = kFusedTagStride / 8 - 1;
constexpr uint32_t kFusedTimeout = 1u;    // status bit: a wait exceeded the limit

// Boundaries of one layer (tag = epoch * stride + layer * 8 + id + 1).  The
// residual stream that a norm prologue reads beside a projection's output
// carries that output's tag, and sits just before it in the arena, so the
// prologue waits for one tag over one range.
enum FusedTag {
  kTagQkv = 0,   // Q/K/V projections
  kTagPart = 1,  // attention partials
  kTagAtt = 2,   // merged attention output
  kTagO = 3,     // O projection, and the residual stream entering the layer
  kTagH = 4,     // GeGLU output
  kTagY = 5,     // down projection, and the residual after attention
};

// One projection weight in the tile layout (hp_common.h).
struct FusedWeight {
  const uint8_t *data;
  const uint16_t *dplane;  // Q6_K d plane, else null
  int32_t type, rows;
  int32_t row_begin;       // first launch row of this weight (the stage's weights end to end)
  int32_t pad;
};

// Launch rows [row_begin, row_begin + rows) of one type go to workgroups
// wg_begin .. wg_begin + wg_count - 1, rows_per_wg each (the last fewer).
struct FusedSeg {
  int32_t row_begin, rows, wg_begin, wg_count, rows_per_wg, type;
};

// The projection of one stage: 1..3 weights of one input size (with pair,
// gate and up: launch rows are the rows of each, both taken by a workgroup).
struct FusedProj {
  FusedWeight w[3];
  FusedSeg seg[3];
  int32_t count, nseg, pair;
  int32_t nb, S, R;
  uint32_t mg_nb, mg_S, mg_R;
  int32_t out_rows;  // rows written to the stage's exchange buffer (pair: rows of gate)
};

struct FusedLayer {
  FusedProj qkv, o, gu, down;
  const float *attn_norm, *q_norm, *k_norm, *post_attn_norm, *ffn_norm, *post_ffw_norm;
  const float *freq_factors;
  _Float16 *k_cache, *v_cache;
  double theta_scale, eps;
  float out_scale;
  int32_t nq, nkv, capacity, window, rope_dims, chunks;
  int32_t k_off, v_off;  // rows of k and v in the Q/K/V buffer (v_off == k_off: shared value)
  int32_t rope_key;      // layers with equal keys have equal RoPE parameters
  int32_t pad;
};

// Device control words (zeroed when allocated).
struct FusedCtl {
  uint32_t epoch;   // advanced by the last workgroup of each launch
  uint32_t done;    // workgroups finished in the current launch
  uint32_t status;  // sticky error bits (kFusedTimeout)
  uint32_t pad[61];
};

// Byte offsets of the exchange buffers (8 bytes per value) in the arena;
// o starts right after hid, y right after x1.
struct FusedXchg {
  uint32_t hid, qkv, part, att, o, x1, h, y;
  uint32_t part_slots;  // nkv * chunks * kAttnMaxGroup of the largest layer
  uint32_t total;
};

struct FusedArgs {
  const FusedLayer *layers;  // device copy, n_layers entries
  int32_t n_layers, hidden_n;
  float *hidden;             // [hidden_n] residual stream (read at layer 0, written at the end)
  const float *out_norm;     // output_norm weight, or null
  float *out;                // rmsNormRows(hidden, out_norm) when out_norm
  const int32_t *position;
  uint8_t *xchg;
  uint32_t xchg_bytes;       // the arena's size (the bound of its buffer resource)
  FusedCtl *ctl;
  const uint16_t *gelu_lut;
  uint64_t spin_ticks;       // bound of one wait (s_memrealtime ticks, 100 MHz)
  FusedXchg x;
  int32_t G;                 // query heads per kv head (every layer)
  int32_t lds_bytes;         // dynamic LDS of the launch
  // optional stage timeline: non-null, workgroup w stamps s_memrealtime at
  // eight points of stage s of layer l into trace[((w * n_layers + l) * 6 +
  // s) * 8 + k]: k = 0 stage start, 1 loads issued, 2 input arrived, 3
  // prologue done, 4 weights in registers, 5 products done, 6 chains done,
  // 7 end (points a stage does not have stay 0)
  uint64_t *trace;
};

// LDS the fused stages need for these layers (0: some stage does not fit).
size_t fused_lds_bytes(const FusedLayer *layers, int n_layers, int hidden_n);
// Launch on `s` (grid = num_cus workgroups of kFusedThreads threads).
hipError_t launch_decode_fused(const FusedArgs &a, int num_cus, hipStream_t s);
// Whether G query heads per kv head has a fused kernel.
bool fused_group_supported(int G);
// Workgroups of the G kernel that fit on one CU with `lds` dynamic LDS.
int fused_blocks_per_cu(int G, size_t lds);
// Static LDS of the G kernel (beside the dynamic part).
size_t fused_static_lds(int G);
// Task slots of one thread in a projection stage: Q4_K and Q6_K.
constexpr int kFusedSlotsQ4 = 4, kFusedSlotsQ6 = 2;

}  // namespace hp
