// capi.hip -- C ABI of the gfx950 runner (include/hp_hip.h): device setup,
// resident weight handles, shape checks and kernel sequencing.
//
// Shape and type checks follow packages/engine/wasm-kernels/src/lib.rs
// (224-298, 300-426: saturating products, ERR_SHAPE before ERR_TYPE for the
// activation/output lengths) and the resident wrappers in
// packages/engine/src/runner/wasm/wasm-kernels.ts (520-749: handle shape must
// match the call).
#include "../../include/hp_gguf.h"
#include "../../include/hp_hip.h"
#include "hp_common.h"
#include "hp_fused.h"
#include "hp_scratch.h"

#include <algorithm>
#include <atomic>
#include <climits>
#include <cstring>
#include <cmath>
#include <map>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

// Selection state of hp_hip_topk_device_noalloc: one batch of kTopkMaxRows
// rows at the largest top-k shape (n = 524288, k = 64) needs 8,454,400
// bytes.  Every device the library runs on holds its own copy for the life
// of the process; host code reaches it only through the address that
// hipGetSymbolAddress returns on that device (State::static_scratch).
constexpr size_t kNoAllocScratchBytes = (8u << 20) + (512u << 10);
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace {

using namespace hp;

struct Handle {
  int type = 0;
  size_t input_size = 0, row_count = 0, byte_length = 0;
  TileGeom g{};
  int tiles = 0;
  uint8_t *data = nullptr;     // tiles (+ Q6_K d plane at the end)
  uint16_t *dplane = nullptr;  // Q6_K only
  // matrix-core layout (16-row tile segments), or null for a weight kept in
  // one layout (the matrix-core kernels then read its tiles)
  uint8_t *segs = nullptr;
  size_t seg_bytes = 0;
  uint32_t *f16_flag = nullptr;  // set by the Q6_K repack (launch_repack)
  // The matrix-core kernels' f16 weight operands sc * q are exact for every
  // block (always for Q4_K; for Q6_K unless the repack set f16_flag).  When
  // false the launches that would use matrix cores run the vector-ALU kernels.
  bool f16_exact = true;
  uint32_t generation = 0;
  bool live = false;
};

struct ProfileSlot {
  std::vector<std::pair<hipEvent_t, hipEvent_t>> pending;
  double total_ms = 0;
  uint64_t launches = 0;
};

// Device memory for the scratch pool (hp_scratch.h).
struct HipAlloc {
  bool alloc(void **p, size_t bytes) { return hipMalloc(p, bytes) == hipSuccess; }
  void free(void *p) { (void)hipFree(p); }
  bool zero(void *p, size_t bytes, void *stream) {
    hipStream_t q = static_cast<hipStream_t>(stream);
    return hipMemsetAsync(p, 0, bytes, q) == hipSuccess && hipStreamSynchronize(q) == hipSuccess;
  }
};

struct State {
  std::recursive_mutex mu;
  bool ready = false;
  int device = -1;
  int num_cus = 0;
  size_t max_lds = 0;
  hipStream_t stream = nullptr;
  std::vector<Handle> handles;
  float *io_in = nullptr, *io_out[kMaxWeights] = {nullptr, nullptr, nullptr, nullptr};
  size_t io_in_cap = 0, io_out_cap[kMaxWeights] = {0, 0, 0, 0};
  void *topk_out = nullptr;  // ids + values of the host-pointer top-k entry points
  size_t topk_out_cap = 0;
  uint64_t matmul_calls = 0, launches = 0;
  int matvec_kernel = 0;  // 0 auto, 1 vector ALU, 2 matrix cores, 3 half-split, 4 prefill,
                          // 5 fast prefill, 6 wide, 7 wide (whole tasks), 8 wide (half tasks)
  // set while a host-pointer matmul entry point runs: the automatic policy then
  // keeps to the bit-exact kernels, as the reference's resident calls are
  bool host_exact = false;
  // pre-quantised input images between the launches of a draft step (a
  // test switch: off, every vector-ALU launch quantises its own input)
  bool images = true;
  bool prefill_folds = true;  // hp_hip_set_prefill_folds
  bool both_layouts = true;   // hp_hip_set_weight_layouts: uploads keep the segment copy
  bool profiling = false;
  ProfileSlot prof[HP_KERNEL_COUNT];
  std::vector<hipEvent_t> event_pool;
  // GGUF loader: pinned staging (two chunks per reader), one copy stream and
  // two events per reader, and the device staging of a batch of tensors.
  uint8_t *pinned = nullptr;
  size_t pinned_cap = 0;
  std::vector<hipStream_t> copy_streams;
  std::vector<hipEvent_t> copy_events;
  uint8_t *load_staging = nullptr;
  size_t load_staging_cap = 0;
  // sampling outputs of the host-pointer entry point: rng state, tokens,
  // kept counts and probabilities
  void *sample_out = nullptr;
  size_t sample_out_cap = 0;
  // intermediate device memory of the asynchronous entry points, per stream
  ScratchPool<HipAlloc> pool;
  // device address of the file-scope `scratch` array on `device`, looked up
  // by ensure_init (the allocation-free entry point's only scratch)
  uint8_t *static_scratch = nullptr;
  uint16_t *gelu_lut = nullptr;  // the GeGLU launches' gelu table (ensure_init)
  // persistent decode step (decode_fused.hip): 1 runs it for one-token calls
  // that it covers, 0 keeps the launch sequence; the bound of one of its
  // waits in s_memrealtime ticks (100 MHz); device copies of its layer
  // tables by content, kept until hp_hip_shutdown (a captured graph may
  // still point at one)
  int fused_mode = 0;  // the persistent one-token step is opt-in (hp_hip_set_decode_fused)
  uint64_t fused_spin = 100000000ull;
  uint64_t *fused_trace = nullptr;  // stage timeline buffer (hp_hip_set_fused_trace), or null
  size_t fused_trace_len = 0;
  std::map<std::vector<uint8_t>, void *> fused_tables;
  // device buffers of hp_hip_device_alloc: base address -> bytes (copies are
  // checked against them), freed by hp_hip_device_free or hp_hip_shutdown
  std::map<uintptr_t, size_t> dev_bufs;
};

State &st() {
  static State s;
  return s;
}

thread_local std::string g_last_error;

int32_t fail(int32_t code, const std::string &msg) {
  g_last_error = msg;
  return code;
}

int32_t hip_fail(hipError_t e, const char *what) {
  return fail(HP_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

#define HP_HIP_TRY(expr)                         \
  do {                                           \
    hipError_t _e = (expr);                      \
    if (_e != hipSuccess) return hip_fail(_e, #expr); \
  } while (0)

size_t sat_mul(size_t a, size_t b) {
  size_t r;
  if (__builtin_mul_overflow(a, b, &r)) return (size_t)-1;
  return r;
}

size_t row_bytes_for(int type, size_t input_size) {
  if (input_size % kQK != 0) return 0;
  if (type == kTypeQ4K) return input_size / kQK * 144;
  if (type == kTypeQ6K) return input_size / kQK * 210;
  return 0;
}

double gelu_constant();

int32_t ensure_init(int device) {
  State &s = st();
  if (s.ready) return HP_OK;
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return fail(HP_ERR_NODEV, "no HIP device available");
  if (device < 0 || device >= n) return fail(HP_ERR_ARG, "device index out of range");
  HP_HIP_TRY(hipSetDevice(device));
  HP_HIP_TRY(hipDeviceGetAttribute(&s.num_cus, hipDeviceAttributeMultiprocessorCount, device));
  int lds = 0;
  HP_HIP_TRY(hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerBlock, device));
  s.max_lds = (size_t)lds;
  HP_HIP_TRY(hipStreamCreateWithFlags(&s.stream, hipStreamNonBlocking));
  // this device's copy of the static scratch: the array's name is a host
  // stand-in, only this address reaches its device memory
  void *sym = nullptr;
  HP_HIP_TRY(hipGetSymbolAddress(&sym, HIP_SYMBOL(scratch)));
  if (!sym) return fail(HP_ERR_HIP, "hipGetSymbolAddress(scratch) returned null");
  s.static_scratch = static_cast<uint8_t *>(sym);
  // the gelu table of the GeGLU launches (hp_gelu.h gelu_lut), built once
  if (hipMalloc((void **)&s.gelu_lut, 65536 * sizeof(uint16_t)) != hipSuccess) {
    s.gelu_lut = nullptr;
    return fail(HP_ERR_OOM, "gelu table allocation failed");
  }
  HP_HIP_TRY(launch_gelu_lut(gelu_constant(), s.gelu_lut, s.stream));
  HP_HIP_TRY(hipStreamSynchronize(s.stream));
  s.device = device;
  s.ready = true;
  return HP_OK;
}

Handle *lookup(uint64_t id) {
  State &s = st();
  const uint64_t idx = (id & 0xffffffffu);
  const uint32_t gen = (uint32_t)(id >> 32);
  if (idx == 0 || idx > s.handles.size()) return nullptr;
  Handle &h = s.handles[idx - 1];
  if (!h.live || h.generation != gen) return nullptr;
  return &h;
}

int32_t grow(void **p, size_t *cap, size_t bytes) {
  if (*cap >= bytes && *p) return HP_OK;
  State &s = st();
  if (*p) {
    HP_HIP_TRY(hipStreamSynchronize(s.stream));
    HP_HIP_TRY(hipFree(*p));
    *p = nullptr;
    *cap = 0;
  }
  size_t want = bytes < 4096 ? 4096 : bytes;
  if (hipMalloc(p, want) != hipSuccess) {
    *p = nullptr;
    return fail(HP_ERR_OOM, "device allocation failed");
  }
  *cap = want;
  return HP_OK;
}

// Scratch of `kind` for work queued on `stream` (hp_scratch.h): per stream,
// grow-only, and never grown while the stream captures a graph.
int32_t stream_scratch(hipStream_t stream, int kind, size_t bytes, void **out, bool zero = false) {
  State &s = st();
  void *key = stream ? static_cast<void *>(stream) : static_cast<void *>(s.stream);
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &cs) != hipSuccess) cs = hipStreamCaptureStatusNone;
  switch (s.pool.get(key, kind, bytes, cs != hipStreamCaptureStatusNone, zero, out)) {
    case kScratchOk: return HP_OK;
    case kScratchCapturing:
      return fail(HP_ERR_ARG, "scratch must be sized by an uncaptured call of this shape before graph capture");
    case kScratchZeroFailed: return fail(HP_ERR_HIP, "clearing scratch failed");
    default: return fail(HP_ERR_OOM, "device allocation failed");
  }
}

hipEvent_t take_event() {
  State &s = st();
  if (!s.event_pool.empty()) {
    hipEvent_t e = s.event_pool.back();
    s.event_pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

// Records a start event when profiling; returns it (or null).
hipEvent_t prof_begin(hipStream_t stream) {
  State &s = st();
  if (!s.profiling) return nullptr;
  hipEvent_t e = take_event();
  if (e) (void)hipEventRecord(e, stream);
  return e;
}

void prof_end(int kernel, hipEvent_t start, hipStream_t stream) {
  State &s = st();
  if (!start) return;
  hipEvent_t e = take_event();
  if (!e) return;
  (void)hipEventRecord(e, stream);
  s.prof[kernel].pending.emplace_back(start, e);
}

void prof_collect() {
  State &s = st();
  for (int k = 0; k < HP_KERNEL_COUNT; k++) {
    for (auto &pr : s.prof[k].pending) {
      float ms = 0.0f;
      if (hipEventSynchronize(pr.second) == hipSuccess && hipEventElapsedTime(&ms, pr.first, pr.second) == hipSuccess) {
        s.prof[k].total_ms += ms;
        s.prof[k].launches += 1;
      }
      s.event_pool.push_back(pr.first);
      s.event_pool.push_back(pr.second);
    }
    s.prof[k].pending.clear();
  }
}

// sqrt(2/pi) as Math.sqrt(2 / Math.PI) evaluates it (IEEE f64 divide and sqrt).
double gelu_constant() { return std::sqrt(2.0 / 3.141592653589793); }

// Column chunk such that the matvec launch's LDS fits the device limit.
int cols_per_launch(const TileGeom &g, size_t max_lds) {
  for (int c = kMaxCols; c >= 1; c--) {
    size_t x = (size_t)c * g.nb * kQ8BlockBytes + (size_t)((c * g.nb + 3) & ~3) * 4;
    if (x <= max_lds) return c;
  }
  return 0;
}

// Kernel choice.  The matrix-core kernel's cost barely grows with the column
// count but each wave walks its 16-row tile block by block, so it needs many
// tiles to hide memory latency; the vector-ALU kernel's cost grows with the
// columns (and it spills registers beyond four).  Measured on MI355X: the
// matrix cores win from five columns on, and from two columns on when the
// launch has >= 1024 tiles (16 rows each); one column stays on the vector
// ALU.  Both need their LDS (the columns' Q8_K for every block) to fit.
// Prefill kernels (matrix cores, columns in tiles of 64, weights read once per
// column tile) for many columns.  From kFastMinCols columns the automatic
// policy takes the fast one, whose outputs agree with the reference within the
// 1e-4 relative tolerance of projections (M >= 64 prefill chunks); selector 4
// forces the bit-exact one, 5 the fast one.  Below kPrefillMinCols the decode
// kernels, which read the weights once per 8 columns, are as fast.
constexpr size_t kPrefillMinCols = 32;
constexpr size_t kFastMinCols = 64;

// 0: not a prefill launch, 1: bit-exact prefill, 2: fast prefill
// f16ok: the matrix-core kernels can take every weight of the launch
// (mfma_ok: exact f16 operands, tiles they can address); otherwise no prefill
// kernel applies, forced or not.
int prefill_kind(size_t cols, bool f16ok) {
  const State &s = st();
  const int forced = s.matvec_kernel;
  if (!f16ok) return 0;
  const bool exact_fits = prefill_lds_bytes() <= s.max_lds;
  const bool fast_fits = prefill_fast_lds_bytes() <= s.max_lds;
  if (forced == 4) return exact_fits ? 1 : 0;
  if (forced == 5) return fast_fits ? 2 : 0;
  if (forced != 0) return 0;
  if (cols >= kFastMinCols && fast_fits && !s.host_exact) return 2;
  if (cols >= kPrefillMinCols && exact_fits) return 1;
  return 0;
}

bool use_mfma(size_t cols, int nb, int tiles16, bool f16ok) {
  const State &s = st();
  const int forced = s.matvec_kernel;
  const size_t lds = mfma_lds_bytes(cols < 8 ? (int)cols : 8, nb);
  if (!f16ok || forced == 1 || forced == 3 || lds > s.max_lds) return false;
  if (forced == 2) return true;
  if (cols < 2 || lds > 64 * 1024) return false;
  return cols >= 5 || tiles16 >= 1024;
}

// Half-split vector-ALU kernel (two lanes per row-block).  It halves each
// wave's work and doubles the waves, which pays while the launch has few
// tiles (small projections are latency-bound) and costs throughput on large
// ones.  Measured on MI355X: faster for one column up to ~2048 tiles (Q/K/V
// 512, 10240 rows 1707: 7.39 against 7.75 us) and for two to four columns up
// to ~1024 tiles; slower for gate/up (3414 tiles), the head, and 40-block
// rows (S = 20: down 15.6 against 13.2 us).
bool use_half(int cols, const TileGeom &g, int tiles, int rows) {
  const int forced = st().matvec_kernel;
  if (cols > 4 || g.S > 32 || rows >= (1 << 20)) return false;  // (rows: the kernel's index range)
  if (forced == 3) return true;
  if (forced != 0 || g.S > 16) return false;
  return tiles <= (cols == 1 ? 2048 : 1024);
}

// Wide kernel (kquant_wide.hip): one workgroup per block of rows, every
// block of each row, products chained in LDS.  Needs one weight type (Q4_K or
// Q6_K) across the launch, at most four columns and its LDS within the device
// limit.  Automatic for long rows (40 blocks and more: the FFN down
// projection) at one to four columns, where the one-wave-per-tile kernel
// leaves most SIMDs idle (down, measured: 13.2 -> 10.6 us at one column,
// 19.5 -> 14.6 at two, 30.9 -> 23.1 at four); selector 6 forces it wherever it
// applies.
int wide_rows_for(int rows, int nb, int cols, int type) {
  const State &s = st();
  int r = (rows + s.num_cus - 1) / s.num_cus;
  while (r > 1 && wide_lds_bytes(cols, nb, type, r) > s.max_lds) r = (r + 1) / 2;
  return r;
}

int g_nb_of(Handle *const *hs) { return hs[0]->g.nb; }

// The matrix-core kernels can take these weights: their f16 operands are
// exact, and when the launch reads its weights from their tiles (one of them
// kept without segments makes every weight of the launch read that way),
// each fits the kernels' 32-bit tile offsets (under 4 GiB).
bool mfma_ok(size_t count, Handle *const *hs) {
  bool tiles = false;
  for (size_t i = 0; i < count; i++) tiles = tiles || !hs[i]->segs;
  for (size_t i = 0; i < count; i++)
    if (!hs[i]->f16_exact || (tiles && hs[i]->byte_length >= ((size_t)1 << 32))) return false;
  return true;
}

bool use_wide(size_t count, Handle *const *hs, size_t cols) {
  const State &s = st();
  const int forced = s.matvec_kernel;
  if (cols < 1 || cols > 4 || (forced != 0 && forced < 6)) return false;
  const int type = hs[0]->type;
  if (type != kTypeQ4K && type != kTypeQ6K) return false;
  size_t rows = 0;
  for (size_t i = 0; i < count; i++) {
    if (hs[i]->type != type) return false;
    rows += hs[i]->row_count;
  }
  const int nb = hs[0]->g.nb;
  if (nb > 256 || rows >= (1u << 20)) return false;  // div_magic's exact range
  if (wide_lds_bytes((int)cols, nb, type, wide_rows_for((int)rows, nb, (int)cols, type)) > s.max_lds)
    return false;
  if (forced >= 6) return true;
  return nb >= 40;  // 1..4 columns (checked above)
}

// Tasks of the wide kernel: whole row-blocks (up to 512 threads) or half
// row-blocks (lane classes 4h .. 4h+3, up to 1024 threads).  Selector 7
// forces whole, 8 half; both give the same bits.
// Half tasks exist for launches without the norm prologue or GeGLU at one or
// two columns.
int wide_half_for(bool norm, bool pair, int cols) {
  const int forced = st().matvec_kernel;
  if (norm || pair || cols > 2 || forced == 7) return 0;
  if (forced == 8) return 1;
  return cols == 1 ? 1 : 0;
}

// The wide kernel for gate/up + GeGLU (equal rows, one type) at one to four
// columns (the FFN gate/up + GeGLU + down, measured: 42.3 -> 31.4 us at two
// columns, 56.0 -> 45.5 at four against the matrix-core gate/up and its GeGLU
// launch).
bool use_wide_pair(Handle *const *hs, size_t cols) {
  const State &s = st();
  const int forced = s.matvec_kernel;
  if (cols < 1 || cols > 4 || (forced != 0 && forced < 6)) return false;
  const int type = hs[0]->type;
  if ((type != kTypeQ4K && type != kTypeQ6K) || hs[1]->type != type || hs[0]->row_count != hs[1]->row_count)
    return false;
  const int nb = hs[0]->g.nb;
  const size_t rows = hs[0]->row_count;
  if (nb > 256 || 2 * rows >= (1u << 20)) return false;
  const int r = wide_rows_for((int)(2 * rows), nb, (int)cols, type) / 2;
  if (r < 1 || wide_lds_bytes((int)cols, nb, type, 2 * r) > s.max_lds) return false;
  return true;  // 1..4 columns (checked above)
}

// One matvec launch per column chunk covering every weight (multi == one
// launch, lib.rs:300-426); each launch quantises its columns in its prologue.
int32_t run_norm(const float *y, int rows, int n, const float *w_post, const float *x_res, float scale, float *x_out,
                 const float *w_next, float *next_out, double eps, hipStream_t stream, uint8_t *q8img = nullptr,
                 uint8_t *xt = nullptr, const PrefillParts *y_parts = nullptr, bool next_image_only = false,
                 bool x16 = false);

// Whether a one-column launch over these weights runs a vector-ALU kernel,
// which can form its input with the norm prologue.
bool norm_prologue_ok(size_t count, Handle *const *hs, size_t cols) {
  const bool f16 = mfma_ok(count, hs);
  if (cols != 1 || hs[0]->g.nb > 16 || prefill_kind(cols, f16) != 0) return false;
  int tiles16 = 0;
  for (size_t i = 0; i < count; i++) tiles16 += (int)((hs[i]->row_count + 15) / 16);
  return !use_mfma(cols, hs[0]->g.nb, tiles16, f16);
}

// Whether a launch of `cols` columns (2 or more) runs the vector-ALU kernels
// in one chunk, so it can take its input as a pre-quantised image.
bool image_input_ok(size_t count, Handle *const *hs, size_t cols) {
  const bool f16 = mfma_ok(count, hs);
  if (cols < 2 || prefill_kind(cols, f16) != 0) return false;
  int tiles16 = 0;
  for (size_t i = 0; i < count; i++) tiles16 += (int)((hs[i]->row_count + 15) / 16);
  return !use_mfma(cols, hs[0]->g.nb, tiles16, f16) && cols_per_launch(hs[0]->g, st().max_lds) >= (int)cols;
}

// norm != null: the input is formed from a residual stream (NormIn) -- in the
// launch's prologue when the launch runs a vector-ALU kernel, else by the norm
// kernel into norm_scratch first.
// q8img_in (2 or more columns): the input already quantised, as written by
// the norm or GeGLU kernels (q8_image_bytes(cols, nb)); used when the launch
// runs the vector-ALU kernels in one chunk.  img_scratch: where a norm run
// here writes that image for the launch.
int32_t run_matvec(size_t count, Handle *const *hs, const float *d_input, size_t input_size, size_t cols,
                   float *const *d_outs, hipStream_t stream, const NormIn *norm = nullptr,
                   float *norm_scratch = nullptr, uint8_t *img_scratch = nullptr, const uint8_t *q8img_in = nullptr,
                   const PrefillParts *norm_parts = nullptr, PrefillParts *defer = nullptr,
                   bool tiles_in = false, const GegluTail *tail_in = nullptr) {
  if (defer) defer->ks = 1;
  State &s = st();
  if (cols == 0) return HP_OK;
  if (tail_in && !tail_in->part) tail_in = nullptr;
  const bool image_ok = s.images && cols >= 2 && image_input_ok(count, hs, cols);
  const bool f16 = mfma_ok(count, hs);
  const bool wide = prefill_kind(cols, f16) == 0 && use_wide(count, hs, cols);
  const bool wide_norm = wide && cols == 1 && g_nb_of(hs) <= 16;  // the wide kernel's norm prologue
  const int kind = prefill_kind(cols, f16);
  if (kind && cols > 65535) return fail(HP_ERR_SHAPE, "too many columns");
  // a deferred GeGLU tail is completed by the fast prefill kernel's pre-pass
  if (tail_in && (kind != 2 || norm || tiles_in)) return fail(HP_ERR_ARG, "deferred GeGLU tail needs the fast prefill");
  MfmaLaunch l{};
  l.count = (int)count;
  l.k = (int)input_size;
  l.cols = (int)cols;
  l.S = hs[0]->g.S;
  l.R = hs[0]->g.R;
  for (size_t i = 0; i < count; i++) {
    l.seg[i] = hs[i]->segs;
    l.wt[i] = hs[i]->data;
    l.dplane[i] = hs[i]->dplane;
    l.type[i] = hs[i]->type;
    l.rows[i] = (int)hs[i]->row_count;
    l.out[i] = d_outs[i];
  }
  uint8_t *pre = nullptr;  // the prefill kernels' scratch
  if (kind) {
    const size_t need = kind == 2 ? prefill_fast_bytes(l, s.num_cus) : prefill_q8k_bytes((int)input_size, (int)cols);
    void *p = nullptr;
    int32_t rc = stream_scratch(stream, kScratchPrefill, need, &p);
    if (rc != HP_OK) return rc;
    pre = static_cast<uint8_t *>(p);
  }
  // the norm kernel below, or the producer of d_input (tiles_in: the prefill
  // attention's slice merge), wrote the fast prefill's tiles
  bool tiles_ready = s.prefill_folds && tiles_in && kind == 2 && input_size % kQK == 0;
  const bool y_split = norm_parts && norm_parts->ks > 1;  // the norm's y as partial sums
  if (norm && (y_split || (wide ? !wide_norm : !norm_prologue_ok(count, hs, cols)))) {
    uint8_t *img = image_ok && img_scratch ? img_scratch : nullptr;
    tiles_ready = s.prefill_folds && kind == 2 && input_size % kQK == 0;
    // with its tiles written, the fast prefill kernel does not read the f32
    // input (kept for an image: storing it measured faster for the drafts)
    int32_t rc = run_norm(norm->y, (int)cols, (int)input_size, norm->w_post, norm->mode == 2 ? norm->x_res : nullptr,
                          norm->scale, norm->x_out, norm->w_next, norm_scratch, norm->eps, stream, img,
                          tiles_ready ? pre : nullptr, norm_parts, tiles_ready, true);
    if (rc != HP_OK) return rc;
    d_input = norm_scratch;
    norm = nullptr;
    q8img_in = img;
  }
  if (!image_ok) q8img_in = nullptr;
  const TileGeom g = hs[0]->g;
  MatvecArgs a{};
  if (norm) a.norm = *norm;
  a.count = (int)count;
  a.g = g;
  a.k = (int)input_size;
  int tiles = 0;
  for (size_t i = 0; i < count; i++) {
    a.w[i].data = hs[i]->data;
    a.w[i].dplane = hs[i]->dplane;
    a.w[i].out = d_outs[i];
    a.w[i].type = hs[i]->type;
    a.w[i].rows = (int)hs[i]->row_count;
    a.w[i].tiles = hs[i]->tiles;
    a.w[i].tile_begin = tiles;
    tiles += hs[i]->tiles;
  }
  a.total_tiles = tiles;
  a.Rh = g.S <= 32 ? 32 / g.S : 0;
  int rows_all = 0;
  for (size_t i = 0; i < count; i++) {
    a.w[i].row_begin = rows_all;
    rows_all += (int)hs[i]->row_count;
  }
  a.total_rows = rows_all;
  a.total_units = a.Rh ? (rows_all + a.Rh - 1) / a.Rh : 0;
  if (kind) {
    hipEvent_t e1 = prof_begin(stream);
    if (kind == 2) {
      const size_t part_bytes = defer ? prefill_fast_part_bytes(l, s.num_cus) : 0;
      if (part_bytes) {
        void *p = nullptr;
        int32_t rc = stream_scratch(stream, kScratchParts, part_bytes, &p);
        if (rc != HP_OK) return rc;
        defer->part = static_cast<float *>(p);
      }
      HP_HIP_TRY(launch_prefill_fast(l, d_input, pre, s.num_cus, stream, tiles_ready, part_bytes ? defer : nullptr,
                                     tail_in));
      if (part_bytes) s.launches--;  // no reduction launch
    } else {
      HP_HIP_TRY(launch_q8k_prefill(d_input, (int)input_size, (int)cols, pre, stream));
      HP_HIP_TRY(launch_prefill(l, pre, s.num_cus, stream));
    }
    prof_end(HP_KERNEL_MATVEC, e1, stream);
    s.launches += kind == 2 ? prefill_fast_launches(l, s.num_cus) - (tiles_ready ? 1 : 0) : 2;
    s.matmul_calls++;
    return HP_OK;
  }
  if (wide) {
    a.wide_rows = wide_rows_for(rows_all, g.nb, (int)cols, hs[0]->type);
    a.wide_half = wide_half_for(norm != nullptr, false, (int)cols);
    a.mg_nb = div_magic(g.nb);
    a.mg_S = div_magic(g.S);
    a.mg_R = div_magic(g.R);
    a.x = d_input;
    a.cols = (int)cols;
    a.out_col0 = 0;
    a.q8img = q8img_in;
    hipEvent_t e1 = prof_begin(stream);
    HP_HIP_TRY(launch_matvec_wide(a, stream));
    prof_end(HP_KERNEL_MATVEC, e1, stream);
    s.launches++;
    s.matmul_calls++;
    return HP_OK;
  }
  int tiles16 = 0;
  for (size_t i = 0; i < count; i++) tiles16 += (int)((hs[i]->row_count + 15) / 16);
  if (use_mfma(cols, g.nb, tiles16, f16)) {
    MfmaLaunch l{};
    l.count = (int)count;
    l.k = (int)input_size;
    l.S = g.S;
    l.R = g.R;
    for (size_t i = 0; i < count; i++) {
      l.seg[i] = hs[i]->segs;
      l.wt[i] = hs[i]->data;
      l.dplane[i] = hs[i]->dplane;
      l.type[i] = hs[i]->type;
      l.rows[i] = (int)hs[i]->row_count;
    }
    for (size_t m0 = 0; m0 < cols; m0 += 8) {
      const int c = (int)((cols - m0) < 8 ? (cols - m0) : 8);
      l.x = d_input + m0 * input_size;
      l.cols = c;
      l.out_col0 = (int)m0;
      for (size_t i = 0; i < count; i++) l.out[i] = d_outs[i];
      hipEvent_t e1 = prof_begin(stream);
      HP_HIP_TRY(launch_matvec_mfma(l, s.num_cus, stream));
      prof_end(HP_KERNEL_MATVEC, e1, stream);
      s.launches++;
    }
    s.matmul_calls++;
    return HP_OK;
  }
  const int chunk = cols_per_launch(g, s.max_lds);
  if (chunk <= 0) return fail(HP_ERR_SHAPE, "input_size too large for the matvec LDS budget");
  a.q8img = q8img_in;  // one chunk (image_input_ok)
  for (size_t m0 = 0; m0 < cols; m0 += (size_t)chunk) {
    const int c = (int)((cols - m0) < (size_t)chunk ? (cols - m0) : (size_t)chunk);
    a.x = d_input + m0 * input_size;
    a.cols = c;
    a.out_col0 = (int)m0;
    hipEvent_t e1 = prof_begin(stream);
    if (use_half(c, g, a.total_tiles, a.total_rows))
      HP_HIP_TRY(launch_matvec_half(a, s.num_cus, stream));
    else
      HP_HIP_TRY(launch_matvec(a, s.num_cus, stream));
    prof_end(HP_KERNEL_MATVEC, e1, stream);
    s.launches++;
  }
  s.matmul_calls++;
  return HP_OK;
}

// gate/up projections + GeGLU into d_out ([cols][rows]).  One fused
// vector-ALU launch when the kernel policy would run the full vector-ALU
// kernel on this launch (one column of large projections); the fast prefill
// kernel with gate and up rows in one tile when the policy takes it (gate and
// up of one type); otherwise the
// projections (one launch, any kernel) into scratch, then the GeGLU kernel.
// Both give the same bits.
// q8img_out (2 or more columns): when the GeGLU runs as its own launch it also
// writes d_out as a matvec input image there, and *q8img_written says so.
int32_t run_matvec_geglu(Handle *hg, Handle *hu, const float *d_input, size_t input_size, size_t cols,
                         float *d_out, hipStream_t stream, const NormIn *norm = nullptr,
                         float *norm_scratch = nullptr, uint8_t *q8img_out = nullptr,
                         bool *q8img_written = nullptr, const PrefillParts *norm_parts = nullptr,
                         GegluTail *tail_out = nullptr) {
  if (q8img_written) *q8img_written = false;
  if (tail_out) *tail_out = GegluTail{};
  State &s = st();
  if (cols == 0) return HP_OK;
  const size_t rows = hg->row_count;
  const TileGeom g = hg->g;
  const int tiles16 = 2 * (int)((rows + 15) / 16);
  Handle *pair[2] = {hg, hu};
  const bool f16 = mfma_ok(2, pair);
  const bool wide = prefill_kind(cols, f16) == 0 && hg->type == hu->type && use_wide_pair(pair, cols);
  const bool fused = !wide && cols <= 4 && s.matvec_kernel <= 1 && !use_mfma(cols, g.nb, tiles16, f16) &&
                     !use_half((int)cols, g, 2 * hg->tiles, (int)(2 * rows)) && cols_per_launch(g, s.max_lds) >= (int)cols;
  // fast prefill: gate and up rows in one tile, GeGLU in its epilogue
  const bool fast = prefill_kind(cols, f16) == 2 && hg->type == hu->type;
  MfmaLaunch l{};
  uint8_t *pre = nullptr;  // its scratch, tiles first
  if (fast) {
    l.count = 2;
    l.k = (int)input_size;
    l.S = g.S;
    l.R = g.R;
    l.cols = (int)cols;
    for (int i = 0; i < 2; i++) {
      l.seg[i] = pair[i]->segs;
      l.wt[i] = pair[i]->data;
      l.dplane[i] = pair[i]->dplane;
      l.type[i] = pair[i]->type;
      l.rows[i] = (int)rows;
    }
    void *p = nullptr;
    int32_t rc = stream_scratch(stream, kScratchPrefill, prefill_fast_geglu_bytes(l, s.num_cus), &p);
    if (rc != HP_OK) return rc;
    pre = static_cast<uint8_t *>(p);
  }
  bool tiles_ready = false;  // the norm kernel wrote the fast prefill's tiles
  const bool y_split = norm_parts && norm_parts->ks > 1;  // the norm's y as partial sums
  if (norm && (y_split || !((fused || wide) && cols == 1 && g.nb <= 16))) {
    tiles_ready = s.prefill_folds && fast && input_size % kQK == 0;
    int32_t rc = run_norm(norm->y, (int)cols, (int)input_size, norm->w_post, norm->mode == 2 ? norm->x_res : nullptr,
                          norm->scale, norm->x_out, norm->w_next, norm_scratch, norm->eps, stream, nullptr,
                          tiles_ready ? pre : nullptr, norm_parts, tiles_ready, true);
    if (rc != HP_OK) return rc;
    d_input = norm_scratch;
    norm = nullptr;
  }
  if (wide) {
    MatvecArgs a{};
    if (norm) a.norm = *norm;
    a.count = 2;
    a.g = g;
    a.k = (int)input_size;
    for (int i = 0; i < 2; i++) {
      a.w[i].data = pair[i]->data;
      a.w[i].dplane = pair[i]->dplane;
      a.w[i].out = nullptr;
      a.w[i].type = pair[i]->type;
      a.w[i].rows = (int)rows;
      a.w[i].tiles = pair[i]->tiles;
      a.w[i].row_begin = i * (int)rows;
    }
    a.total_rows = (int)rows;
    a.wide_rows = wide_rows_for((int)(2 * rows), g.nb, (int)cols, hg->type) / 2;
    if (a.wide_rows < 1) a.wide_rows = 1;
    a.wide_half = wide_half_for(norm != nullptr, true, (int)cols);
    a.mg_nb = div_magic(g.nb);
    a.mg_S = div_magic(g.S);
    a.mg_R = div_magic(g.R);
    a.x = d_input;
    a.cols = (int)cols;
    a.out_col0 = 0;
    a.pair_out = d_out;
    a.gelu_lut = s.gelu_lut;
    hipEvent_t e1 = prof_begin(stream);
    HP_HIP_TRY(launch_matvec_wide(a, stream));
    prof_end(HP_KERNEL_MATVEC, e1, stream);
    s.launches++;
    s.matmul_calls++;
    return HP_OK;
  }
  if (fused) {
    MatvecArgs a{};
    if (norm) a.norm = *norm;
    a.count = 2;
    a.g = g;
    a.k = (int)input_size;
    Handle *hs[2] = {hg, hu};
    for (int i = 0; i < 2; i++) {
      a.w[i].data = hs[i]->data;
      a.w[i].dplane = hs[i]->dplane;
      a.w[i].out = nullptr;
      a.w[i].type = hs[i]->type;
      a.w[i].rows = (int)rows;
      a.w[i].tiles = hs[i]->tiles;
      a.w[i].tile_begin = i * hs[0]->tiles;
    }
    a.total_tiles = 2 * hg->tiles;
    a.x = d_input;
    a.cols = (int)cols;
    a.out_col0 = 0;
    a.pair_out = d_out;
    a.gelu_lut = s.gelu_lut;
    hipEvent_t e1 = prof_begin(stream);
    HP_HIP_TRY(launch_matvec_pair(a, s.num_cus, stream));
    prof_end(HP_KERNEL_MATVEC, e1, stream);
    s.launches++;
    s.matmul_calls++;
    return HP_OK;
  }
  if (fast) {
    // tail_out: the trailing tiles' range sums go to their own scratch for
    // the consumer's pre-pass, in place of the tail launch
    float *tail_part = nullptr;
    const size_t tail_bytes = tail_out ? prefill_fast_geglu_tail_bytes(l, s.num_cus) : 0;
    if (tail_bytes) {
      void *p = nullptr;
      int32_t rc = stream_scratch(stream, kScratchGeglu, tail_bytes, &p);
      if (rc != HP_OK) return rc;
      tail_part = static_cast<float *>(p);
    }
    hipEvent_t e1 = prof_begin(stream);
    HP_HIP_TRY(launch_prefill_fast_geglu(l, d_input, pre, s.gelu_lut, d_out, s.num_cus, stream, tiles_ready,
                                         tail_part ? tail_out : nullptr, tail_part));
    prof_end(HP_KERNEL_MATVEC, e1, stream);
    s.launches += prefill_fast_geglu_launches(l, s.num_cus) - (tiles_ready ? 1 : 0) - (tail_part ? 1 : 0);
    s.matmul_calls++;
    return HP_OK;
  }
  void *sums = nullptr;
  int32_t rc = stream_scratch(stream, kScratchGeglu, 2 * cols * rows * sizeof(float), &sums);
  if (rc != HP_OK) return rc;
  Handle *hs[2] = {hg, hu};
  float *outs[2] = {static_cast<float *>(sums), static_cast<float *>(sums) + cols * rows};
  rc = run_matvec(2, hs, d_input, input_size, cols, outs, stream);
  if (rc != HP_OK) return rc;
  hipEvent_t e2 = prof_begin(stream);
  if (q8img_out && s.images && cols >= 2 && rows % kQK == 0) {
    HP_HIP_TRY(launch_geglu_q8k(outs[0], outs[1], (int)rows, (int)cols, s.gelu_lut, d_out, q8img_out, stream));
    if (q8img_written) *q8img_written = true;
  } else {
    HP_HIP_TRY(launch_geglu(outs[0], outs[1], cols * rows, s.gelu_lut, d_out, s.num_cus, stream));
  }
  prof_end(HP_KERNEL_GEGLU, e2, stream);
  s.launches++;
  return HP_OK;
}

// Scope of a host-pointer matmul entry point (hp_hip_matmul, _multi, _geglu,
// _topk, _topk_sample): these replace the reference's resident matmul calls,
// whose results are bit-exact, so the automatic kernel policy does not pick
// the fast prefill kernel inside them (selector 5 still forces it).
struct HostExactScope {
  bool prev;
  HostExactScope() : prev(st().host_exact) { st().host_exact = true; }
  ~HostExactScope() { st().host_exact = prev; }
};

int32_t geglu_pair_check(uint64_t gate, uint64_t up, size_t input_len, size_t input_size, size_t cols,
                         size_t output_len, Handle **hg, Handle **hu) {
  *hg = lookup(gate);
  *hu = lookup(up);
  if (!*hg || !*hu) return fail(HP_ERR_HANDLE, "unknown weight handle");
  if ((*hg)->input_size != input_size || (*hu)->input_size != input_size || input_len != sat_mul(input_size, cols))
    return fail(HP_ERR_SHAPE, "gate/up input shape mismatch");
  if ((*hg)->row_count != (*hu)->row_count) return fail(HP_ERR_SHAPE, "gate and up row counts differ");
  if (output_len != sat_mul((*hg)->row_count, cols)) return fail(HP_ERR_SHAPE, "output length mismatch");
  return HP_OK;
}

// Handle::f16_exact from the Q6_K repack's flag, once the repack has finished.
hipError_t read_f16_flag(Handle &h) {
  if (h.type != kTypeQ6K) return hipSuccess;
  uint32_t v = 1;
  const hipError_t e = hipMemcpy(&v, h.f16_flag, sizeof v, hipMemcpyDeviceToHost);
  h.f16_exact = e == hipSuccess && v == 0;
  return e;
}

// Uploads one weight.  With sync == false (device source only) the repack is
// left queued on the library stream; the caller synchronises before it
// reuses or frees the source, then calls read_f16_flag.
int32_t upload_common(int32_t type_id, const void *src, bool src_device, size_t weight_len, size_t input_size,
                      size_t row_count, uint64_t *out_handle, bool sync = true) {
  State &s = st();
  if (!out_handle || !src) return fail(HP_ERR_ARG, "null pointer");
  int32_t rc = ensure_init(s.ready ? s.device : 0);
  if (rc != HP_OK) return rc;
  if (input_size == 0 || row_count == 0) return fail(HP_ERR_SHAPE, "resident weight shape mismatch");
  if (type_id != kTypeQ4K && type_id != kTypeQ6K) return fail(HP_ERR_TYPE, "unsupported quantized type");
  const size_t rb = row_bytes_for(type_id, input_size);
  if (rb == 0) return fail(HP_ERR_TYPE, "input_size is not a multiple of 256");
  if (weight_len != sat_mul(rb, row_count)) return fail(HP_ERR_SHAPE, "weight byte length mismatch");
  if (row_count > (size_t)0x7fffffff / 64 || input_size / kQK > 4096) return fail(HP_ERR_SHAPE, "weight too large");

  if (src_device && reinterpret_cast<uintptr_t>(src) % 16 != 0)
    return fail(HP_ERR_ARG, "device weight buffer must be 16-byte aligned");
  Handle h;
  h.type = type_id;
  h.input_size = input_size;
  h.row_count = row_count;
  h.byte_length = weight_len;
  h.g = choose_geometry((int)(input_size / kQK));
  h.tiles = (int)((row_count + h.g.R - 1) / h.g.R);
  // one allocation: the tiles (+ Q6_K d plane), the segments unless the
  // weight is kept in one layout, then the repack's f16 flag
  const int nb = (int)(input_size / kQK);
  const size_t tile_bytes = (weight_len + 255) & ~(size_t)255;
  h.seg_bytes = s.both_layouts ? mfma_segment_bytes(type_id, (int)row_count, nb) : 0;
  if (hipMalloc((void **)&h.data, tile_bytes + h.seg_bytes + 256) != hipSuccess)
    return fail(HP_ERR_OOM, "weight allocation failed");
  if (s.both_layouts) h.segs = h.data + tile_bytes;
  h.f16_flag = reinterpret_cast<uint32_t *>(h.data + tile_bytes + h.seg_bytes);
  h.f16_exact = type_id != kTypeQ6K;  // Q6_K: read_f16_flag after the repack
  if (type_id == kTypeQ6K) h.dplane = reinterpret_cast<uint16_t *>(h.data + row_count * (input_size / kQK) * 208);

  const uint8_t *raw = static_cast<const uint8_t *>(src);
  uint8_t *staging = nullptr;
  if (!src_device) {
    if (hipMalloc((void **)&staging, weight_len) != hipSuccess) {
      (void)hipFree(h.data);
      return fail(HP_ERR_OOM, "staging allocation failed");
    }
    hipError_t e = hipMemcpyAsync(staging, src, weight_len, hipMemcpyHostToDevice, s.stream);
    if (e != hipSuccess) {
      (void)hipFree(staging);
      (void)hipFree(h.data);
      return hip_fail(e, "hipMemcpyAsync(weights)");
    }
    raw = staging;
  }
  hipError_t e = hipMemsetAsync(h.f16_flag, 0, sizeof(uint32_t), s.stream);
  if (e == hipSuccess) e = launch_repack(type_id, raw, (int)row_count, h.g, h.data, h.dplane, h.f16_flag, s.stream);
  if (e == hipSuccess && h.segs) e = launch_repack_mfma(type_id, raw, (int)row_count, nb, h.segs, s.stream);
  if (e == hipSuccess && (sync || !src_device)) e = hipStreamSynchronize(s.stream);
  if (staging) (void)hipFree(staging);
  if (e == hipSuccess && (sync || !src_device)) e = read_f16_flag(h);
  if (e != hipSuccess) {
    (void)hipStreamSynchronize(s.stream);
    (void)hipFree(h.data);
    return hip_fail(e, "repack");
  }
  // reuse a free slot
  size_t slot = s.handles.size();
  for (size_t i = 0; i < s.handles.size(); i++)
    if (!s.handles[i].live) {
      slot = i;
      break;
    }
  if (slot == s.handles.size()) s.handles.emplace_back();
  h.generation = s.handles[slot].generation + 1;
  h.live = true;
  s.handles[slot] = h;
  *out_handle = ((uint64_t)h.generation << 32) | (uint64_t)(slot + 1);
  return HP_OK;
}

// ---- GGUF -> HBM loader ----------------------------------------------------
// Tensor bytes go file -> pinned host chunk (pread) -> device staging
// (hipMemcpyAsync) -> repack into the resident layouts.  Readers work on
// interleaved chunks (chunk c on reader c % n), each with two pinned chunks
// and its own stream, so one chunk's DMA overlaps the next chunk's read.
constexpr size_t kLoadChunk = 8u << 20;
constexpr int kLoadMaxReaders = 8;
constexpr size_t kLoadBatch = 1ull << 30;  // device staging per batch of tensors

void release_loader(State &s) {
  for (hipStream_t q : s.copy_streams) (void)hipStreamDestroy(q);
  for (hipEvent_t e : s.copy_events) (void)hipEventDestroy(e);
  s.copy_streams.clear();
  s.copy_events.clear();
  if (s.pinned) (void)hipHostFree(s.pinned);
  s.pinned = nullptr;
  s.pinned_cap = 0;
  if (s.load_staging) (void)hipFree(s.load_staging);
  s.load_staging = nullptr;
  s.load_staging_cap = 0;
}

int load_readers() {
  const unsigned hw = std::thread::hardware_concurrency();
  const int n = hw == 0 ? 4 : (int)hw;
  return std::max(1, std::min(kLoadMaxReaders, n));
}

int32_t ensure_loader(State &s, int readers) {
  const size_t need = (size_t)readers * 2 * kLoadChunk;
  if (s.pinned_cap < need) {
    if (s.pinned) (void)hipHostFree(s.pinned);
    s.pinned = nullptr;
    s.pinned_cap = 0;
    HP_HIP_TRY(hipHostMalloc((void **)&s.pinned, need, hipHostMallocDefault));
    s.pinned_cap = need;
  }
  while ((int)s.copy_streams.size() < readers) {
    hipStream_t q;
    HP_HIP_TRY(hipStreamCreateWithFlags(&q, hipStreamNonBlocking));
    s.copy_streams.push_back(q);
  }
  while ((int)s.copy_events.size() < 2 * readers) {
    hipEvent_t e;
    HP_HIP_TRY(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    s.copy_events.push_back(e);
  }
  return HP_OK;
}

struct CopyJob {
  uint64_t file_offset;
  size_t length;
  uint8_t *dst;
};

// Copies every job's file range into device memory; returns once all copies
// have landed.  Jobs are cut into kLoadChunk pieces dealt round-robin.
int32_t stream_ranges(const hp_gguf_t *g, const std::vector<CopyJob> &jobs) {
  State &s = st();
  struct Piece {
    uint64_t off;
    size_t n;
    uint8_t *dst;
  };
  std::vector<Piece> pieces;
  for (const CopyJob &j : jobs)
    for (size_t done = 0; done < j.length; done += kLoadChunk)
      pieces.push_back({j.file_offset + done, std::min(kLoadChunk, j.length - done), j.dst + done});
  if (pieces.empty()) return HP_OK;
  const int readers = (int)std::min<size_t>((size_t)load_readers(), pieces.size());
  int32_t rc = ensure_loader(s, readers);
  if (rc != HP_OK) return rc;
  std::atomic<int32_t> status{HP_OK};
  std::mutex msg_mu;
  std::string msg;
  auto note = [&](int32_t code, const std::string &m) {
    int32_t ok = HP_OK;
    if (status.compare_exchange_strong(ok, code)) {
      std::lock_guard<std::mutex> lk(msg_mu);
      msg = m;
    }
  };
  auto reader = [&](int t) {
    hipStream_t q = s.copy_streams[t];
    bool used[2] = {false, false};
    for (size_t p = (size_t)t, round = 0; p < pieces.size(); p += (size_t)readers, round++) {
      if (status.load() != HP_OK) break;
      const int b = (int)(round & 1);
      hipEvent_t ev = s.copy_events[2 * t + b];
      uint8_t *buf = s.pinned + ((size_t)t * 2 + b) * kLoadChunk;
      if (used[b] && hipEventSynchronize(ev) != hipSuccess) {
        note(HP_ERR_HIP, "hipEventSynchronize(loader)");
        break;
      }
      if (hp_gguf_read(g, pieces[p].off, buf, pieces[p].n) != 0) {
        note(HP_ERR_IO, "read of " + std::to_string(pieces[p].n) + " bytes at offset " + std::to_string(pieces[p].off) +
                            " failed");
        break;
      }
      hipError_t e = hipMemcpyAsync(pieces[p].dst, buf, pieces[p].n, hipMemcpyHostToDevice, q);
      if (e == hipSuccess) e = hipEventRecord(ev, q);
      if (e != hipSuccess) {
        note(HP_ERR_HIP, std::string("hipMemcpyAsync(loader): ") + hipGetErrorString(e));
        break;
      }
      used[b] = true;
    }
    if (hipStreamSynchronize(q) != hipSuccess) note(HP_ERR_HIP, "hipStreamSynchronize(loader)");
  };
  std::vector<std::thread> pool;
  for (int t = 1; t < readers; t++) pool.emplace_back(reader, t);
  reader(0);
  for (std::thread &th : pool) th.join();
  if (status.load() != HP_OK) return fail(status.load(), msg);
  return HP_OK;
}

// ggml type id -> runner type id (lib.rs:12-17), 0 when the runner has none.
int32_t runner_type(uint32_t ggml) {
  switch (ggml) {
    case HP_GGML_Q4_K: return kTypeQ4K;
    case HP_GGML_Q6_K: return kTypeQ6K;
    default: return 0;
  }
}

// resolveGenerationSamplingOptions' checks (generation.ts:49-60) on the
// resolved options the entry points take.
int32_t sampling_check(const hp_hip_sampling_t *o, size_t k) {
  if (!o) return fail(HP_ERR_ARG, "null sampling options");
  if (!std::isfinite(o->temperature) || o->temperature < 0)
    return fail(HP_ERR_ARG, "temperature must be a finite number greater than or equal to 0.");
  if (!std::isfinite(o->top_p) || o->top_p <= 0 || o->top_p > 1)
    return fail(HP_ERR_ARG, "topP must be a finite number in the range (0, 1].");
  if (o->top_k < 1) return fail(HP_ERR_ARG, "topK must be a positive finite number.");
  if (k == 0 || k > 64) return fail(HP_ERR_ARG, "k must be in 1..64");
  return HP_OK;
}

SampleParams sample_params(const hp_hip_sampling_t *o) {
  SampleParams p;
  p.do_sample = o->do_sample ? 1 : 0;
  p.top_k = o->top_k;
  p.temperature = o->temperature;
  p.top_p = o->top_p;
  return p;
}

constexpr size_t kNormMaxN = 4096;

int32_t attention_check(const hp_hip_attention_config_t *c) {
  if (!c) return fail(HP_ERR_ARG, "null attention config");
  if (c->head_dim != kHeadDim) return fail(HP_ERR_SHAPE, "head_dim must be 256");
  if (c->head_count < 1 || c->head_count_kv < 1 || c->head_count % c->head_count_kv != 0 ||
      c->head_count / c->head_count_kv > kAttnMaxGroup)
    return fail(HP_ERR_HEADS, "head_count must be a multiple (at most 8x) of head_count_kv");
  if (c->rope_dims < 0 || c->rope_dims > kHeadDim || c->rope_dims % 2 != 0)
    return fail(HP_ERR_ARG, "rope_dims must be even and at most head_dim");
  if (c->rope_dims > 0 && !(c->rope_freq_base > 0.0 && std::isfinite(c->rope_freq_base)))
    return fail(HP_ERR_ARG, "rope_freq_base must be positive");
  if (c->capacity < 1 || c->sliding_window < 0) return fail(HP_ERR_ARG, "bad KV capacity or window");
  if (!(c->epsilon >= 0.0)) return fail(HP_ERR_ARG, "epsilon must be >= 0");
  return HP_OK;
}

QkvPostArgs qkv_post_args(const hp_hip_attention_config_t *c) {
  QkvPostArgs a{};
  a.nq = c->head_count;
  a.nkv = c->head_count_kv;
  a.capacity = c->capacity;
  a.rope_dims = c->rope_dims;
  // thetaScale = Math.pow(freqBase, -2 / nDims) (layers.ts:1013)
  a.theta_scale = c->rope_dims > 0 ? std::pow(c->rope_freq_base, -2.0 / (double)c->rope_dims) : 1.0;
  a.freq_factors = c->d_rope_freq_factors;
  a.eps = c->epsilon;
  a.tokens = 1;
  return a;
}

AttnArgs attn_args(const hp_hip_attention_config_t *c) {
  const QkvPostArgs p = qkv_post_args(c);
  AttnArgs a{};
  a.nq = c->head_count;
  a.nkv = c->head_count_kv;
  a.capacity = c->capacity;
  a.window = c->sliding_window;
  a.rope_dims = p.rope_dims;
  a.theta_scale = p.theta_scale;
  a.freq_factors = p.freq_factors;
  a.eps = p.eps;
  a.tokens = 1;
  return a;
}

int32_t run_attention(AttnArgs a, float *partials, hipStream_t stream) {
  hipEvent_t e = prof_begin(stream);
  HP_HIP_TRY(launch_attention(a, partials, stream));
  prof_end(HP_KERNEL_ATTENTION, e, stream);
  st().launches += 2;
  return HP_OK;
}

int32_t run_norm(const float *y, int rows, int n, const float *w_post, const float *x_res, float scale, float *x_out,
                 const float *w_next, float *next_out, double eps, hipStream_t stream, uint8_t *q8img,
                 uint8_t *xt, const PrefillParts *y_parts, bool next_image_only, bool x16) {
  NormArgs a{};
  a.x16 = x16 ? 1 : 0;
  a.q8img = q8img;
  a.xt = xt;
  a.next_image_only = next_image_only && (q8img || xt) ? 1 : 0;
  if (y_parts && y_parts->ks > 1) {
    // y is the projection's block-range partial sums
    a.y_ks = y_parts->ks;
    a.y_stride = y_parts->stride;
  }
  a.y = y;
  a.w_post = w_post;
  a.x_res = x_res;
  a.scale = scale;
  a.x_out = x_out;
  a.w_next = w_next;
  a.next_out = next_out;
  a.n = n;
  a.rows = rows;
  a.eps = eps;
  hipEvent_t e = prof_begin(stream);
  HP_HIP_TRY(launch_norm_residual(a, stream));
  prof_end(HP_KERNEL_NORM, e, stream);
  st().launches++;
  return HP_OK;
}

// Weights of one decode layer, looked up and checked against each other.
struct LayerHandles {
  Handle *q, *k, *v, *o, *gate, *up, *down;
  Handle *inp_gate, *proj;  // the per-layer input step, or null
};

int32_t decode_layer_check(const hp_hip_decode_layer_t &L, size_t hidden, LayerHandles *out) {
  int32_t rc = attention_check(&L.attention);
  if (rc != HP_OK) return rc;
  LayerHandles h{};
  h.q = lookup(L.attn_q);
  h.k = lookup(L.attn_k);
  h.v = L.attn_v ? lookup(L.attn_v) : nullptr;
  h.o = lookup(L.attn_output);
  h.gate = lookup(L.ffn_gate);
  h.up = lookup(L.ffn_up);
  h.down = lookup(L.ffn_down);
  if (!h.q || !h.k || (L.attn_v && !h.v) || !h.o || !h.gate || !h.up || !h.down)
    return fail(HP_ERR_HANDLE, "unknown weight handle in decode layer");
  const size_t qd = (size_t)L.attention.head_count * kHeadDim, kd = (size_t)L.attention.head_count_kv * kHeadDim;
  if (h.q->input_size != hidden || h.k->input_size != hidden || (h.v && h.v->input_size != hidden) ||
      h.q->row_count != qd || h.k->row_count != kd || (h.v && h.v->row_count != kd))
    return fail(HP_ERR_SHAPE, "attention projection shapes do not match the attention config");
  if (h.o->input_size != qd || h.o->row_count != hidden)
    return fail(HP_ERR_SHAPE, "attn_output shape mismatch");
  if (h.gate->input_size != hidden || h.up->input_size != hidden || h.gate->row_count != h.up->row_count ||
      h.down->input_size != h.gate->row_count || h.down->row_count != hidden)
    return fail(HP_ERR_SHAPE, "FFN shape mismatch");
  if (!L.d_attn_norm || !L.d_attn_q_norm || !L.d_attn_k_norm || !L.d_post_attention_norm || !L.d_ffn_norm ||
      !L.d_post_ffw_norm || !L.d_key_cache || !L.d_value_cache)
    return fail(HP_ERR_ARG, "null norm weight or cache in decode layer");
  if (L.reserved != 0) return fail(HP_ERR_ARG, "reserved field must be 0");
  if (L.inp_gate || L.proj) {
    h.inp_gate = lookup(L.inp_gate);
    h.proj = lookup(L.proj);
    if (!h.inp_gate || !h.proj) return fail(HP_ERR_HANDLE, "unknown per-layer input handle in decode layer");
    if (h.inp_gate->input_size != hidden || h.proj->row_count != hidden ||
        h.proj->input_size != h.inp_gate->row_count)
      return fail(HP_ERR_SHAPE, "per-layer input shape mismatch");
    if (!L.d_post_norm || !L.d_per_layer_input) return fail(HP_ERR_ARG, "null per-layer input or post_norm");
  }
  *out = h;
  return HP_OK;
}

int32_t topk_check(size_t rows, size_t n, size_t k) {
  if (k == 0 || k > 64) return fail(HP_ERR_ARG, "k must be in 1..64");
  if (n == 0 || n > 524288 || rows > 65535) return fail(HP_ERR_SHAPE, "topk supports 1..524288 values per row");
  return HP_OK;
}

// Enqueue top-k of device logits into device ids/values, in batches of
// kTopkMaxRows rows.  The selection scratch is zeroed when allocated; the
// kernels return their counters to zero, so later calls need no clearing
// (and a captured call records no memset).
int32_t run_topk(const float *d_logits, size_t rows, size_t n, size_t k, double cap, uint32_t *d_ids, float *d_vals,
                 hipStream_t stream) {
  State &s = st();
  const size_t batch = rows < (size_t)kTopkMaxRows ? rows : (size_t)kTopkMaxRows;
  const size_t bytes = topk_scratch_bytes((int)batch, (int)n, (int)k);
  void *sel = nullptr;
  int32_t rc = stream_scratch(stream, kScratchTopk, bytes, &sel, true);
  if (rc != HP_OK) return rc;
  hipEvent_t e = prof_begin(stream);
  for (size_t r0 = 0; r0 < rows; r0 += batch) {
    const size_t nr = rows - r0 < batch ? rows - r0 : batch;
    HP_HIP_TRY(launch_topk(d_logits + r0 * n, (int)nr, (int)n, (int)k, cap,
                           static_cast<uint8_t *>(sel), d_ids + r0 * k, d_vals + r0 * k, stream));
    s.launches += 3;
  }
  prof_end(HP_KERNEL_TOPK, e, stream);
  return HP_OK;
}

// Scratch for [rows][k] ids + values; returns device pointers.
int32_t topk_outputs(size_t rows, size_t k, uint32_t **ids, float **vals) {
  State &s = st();
  const size_t bytes = rows * k * 8;
  int32_t rc = grow(&s.topk_out, &s.topk_out_cap, bytes);
  if (rc != HP_OK) return rc;
  *ids = static_cast<uint32_t *>(s.topk_out);
  *vals = reinterpret_cast<float *>(static_cast<uint8_t *>(s.topk_out) + rows * k * 4);
  return HP_OK;
}

// ---- persistent decode step (decode_fused.hip) ------------------------

// The weights hs[0 .. count) (one input size) of a stage, their rows split
// over workgroups [wg0, wg0 + wgs): one segment per weight (gate/up: one,
// both weights' rows), workgroup counts in proportion to weight bytes.
// false: a workgroup's share would not fit the stage's per-thread task slots.
bool fused_proj(FusedProj &P, Handle *const *hs, int count, bool pair, int wg0, int wgs) {
  P = FusedProj{};
  const TileGeom g = hs[0]->g;
  P.count = count;
  P.pair = pair ? 1 : 0;
  P.nb = g.nb;
  P.S = g.S;
  P.R = g.R;
  P.mg_nb = div_magic(g.nb);
  P.mg_S = div_magic(g.S);
  P.mg_R = div_magic(g.R);
  int row = 0;
  for (int i = 0; i < 3; i++) {
    const Handle *h = hs[i < count ? i : 0];  // unused entries repeat weight 0 (offset 0)
    P.w[i].data = h->data;
    P.w[i].dplane = h->dplane;
    P.w[i].type = h->type;
    P.w[i].rows = (int)h->row_count;
    P.w[i].row_begin = i < count ? (pair ? 0 : row) : INT_MAX;
    if (i < count && !pair) row += (int)h->row_count;
  }
  P.out_rows = pair ? (int)hs[0]->row_count : row;
  auto slots_ok = [&](int type, int rpw) {
    const int tasks = (pair ? 2 : 1) * rpw * g.nb;
    return (tasks + kFusedThreads - 1) / kFusedThreads <= (type == kTypeQ4K ? kFusedSlotsQ4 : kFusedSlotsQ6);
  };
  if (pair) {
    const int rows = (int)hs[0]->row_count;
    const int rpw = (rows + wgs - 1) / wgs;
    P.nseg = 1;
    P.seg[0] = {0, rows, wg0, (rows + rpw - 1) / rpw, rpw, hs[0]->type};
    return slots_ok(hs[0]->type, rpw);
  }
  double total = 0;
  double bytes[3] = {0, 0, 0};
  for (int i = 0; i < count; i++) {
    bytes[i] = (double)hs[i]->row_count * (double)row_bytes_for(hs[i]->type, hs[i]->input_size);
    total += bytes[i];
  }
  int n[3] = {0, 0, 0}, sum = 0;
  for (int i = 0; i < count; i++) {
    n[i] = std::max(1, (int)((double)wgs * bytes[i] / total));
    sum += n[i];
  }
  while (sum > wgs) {  // trim the largest share
    int j = 0;
    for (int i = 1; i < count; i++)
      if (n[i] > n[j]) j = i;
    if (n[j] <= 1) return false;
    n[j]--;
    sum--;
  }
  P.nseg = count;
  int wg = wg0, rb = 0;
  for (int i = 0; i < count; i++) {
    const int rows = (int)hs[i]->row_count;
    const int rpw = (rows + n[i] - 1) / n[i];
    const int cnt = (rows + rpw - 1) / rpw;
    P.seg[i] = {rb, rows, wg, cnt, rpw, hs[i]->type};
    if (!slots_ok(hs[i]->type, rpw)) return false;
    wg += cnt;
    rb += rows;
  }
  return wg <= wg0 + wgs;
}

// The persistent step's layer table, exchange layout, LDS and kernel choice
// for these layers, or false when some layer is outside what it covers (the
// caller then runs the launch sequence).
struct FusedPlan {
  std::vector<FusedLayer> layers;
  FusedXchg x{};
  size_t lds = 0;
  int G = 0;
};

bool fused_plan(const hp_hip_decode_layer_t *layers, const std::vector<LayerHandles> &hs, size_t hidden,
                FusedPlan *out) {
  State &s = st();
  const int W = s.num_cus;
  if (W < 8 || hidden % kQK != 0 || hidden > 16 * (size_t)kQK || hs.size() > (size_t)kFusedMaxLayers) return false;
  FusedPlan p;
  p.layers.resize(hs.size());
  size_t qkv_max = 0, att_max = 0, ffn_max = 0, slots_max = 0;
  for (size_t i = 0; i < hs.size(); i++) {
    const hp_hip_decode_layer_t &Ls = layers[i];
    const LayerHandles &H = hs[i];
    const hp_hip_attention_config_t &c = Ls.attention;
    const int G = c.head_count / c.head_count_kv;
    if (i == 0) p.G = G;
    if (G != p.G || !fused_group_supported(G)) return false;
    if (c.rope_dims != 0 && c.rope_dims != 128 && c.rope_dims != kHeadDim) return false;  // RoPE pairs within a lane
    const int chunks = (c.capacity + kAttnChunk - 1) / kAttnChunk;
    if (chunks > 128 || c.head_count * 4 > 65535) return false;
    if (H.gate->type != H.up->type) return false;
    if (H.inp_gate) return false;  // the per-layer input step runs in the launch sequence
    FusedLayer &D = p.layers[i];
    D = FusedLayer{};
    Handle *qkv[3] = {H.q, H.k, H.v};
    if (!fused_proj(D.qkv, qkv, H.v ? 3 : 2, false, 0, W)) return false;
    // O skips the workgroups that merge attention (they finish that stage last)
    const int merge_wgs = c.head_count * 4;
    const int o0 = W - merge_wgs >= W / 2 ? merge_wgs : 0;
    Handle *o[1] = {H.o};
    if (!fused_proj(D.o, o, 1, false, o0, W - o0)) return false;
    Handle *gu[2] = {H.gate, H.up};
    if (!fused_proj(D.gu, gu, 2, true, 0, W)) return false;
    Handle *dn[1] = {H.down};
    if (!fused_proj(D.down, dn, 1, false, 0, W)) return false;
    D.attn_norm = Ls.d_attn_norm;
    D.q_norm = Ls.d_attn_q_norm;
    D.k_norm = Ls.d_attn_k_norm;
    D.post_attn_norm = Ls.d_post_attention_norm;
    D.ffn_norm = Ls.d_ffn_norm;
    D.post_ffw_norm = Ls.d_post_ffw_norm;
    const AttnArgs aa = attn_args(&c);
    D.freq_factors = aa.freq_factors;
    D.k_cache = reinterpret_cast<_Float16 *>(Ls.d_key_cache);
    D.v_cache = reinterpret_cast<_Float16 *>(Ls.d_value_cache);
    D.theta_scale = aa.theta_scale;
    D.eps = aa.eps;
    D.out_scale = Ls.layer_output_scale;
    D.nq = c.head_count;
    D.nkv = c.head_count_kv;
    D.capacity = c.capacity;
    D.window = c.sliding_window;
    D.rope_dims = c.rope_dims;
    D.chunks = chunks;
    D.k_off = (int)H.q->row_count;
    D.v_off = H.v ? (int)(H.q->row_count + H.k->row_count) : D.k_off;
    // layers with the same RoPE parameters share a key (the first such layer's index)
    D.rope_key = (int)i;
    for (size_t j = 0; j < i; j++) {
      const hp_hip_attention_config_t &cj = layers[j].attention;
      if (cj.rope_dims == c.rope_dims && cj.rope_freq_base == c.rope_freq_base &&
          cj.d_rope_freq_factors == c.d_rope_freq_factors) {
        D.rope_key = (int)j;
        break;
      }
    }
    qkv_max = std::max(qkv_max, (size_t)D.qkv.out_rows);
    att_max = std::max(att_max, (size_t)c.head_count * kHeadDim);
    ffn_max = std::max(ffn_max, H.gate->row_count);
    slots_max = std::max(slots_max, (size_t)c.head_count_kv * chunks * kAttnMaxGroup);
  }
  p.lds = fused_lds_bytes(p.layers.data(), (int)p.layers.size(), (int)hidden);
  if (p.lds == 0 || p.lds + fused_static_lds(p.G) > s.max_lds) return false;
  if (fused_blocks_per_cu(p.G, p.lds) < 1) return false;
  // the exchange arena (8 bytes per value; o right after hid, y right after x1)
  auto al = [](size_t b) { return (b + 255) & ~(size_t)255; };
  size_t off = 0;
  auto take = [&](size_t values) {
    const size_t o = off;
    off += al(values * 8);
    return (uint32_t)o;
  };
  p.x.hid = take(hidden);
  p.x.o = take(hidden);
  p.x.x1 = take(hidden);
  p.x.y = take(hidden);
  p.x.qkv = take(qkv_max);
  p.x.att = take(att_max);
  p.x.h = take(ffn_max);
  p.x.part_slots = (uint32_t)slots_max;
  p.x.part = take(slots_max * (kHeadDim + 2));
  p.x.total = (uint32_t)off;
  if (p.x.o != p.x.hid + hidden * 8 || p.x.y != p.x.x1 + hidden * 8 || off >= (1u << 31)) return false;
  *out = std::move(p);
  return true;
}

// The device copy of a layer table (uploaded once per distinct content).
int32_t fused_table(const std::vector<FusedLayer> &layers, hipStream_t stream, const FusedLayer **out) {
  State &s = st();
  constexpr size_t kDesc = 1024;
  std::vector<uint8_t> bytes(layers.size() * kDesc, 0);
  for (size_t i = 0; i < layers.size(); i++) std::memcpy(bytes.data() + i * kDesc, &layers[i], sizeof(FusedLayer));
  auto it = s.fused_tables.find(bytes);
  if (it != s.fused_tables.end()) {
    *out = static_cast<const FusedLayer *>(it->second);
    return HP_OK;
  }
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &cs) != hipSuccess) cs = hipStreamCaptureStatusNone;
  if (cs != hipStreamCaptureStatusNone)
    return fail(HP_ERR_ARG, "decode layers: a captured call must follow an uncaptured call with the same layers");
  void *d = nullptr;
  if (hipMalloc(&d, bytes.size()) != hipSuccess) return fail(HP_ERR_OOM, "device allocation failed");
  if (hipMemcpyAsync(d, bytes.data(), bytes.size(), hipMemcpyHostToDevice, stream) != hipSuccess ||
      hipStreamSynchronize(stream) != hipSuccess) {
    (void)hipFree(d);
    return fail(HP_ERR_HIP, "uploading the decode layer table failed");
  }
  s.fused_tables.emplace(std::move(bytes), d);
  *out = static_cast<const FusedLayer *>(d);
  return HP_OK;
}

// Enqueue the persistent step for one token through every layer.
int32_t run_fused(const FusedPlan &p, size_t hidden, float *d_hidden, const int32_t *d_position,
                  const float *d_output_norm, float *d_output, hipStream_t strm) {
  State &s = st();
  const FusedLayer *table = nullptr;
  int32_t rc = fused_table(p.layers, strm, &table);
  if (rc != HP_OK) return rc;
  void *arena = nullptr;
  rc = stream_scratch(strm, kScratchFused, sizeof(FusedCtl) + p.x.total, &arena, true);
  if (rc != HP_OK) return rc;
  FusedArgs a{};
  a.layers = table;
  a.n_layers = (int)p.layers.size();
  a.hidden_n = (int)hidden;
  a.hidden = d_hidden;
  a.out_norm = d_output_norm;
  a.out = d_output;
  a.position = d_position;
  a.ctl = static_cast<FusedCtl *>(arena);
  a.xchg = static_cast<uint8_t *>(arena) + sizeof(FusedCtl);
  a.xchg_bytes = p.x.total;
  a.gelu_lut = s.gelu_lut;
  a.spin_ticks = s.fused_spin;
  a.x = p.x;
  a.G = p.G;
  a.lds_bytes = (int)p.lds;
  const size_t stamps = (size_t)s.num_cus * p.layers.size() * 6 * 8;
  a.trace = s.fused_trace && s.fused_trace_len >= stamps ? s.fused_trace : nullptr;
  hipEvent_t e = prof_begin(strm);
  HP_HIP_TRY(launch_decode_fused(a, s.num_cus, strm));
  prof_end(HP_KERNEL_MATVEC, e, strm);
  s.launches++;
  return HP_OK;
}

}  // namespace

extern "C" {

const char *hp_hip_status_string(int32_t status) {
  switch (status) {
    case HP_OK: return "ok";
    case HP_ERR_SHAPE: return "shape mismatch";
    case HP_ERR_HEADS: return "head count mismatch";
    case HP_ERR_TYPE: return "unsupported type";
    case HP_ERR_HIP: return "HIP runtime error";
    case HP_ERR_HANDLE: return "unknown weight handle";
    case HP_ERR_ARG: return "invalid argument";
    case HP_ERR_NODEV: return "no GPU available";
    case HP_ERR_OOM: return "device out of memory";
    case HP_ERR_FORMAT: return "malformed GGUF";
    case HP_ERR_IO: return "file read error";
    default: return "unknown status";
  }
}

const char *hp_hip_last_error(void) { return g_last_error.c_str(); }

int32_t hp_hip_init(int32_t device) {
  State &s = st();
  std::lock_guard<std::recursive_mutex> lock(s.mu);
  if (s.ready && s.device != device) return fail(HP_ERR_ARG, "already initialised on another device");
  return ensure_init(device);
}

int32_t hp_hip_device_count(int32_t *count) {
  if (!count) return fail(HP_ERR_ARG, "null pointer");
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) n = 0;
  *count = n;
  return HP_OK;
}

int32_t hp_hip_shutdown(void) {
  State &s = st();
  std::lock_guard<std::recursive_mutex> lock(s.mu);
  if (!s.ready) return HP_OK;
  (void)hipStreamSynchronize(s.stream);
  for (auto &h : s.handles)
    if (h.live) {
      (void)hipFree(h.data);  // both layouts
      h.live = false;
    }
  if (s.io_in) (void)hipFree(s.io_in);
  s.io_in = nullptr;
  s.io_in_cap = 0;
  for (int i = 0; i < kMaxWeights; i++) {
    if (s.io_out[i]) (void)hipFree(s.io_out[i]);
    s.io_out[i] = nullptr;
    s.io_out_cap[i] = 0;
  }
  if (s.topk_out) (void)hipFree(s.topk_out);
  if (s.gelu_lut) (void)hipFree(s.gelu_lut);
  s.gelu_lut = nullptr;
  if (s.sample_out) (void)hipFree(s.sample_out);
  s.sample_out = nullptr;
  s.sample_out_cap = 0;
  s.topk_out = nullptr;
  s.topk_out_cap = 0;
  (void)hipDeviceSynchronize();
  s.pool.release_all();
  for (auto &kv : s.fused_tables) (void)hipFree(kv.second);
  s.fused_tables.clear();
  for (auto &kv : s.dev_bufs) (void)hipFree(reinterpret_cast<void *>(kv.first));
  s.dev_bufs.clear();
  prof_collect();
  for (hipEvent_t e : s.event_pool) (void)hipEventDestroy(e);
  s.event_pool.clear();
  release_loader(s);
  (void)hipStreamDestroy(s.stream);
  s.stream = nullptr;
  s.static_scratch = nullptr;
  s.ready = false;
  return HP_OK;
}

int32_t hp_hip_weight_upload(int32_t type_id, const uint8_t *weight, size_t weight_len, size_t input_size,
                             size_t row_count, uint64_t *out_handle) {
  std::lock_guard<std::recursive_mutex> lock(st().mu);
  return upload_common(type_id, weight, false, weight_len, input_size, row_count, out_handle);
}

int32_t hp_hip_weight_upload_device(int32_t type_id, const void *d_weight, size_t weight_len, size_t input_size,
                                    size_t row_count, uint64_t *out_handle) {
  std::lock_guard<std::recursive_mutex> lock(st().mu);
  return upload_common(type_id, d_weight, true, weight_len, input_size, row_count, out_handle);
}

int32_t hp_hip_weight_upload_gguf(const hp_gguf_t *g, size_t count, const uint64_t *tensor_indices,
                                  uint64_t *handles, int32_t *statuses) {
  State &s = st();
  std::lock_guard<std::recursive_mutex> lock(s.mu);
  if (!g || (count && (!tensor_indices || !handles || !statuses))) return fail(HP_ERR_ARG, "null pointer");
  int32_t rc = ensure_init(s.ready ? s.device : 0);
  if (rc != HP_OK) return rc;
  uint64_t tensor_count = 0, file_size = 0;
  hp_gguf_header(g, nullptr, &tensor_count, nullptr, nullptr, nullptr, &file_size);
  // validate everything first: the call uploads all or nothing
  std::vector<hp_gguf_tensor_t> info(count);
  for (size_t i = 0; i < count; i++) {
    handles[i] = 0;
    statuses[i] = HP_ERR_TYPE;
    if (tensor_indices[i] >= tensor_count) return fail(HP_ERR_ARG, "tensor index out of range");
    hp_gguf_tensor_info(g, tensor_indices[i], &info[i]);
    const hp_gguf_tensor_t &t = info[i];
    const int32_t type = runner_type(t.type_id);
    if (type == 0) continue;  // the caller falls back, as for createWasmQuantizedWeightHandle -> undefined
    const std::string name(t.name, t.name_length);
    const size_t input_size = t.n_dims >= 1 ? t.dims[0] : 0, rows = t.n_dims >= 2 ? t.dims[1] : 0;
    const size_t rb = row_bytes_for(type, input_size);
    if (t.n_dims < 2 || !t.storage_known || rb == 0 || t.byte_length != sat_mul(rb, rows))
      return fail(HP_ERR_SHAPE, "tensor " + name + " is not a [rows][input] weight of whole blocks");
    if (t.data_offset > file_size || t.byte_length > file_size - t.data_offset)
      return fail(HP_ERR_IO, "tensor " + name + " data runs past the end of the file");
    statuses[i] = HP_OK;
  }
  // batches of tensors whose bytes fit the device staging (a larger tensor goes alone)
  size_t begin = 0;
  while (begin < count) {
    size_t end = begin, bytes = 0;
    while (end < count && (statuses[end] != HP_OK || bytes == 0 || bytes + info[end].byte_length <= kLoadBatch)) {
      if (statuses[end] == HP_OK) bytes += (bytes % 256 ? 256 - bytes % 256 : 0) + info[end].byte_length;
      end++;
    }
    if (bytes > 0) {
      rc = grow((void **)&s.load_staging, &s.load_staging_cap, bytes);
      std::vector<CopyJob> jobs;
      std::vector<size_t> at(end - begin);
      size_t off = 0;
      for (size_t i = begin; i < end && rc == HP_OK; i++) {
        if (statuses[i] != HP_OK) continue;
        off = (off + 255) & ~(size_t)255;
        at[i - begin] = off;
        jobs.push_back({info[i].data_offset, (size_t)info[i].byte_length, s.load_staging + off});
        off += info[i].byte_length;
      }
      if (rc == HP_OK) rc = stream_ranges(g, jobs);
      for (size_t i = begin; i < end && rc == HP_OK; i++) {
        if (statuses[i] != HP_OK) continue;
        const hp_gguf_tensor_t &t = info[i];
        rc = upload_common(runner_type(t.type_id), s.load_staging + at[i - begin], true, t.byte_length, t.dims[0],
                           t.dims[1], &handles[i], false);
      }
      // the next batch overwrites the staging the queued repacks read
      if (rc == HP_OK && hipStreamSynchronize(s.stream) != hipSuccess) rc = fail(HP_ERR_HIP, "repack (GGUF load)");
      for (size_t i = begin; i < end && rc == HP_OK; i++) {
        Handle *h = handles[i] ? lookup(handles[i]) : nullptr;
        if (h && read_f16_flag(*h) != hipSuccess) rc = fail(HP_ERR_HIP, "repack flag (GGUF load)");
      }
    }
    if (rc != HP_OK) {
      const std::string why = g_last_error;
      (void)hipStreamSynchronize(s.stream);
      for (size_t i = 0; i < count; i++)
        if (handles[i]) {
          Handle *h = lookup(handles[i]);
          if (h) {
            (void)hipFree(h->data);
            h->data = h->segs = nullptr;
            h->dplane = nullptr;
            h->f16_flag = nullptr;
            h->live = false;
          }
          handles[i] = 0;
        }
      release_loader(s);
      return fail(rc, why);
    }
    begin = end;
  }
  release_loader(s);  // staging is only needed while loading
  return HP_OK;
}

int32_t hp_hip_weight_release(uint64_t handle) {
  State &s = st();
  std::lock_guard<std::recursive_mutex> lock(s.mu);
  Handle *h = lookup(handle);
  if (!h) return fail(HP_ERR_HANDLE, "unknown weight handle");
  (void)hipStreamSynchronize(s.stream);
  (void)hipFree(h->data);  // every layout of the weight
  h->data = nullptr;
  h->segs = nullptr;
  h->dplane = nullptr;
  h->f16_flag = nullptr;
  h->live = false;
  return HP_OK;
}

int32_t hp_hip_weight_info(uint64_t handle, int32_t *type_id, size_t *input_size, size_t *row_count,
                           size_t *byte_length) {
  std::lock_guard<std::recursive_mutex> lock(st().mu);
  Handle *h = lookup(handle);
  if (!h) return fail(HP_ERR_HANDLE, "unknown weight handle");
  if (type_id) *type_id = h->type;
  if (input_size) *input_size = h->input_size;
  if (row_count) *row_count = h->row_count;
  if (byte_length) *byte_length = h->byte_length;
  return HP_OK;
}

int32_t hp_hip_matmul_multi_device(size_t count, const uint64_t *handles, const float *d_input, size_t input_len,
                                   size_t input_size, size_t column_count, float *const *d_outputs,
                                   const size_t *output_lens, void *stream) {
  State &s = st();
  std::lock_guard<std::recursive_mutex> lock(s.mu);
  int32_t rc = ensure_init(s.ready ? s.device : 0);
  if (rc != HP_OK) return rc;
  if (count == 0 || count > (size_t)kMaxWeights || input_len != sat_mul(input_size, column_count))
    return fail(HP_ERR_SHAPE, "multi matmul shape mismatch");
  if (!handles || !output_lens || !d_outputs || (column_count && !d_input)) return fail(HP_ERR_ARG, "null pointer");
  Handle *hs[kMaxWeights];
  for (size_t i = 0; i < count; i++) {
    hs[i] = lookup(handles[i]);
    if (!hs[i]) return fail(HP_ERR_HANDLE, "unknown weight handle");
    if (hs[i]->input_size != input_size) return fail(HP_ERR_SHAPE, "handle input size mismatch");
    if (output_lens[i] != sat_mul(hs[i]->row_count, column_count))
      return fail(HP_ERR_SHAPE, "output length mismatch");
    if (column_count && !d_outputs[i]) return fail(HP_ERR_ARG, "null output");
  }
  if (reinterpret_cast<uintptr_t>(d_input) % 16 != 0) return fail(HP_ERR_ARG, "input must be 16-byte aligned");
  hipStream_t strm = stream ? static_cast<hipStream_t>(stream) : s.stream;
  return run_matvec(count, hs, d_input, input_size, column_count, d_outputs, strm);
}

int32_t hp_hip_matmul_multi(size_t count, const uint64_t *handles, const float *input, size_t input_len,
                            size_t input_size, size_t column_count, float *const *outputs,
                            const size_t *output_lens) {
  State &s = st();
  std::lock_guard<std::recursive_mutex> lock(s.mu);
  HostExactScope exact;
  int32_t rc = ensure_init(s.ready ? s.device : 0);
  if (rc != HP_OK) return rc;
  if (count == 0 || count > (size_t)kMaxWeights || input_len != sat_mul(input_size, column_count))
    return fail(HP_ERR_SHAPE, "multi matmul shape mismatch");
  if (!handles || !output_lens || !outputs || (column_count && !input)) return fail(HP_ERR_ARG, "null pointer");
  Handle *hs[kMaxWeights];
  for (size_t i = 0; i < count; i++) {
    hs[i] = lookup(handles[i]);
    if (!hs[i]) return fail(HP_ERR_HANDLE, "unknown weight handle");
    if (hs[i]->input_size != input_size) return fail(HP_ERR_SHAPE, "handle input size mismatch");
    if (output_lens[i] != sat_mul(hs[i]->row_count, column_count))
      return fail(HP_ERR_SHAPE, "output length mismatch");
    if (column_count && !outputs[i]) return fail(HP_ERR_ARG, "null output");
  }
  if (column_count == 0) return HP_OK;
  rc = grow((void **)&s.io_in, &s.io_in_cap, input_len * sizeof(float));
  if (rc != HP_OK) return rc;
  float *douts[kMaxWeights];
  for (size_t i = 0; i < count; i++) {
    rc = grow((void **)&s.io_out[i], &s.io_out_cap[i], output_lens[i] * sizeof(float));
    if (rc != HP_OK) return rc;
    douts[i] = s.io_out[i];
  }
  HP_HIP_TRY(hipMemcpyAsync(s.io_in, input, input_len * sizeof(float), hipMemcpyHostToDevice, s.stream));
  rc = run_matvec(count, hs, s.io_in, input_size, column_count, douts, s.stream);
  if (rc != HP_OK) return rc;
  for (size_t i = 0; i < count; i++)
    HP_HIP_TRY(hipMemcpyAsync(outputs[i], douts[i], output_lens[i] * sizeof(float), hipMemcpyDeviceToHost, s.stream));
  HP_HIP_TRY(hipStreamSynchronize(s.stream));
  return HP_OK;
}

int32_t hp_hip_matmul(uint64_t handle, const float *input, size_t input_len, size_t input_size, size_t row_count,
                      size_t column_count, float *output, size_t output_len) {
  State &s = st();
  std::lock_guard<std::recursive_mutex> lock(s.mu);
  Handle *h = lookup(handle);
  if (!h) return fail(HP_ERR_HANDLE, "unknown weight handle");
  if (h->input_size != input_size || h->row_count != row_count)
    return fail(HP_ERR_SHAPE, "resident handle shape mismatch");
  if (input_len != sat_mul(input_size, column_count) || output_len != sat_mul(row_count, column_count))
    return fail(HP_ERR_SHAPE, "matmul shape mismatch");
  float *outs[1] = {output};
  size_t lens[1] = {output_len};
  return hp_hip_matmul_multi(1, &handle, input, input_len, input_size, column_count, outs, lens);
}

int32_t hp_hip_dequantize(uint64_t handle, size_t row_start, size_t row_count, float *output, size_t output_len) {
  State &s = st();
  std::lock_guard<std::recursive_mutex> lock(s.mu);
  Handle *h = lookup(handle);
  if (!h) return fail(HP_ERR_HANDLE, "unknown weight handle");
  if (!output && row_count) return fail(HP_ERR_ARG, "null pointer");
  if (row_start > h->row_count || row_count > h->row_count - row_start ||
      output_len != sat_mul(row_count, h->input_size))
    return fail(HP_ERR_SHAPE, "dequantize range mismatch");
  if (row_count == 0) return HP_OK;
  float *d = nullptr;
  if (hipMalloc((void **)&d, output_len * sizeof(float)) != hipSuccess) return fail(HP_ERR_OOM, "dequant buffer");
  hipError_t e = launch_dequantize(h->type, h->data, h->dplane, (int)h->row_count, h->g, (int)row_start,
                                   (int)row_count, d, s.stream);
  if (e == hipSuccess) e = hipMemcpyAsync(output, d, output_len * sizeof(float), hipMemcpyDeviceToHost, s.stream);
  if (e == hipSuccess) e = hipStreamSynchronize(s.stream);
  (void)hipFree(d);
  if (e != hipSuccess) return hip_fail(e, "dequantize");
  return HP_OK;
}

int32_t hp_hip_topk_device(const float *d_logits, size_t rows, size_t n, size_t k, double softcap,
                           uint32_t *d_ids, float *d_values, void *stream) {
  State &s = st();
  std::lock_guard<std::recursive_mutex> lock(s.mu);
  int32_t rc = ensure_init(s.ready ? s.device : 0);
  if (rc != HP_OK) return rc;
  rc = topk_check(rows, n, k);
  if (rc != HP_OK) return rc;
  if (rows == 0) return HP_OK;
  if (!d_logits || !d_ids || !d_values) return fail(HP_ERR_ARG, "null pointer");
  hipStream_t strm = stream ? static_cast<hipStream_t>(stream) : s.stream;
  return run_topk(d_logits, rows, n, k, softcap, d_ids, d_values, strm);
}

int32_t hp_hip_topk_device_noalloc(const float *d_logits, size_t rows, size_t n, size_t k, double softcap,
                                   uint32_t *d_ids, float *d_values, void *stream) {
  State &s = st();
  std::lock_guard<std::recursive_mutex> lock(s.mu);
  if (!s.ready || !s.static_scratch)
    return fail(HP_ERR_ARG, "hp_hip_init must run before hp_hip_topk_device_noalloc");
  int32_t rc = topk_check(rows, n, k);
  if (rc != HP_OK) return rc;
  if (rows == 0) return HP_OK;
  if (!d_logits || !d_ids || !d_values) return fail(HP_ERR_ARG, "null pointer");
  const size_t batch = rows < (size_t)kTopkMaxRows ? rows : (size_t)kTopkMaxRows;
  if (topk_scratch_bytes((int)batch, (int)n, (int)k) > kNoAllocScratchBytes)
    return fail(HP_ERR_SHAPE, "top-k selection state exceeds the static scratch of " +
                                  std::to_string(kNoAllocScratchBytes) + " bytes");
  hipStream_t strm = stream ? static_cast<hipStream_t>(stream) : s.stream;
  // the array keeps the last call's contents: its counters start at zero here
  HP_HIP_TRY(launch_topk_clear(s.static_scratch, strm));
  s.launches++;
  for (size_t r0 = 0; r0 < rows; r0 += batch) {
    const size_t nr = rows - r0 < batch ? rows - r0 : batch;
    HP_HIP_TRY(launch_topk(d_logits + r0 * n, (int)nr, (int)n, (int)k, softcap, s.static_scratch, d_ids + r0 * k,
                           d_values + r0 * k, strm));
    s.launches += 3;
  }
  return HP_OK;
}

int32_t hp_hip_topk(const float *logits, size_t rows, size_t n, size_t k, double softcap, uint32_t *ids,
                    float *values, size_t out_len) {
  State &s = st();
  std::lock_guard<std::recursive_mutex> lock(s.mu);
  int32_t rc = ensure_init(s.ready ? s.device : 0);
  if (rc != HP_OK) return rc;
  rc = topk_check(rows, n, k);
  if (rc != HP_OK) return rc;
  if (out_len != sat_mul(rows, k)) return fail(HP_ERR_SHAPE, "topk output length mismatch");
  if (rows == 0) return HP_OK;
  if (!logits || !ids || !values) return fail(HP_ERR_ARG, "null pointer");
  rc = grow((void **)&s.io_in, &s.io_in_cap, rows * n * sizeof(float));
  if (rc != HP_OK) return rc;
  uint32_t *d_ids;
  float *d_vals;
  rc = topk_outputs(rows, k, &d_ids, &d_vals);
  if (rc != HP_OK) return rc;
  HP_HIP_TRY(hipMemcpyAsync(s.io_in, logits, rows * n * sizeof(float), hipMemcpyHostToDevice, s.stream));
  rc = run_topk(s.io_in, rows, n, k, softcap, d_ids, d_vals, s.stream);
  if (rc != HP_OK) return rc;
  HP_HIP_TRY(hipMemcpyAsync(ids, d_ids, rows * k * 4, hipMemcpyDeviceToHost, s.stream));
  HP_HIP_TRY(hipMemcpyAsync(values, d_vals, rows * k * 4, hipMemcpyDeviceToHost, s.stream));
  HP_HIP_TRY(hipStreamSynchronize(s.stream));
  return HP_OK;
}

int32_t hp_hip_matmul_topk(uint64_t handle, const float *input, size_t input_len, size_t input_size,
                           size_t column_count, size_t k, double softcap, uint32_t *ids, float *values,
                           size_t out_len) {
  State &s = st();
  std::lock_guard<std::recursive_mutex> lock(s.mu);
  HostExactScope exact;
  Handle *h = lookup(handle);
  if (!h) return fail(HP_ERR_HANDLE, "unknown weight handle");
  if (h->input_size != input_size || input_len != sat_mul(input_size, column_count))
    return fail(HP_ERR_SHAPE, "matmul shape mismatch");
  int32_t rc = topk_check(column_count, h->row_count, k);
  if (rc != HP_OK) return rc;
  if (out_len != sat_mul(column_count, k)) return fail(HP_ERR_SHAPE, "topk output length mismatch");
  if (column_count == 0) return HP_OK;
  if (!input || !ids || !values) return fail(HP_ERR_ARG, "null pointer");
  rc = grow((void **)&s.io_in, &s.io_in_cap, input_len * sizeof(float));
  if (rc != HP_OK) return rc;
  rc = grow((void **)&s.io_out[0], &s.io_out_cap[0], column_count * h->row_count * sizeof(float));
  if (rc != HP_OK) return rc;
  uint32_t *d_ids;
  float *d_vals;
  rc = topk_outputs(column_count, k, &d_ids, &d_vals);
  if (rc != HP_OK) return rc;
  HP_HIP_TRY(hipMemcpyAsync(s.io_in, input, input_len * sizeof(float), hipMemcpyHostToDevice, s.stream));
  float *logits = s.io_out[0];
  rc = run_matvec(1, &h, s.io_in, input_size, column_count, &logits, s.stream);
  if (rc != HP_OK) return rc;
  rc = run_topk(logits, column_count, h->row_count, k, softcap, d_ids, d_vals, s.stream);
  if (rc != HP_OK) return rc;
  HP_HIP_TRY(hipMemcpyAsync(ids, d_ids, column_count * k * 4, hipMemcpyDeviceToHost, s.stream));
  HP_HIP_TRY(hipMemcpyAsync(values, d_vals, column_count * k * 4, hipMemcpyDeviceToHost, s.stream));
  HP_HIP_TRY(hipStreamSynchronize(s.stream));
  return HP_OK;
}

int32_t hp_hip_sample_device(const uint32_t *d_ids, const float *d_values, size_t column_count, size_t k,
                             size_t count, const hp_hip_sampling_t *sampling, uint32_t *d_rng_state,
                             int32_t *d_tokens, double *d_probabilities, int32_t *d_kept, void *stream) {
  State &s = st();
  std::lock_guard<std::recursive_mutex> lock(s.mu);
  int32_t rc = ensure_init(s.ready ? s.device : 0);
  if (rc != HP_OK) return rc;
  rc = sampling_check(sampling, k);
  if (rc != HP_OK) return rc;
  if (count == 0 || count > k) return fail(HP_ERR_ARG, "count must be in 1..k");
  if (column_count == 0) return HP_OK;
  if (column_count > 65535) return fail(HP_ERR_SHAPE, "too many columns");
  if (!d_ids || !d_values || !d_rng_state || !d_tokens || !d_probabilities || !d_kept)
    return fail(HP_ERR_ARG, "null pointer");
  hipStream_t q = stream ? static_cast<hipStream_t>(stream) : s.stream;
  hipEvent_t e = prof_begin(q);
  HP_HIP_TRY(launch_sample(d_ids, d_values, (int)column_count, (int)k, (int)count, sample_params(sampling), d_rng_state,
                           d_tokens, d_probabilities, d_kept, q));
  prof_end(HP_KERNEL_SAMPLE, e, q);
  s.launches++;
  return HP_OK;
}

namespace {
// The head over a device input already ordered on s.stream, top-k of each
// column and, with `sampling`, the sampled token: candidates, tokens,
// probabilities and the advanced generator state copied back; returns once
// they are on the host.
int32_t head_candidates(Handle *h, const float *d_input, size_t input_size, size_t column_count, size_t k,
                        double softcap, const hp_hip_sampling_t *sampling, uint32_t *rng_state, int32_t *tokens,
                        uint32_t *ids, float *values, double *probabilities, int32_t *kept) {
  State &s = st();
  int32_t rc = grow((void **)&s.io_out[0], &s.io_out_cap[0], column_count * h->row_count * sizeof(float));
  uint32_t *d_ids = nullptr;
  float *d_vals = nullptr;
  if (rc == HP_OK) rc = topk_outputs(column_count, k, &d_ids, &d_vals);
  // rng state (16 B slot), tokens, kept, probabilities
  const size_t probs_off = (16 + column_count * 8 + 15) & ~(size_t)15;
  if (rc == HP_OK && sampling) rc = grow(&s.sample_out, &s.sample_out_cap, probs_off + column_count * k * sizeof(double));
  if (rc != HP_OK) return rc;
  float *logits = s.io_out[0];
  rc = run_matvec(1, &h, d_input, input_size, column_count, &logits, s.stream);
  if (rc != HP_OK) return rc;
  rc = run_topk(logits, column_count, h->row_count, k, softcap, d_ids, d_vals, s.stream);
  if (rc != HP_OK) return rc;
  if (sampling) {
    uint8_t *base = static_cast<uint8_t *>(s.sample_out);
    uint32_t *d_rng = reinterpret_cast<uint32_t *>(base);
    int32_t *d_tokens = reinterpret_cast<int32_t *>(base + 16);
    int32_t *d_kept = d_tokens + column_count;
    double *d_probs = reinterpret_cast<double *>(base + probs_off);
    HP_HIP_TRY(hipMemcpyAsync(d_rng, rng_state, 4, hipMemcpyHostToDevice, s.stream));
    const size_t count = h->row_count < k ? h->row_count : k;
    HP_HIP_TRY(launch_sample(d_ids, d_vals, (int)column_count, (int)k, (int)count, sample_params(sampling), d_rng,
                             d_tokens, d_probs, d_kept, s.stream));
    s.launches++;
    HP_HIP_TRY(hipMemcpyAsync(tokens, d_tokens, column_count * 4, hipMemcpyDeviceToHost, s.stream));
    HP_HIP_TRY(hipMemcpyAsync(kept, d_kept, column_count * 4, hipMemcpyDeviceToHost, s.stream));
    HP_HIP_TRY(hipMemcpyAsync(probabilities, d_probs, column_count * k * 8, hipMemcpyDeviceToHost, s.stream));
    HP_HIP_TRY(hipMemcpyAsync(rng_state, d_rng, 4, hipMemcpyDeviceToHost, s.stream));
  }
  HP_HIP_TRY(hipMemcpyAsync(ids, d_ids, column_count * k * 4, hipMemcpyDeviceToHost, s.stream));
  HP_HIP_TRY(hipMemcpyAsync(values, d_vals, column_count * k * 4, hipMemcpyDeviceToHost, s.stream));
  HP_HIP_TRY(hipStreamSynchronize(s.stream));
  return HP_OK;
}

// The allocation [base, base + bytes) of hp_hip_device_alloc that holds
// [p, p + n), or false.
bool in_device_buffer(const void *p, size_t n) {
  const State &s = st();
  const uintptr_t a = reinterpret_cast<uintptr_t>(p);
  auto it = s.dev_bufs.upper_bound(a);
  if (it == s.dev_bufs.begin()) return false;
  --it;
  return a >= it->first && n <= it->second && a - it->first <= it->second - n;
}
}  // namespace

int32_t hp_hip_matmul_topk_sample(uint64_t handle, const float *input, size_t input_len, size_t input_size,
                                  size_t column_count, size_t k, double softcap, const hp_hip_sampling_t *sampling,
                                  uint32_t *rng_state, int32_t *tokens, uint32_t *ids, float *values,
                                  double *probabilities, int32_t *kept, size_t out_len) {
  State &s = st();
  std::lock_guard<std::recursive_mutex> lock(s.mu);
  HostExactScope exact;
  Handle *h = lookup(handle);
  if (!h) return fail(HP_ERR_HANDLE, "unknown weight handle");
  if (h->input_size != input_size || input_len != sat_mul(input_size, column_count))
    return fail(HP_ERR_SHAPE, "matmul shape mismatch");
  int32_t rc = topk_check(column_count, h->row_count, k);
  if (rc != HP_OK) return rc;
  rc = sampling_check(sampling, k);
  if (rc != HP_OK) return rc;
  if (out_len != sat_mul(column_count, k)) return fail(HP_ERR_SHAPE, "topk output length mismatch");
  if (column_count == 0) return HP_OK;
  if (!input || !rng_state || !tokens || !ids || !values || !probabilities || !kept)
    return fail(HP_ERR_ARG, "null pointer");
  rc = grow((void **)&s.io_in, &s.io_in_cap, input_len * sizeof(float));
  if (rc != HP_OK) return rc;
  HP_HIP_TRY(hipMemcpyAsync(s.io_in, input, input_len * sizeof(float), hipMemcpyHostToDevice, s.stream));
  return head_candidates(h, s.io_in, input_size, column_count, k, softcap, sampling, rng_state, tokens, ids, values,
                         probabilities, kept);
}

int32_t hp_hip_matmul_topk_sample_device(uint64_t handle, const float *d_input, size_t input_len, size_t input_size,
                                         size_t column_count, size_t k, double softcap,
                                         const hp_hip_sampling_t *sampling, uint32_t *rng_state, int32_t *tokens,
                                         uint32_t *ids, float *values, double *probabilities, int32_t *kept,
                                         size_t out_len) {
  State &s = st();
  std::lock_guard<std::recursive_mutex> lock(s.mu);
  int32_t rc = ensure_init(s.ready ? s.device : 0);
  if (rc != HP_OK) return rc;
  Handle *h = lookup(handle);
  if (!h) return fail(HP_ERR_HANDLE, "unknown weight handle");
  if (h->input_size != input_size || input_len != sat_mul(input_size, column_count))
    return fail(HP_ERR_SHAPE, "matmul shape mismatch");
  rc = topk_check(column_count, h->row_count, k);
  if (rc != HP_OK) return rc;
  if (sampling) {
    rc = sampling_check(sampling, k);
    if (rc != HP_OK) return rc;
  }
  if (out_len != sat_mul(column_count, k)) return fail(HP_ERR_SHAPE, "topk output length mismatch");
  if (column_count == 0) return HP_OK;
  if (!d_input || !ids || !values) return fail(HP_ERR_ARG, "null pointer");
  if (sampling && (!rng_state || !tokens || !probabilities || !kept)) return fail(HP_ERR_ARG, "null pointer");
  if (reinterpret_cast<uintptr_t>(d_input) % 16 != 0) return fail(HP_ERR_ARG, "input must be 16-byte aligned");
  return head_candidates(h, d_input, input_size, column_count, k, softcap, sampling, rng_state, tokens, ids, values,
                         probabilities, kept);
}

int32_t hp_hip_device_alloc(size_t bytes, void **d_out) {
  State &s = st();
  std::lock_guard<std::recursive_mutex> lock(s.mu);
  if (!d_out) return fail(HP_ERR_ARG, "null pointer");
  *d_out = nullptr;
  int32_t rc = ensure_init(s.ready ? s.device : 0);
  if (rc != HP_OK) return rc;
  if (bytes == 0) return fail(HP_ERR_ARG, "zero-byte buffer");
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  HP_HIP_TRY(hipStreamIsCapturing(s.stream, &cs));
  if (cs != hipStreamCaptureStatusNone) return fail(HP_ERR_ARG, "no allocation while the library stream captures");
  void *p = nullptr;
  if (hipMalloc(&p, bytes) != hipSuccess) {
    (void)hipGetLastError();
    return fail(HP_ERR_OOM, "device allocation failed");
  }
  if (hipMemsetAsync(p, 0, bytes, s.stream) != hipSuccess || hipStreamSynchronize(s.stream) != hipSuccess) {
    (void)hipFree(p);
    return fail(HP_ERR_HIP, "device allocation could not be cleared");
  }
  s.dev_bufs[reinterpret_cast<uintptr_t>(p)] = bytes;
  *d_out = p;
  return HP_OK;
}

int32_t hp_hip_device_free(void *d) {
  State &s = st();
  std::lock_guard<std::recursive_mutex> lock(s.mu);
  if (!d) return HP_OK;
  auto it = s.dev_bufs.find(reinterpret_cast<uintptr_t>(d));
  if (it == s.dev_bufs.end()) return fail(HP_ERR_ARG, "not a buffer of hp_hip_device_alloc");
  HP_HIP_TRY(hipStreamSynchronize(s.stream));  // work queued on the buffer has finished
  HP_HIP_TRY(hipFree(d));
  s.dev_bufs.erase(it);
  return HP_OK;
}

int32_t hp_hip_copy_to_device(void *d_dst, const void *src, size_t bytes, void *stream) {
  State &s = st();
  std::lock_guard<std::recursive_mutex> lock(s.mu);
  if (bytes == 0) return HP_OK;
  if (!d_dst || !src) return fail(HP_ERR_ARG, "null pointer");
  if (!in_device_buffer(d_dst, bytes)) return fail(HP_ERR_ARG, "destination outside the buffers of hp_hip_device_alloc");
  hipStream_t strm = stream ? static_cast<hipStream_t>(stream) : s.stream;
  HP_HIP_TRY(hipMemcpyAsync(d_dst, src, bytes, hipMemcpyHostToDevice, strm));
  HP_HIP_TRY(hipStreamSynchronize(strm));
  return HP_OK;
}

int32_t hp_hip_copy_to_host(void *dst, const void *d_src, size_t bytes, void *stream) {
  State &s = st();
  std::lock_guard<std::recursive_mutex> lock(s.mu);
  if (bytes == 0) return HP_OK;
  if (!dst || !d_src) return fail(HP_ERR_ARG, "null pointer");
  if (!in_device_buffer(d_src, bytes)) return fail(HP_ERR_ARG, "source outside the buffers of hp_hip_device_alloc");
  hipStream_t strm = stream ? static_cast<hipStream_t>(stream) : s.stream;
  HP_HIP_TRY(hipMemcpyAsync(dst, d_src, bytes, hipMemcpyDeviceToHost, strm));
  HP_HIP_TRY(hipStreamSynchronize(strm));
  return HP_OK;
}

int32_t hp_hip_matmul_geglu_device(uint64_t gate, uint64_t up, const float *d_input, size_t input_len,
                                   size_t input_size, size_t column_count, float *d_output, size_t output_len,
                                   void *stream) {
  State &s = st();
  std::lock_guard<std::recursive_mutex> lock(s.mu);
  int32_t rc = ensure_init(s.ready ? s.device : 0);
  if (rc != HP_OK) return rc;
  Handle *hg, *hu;
  rc = geglu_pair_check(gate, up, input_len, input_size, column_count, output_len, &hg, &hu);
  if (rc != HP_OK) return rc;
  if (column_count == 0) return HP_OK;
  if (!d_input || !d_output) return fail(HP_ERR_ARG, "null pointer");
  if (reinterpret_cast<uintptr_t>(d_input) % 16 != 0) return fail(HP_ERR_ARG, "input must be 16-byte aligned");
  hipStream_t strm = stream ? static_cast<hipStream_t>(stream) : s.stream;
  return run_matvec_geglu(hg, hu, d_input, input_size, column_count, d_output, strm);
}

int32_t hp_hip_matmul_geglu(uint64_t gate, uint64_t up, const float *input, size_t input_len, size_t input_size,
                            size_t column_count, float *output, size_t output_len) {
  State &s = st();
  std::lock_guard<std::recursive_mutex> lock(s.mu);
  HostExactScope exact;
  int32_t rc = ensure_init(s.ready ? s.device : 0);
  if (rc != HP_OK) return rc;
  Handle *hg, *hu;
  rc = geglu_pair_check(gate, up, input_len, input_size, column_count, output_len, &hg, &hu);
  if (rc != HP_OK) return rc;
  if (column_count == 0) return HP_OK;
  if (!input || !output) return fail(HP_ERR_ARG, "null pointer");
  rc = grow((void **)&s.io_in, &s.io_in_cap, input_len * sizeof(float));
  if (rc == HP_OK) rc = grow((void **)&s.io_out[0], &s.io_out_cap[0], output_len * sizeof(float));
  if (rc != HP_OK) return rc;
  HP_HIP_TRY(hipMemcpyAsync(s.io_in, input, input_len * sizeof(float), hipMemcpyHostToDevice, s.stream));
  rc = run_matvec_geglu(hg, hu, s.io_in, input_size, column_count, s.io_out[0], s.stream);
  if (rc != HP_OK) return rc;
  HP_HIP_TRY(hipMemcpyAsync(output, s.io_out[0], output_len * sizeof(float), hipMemcpyDeviceToHost, s.stream));
  HP_HIP_TRY(hipStreamSynchronize(s.stream));
  return HP_OK;
}

int32_t hp_hip_geglu_device(const float *d_gate, const float *d_up, size_t n, float *d_output, void *stream) {
  State &s = st();
  std::lock_guard<std::recursive_mutex> lock(s.mu);
  int32_t rc = ensure_init(s.ready ? s.device : 0);
  if (rc != HP_OK) return rc;
  if (n == 0) return HP_OK;
  if (!d_gate || !d_up || !d_output) return fail(HP_ERR_ARG, "null pointer");
  hipStream_t strm = stream ? static_cast<hipStream_t>(stream) : s.stream;
  hipEvent_t e = prof_begin(strm);
  HP_HIP_TRY(launch_geglu(d_gate, d_up, n, s.gelu_lut, d_output, s.num_cus, strm));
  prof_end(HP_KERNEL_GEGLU, e, strm);
  s.launches++;
  return HP_OK;
}

int32_t hp_hip_geglu(const float *gate, const float *up, size_t n, float *output) {
  State &s = st();
  std::lock_guard<std::recursive_mutex> lock(s.mu);
  int32_t rc = ensure_init(s.ready ? s.device : 0);
  if (rc != HP_OK) return rc;
  if (n == 0) return HP_OK;
  if (!gate || !up || !output) return fail(HP_ERR_ARG, "null pointer");
  rc = grow((void **)&s.io_in, &s.io_in_cap, 2 * n * sizeof(float));
  if (rc != HP_OK) return rc;
  rc = grow((void **)&s.io_out[0], &s.io_out_cap[0], n * sizeof(float));
  if (rc != HP_OK) return rc;
  HP_HIP_TRY(hipMemcpyAsync(s.io_in, gate, n * 4, hipMemcpyHostToDevice, s.stream));
  HP_HIP_TRY(hipMemcpyAsync(s.io_in + n, up, n * 4, hipMemcpyHostToDevice, s.stream));
  HP_HIP_TRY(launch_geglu(s.io_in, s.io_in + n, n, s.gelu_lut, s.io_out[0], s.num_cus, s.stream));
  s.launches++;
  HP_HIP_TRY(hipMemcpyAsync(output, s.io_out[0], n * 4, hipMemcpyDeviceToHost, s.stream));
  HP_HIP_TRY(hipStreamSynchronize(s.stream));
  return HP_OK;
}

int32_t hp_hip_quantize_q8_k(const float *input, size_t input_len, size_t input_size, size_t column_count,
                             int8_t *qs, float *d, int16_t *bsums32) {
  State &s = st();
  std::lock_guard<std::recursive_mutex> lock(s.mu);
  int32_t rc = ensure_init(s.ready ? s.device : 0);
  if (rc != HP_OK) return rc;
  if (input_size == 0 || input_size % kQK != 0) return fail(HP_ERR_TYPE, "input_size is not a multiple of 256");
  if (input_len != sat_mul(input_size, column_count)) return fail(HP_ERR_SHAPE, "q8_k input length mismatch");
  if (column_count == 0) return HP_OK;
  if (!input || !qs || !d || !bsums32) return fail(HP_ERR_ARG, "null pointer");
  const size_t nb = input_size / kQK;
  uint8_t *buf = nullptr;
  const size_t bytes = input_len * 4 + input_len + column_count * nb * 4 + input_len / 32 * 2;
  if (hipMalloc((void **)&buf, bytes) != hipSuccess) return fail(HP_ERR_OOM, "q8_k buffer");
  float *dx = reinterpret_cast<float *>(buf);
  int8_t *dq = reinterpret_cast<int8_t *>(buf + input_len * 4);
  float *dd = reinterpret_cast<float *>(buf + input_len * 5);
  int16_t *db = reinterpret_cast<int16_t *>(buf + input_len * 5 + column_count * nb * 4);
  hipError_t e = hipMemcpyAsync(dx, input, input_len * 4, hipMemcpyHostToDevice, s.stream);
  if (e == hipSuccess) e = launch_q8k_natural(dx, (int)input_size, (int)column_count, dq, dd, db, s.stream);
  if (e == hipSuccess) e = hipMemcpyAsync(qs, dq, input_len, hipMemcpyDeviceToHost, s.stream);
  if (e == hipSuccess) e = hipMemcpyAsync(d, dd, column_count * nb * 4, hipMemcpyDeviceToHost, s.stream);
  if (e == hipSuccess) e = hipMemcpyAsync(bsums32, db, input_len / 32 * 2, hipMemcpyDeviceToHost, s.stream);
  if (e == hipSuccess) e = hipStreamSynchronize(s.stream);
  (void)hipFree(buf);
  if (e != hipSuccess) return hip_fail(e, "quantize_q8_k");
  return HP_OK;
}

int32_t hp_hip_set_matvec_kernel(int32_t which) {
  State &s = st();
  std::lock_guard<std::recursive_mutex> lock(s.mu);
  if (which < 0 || which > 8) return fail(HP_ERR_ARG, "kernel selector must be 0..8");
  s.matvec_kernel = which;
  return HP_OK;
}

int32_t hp_hip_set_input_images(int32_t enable) {
  State &s = st();
  std::lock_guard<std::recursive_mutex> lock(s.mu);
  s.images = enable != 0;
  return HP_OK;
}

int32_t hp_hip_set_prefill_folds(int32_t enable) {
  State &s = st();
  std::lock_guard<std::recursive_mutex> lock(s.mu);
  s.prefill_folds = enable != 0;
  return HP_OK;
}

int32_t hp_hip_set_weight_layouts(int32_t both) {
  State &s = st();
  std::lock_guard<std::recursive_mutex> lock(s.mu);
  s.both_layouts = both != 0;
  return HP_OK;
}

int32_t hp_hip_stats(hp_hip_stats_t *out) {
  State &s = st();
  std::lock_guard<std::recursive_mutex> lock(s.mu);
  if (!out) return fail(HP_ERR_ARG, "null pointer");
  hp_hip_stats_t r{};
  for (auto &h : s.handles)
    if (h.live) {
      r.handle_count++;
      r.resident_bytes += h.byte_length + h.seg_bytes;
    }
  r.scratch_bytes = s.io_in_cap + s.topk_out_cap + s.sample_out_cap + s.pool.stats().live_bytes +
                    s.pool.stats().retired_bytes;
  for (int i = 0; i < kMaxWeights; i++) r.scratch_bytes += s.io_out_cap[i];
  r.matmul_calls = s.matmul_calls;
  r.kernel_launches = s.launches;
  r.device = s.device;
  r.compute_units = s.num_cus;
  *out = r;
  return HP_OK;
}

int32_t hp_hip_synchronize(void) {
  State &s = st();
  std::lock_guard<std::recursive_mutex> lock(s.mu);
  if (!s.ready) return HP_OK;
  HP_HIP_TRY(hipStreamSynchronize(s.stream));
  return HP_OK;
}

int32_t hp_hip_profile(int32_t enable) {
  State &s = st();
  std::lock_guard<std::recursive_mutex> lock(s.mu);
  prof_collect();
  for (auto &p : s.prof) {
    p.total_ms = 0;
    p.launches = 0;
  }
  s.profiling = enable != 0;
  return HP_OK;
}

namespace {
__global__ void empty_kernel() {}
}  // namespace

int32_t hp_hip_empty_launches(size_t count, void *stream) {
  State &s = st();
  std::lock_guard<std::recursive_mutex> lock(s.mu);
  int32_t rc = ensure_init(s.ready ? s.device : 0);
  if (rc != HP_OK) return rc;
  if (count < 1 || count > 65536) return fail(HP_ERR_ARG, "count must be 1..65536");
  hipStream_t strm = stream ? static_cast<hipStream_t>(stream) : s.stream;
  for (size_t i = 0; i < count; i++) {
    hipLaunchKernelGGL(empty_kernel, dim3(1), dim3(64), 0, strm);
    HP_HIP_TRY(hipGetLastError());
  }
  return HP_OK;
}

int32_t hp_hip_profile_read(int32_t kernel, double *total_ms, uint64_t *launches) {
  State &s = st();
  std::lock_guard<std::recursive_mutex> lock(s.mu);
  if (kernel < 0 || kernel >= HP_KERNEL_COUNT) return fail(HP_ERR_ARG, "kernel id out of range");
  prof_collect();
  if (total_ms) *total_ms = s.prof[kernel].total_ms;
  if (launches) *launches = s.prof[kernel].launches;
  return HP_OK;
}

int32_t hp_hip_rms_norm_device(const float *d_input, size_t rows, size_t n, const float *d_weight,
                               double epsilon, float *d_output, void *stream) {
  State &s = st();
  std::lock_guard<std::recursive_mutex> lock(s.mu);
  int32_t rc = ensure_init(s.ready ? s.device : 0);
  if (rc != HP_OK) return rc;
  if (n == 0 || n > kNormMaxN) return fail(HP_ERR_SHAPE, "norm width must be 1..4096");
  if (rows > 65535) return fail(HP_ERR_SHAPE, "too many rows");
  if (rows == 0) return HP_OK;
  if (!d_input || !d_output) return fail(HP_ERR_ARG, "null pointer");
  hipStream_t strm = stream ? static_cast<hipStream_t>(stream) : s.stream;
  return run_norm(d_input, (int)rows, (int)n, nullptr, nullptr, 1.0f, nullptr, d_weight, d_output, epsilon, strm);
}

int32_t hp_hip_residual_norm_device(const float *d_branch, size_t rows, size_t n, const float *d_post_weight,
                                    const float *d_residual, float scale, float *d_residual_out,
                                    const float *d_next_weight, float *d_next_out, double epsilon,
                                    void *stream) {
  State &s = st();
  std::lock_guard<std::recursive_mutex> lock(s.mu);
  int32_t rc = ensure_init(s.ready ? s.device : 0);
  if (rc != HP_OK) return rc;
  if (n == 0 || n > kNormMaxN) return fail(HP_ERR_SHAPE, "norm width must be 1..4096");
  if (rows > 65535) return fail(HP_ERR_SHAPE, "too many rows");
  if (rows == 0) return HP_OK;
  if (!d_branch || !d_residual || !d_residual_out) return fail(HP_ERR_ARG, "null pointer");
  hipStream_t strm = stream ? static_cast<hipStream_t>(stream) : s.stream;
  return run_norm(d_branch, (int)rows, (int)n, d_post_weight, d_residual, scale, d_residual_out, d_next_weight,
                  d_next_out, epsilon, strm);
}

int32_t hp_hip_attention_prep_device(const hp_hip_attention_config_t *config, size_t token_count, const float *d_q,
                                     const float *d_k, const float *d_v, const float *d_q_norm,
                                     const float *d_k_norm, const int32_t *d_position, float *d_q_out,
                                     uint16_t *d_key_cache, uint16_t *d_value_cache, void *stream) {
  State &s = st();
  std::lock_guard<std::recursive_mutex> lock(s.mu);
  int32_t rc = ensure_init(s.ready ? s.device : 0);
  if (rc != HP_OK) return rc;
  rc = attention_check(config);
  if (rc != HP_OK) return rc;
  if (token_count < 1 || token_count > (size_t)kMaxChunkTokens || token_count > (size_t)config->capacity)
    return fail(HP_ERR_SHAPE, "token_count must be 1..min(4096, capacity)");
  if (!d_q || !d_k || !d_q_norm || !d_k_norm || !d_position || !d_q_out || !d_key_cache || !d_value_cache)
    return fail(HP_ERR_ARG, "null pointer");
  hipStream_t strm = stream ? static_cast<hipStream_t>(stream) : s.stream;
  QkvPostArgs a = qkv_post_args(config);
  a.q = d_q;
  a.k = d_k;
  a.v = d_v ? d_v : d_k;
  a.wq = d_q_norm;
  a.wk = d_k_norm;
  a.position = d_position;
  a.q_out = d_q_out;
  a.k_cache = reinterpret_cast<_Float16 *>(d_key_cache);
  a.v_cache = reinterpret_cast<_Float16 *>(d_value_cache);
  a.tokens = (int)token_count;
  HP_HIP_TRY(launch_qkv_post(a, strm));
  s.launches++;
  return HP_OK;
}

int32_t hp_hip_gqa_attention_device(const hp_hip_attention_config_t *config, size_t token_count, const float *d_q,
                                    const uint16_t *d_key_cache, const uint16_t *d_value_cache,
                                    const int32_t *d_position, float *d_output, void *stream) {
  State &s = st();
  std::lock_guard<std::recursive_mutex> lock(s.mu);
  int32_t rc = ensure_init(s.ready ? s.device : 0);
  if (rc != HP_OK) return rc;
  rc = attention_check(config);
  if (rc != HP_OK) return rc;
  if (token_count < 1 || token_count > (size_t)kMaxChunkTokens || token_count > (size_t)config->capacity)
    return fail(HP_ERR_SHAPE, "token_count must be 1..min(4096, capacity)");
  if (!d_q || !d_key_cache || !d_value_cache || !d_position || !d_output) return fail(HP_ERR_ARG, "null pointer");
  hipStream_t strm = stream ? static_cast<hipStream_t>(stream) : s.stream;
  const bool prefill = token_count > (size_t)kMaxTokens;
  const int ranges = prefill ? attn_prefill_ranges((int)token_count, config->head_count, config->head_count_kv,
                                                   config->capacity, s.num_cus)
                             : 0;
  void *partials = nullptr;
  rc = stream_scratch(strm, kScratchAttn,
                      (prefill ? attn_prefill_partial_floats(config->head_count_kv, (int)token_count, ranges)
                               : attn_partial_floats(config->head_count_kv, config->capacity, (int)token_count)) *
                          sizeof(float),
                      &partials);
  if (rc != HP_OK) return rc;
  AttnArgs a = attn_args(config);
  a.q = d_q;
  a.k_cache = reinterpret_cast<_Float16 *>(const_cast<uint16_t *>(d_key_cache));  // read only: prep == 0
  a.v_cache = reinterpret_cast<_Float16 *>(const_cast<uint16_t *>(d_value_cache));
  a.position = d_position;
  a.out = d_output;
  a.tokens = (int)token_count;
  if (!prefill) return run_attention(a, static_cast<float *>(partials), strm);
  hipEvent_t e = prof_begin(strm);
  HP_HIP_TRY(launch_attention_prefill(a, static_cast<float *>(partials), ranges, strm));
  prof_end(HP_KERNEL_ATTENTION, e, strm);
  s.launches += 2;
  return HP_OK;
}

int32_t hp_hip_decode_layers_device(const hp_hip_decode_layer_t *layers, size_t layer_count, size_t token_count,
                                    float *d_hidden, const int32_t *d_position, const float *d_output_norm,
                                    float *d_output, void *stream) {
  State &s = st();
  std::lock_guard<std::recursive_mutex> lock(s.mu);
  int32_t rc = ensure_init(s.ready ? s.device : 0);
  if (rc != HP_OK) return rc;
  if (token_count < 1 || token_count > (size_t)kMaxLayerTokens)
    return fail(HP_ERR_SHAPE, "token_count must be 1.." + std::to_string(kMaxLayerTokens));
  if (layer_count == 0) return fail(HP_ERR_ARG, "no layers (the final norm alone: hp_hip_rms_norm_device)");
  if (!d_hidden || !d_position || !layers || (d_output_norm && !d_output)) return fail(HP_ERR_ARG, "null pointer");
  if (reinterpret_cast<uintptr_t>(d_hidden) % 16 != 0) return fail(HP_ERR_ARG, "hidden must be 16-byte aligned");
  std::vector<LayerHandles> hs(layer_count);
  size_t hidden = lookup(layers[0].attn_q) ? lookup(layers[0].attn_q)->input_size : 0;
  size_t qmax = 0, kvmax = 0, ffmax = 0, pmax = 0;
  int min_cap = INT32_MAX;
  for (size_t i = 0; i < layer_count; i++) {
    rc = decode_layer_check(layers[i], hidden, &hs[i]);
    if (rc != HP_OK) return rc;
    const hp_hip_attention_config_t &c = layers[i].attention;
    qmax = std::max(qmax, (size_t)c.head_count * kHeadDim);
    kvmax = std::max(kvmax, (size_t)c.head_count_kv * kHeadDim);
    ffmax = std::max(ffmax, hs[i].gate->row_count);
    if (hs[i].inp_gate) pmax = std::max(pmax, hs[i].inp_gate->row_count);
    min_cap = std::min(min_cap, c.capacity);
  }
  if (hidden == 0 || hidden > kNormMaxN) return fail(HP_ERR_SHAPE, "hidden size must be 1..4096");
  if (token_count == 1 && s.fused_mode != 0 && s.matvec_kernel == 0) {
    // one token: the persistent step, when these layers are within what it covers
    FusedPlan plan;
    if (fused_plan(layers, hs, hidden, &plan))
      return run_fused(plan, hidden, d_hidden, d_position, d_output_norm, d_output,
                       stream ? static_cast<hipStream_t>(stream) : s.stream);
  }
  // Chunks of tokens go through every layer in turn, each chunk spanning
  // fewer positions than the smallest KV ring holds, so a chunk's appends
  // never overwrite keys that its own tokens still attend to
  // (slidingRingChunkTokenCount, wasm/segment-runner.ts:181-207).
  const size_t chunk = std::min<size_t>({token_count, (size_t)min_cap, (size_t)kMaxChunkTokens});
  const size_t last = token_count - (token_count - 1) / chunk * chunk;  // tokens of the last chunk
  size_t partials = 0;
  for (size_t i = 0; i < layer_count; i++) {
    const hp_hip_attention_config_t &c = layers[i].attention;
    for (size_t mc : {chunk, last}) {
      const size_t need =
          mc <= (size_t)kMaxTokens
              ? attn_partial_floats(c.head_count_kv, c.capacity, (int)mc)
              : attn_prefill_partial_floats(
                    c.head_count_kv, (int)mc,
                    attn_prefill_ranges((int)mc, c.head_count, c.head_count_kv, c.capacity, s.num_cus));
      partials = std::max(partials, need);
    }
  }
  const size_t M = chunk;  // rows of every scratch buffer
  // scratch ([M] rows each): xn, q, k, v, q after RoPE, attention, o, x1, h, y;
  // attention partials; RoPE tables [M][128] cos, sin
  // (2..8 tokens) the Q/K/V and down inputs as pre-quantised images
  auto al = [](size_t n) { return (n + 63) & ~(size_t)63; };
  const bool images = M >= 2 && M <= (size_t)kMaxTokens;
  const size_t img_x = images ? q8_image_bytes((int)M, (int)(hidden / kQK)) / sizeof(float) : 0;
  const size_t img_h = images ? q8_image_bytes((int)M, (int)(ffmax / kQK)) / sizeof(float) : 0;
  // (per-layer input step) the FFN residual x2, the gate and the gelu product
  const size_t sizes[16] = {al(M * hidden), al(M * qmax),   al(M * kvmax),  al(M * kvmax),
                            al(M * qmax),   al(M * qmax),   al(M * hidden), al(M * hidden),
                            al(M * ffmax),  al(M * hidden), al(partials),   al(M * kHeadDim / 2 * 4),
                            al(img_x),      al(img_h),      al(pmax ? M * hidden : 0), al(M * 2 * pmax)};
  size_t total = 0;
  for (size_t z : sizes) total += z;
  hipStream_t strm = stream ? static_cast<hipStream_t>(stream) : s.stream;
  void *dscr = nullptr;
  rc = stream_scratch(strm, kScratchDecode, total * sizeof(float), &dscr);
  if (rc != HP_OK) return rc;
  float *buf[16];
  float *p = static_cast<float *>(dscr);
  for (int i = 0; i < 16; i++) {
    buf[i] = p;
    p += sizes[i];
  }
  float *xn = buf[0], *q = buf[1], *k = buf[2], *v = buf[3], *qr = buf[4], *att = buf[5], *o = buf[6],
        *x1 = buf[7], *h = buf[8], *y = buf[9], *part = buf[10];
  double2 *rope_table = reinterpret_cast<double2 *>(buf[11]);
  uint8_t *imgx_buf = images && hidden % kQK == 0 ? reinterpret_cast<uint8_t *>(buf[12]) : nullptr;
  uint8_t *imgh_buf = images && ffmax % kQK == 0 ? reinterpret_cast<uint8_t *>(buf[13]) : nullptr;
  float *x2 = buf[14], *pg = buf[15];

  for (size_t c0 = 0; c0 < token_count; c0 += chunk) {
    const size_t Mc = std::min(chunk, token_count - c0);
    float *hid = d_hidden + c0 * hidden;
    uint8_t *imgx = Mc >= 2 && Mc <= (size_t)kMaxTokens ? imgx_buf : nullptr;
    uint8_t *imgh = Mc >= 2 && Mc <= (size_t)kMaxTokens ? imgh_buf : nullptr;
    // The norms ride in the prologues of the launches that consume them (one
    // token): the Q/K/V launch forms attn_norm(previous residual), the gate/up
    // launch ffn_norm(residual after attention).  With several tokens, or a
    // forced matrix-core kernel, they run as norm launches into xn.
    NormIn nin{};
    // a fast prefill O or down launch leaves its block-range sums (ks > 1)
    // in a scratch buffer for the norm launch after it to add
    PrefillParts qp{}, op{}, dp{};
    nin.mode = 1;
    nin.y = hid;
    nin.w_next = layers[0].d_attn_norm;
    nin.scale = 1.0f;
    nin.eps = layers[0].attention.epsilon;
    for (size_t i = 0; i < layer_count; i++) {
      const hp_hip_decode_layer_t &L = layers[i];
      const LayerHandles &H = hs[i];
      const double eps = L.attention.epsilon;
      Handle *qkv[3] = {H.q, H.k, H.v};
      float *qkv_out[3] = {q, k, v};
      rc = run_matvec(H.v ? 3 : 2, qkv, nullptr, hidden, Mc, qkv_out, strm, &nin, xn, imgx, nullptr, &dp,
                      Mc > 1 && s.prefill_folds ? &qp : nullptr);
      if (Mc == 1) qp.ks = 1;
      if (rc != HP_OK) return rc;
      // the RoPE angles depend on the positions and the RoPE parameters only:
      // a layer whose parameters match the previous layer's reads its table
      const hp_hip_attention_config_t *pc = i > 0 ? &layers[i - 1].attention : nullptr;
      const int table_mode = pc && pc->rope_dims == L.attention.rope_dims &&
                                     pc->rope_freq_base == L.attention.rope_freq_base &&
                                     pc->d_rope_freq_factors == L.attention.d_rope_freq_factors
                                 ? 2
                                 : 1;
      AttnArgs aa = attn_args(&L.attention);
      aa.k_cache = reinterpret_cast<_Float16 *>(L.d_key_cache);
      aa.v_cache = reinterpret_cast<_Float16 *>(L.d_value_cache);
      aa.position = d_position;
      aa.pos_offset = (int)c0;
      aa.out = att;
      aa.rope_table = rope_table;
      aa.rope_table_mode = table_mode;
      if (Mc == 1) {
        // one token: norms, RoPE and the cache append inside the attention launch
        aa.prep = 1;
        aa.q = q;
        aa.k = k;
        aa.v = H.v ? v : k;
        aa.wq = L.d_attn_q_norm;
        aa.wk = L.d_attn_k_norm;
      } else {
        // a draft or a prefill chunk: every token's key and value enter the
        // caches first, then each token attends causally
        QkvPostArgs pa = qkv_post_args(&L.attention);
        pa.q = q;
        pa.k = k;
        pa.v = H.v ? v : k;
        if (qp.ks > 1) {
          // the Q/K/V launch left its block-range sums for this launch to add
          pa.q = qp.part + qp.off[0];
          pa.k = qp.part + qp.off[1];
          pa.v = H.v ? qp.part + qp.off[2] : pa.k;
          pa.src_ks = qp.ks;
          pa.src_stride = qp.stride;
        }
        pa.wq = L.d_attn_q_norm;
        pa.wk = L.d_attn_k_norm;
        pa.position = d_position;
        pa.pos_offset = (int)c0;
        // a prefill chunk's queries leave rounded to f16 (the attention's
        // first step), once per query instead of once per window slice
        const bool half_q = s.prefill_folds && Mc > (size_t)kMaxTokens;
        pa.q_out = half_q ? nullptr : qr;
        pa.q_half = half_q ? reinterpret_cast<uint16_t *>(qr) : nullptr;
        pa.k_cache = aa.k_cache;
        pa.v_cache = aa.v_cache;
        pa.tokens = (int)Mc;
        pa.rope_table = rope_table;
        pa.rope_table_mode = table_mode;
        hipEvent_t e = prof_begin(strm);
        HP_HIP_TRY(launch_qkv_post(pa, strm));
        prof_end(HP_KERNEL_ATTENTION, e, strm);
        s.launches++;
        aa.q = half_q ? nullptr : qr;
        aa.q_half = pa.q_half;
        aa.tokens = (int)Mc;
      }
      bool o_tiles = false;  // the attention left O's activation tiles
      if (Mc <= (size_t)kMaxTokens) {
        rc = run_attention(aa, part, strm);
      } else {
        const int ranges = attn_prefill_ranges((int)Mc, L.attention.head_count, L.attention.head_count_kv,
                                               L.attention.capacity, s.num_cus);
        // O on the fast prefill kernel: the slice merge writes its
        // activation tiles into O's prefill scratch (the pre-pass launch
        // they replace would write the same bytes there)
        if (s.prefill_folds && prefill_kind(Mc, mfma_ok(1, &H.o)) == 2 && H.o->input_size % kQK == 0 &&
            H.o->input_size == (size_t)L.attention.head_count * kHeadDim) {
          MfmaLaunch lo{};
          lo.count = 1;
          lo.k = (int)H.o->input_size;
          lo.cols = (int)Mc;
          lo.rows[0] = (int)H.o->row_count;
          void *pre = nullptr;
          rc = stream_scratch(strm, kScratchPrefill, prefill_fast_bytes(lo, s.num_cus), &pre);
          if (rc != HP_OK) return rc;
          aa.o_tiles = static_cast<uint8_t *>(pre);
          o_tiles = true;
        }
        hipEvent_t e = prof_begin(strm);
        HP_HIP_TRY(launch_attention_prefill(aa, part, ranges, strm));
        prof_end(HP_KERNEL_ATTENTION, e, strm);
        s.launches += 2;
      }
      if (rc != HP_OK) return rc;
      Handle *oh[1] = {H.o};
      float *oo[1] = {o};
      const bool defer = s.prefill_folds && H.o->row_count == hidden;
      rc = run_matvec(1, oh, att, H.o->input_size, Mc, oo, strm, nullptr, nullptr, nullptr, nullptr, nullptr,
                      defer ? &op : nullptr, o_tiles);
      if (rc != HP_OK) return rc;
      if (!defer) op.ks = 1;
      NormIn fin{};
      fin.mode = 2;
      fin.y = op.ks > 1 ? op.part : o;
      fin.w_post = L.d_post_attention_norm;
      fin.x_res = hid;
      fin.scale = 1.0f;
      fin.x_out = x1;
      fin.w_next = L.d_ffn_norm;
      fin.eps = eps;
      bool h_img = false;
      // down on the fast prefill kernel: its pre-pass completes the gate/up
      // launch's trailing tiles (no tail launch)
      Handle *dh[1] = {H.down};
      const bool down_fast = s.prefill_folds && prefill_kind(Mc, mfma_ok(1, dh)) == 2 && H.down->input_size % kQK == 0;
      GegluTail gtail{};
      rc = run_matvec_geglu(H.gate, H.up, nullptr, hidden, Mc, h, strm, &fin, xn, imgh, &h_img, &op,
                            down_fast ? &gtail : nullptr);
      if (rc != HP_OK) return rc;
      float *yo[1] = {y};
      rc = run_matvec(1, dh, h, H.down->input_size, Mc, yo, strm, nullptr, nullptr, nullptr, h_img ? imgh : nullptr,
                      nullptr, s.prefill_folds && H.down->row_count == hidden ? &dp : nullptr, false, &gtail);
      if (rc != HP_OK) return rc;
      if (H.down->row_count != hidden) dp.ks = 1;
      nin.mode = 2;
      nin.y = dp.ks > 1 ? dp.part : y;
      nin.w_post = L.d_post_ffw_norm;
      nin.x_res = x1;
      nin.scale = L.layer_output_scale;
      nin.x_out = hid;
      nin.w_next = i + 1 < layer_count ? layers[i + 1].d_attn_norm : nullptr;
      nin.eps = eps;
      if (H.inp_gate) {
        // applyPerLayerInput: the FFN residual x2 (no scale yet), gate =
        // inp_gate . x2, mixed = f32(gelu(gate) * input) (the GeGLU product
        // with the per-layer input as `up`), y = proj . mixed; the next norm
        // forms f32((x2 + post_norm(y)) * scale)
        rc = run_norm(nin.y, (int)Mc, (int)hidden, L.d_post_ffw_norm, x1, 1.0f, x2, nullptr, nullptr, eps, strm,
                      nullptr, nullptr, &dp);
        if (rc != HP_OK) return rc;
        dp.ks = 1;
        const size_t P = H.inp_gate->row_count;
        Handle *gh[1] = {H.inp_gate};
        float *go[1] = {pg};
        rc = run_matvec(1, gh, x2, hidden, Mc, go, strm);
        if (rc != HP_OK) return rc;
        float *mixed = pg + Mc * P;
        HP_HIP_TRY(launch_geglu(pg, L.d_per_layer_input + c0 * P, Mc * P, s.gelu_lut, mixed, s.num_cus, strm));
        s.launches++;
        Handle *ph[1] = {H.proj};
        float *po[1] = {y};
        rc = run_matvec(1, ph, mixed, P, Mc, po, strm);
        if (rc != HP_OK) return rc;
        nin.y = y;
        nin.w_post = L.d_post_norm;
        nin.x_res = x2;
      }
    }
    // the last layer's post-FFN residual (or per-layer input residual), then output_norm
    rc = run_norm(nin.y, (int)Mc, (int)hidden, nin.w_post, nin.x_res, nin.scale, hid, d_output_norm,
                  d_output_norm ? d_output + c0 * hidden : nullptr, nin.eps, strm, nullptr, nullptr, &dp);
    if (rc != HP_OK) return rc;
  }
  return HP_OK;
}

int32_t hp_hip_set_decode_fused(int32_t mode) {
  if (mode != 0 && mode != 1) return fail(HP_ERR_ARG, "mode must be 0 or 1");
  State &s = st();
  std::lock_guard<std::recursive_mutex> lock(s.mu);
  s.fused_mode = mode;
  return HP_OK;
}

int32_t hp_hip_set_fused_wait_limit(uint64_t ticks) {
  State &s = st();
  std::lock_guard<std::recursive_mutex> lock(s.mu);
  s.fused_spin = ticks == 0 ? 100000000ull : ticks;
  return HP_OK;
}

int32_t hp_hip_set_fused_trace(uint64_t *d_stamps, size_t len) {
  State &s = st();
  std::lock_guard<std::recursive_mutex> lock(s.mu);
  s.fused_trace = d_stamps;
  s.fused_trace_len = d_stamps ? len : 0;
  return HP_OK;
}

int32_t hp_hip_release_stream_scratch(void *stream) {
  State &s = st();
  std::lock_guard<std::recursive_mutex> lock(s.mu);
  if (!s.ready) return HP_OK;
  if (!stream) return fail(HP_ERR_ARG, "the library stream's scratch lives until hp_hip_shutdown");
  hipStream_t strm = static_cast<hipStream_t>(stream);
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  HP_HIP_TRY(hipStreamIsCapturing(strm, &cs));
  if (cs != hipStreamCaptureStatusNone) return fail(HP_ERR_ARG, "the stream is capturing");
  HP_HIP_TRY(hipStreamSynchronize(strm));
  s.pool.release_stream(stream);
  return HP_OK;
}

int32_t hp_hip_decode_fused_status(void *stream) {
  State &s = st();
  std::lock_guard<std::recursive_mutex> lock(s.mu);
  if (!s.ready) return HP_OK;
  hipStream_t strm = stream ? static_cast<hipStream_t>(stream) : s.stream;
  void *arena = nullptr;
  // an existing arena only (a zero-byte request never allocates one anew)
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(strm, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone)
    return fail(HP_ERR_ARG, "hp_hip_decode_fused_status cannot run under graph capture");
  if (s.pool.peek(static_cast<void *>(strm), kScratchFused, &arena) != kScratchOk || !arena) return HP_OK;
  HP_HIP_TRY(hipStreamSynchronize(strm));
  uint32_t status = 0;
  FusedCtl *ctl = static_cast<FusedCtl *>(arena);
  HP_HIP_TRY(hipMemcpy(&status, &ctl->status, sizeof(status), hipMemcpyDeviceToHost));
  if (status == 0) return HP_OK;
  const uint32_t zero = 0;
  HP_HIP_TRY(hipMemcpy(&ctl->status, &zero, sizeof(zero), hipMemcpyHostToDevice));
  return fail(HP_ERR_HIP, "persistent decode step: a stage waited past its time limit (status " +
                              std::to_string(status) + "); outputs of the failed steps are invalid");
}

}  // extern "C"
