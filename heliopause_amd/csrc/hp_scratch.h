// hp_scratch.h -- device scratch of the *_device entry points: one set per
// stream, grow-only, never freed while a captured graph may still hold it.
//
// The asynchronous entry points (decode layers, attention, top-k, the
// prefill pre-pass, the gate/up sums of a split GeGLU) keep intermediate
// results in library-owned device memory.  Two rules make that safe under
// HIP graph capture and across caller streams:
//   * Each (stream, kind) pair owns its buffer, so calls queued on different
//     streams never share intermediate memory.  A captured graph keeps the
//     buffers of the stream it was captured on.
//   * A buffer that is too small is replaced by a larger one, and the old one
//     is retired, not freed: a graph captured earlier may still point at it.
//     Retired and live buffers are freed by release_stream(stream)
//     (hp_hip_release_stream_scratch: the caller is done with the stream and
//     with every graph captured on it) or by release_all() (hp_hip_shutdown),
//     never otherwise.  Growth itself is refused while the stream is
//     capturing (the allocation would not be part of the graph), so a
//     captured call must follow an uncaptured call of the same shape.
// Capacities grow at least 2x, so retired memory stays below the live size.
//
// Host-only C++ with the allocator as a template parameter, so the policy
// can be exercised on the CPU with a recording allocator.
#ifndef HP_SCRATCH_H
#define HP_SCRATCH_H

#include <stddef.h>
#include <stdint.h>

#include <map>
#include <utility>
#include <vector>

namespace hp {

enum ScratchKind {
  kScratchDecode = 0,   // activations of a decode step
  kScratchAttn = 1,     // attention partials
  kScratchTopk = 2,     // top-k selection state (zeroed when allocated)
  kScratchPrefill = 3,  // Q8_K / f16 images of a prefill launch
  kScratchGeglu = 4,    // gate and up sums ahead of a GeGLU launch
  kScratchParts = 5,    // block-range sums of a prefill launch that a norm launch adds
  kScratchFused = 6,    // exchange arena and control words of the persistent decode step (zeroed when allocated)
  kScratchKinds = 7
};

enum ScratchStatus { kScratchOk = 0, kScratchCapturing = 1, kScratchNoMemory = 2, kScratchZeroFailed = 3 };

// Alloc provides:
//   bool alloc(void **p, size_t bytes);            device allocation
//   void free(void *p);                            device free
//   bool zero(void *p, size_t bytes, void *stream) clear, complete on return
template <class Alloc>
class ScratchPool {
 public:
  struct Stats {
    uint64_t live_bytes = 0;     // buffers currently handed out
    uint64_t retired_bytes = 0;  // replaced buffers kept until release_all
    uint64_t allocations = 0;
    uint64_t frees = 0;          // buffers freed (only release_all frees)
  };

  explicit ScratchPool(Alloc a = Alloc()) : alloc_(a) {}

  // A buffer of at least `bytes` for (stream, kind) in *out.
  int get(void *stream, int kind, size_t bytes, bool capturing, bool zero, void **out) {
    Buf &b = sets_[stream].buf[kind];
    if (b.p && b.cap >= bytes) {
      *out = b.p;
      return kScratchOk;
    }
    if (capturing) return kScratchCapturing;
    size_t want = bytes < 4096 ? 4096 : bytes;
    if (b.p && want < 2 * b.cap) want = 2 * b.cap;
    void *p = nullptr;
    if (!alloc_.alloc(&p, want) || !p) return kScratchNoMemory;
    if (zero && !alloc_.zero(p, want, stream)) {
      alloc_.free(p);
      return kScratchZeroFailed;
    }
    stats_.allocations++;
    if (b.p) {
      retired_.push_back(Retired{b, stream});
      stats_.retired_bytes += b.cap;
      stats_.live_bytes -= b.cap;
    }
    b.p = p;
    b.cap = want;
    stats_.live_bytes += want;
    *out = p;
    return kScratchOk;
  }

  // The live buffer of (stream, kind) in *out, if there is one (never allocates).
  int peek(void *stream, int kind, void **out) const {
    auto it = sets_.find(stream);
    if (it == sets_.end() || !it->second.buf[kind].p) return kScratchNoMemory;
    *out = it->second.buf[kind].p;
    return kScratchOk;
  }

  // Frees the live and retired buffers of one stream.  The caller has
  // synchronised the stream and no graph captured on it is replayed
  // afterwards.  Returns the bytes freed.
  uint64_t release_stream(void *stream) {
    uint64_t freed = 0;
    auto it = sets_.find(stream);
    if (it != sets_.end()) {
      for (Buf &b : it->second.buf)
        if (b.p) {
          alloc_.free(b.p);
          stats_.frees++;
          stats_.live_bytes -= b.cap;
          freed += b.cap;
        }
      sets_.erase(it);
    }
    std::vector<Retired> keep;
    for (Retired &r : retired_) {
      if (r.stream == stream) {
        alloc_.free(r.buf.p);
        stats_.frees++;
        stats_.retired_bytes -= r.buf.cap;
        freed += r.buf.cap;
      } else {
        keep.push_back(r);
      }
    }
    retired_.swap(keep);
    return freed;
  }

  // Streams that hold buffers.
  size_t stream_count() const { return sets_.size(); }

  // Frees every buffer, live and retired.  The caller has synchronised the
  // device and no graph that holds these buffers is replayed afterwards.
  void release_all() {
    for (auto &kv : sets_)
      for (Buf &b : kv.second.buf)
        if (b.p) {
          alloc_.free(b.p);
          stats_.frees++;
          b = Buf();
        }
    for (Retired &r : retired_) {
      alloc_.free(r.buf.p);
      stats_.frees++;
    }
    sets_.clear();
    retired_.clear();
    stats_.live_bytes = stats_.retired_bytes = 0;
  }

  const Stats &stats() const { return stats_; }

 private:
  struct Buf {
    void *p = nullptr;
    size_t cap = 0;
  };
  struct Set {
    Buf buf[kScratchKinds];
  };
  struct Retired {
    Buf buf;
    void *stream;
  };
  Alloc alloc_;
  std::map<void *, Set> sets_;
  std::vector<Retired> retired_;
  Stats stats_;
};

}  // namespace hp

#endif
