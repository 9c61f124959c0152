// CPU check of the scratch policy in heliopause_amd/csrc/hp_scratch.h with a
// recording allocator: a buffer handed out (as a captured graph would hold
// it) stays allocated until release_all or its stream's release_stream,
// growth is refused while capturing, streams never share a buffer.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <set>

#include "hp_scratch.h"

namespace {

struct Recorder {
  std::set<void *> live;
  int frees = 0, zeros = 0;
  bool fail_next = false;
};
Recorder rec;

struct FakeAlloc {
  bool alloc(void **p, size_t bytes) {
    if (rec.fail_next) {
      rec.fail_next = false;
      return false;
    }
    *p = std::malloc(bytes);
    std::memset(*p, 0xAB, bytes);
    rec.live.insert(*p);
    return true;
  }
  void free(void *p) {
    if (!rec.live.erase(p)) {
      std::printf("FAIL free of an unknown pointer\n");
      std::exit(1);
    }
    rec.frees++;
    std::free(p);
  }
  bool zero(void *p, size_t bytes, void *) {
    std::memset(p, 0, bytes);
    rec.zeros++;
    return true;
  }
};

int failures = 0;
void check(bool ok, const char *what) {
  if (!ok) {
    std::printf("FAIL %s\n", what);
    failures++;
  }
}

}  // namespace

int main() {
  using Pool = hp::ScratchPool<FakeAlloc>;
  Pool pool;
  void *s1 = reinterpret_cast<void *>(0x1000), *s2 = reinterpret_cast<void *>(0x2000);
  void *a = nullptr, *b = nullptr, *c = nullptr, *d = nullptr;

  check(pool.get(s1, hp::kScratchDecode, 10000, false, false, &a) == hp::kScratchOk && a, "first allocation");
  // a captured graph now holds `a`; an equal or smaller request reuses it, even while capturing
  check(pool.get(s1, hp::kScratchDecode, 9000, true, false, &b) == hp::kScratchOk && b == a, "reuse under capture");
  // growth while capturing is refused and allocates nothing
  const size_t live_before = rec.live.size();
  check(pool.get(s1, hp::kScratchDecode, 50000, true, false, &c) == hp::kScratchCapturing, "growth refused");
  check(rec.live.size() == live_before, "refused growth allocates nothing");
  // growth outside capture: a new buffer, the old one still allocated
  check(pool.get(s1, hp::kScratchDecode, 50000, false, false, &c) == hp::kScratchOk && c != a, "growth");
  check(rec.live.count(a) == 1, "grown-out buffer stays allocated");
  check(rec.frees == 0, "no free before release_all");
  check(pool.stats().retired_bytes >= 10000, "retired bytes counted");
  // each growth at least doubles the capacity: 50001 bytes take a buffer of
  // at least 100000, which then serves up to that size
  check(pool.get(s1, hp::kScratchDecode, 50001, false, false, &d) == hp::kScratchOk && d != c, "second growth");
  void *d2 = nullptr;
  check(pool.get(s1, hp::kScratchDecode, 100000, false, false, &d2) == hp::kScratchOk && d2 == d, "2x growth");
  check(rec.live.count(a) == 1 && rec.live.count(c) == 1, "both grown-out buffers stay allocated");
  // another stream and another kind get their own buffers
  check(pool.get(s2, hp::kScratchDecode, 100, false, false, &d) == hp::kScratchOk && d != c && d != a && d != d2,
        "per-stream buffer");
  void *e = nullptr;
  check(pool.get(s1, hp::kScratchAttn, 100, false, false, &e) == hp::kScratchOk && e != c && e != d,
        "per-kind buffer");
  // zeroed kinds are cleared when allocated, and only then
  void *z = nullptr, *z2 = nullptr;
  check(pool.get(s1, hp::kScratchTopk, 4096, false, true, &z) == hp::kScratchOk, "zeroed allocation");
  bool all_zero = true;
  for (int i = 0; i < 4096; i++) all_zero = all_zero && static_cast<unsigned char *>(z)[i] == 0;
  check(all_zero && rec.zeros == 1, "cleared on allocation");
  check(pool.get(s1, hp::kScratchTopk, 4000, false, true, &z2) == hp::kScratchOk && z2 == z && rec.zeros == 1,
        "not cleared again");
  // allocation failure leaves the old buffer in place
  rec.fail_next = true;
  void *f = nullptr;
  check(pool.get(s2, hp::kScratchDecode, 1 << 20, false, false, &f) == hp::kScratchNoMemory, "allocation failure");
  check(pool.get(s2, hp::kScratchDecode, 100, false, false, &f) == hp::kScratchOk && f == d, "old buffer kept");
  check(rec.frees == 0, "still no free before release_all");
  // releasing one stream frees its live and retired buffers only
  void *s3 = reinterpret_cast<void *>(0x3000), *g1 = nullptr, *g2 = nullptr;
  check(pool.get(s3, hp::kScratchDecode, 5000, false, false, &g1) == hp::kScratchOk, "third stream");
  check(pool.get(s3, hp::kScratchDecode, 20000, false, false, &g2) == hp::kScratchOk && g2 != g1, "third grows");
  void *g3 = nullptr;
  check(pool.get(s3, hp::kScratchAttn, 100, false, false, &g3) == hp::kScratchOk, "third stream, second kind");
  const size_t streams = pool.stream_count();
  const size_t before = rec.live.size();
  const uint64_t freed = pool.release_stream(s3);
  check(rec.live.size() == before - 3 && !rec.live.count(g1) && !rec.live.count(g2) && !rec.live.count(g3),
        "release_stream frees that stream's live and retired buffers");
  check(freed >= 5000 + 20000 + 100 && pool.stream_count() == streams - 1, "release_stream bytes and streams");
  check(rec.live.count(a) == 1 && rec.live.count(c) == 1 && rec.live.count(d) == 1, "other streams untouched");
  void *g4 = nullptr;
  check(pool.get(s3, hp::kScratchDecode, 100, false, false, &g4) == hp::kScratchOk, "a released stream starts anew");
  check(pool.release_stream(reinterpret_cast<void *>(0x9999)) == 0, "an unknown stream frees nothing");
  const size_t held = rec.live.size();
  const int frees_before = rec.frees;
  const uint64_t stat_frees_before = pool.stats().frees;
  pool.release_all();
  check(rec.live.empty() && rec.frees == frees_before + (int)held, "release_all frees live and retired buffers");
  check(pool.stats().frees == stat_frees_before + held && pool.stats().live_bytes == 0 &&
            pool.stats().retired_bytes == 0,
        "stats after release");
  if (failures) return 1;
  std::printf("scratch policy ok\n");
  return 0;
}
