// CPU check of the scratch policy in heliopause_amd/csrc/hp_scratch.h with a
// recording allocator: a buffer handed out (as a captured graph would hold
// it) stays allocated until release_all, growth is refused while capturing,
// streams never share a buffer, and only release_all frees.
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
  const size_t held = rec.live.size();
  pool.release_all();
  check(rec.live.empty() && rec.frees == (int)held, "release_all frees live and retired buffers");
  check(pool.stats().frees == (uint64_t)held && pool.stats().live_bytes == 0, "stats after release");
  if (failures) return 1;
  std::printf("scratch policy ok\n");
  return 0;
}
