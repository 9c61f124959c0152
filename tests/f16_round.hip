// CPU check of rs_f16_bits (heliopause_amd/csrc/hp_attn.h), the device
// kernels' f32 -> f16 rounding of the query, against the oracle's
// restatement of float32_to_float16 (lib.rs:2534-2569) on every one of the
// 2^32 f32 bit patterns.  Host code only; no GPU is involved.
#include <cstdio>
#include <cstring>
#include <thread>
#include <vector>

#include "hp_attn.h"

extern "C" uint16_t hpo_f32_to_f16_rust(float v);

int main() {
  const unsigned threads = 8;
  std::vector<unsigned long long> bad(threads, 0), first(threads, ~0ull);
  std::vector<std::thread> pool;
  for (unsigned t = 0; t < threads; t++)
    pool.emplace_back([&, t] {
      const unsigned long long span = (1ull << 32) / threads;
      for (unsigned long long b = t * span; b < (t + 1) * span; b++) {
        float f;
        const uint32_t u = (uint32_t)b;
        memcpy(&f, &u, 4);
        if (hp::rs_f16_bits(u) != hpo_f32_to_f16_rust(f)) {
          if (!bad[t]) first[t] = b;
          bad[t]++;
        }
      }
    });
  for (auto &th : pool) th.join();
  unsigned long long total = 0;
  for (unsigned t = 0; t < threads; t++) {
    total += bad[t];
    if (bad[t]) printf("first mismatch %08llx\n", first[t]);
  }
  printf("f16 rounding mismatches %llu\n", total);
  return total ? 1 : 0;
}
