/*
 * hp_synth.c -- host-side SplitMix64 stream for the synthetic workloads.
 *
 * Draw i (0-based, counted from `start`) of stream `seed` is
 * mix(seed + (start + i + 1) * 0x9E3779B97F4A7C15), the counter form that
 * heliopause_amd/synthetic.py defines; this file only computes it faster
 * than numpy for the half-gigabyte output head and the 42-layer model
 * (threads split the range; the result does not depend on the split).
 */
#include <pthread.h>
#include <stdint.h>

static uint64_t mix(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

typedef struct {
  uint64_t seed, first, count;
  uint64_t *out;
} Job;

static void *run(void *p) {
  const Job *j = (const Job *)p;
  uint64_t z = j->seed + (j->first + 1) * 0x9E3779B97F4A7C15ull;
  for (uint64_t i = 0; i < j->count; i++, z += 0x9E3779B97F4A7C15ull) j->out[i] = mix(z);
  return 0;
}

/* out[0 .. n) = draws start .. start + n - 1 of stream seed; 0 on success. */
int hp_synth_splitmix64(uint64_t seed, uint64_t start, uint64_t n, uint64_t *out, int threads) {
  if (threads < 1) threads = 1;
  if (threads > 64) threads = 64;
  if (n < (1u << 20)) threads = 1;
  pthread_t th[64];
  Job jobs[64];
  const uint64_t per = (n + (uint64_t)threads - 1) / (uint64_t)threads;
  int started = 0;
  for (int t = 0; t < threads; t++) {
    const uint64_t a = (uint64_t)t * per;
    if (a >= n) break;
    jobs[t].seed = seed;
    jobs[t].first = start + a;
    jobs[t].count = n - a < per ? n - a : per;
    jobs[t].out = out + a;
    if (t == 0) continue;
    if (pthread_create(&th[t], 0, run, &jobs[t]) != 0) {
      run(&jobs[t]);
      jobs[t].count = 0;
    }
    started = t;
  }
  run(&jobs[0]);
  for (int t = 1; t <= started; t++)
    if (jobs[t].count) pthread_join(th[t], 0);
  return 0;
}
