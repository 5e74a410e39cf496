// Host build of the engine's deal (cugo_amd/csrc/engine.h create_env + pack_row) as a
// small C library for tests/test_cpu_engine_host.py, which compares whole rows with the
// oracle's create.  TEST INFRASTRUCTURE ONLY.
#include <cstdint>

#include "engine.h"

using namespace cugo_amd;

extern "C" {

// rows [n, 31] words: the row create_env deals from seeds[i] with first player first[i] & 1.
void host_create_rows(const int64_t* seeds, const int64_t* first, int64_t n, uint64_t* rows) {
  for (int64_t i = 0; i < n; ++i)
    pack_row(create_env((u64)seeds[i], (u32)(first[i] & 1)), rows + i * kRowWords);
}

// Up to `count` seeds from start, start + step, ... whose 28 deal draws include one in
// Lemire's rejection zone (the draw-by-draw path of create_env); returns how many.
int64_t host_rejection_seeds(uint64_t start, uint64_t step, int64_t count, int64_t* out) {
  int64_t found = 0;
  for (uint64_t seed = start; found < count; seed += step) {
    u64 s = seed;
    for (u32 k = 0; k < 28; ++k) {
      const u64 product = (u64)(u32)(sm_next(s) >> 32) * (50u - k);
      if ((u32)product < 50u - k) {
        out[found++] = (int64_t)seed;
        break;
      }
    }
  }
  return found;
}

}  // extern "C"
