/* Emits the stop-points feature table as C float literals (hex, exact):
 * entry p = log2f(1 + p) / 12, clamped to 1 (include/cugo/game/torch50.h:405-408),
 * evaluated with this host's C library, as the reference engine evaluates it. */
#include <math.h>
#include <stdio.h>

int main(void) {
  for (int p = 0; p < 4095; ++p) {
    volatile float one = 1.0f;
    const float bits = log2f(one + (float)p) / 12.0f;
    const float v = bits > 1.0f ? 1.0f : bits;
    printf("%af,%s", (double)v, (p % 4 == 3) ? "\n" : " ");
  }
  printf("\n");
  return 0;
}
