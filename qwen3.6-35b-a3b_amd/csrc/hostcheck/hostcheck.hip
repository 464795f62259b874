// Host-callable builds of device helpers whose arithmetic the CPU tests check directly (no GPU
// needed): libmoe_hostcheck.so, test infrastructure only; the product library does not link it.
#include "../router_dev.h"

extern "C" {

// R1's certified rounding: 1 and *bits = the bf16 of s when no rounding midpoint lies within
// `bound` of s, else 0.
int moe_hostcheck_round_bf16(double s, double bound, uint32_t* bits) {
  return moe::round_bf16_certified(s, bound, bits) ? 1 : 0;
}

}  // extern "C"
