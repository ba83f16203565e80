/* TEST INFRASTRUCTURE ONLY.  Exports the reference's host-side FP4 -> E4M3
 * expansion (cuda/fp4_unpack.cuh:45-55, compiled from /root/reference by
 * oracle/Makefile) so tests can compare it word by word with our oracle. */
#include "fp4_unpack.cuh"

uint32_t ref_fp4x4_to_e4m3x4(uint32_t p) { return fp4x4_to_e4m3x4(p); }

void ref_fp4x8_to_e4m3x8(uint32_t p, uint32_t *lo, uint32_t *hi) { fp4x8_to_e4m3x8(p, lo, hi); }

uint8_t ref_fp4_code_to_e4m3(uint8_t code) { return fp4_code_to_e4m3_ref(code); }
