/* Host check of the arithmetic identity behind the kernels' div3_rn
 * (rvc-vulkan_amd/csrc/internal.h): for every float32 bit pattern x that is
 * not a NaN,
 *
 *   q0 = RN(x * RN(1/3)),  q = fma(fma(-q0, 3, x), RN(1/3), q0),
 *   (q0 == 0 || |q0| == inf) ? q0 : q   ==   RN(x / 3)   bit for bit.
 *
 * The decoder averages its three ResBlock outputs as ((o1 + o2) + o3) / 3
 * (runtime/models/vits.py:2225-2227); the identity lets the GPU form that
 * quotient without the full division sequence and stay bit-identical.
 * Built with contraction off so x * r is rounded on its own, as __fmul_rn
 * rounds it on the device.  Prints the number of patterns checked and of
 * mismatches; exits 1 on any mismatch. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float from_bits(uint32_t u) {
  float x;
  memcpy(&x, &u, 4);
  return x;
}
static uint32_t to_bits(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  return u;
}

int main(void) {
  const float r = 0x1.555556p-2f;
  long long checked = 0, bad = 0;
  if (to_bits(r) != to_bits(1.0f / 3.0f)) {
    printf("r is not RN(1/3)\n");
    return 1;
  }
#pragma omp parallel for reduction(+ : checked, bad) schedule(static)
  for (long long i = 0; i < (1LL << 32); ++i) {
    const float x = from_bits((uint32_t)i);
    if (isnan(x)) continue;
    ++checked;
    const float q0 = x * r;
    const float q = fmaf(fmaf(-q0, 3.0f, x), r, q0);
    const float got = (q0 == 0.0f || isinf(q0)) ? q0 : q;
    if (to_bits(got) != to_bits(x / 3.0f)) ++bad;
  }
  printf("checked %lld mismatches %lld\n", checked, bad);
  return bad != 0;
}
