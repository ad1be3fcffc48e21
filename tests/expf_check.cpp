// Checks the restatement of glibc's expf that the device's output post-processing computes (the steps of
// expf_glibc in katago-rs_amd/csrc/kgx_post.hip, with the constants of katago-rs_amd/csrc/kgx_expf.h) against the
// host's expf, bit for bit. Arguments: the stride over the float bit patterns of [-110, 90] (1 checks every one).
// Prints the number of floats checked and of mismatches.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "../katago-rs_amd/csrc/kgx_expf.h"

static float bits_f(uint32_t u) { float f; std::memcpy(&f, &u, 4); return f; }
static uint32_t f_bits(float f) { uint32_t u; std::memcpy(&u, &f, 4); return u; }

static float restated(float x) {
  const uint32_t u = f_bits(x), abstop = (u >> 20) & 0x7ff;
  if (abstop >= (0x42b00000u >> 20)) {
    if (u == 0xff800000u) return 0.f;
    if (abstop >= (0x7f800000u >> 20)) return x + x;
    if (x > bits_f(0x42b17217u)) return bits_f(0x7f800000u);
    if (x < bits_f(0xc2cff1b4u)) return 0.f;
    if (x < bits_f(0xc2ce8ecfu)) return bits_f(1u);
  }
  const double xd = (double)x;
  double kd = std::fma(kgx_exp2f_invln2n, xd, kgx_exp2f_shift);
  uint64_t ki;
  std::memcpy(&ki, &kd, 8);
  kd -= kgx_exp2f_shift;
  const double r = std::fma(kgx_exp2f_invln2n, xd, -kd);
  const uint64_t t = kgx_exp2f_tab[ki % 32] + (ki << 47);
  double sc;
  std::memcpy(&sc, &t, 8);
  const double z = std::fma(kgx_exp2f_c0, r, kgx_exp2f_c1);
  const double r2 = r * r;
  double y = std::fma(kgx_exp2f_c2, r, 1.0);
  y = std::fma(z, r2, y);
  y *= sc;
  return (float)y;
}

int main(int argc, char** argv) {
  const uint64_t stride = argc > 1 ? std::strtoull(argv[1], nullptr, 10) : 1;
  long checked = 0, bad = 0;
  for (uint64_t u = 0; u < 0x100000000ULL; u += stride) {
    const float x = bits_f((uint32_t)u);
    if (!(x >= -110.f && x <= 90.f)) continue;
    checked++;
    const float a = std::exp(x), b = restated(x);
    if (f_bits(a) != f_bits(b)) {
      if (bad < 5) std::printf("mismatch x=%a host=%a restated=%a\n", x, a, b);
      bad++;
    }
  }
  // The special inputs: infinities, NaN, the edges of the underflow and overflow paths.
  const float special[] = {bits_f(0x7f800000u), bits_f(0xff800000u), bits_f(0x7fc00000u), bits_f(0x42b17217u),
                           bits_f(0x42b17218u), bits_f(0xc2cff1b4u), bits_f(0xc2cff1b3u), bits_f(0xc2ce8ecfu),
                           bits_f(0xc2ce8eceu), 0.f, -0.f};
  for (float x : special) {
    checked++;
    const float a = std::exp(x), b = restated(x);
    if (f_bits(a) != f_bits(b) && !(a != a && b != b)) {
      std::printf("mismatch x=%a host=%a restated=%a\n", x, a, b);
      bad++;
    }
  }
  std::printf("%ld %ld\n", checked, bad);
  return 0;
}
