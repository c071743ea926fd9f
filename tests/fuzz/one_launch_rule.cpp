// The one-launch prepare -> GEMM rule (k2w8_gemm_plan.hpp: one_launch_fits) on the
// BASELINE shapes and over a sweep: it admits exactly whole rounds of 256x192 tiles.
#include <cstdio>
#include <cstdlib>

#include "k2w8_gemm_plan.hpp"

#define REQ(c) do { if (!(c)) { std::printf("violated: %s (line %d)\n", #c, __LINE__); std::exit(1); } } while (0)

int main() {
  using k2w8::one_launch_fits;
  const long cus = 256;
  // configs[1] QKV: 16 x 48 = 768 tiles, 3 rounds; the north star: 16 x 64 = 1024, 4
  REQ(one_launch_fits(4096, 4096, 9216, 3072, 3072, 3072, cus));
  REQ(one_launch_fits(4096, 4096, 12288, 3072, 3072, 3072, cus));
  // configs[3] at M=4544: 18 x 48 = 864 tiles, not whole rounds; configs[0]: 16 x 16
  REQ(!one_launch_fits(4544, 4544, 9216, 3072, 3072, 3072, cus));
  REQ(one_launch_fits(4096, 4096, 3072, 3072, 3072, 3072, cus));
  // rows wider than the prepare phase holds, strides that differ, m other than tokens
  REQ(!one_launch_fits(4096, 4096, 12288, 6144, 6144, 6144, cus));
  REQ(!one_launch_fits(4096, 4096, 12288, 3072, 3072, 3136, cus));
  REQ(!one_launch_fits(4096, 4095, 12288, 3072, 3072, 3072, cus));
  REQ(!one_launch_fits(4096, 4096, 12288, 3072, 3072, 3072, 0));
  long admitted = 0;
  for (long m = 1; m <= 20000; m += 37)
    for (long n = 128; n <= 40000; n += 64) {
      const bool fits = one_launch_fits(m, m, n, 3072, 3072, 3072, cus);
      const long tiles = (n % 192 == 0) ? ((m + 255) / 256) * (n / 192) : -1;
      REQ(fits == (tiles > 0 && tiles % cus == 0));
      admitted += fits;
    }
  std::printf("admitted %ld\n", admitted);
  return 0;
}
