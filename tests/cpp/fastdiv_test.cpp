// Host unit test of nvf::FastDiv (the launch-constant divider the kernels use
// for row / column splits): every divisor the ops can see at BASELINE shapes
// plus random and edge divisors, against plain integer division on numerators
// that include 0, 2^32-1 and values around multiples of the divisor.
#include <cstdint>
#include <cstdio>
#include <random>

#include "../../nano_vllm_cpp_amd/csrc/nvf_device.hpp"

int main() {
  std::mt19937_64 rng(7);
  std::vector<uint32_t> divisors = {1, 2, 3, 5, 7, 8, 64, 100, 112, 224, 448, 512, 592, 1536, 2368, 2372,
                                    4736, 18944, 65535, 65536, 65537, 0x7fffffffu, 0x80000000u, 0x80000001u,
                                    0xfffffffeu, 0xffffffffu};
  for (int i = 0; i < 2000; ++i) divisors.push_back((uint32_t)(rng() % 0xffffffffu) + 1);
  for (int i = 0; i < 200; ++i) divisors.push_back((uint32_t)(rng() % 5000) + 1);
  uint64_t checked = 0, bad = 0;
  for (uint32_t d : divisors) {
    const nvf::FastDiv f(d);
    auto check = [&](uint32_t n) {
      ++checked;
      if (f.div(n) != n / d) {
        if (bad++ < 5) std::printf("FastDiv(%u).div(%u) = %u, want %u\n", d, n, f.div(n), n / d);
      }
    };
    for (uint32_t n : {0u, 1u, d - 1, d, d + 1, 0xffffffffu, 0xfffffffeu, 0x80000000u}) check(n);
    for (uint64_t k = 1; k < 64; ++k) {
      const uint64_t n = (uint64_t)d * (rng() % (0xffffffffull / d + 1));
      if (n <= 0xffffffffull) check((uint32_t)n), check((uint32_t)(n - 1 + (n == 0)));
    }
    for (int i = 0; i < 256; ++i) check((uint32_t)rng());
  }
  std::printf("FastDiv: %llu checks, %llu wrong\n", (unsigned long long)checked, (unsigned long long)bad);
  return bad ? 1 : 0;
}
