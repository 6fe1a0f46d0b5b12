// Independent Threefry-2x32-20 implementation for cross-checking the oracle:
// rocRAND's header-only engine (ROCm), run on the host.  Reads lines
// "k0 k1 c0 c1" (hex) on stdin and prints "x0 x1" (hex) per line.
#include <rocrand/rocrand_threefry2x32_20.h>

#include <cstdio>

struct Probe : rocrand_device::threefry2x32_20_engine {
  static uint2 run(uint2 counter, uint2 key) { return threefry_rounds(counter, key); }
};

int main() {
  unsigned k0, k1, c0, c1;
  while (std::scanf("%x %x %x %x", &k0, &k1, &c0, &c1) == 4) {
    const uint2 o = Probe::run(make_uint2(c0, c1), make_uint2(k0, k1));
    std::printf("%08x %08x\n", o.x, o.y);
  }
  return 0;
}
