// Host-side probe of rocRAND's open-source philox4x32-10 (test infrastructure only).
// Reads lines "c0 c1 c2 c3 k0 k1" on stdin and prints the four output words of
// ten rounds, so tests can compare the oracle's Philox restatement with rocRAND's.
#include <rocrand/rocrand_philox4x32_10.h>

#include <cstdio>

struct Probe : rocrand_device::philox4x32_10_engine {
    uint4 run(uint4 c, uint2 k) { return ten_rounds(c, k); }
};

int main() {
    unsigned c0, c1, c2, c3, k0, k1;
    Probe p;
    while (std::scanf("%u %u %u %u %u %u", &c0, &c1, &c2, &c3, &k0, &k1) == 6) {
        uint4 o = p.run(uint4{c0, c1, c2, c3}, uint2{k0, k1});
        std::printf("%u %u %u %u\n", o.x, o.y, o.z, o.w);
    }
    return 0;
}
