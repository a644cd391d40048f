// Host-only check that readout_expf (the readout's exponential, ncas_amd/csrc/nca_device.h) is
// non-decreasing on [-87, 0]: for every pair of adjacent floats d1 < d2 of that range,
// readout_expf(d1) <= readout_expf(d2). The gated-firing decision of the C = 32 streamed kernel
// compares the logit gap with a limit instead of evaluating the exponential, which is exact only
// under this property. Prints the number of decreasing steps; exit status 0 when there are none.
#include <cstdio>
#include <cstring>
#include <thread>
#include <vector>

#include "../ncas_amd/csrc/nca_device.h"

static float from_bits(uint32_t b) {
    float f;
    std::memcpy(&f, &b, 4);
    return f;
}

int main() {
    const uint32_t top = 0x42ae0000u;  // 87.0f
    const int nt = 8;
    std::vector<long> bad(nt, 0);
    std::vector<std::thread> th;
    for (int t = 0; t < nt; ++t) {
        // magnitudes [lo, hi] (inclusive; a chunk's hi is the next chunk's lo, so every adjacent
        // pair is checked), walked from hi down to lo, that is, with the gap d = -m increasing
        const uint32_t lo = (uint32_t)((uint64_t)top * t / nt), hi = (uint32_t)((uint64_t)top * (t + 1) / nt);
        th.emplace_back([lo, hi, t, &bad]() {
            float prev = nca::readout_expf(-from_bits(hi));
            for (uint32_t b = hi; b-- > lo;) {
                const float e = nca::readout_expf(-from_bits(b));
                if (e < prev) ++bad[t];
                prev = e;
            }
        });
    }
    long total = 0;
    for (int t = 0; t < nt; ++t) {
        th[t].join();
        total += bad[t];
    }
    // below -87 the argument is clamped, so the value there is readout_expf(-87)
    if (nca::readout_expf(-1.0e30f) != nca::readout_expf(-87.0f)) ++total;
    std::printf("decreasing steps: %ld\n", total);
    return total != 0;
}
