// Test-input generation for workload-sized parity tests. TEST INFRASTRUCTURE ONLY: this is not a
// restatement of the reference; it fills host arrays with seeded normals far faster than numpy can
// (10^8-value KV histories), deterministically for any thread count.
//
// Element i of a stream draws two 53-bit uniforms from SplitMix64 over the counters 2i and 2i+1
// (the public finalizer, Steele et al. 2014), turns them into one N(0,1) value by Box-Muller in
// double, scales by `std`, and with probability `outlier_frac` (a third counter) replaces it by
// +-outlier_value. The float is rounded to BF16 by round-to-nearest-even.
#include "oracle.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

namespace {

uint64_t mix(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

double unit(uint64_t seed, uint64_t counter) {
    return static_cast<double>(mix(seed + counter * 0x9E3779B97F4A7C15ull) >> 11) * (1.0 / 9007199254740992.0);
}

uint16_t to_bf16(float f) {
    uint32_t b;
    std::memcpy(&b, &f, 4);
    return static_cast<uint16_t>((b + 0x7FFFu + ((b >> 16) & 1u)) >> 16);
}

} // namespace

extern "C" {

void orc_fill_normal_bf16(uint64_t seed, size_t n, float std_dev, float outlier_frac,
                          float outlier_value, uint16_t* out, int32_t threads) {
    const double two_pi = 6.283185307179586476925286766559;
    auto fill = [&](size_t lo, size_t hi) {
        for (size_t i = lo; i < hi; ++i) {
            const double u1 = std::max(unit(seed, 3 * i), 1e-300);
            const double u2 = unit(seed, 3 * i + 1);
            float x = static_cast<float>(std::sqrt(-2.0 * std::log(u1)) * std::cos(two_pi * u2)) * std_dev;
            if (outlier_frac > 0.0f) {
                const uint64_t r = mix(seed ^ (0xD1B54A32D192ED03ull * (i + 1)));
                if (static_cast<double>(r >> 11) * (1.0 / 9007199254740992.0) < outlier_frac) {
                    x = (r & 1u) ? -outlier_value : outlier_value;
                }
            }
            out[i] = to_bf16(x);
        }
    };
    const size_t chunk = size_t{1} << 20;
    const size_t chunks = (n + chunk - 1) / chunk;
    const int32_t nt = static_cast<int32_t>(std::max<size_t>(1, std::min<size_t>(threads > 0 ? threads : 1, chunks)));
    std::vector<std::thread> pool;
    for (int32_t w = 0; w < nt; ++w) {
        pool.emplace_back([&, w]() {
            for (size_t c = w; c < chunks; c += nt) { fill(c * chunk, std::min(n, (c + 1) * chunk)); }
        });
    }
    for (auto& t : pool) { t.join(); }
}

} // extern "C"
