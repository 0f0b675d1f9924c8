// CPU oracle for the MTP verify step. TEST INFRASTRUCTURE ONLY (see oracle.h).
//
// Built with -O3 -ffp-contract=off -fno-fast-math so every float operation is the one written
// here; fused multiply-adds appear only where std::fma is called explicitly.
#include "oracle.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <limits>
#include <thread>
#include <vector>

namespace {

constexpr int kQuantGroup = 64;   // include/ninfer/ops/gqa_attention.h:25-30
constexpr int kCandidateCap = 20; // src/ops/common/sampling_workspace.h:30-31
constexpr int kStatsPerPositionOffset = 4; // src/ops/kernel/speculative_round.cuh:15

float bits_to_f32(uint32_t b) {
    float f;
    std::memcpy(&f, &b, 4);
    return f;
}
uint32_t f32_to_bits(float f) {
    uint32_t b;
    std::memcpy(&b, &f, 4);
    return b;
}

inline float bf16(uint16_t h) { return bits_to_f32(static_cast<uint32_t>(h) << 16); }

// Ordered key: include/ninfer/ops/sampling.h:45-48 ("lower token id breaking ties") as encoded by
// src/ops/kernel/sampling_device.cuh:85-101 (-0 canonicalized to +0, value in the high word,
// 0xffffffff - id in the low word; larger key = better candidate).
uint32_t ordered_float(float v) {
    if (v == 0.0f) { v = 0.0f; }
    const uint32_t bits = f32_to_bits(v);
    return (bits & 0x80000000u) ? ~bits : (bits ^ 0x80000000u);
}

uint64_t sort_key(float v, int32_t idx) {
    return (static_cast<uint64_t>(ordered_float(v)) << 32) |
           static_cast<uint32_t>(0xffffffffu - static_cast<uint32_t>(idx));
}

int32_t key_index(uint64_t key) {
    return static_cast<int32_t>(0xffffffffu - static_cast<uint32_t>(key));
}

float key_float(uint64_t key) {
    const uint32_t o = static_cast<uint32_t>(key >> 32);
    return bits_to_f32((o & 0x80000000u) ? (o ^ 0x80000000u) : ~o);
}

} // namespace

extern "C" {

// ---- scalar numerics -------------------------------------------------------------------------

// IEEE binary32 -> binary16, round to nearest even, with subnormals, overflow to inf and NaN.
// The reference uses the hardware conversion (__float2half_rn,
// src/ops/kernel/gqa_attention_decode_i8.cuh:188-189); this is the same IEEE operation.
uint16_t orc_f32_to_f16_bits(float x) {
    const uint32_t b = f32_to_bits(x);
    const uint16_t sign = static_cast<uint16_t>((b >> 16) & 0x8000u);
    const uint32_t exp = (b >> 23) & 0xffu;
    uint32_t man = b & 0x7fffffu;
    if (exp == 0xffu) { return sign | (man ? 0x7e00u : 0x7c00u); }
    const int32_t e = static_cast<int32_t>(exp) - 127;
    if (e > 15) { return sign | 0x7c00u; }
    if (e >= -14) {
        // normal half: 10 mantissa bits, drop 13
        uint32_t m = man >> 13;
        const uint32_t rem = man & 0x1fffu;
        uint32_t h = (static_cast<uint32_t>(e + 15) << 10) | m;
        if (rem > 0x1000u || (rem == 0x1000u && (m & 1u))) { ++h; }
        return static_cast<uint16_t>(sign | h); // carry into exponent (and to inf) is correct
    }
    if (e < -25) { return sign; } // below half of the smallest subnormal
    // subnormal half: value = man_full * 2^(e-23); half subnormal unit = 2^-24
    man |= 0x800000u;
    const int shift = -e - 14 + 13; // 14..24 bits dropped
    const uint32_t m = man >> shift;
    const uint32_t rem = man & ((1u << shift) - 1u);
    const uint32_t halfway = 1u << (shift - 1);
    uint32_t h = m;
    if (rem > halfway || (rem == halfway && (m & 1u))) { ++h; }
    return static_cast<uint16_t>(sign | h);
}

float orc_f16_bits_to_f32(uint16_t h) {
    const uint32_t sign = static_cast<uint32_t>(h & 0x8000u) << 16;
    const uint32_t exp = (h >> 10) & 0x1fu;
    const uint32_t man = h & 0x3ffu;
    if (exp == 0) {
        const float v = std::ldexp(static_cast<float>(man), -24);
        return sign ? -v : v;
    }
    if (exp == 0x1f) { return bits_to_f32(sign | 0x7f800000u | (man << 13)); }
    return bits_to_f32(sign | ((exp + 112u) << 23) | (man << 13));
}

uint16_t orc_f32_to_bf16_bits(float x) {
    uint32_t b = f32_to_bits(x);
    if ((b & 0x7fffffffu) > 0x7f800000u) { return static_cast<uint16_t>((b >> 16) | 0x40u); }
    const uint32_t lsb = (b >> 16) & 1u;
    b += 0x7fffu + lsb;
    return static_cast<uint16_t>(b >> 16);
}

float orc_bf16_bits_to_f32(uint16_t h) { return bf16(h); }

// Deterministic exp shared (as an algorithm, re-implemented independently on the device) by the
// sampler oracle and the HIP sampler kernels. It replaces the reference's __expf
// (src/ops/kernel/sampling_device.cuh:199), whose bits depend on the NVIDIA device. Method:
// Cody-Waite reduction x = k ln2 + r with ln2 split in two, degree-7 Taylor polynomial for e^r on
// |r| <= ln2/2 in Horner form with explicit fma, then scaling by 2^k in two steps so subnormal
// results stay exact. Measured error below 1 ulp against the correctly rounded exp.
float orc_det_expf(float x) {
    if (!(x == x)) { return x; }
    if (x > 88.72283935546875f) { return std::numeric_limits<float>::infinity(); }
    if (x < -103.97208404541015625f) { return 0.0f; }
    const float k = std::nearbyint(x * 1.44269502162933349609375f);
    float r = std::fma(k, -0.693145751953125f, x);
    r = std::fma(k, -1.428606765330187045e-06f, r);
    float p = 1.9841270114e-04f;             // 1/5040
    p = std::fma(p, r, 1.3888889225e-03f);   // 1/720
    p = std::fma(p, r, 8.3333337680e-03f);   // 1/120
    p = std::fma(p, r, 4.1666667908e-02f);   // 1/24
    p = std::fma(p, r, 1.6666667163e-01f);   // 1/6
    p = std::fma(p, r, 5.0000000000e-01f);   // 1/2
    p = std::fma(p, r, 1.0f);
    p = std::fma(p, r, 1.0f);
    const int ki = static_cast<int>(k);
    // 2^k applied as 2^(k/2) * 2^(k - k/2): each factor is a normal float for k in [-150, 128].
    const int k1 = ki / 2;
    const int k2 = ki - k1;
    const float s1 = bits_to_f32(static_cast<uint32_t>(k1 + 127) << 23);
    const float s2 = bits_to_f32(static_cast<uint32_t>(k2 + 127) << 23);
    return (p * s1) * s2;
}

// SplitMix64 (public algorithm; src/ops/kernel/sampling_device.cuh:53-58).
uint64_t orc_splitmix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

// src/ops/kernel/sampling_device.cuh:62-73.
float orc_sampling_uniform(uint64_t seed, int32_t position, int32_t purpose, uint32_t sub) {
    uint64_t key = seed;
    key = orc_splitmix64(key ^ (static_cast<uint64_t>(static_cast<uint32_t>(position)) *
                                0xD1B54A32D192ED03ull));
    key = orc_splitmix64(key ^ (static_cast<uint64_t>(static_cast<uint32_t>(purpose)) << 21) ^
                         (static_cast<uint64_t>(sub) * 0x2545F4914F6CDD1Dull));
    const uint32_t bits = static_cast<uint32_t>(key >> 40);
    return static_cast<float>(bits) * (1.0f / 16777216.0f);
}

uint64_t orc_sort_key(float v, int32_t idx) { return sort_key(v, idx); }

// ---- INT8 group-64 codec ---------------------------------------------------------------------

// include/ninfer/ops/gqa_attention.h:25-30 (the authoritative contract; the device encoder
// src/ops/kernel/gqa_attention_decode_i8.cuh:184-199 and gqa_attention_kv_quant.cuh:50-55 agree):
//   a = max|x|, scale_bits = FP16_RNE(a/127), s = FP32(scale_bits), inv = s==0 ? 0 : FP32(1/s),
//   code = s==0 ? 0 : clamp(RNE(FP32(x*inv)), -127, 127).
void orc_quantize_group(const uint16_t* src_bf16, int32_t n, int8_t* codes, uint16_t* scale_bits) {
    float a = 0.0f;
    for (int32_t i = 0; i < n; ++i) { a = std::max(a, std::fabs(bf16(src_bf16[i]))); }
    const uint16_t sb = orc_f32_to_f16_bits(a > 0.0f ? a / 127.0f : 0.0f);
    *scale_bits = sb;
    const float s = orc_f16_bits_to_f32(sb);
    const float inv = s > 0.0f ? 1.0f / s : 0.0f;
    for (int32_t i = 0; i < n; ++i) {
        if (inv == 0.0f) {
            codes[i] = 0;
            continue;
        }
        const float prod = bf16(src_bf16[i]) * inv;
        float r = std::nearbyint(prod);
        r = std::max(-127.0f, std::min(127.0f, r));
        codes[i] = static_cast<int8_t>(r);
    }
}

// Restates the A2 append (include/ninfer/ops/gqa_attention.h:75-81) with the cache layout of
// src/core/kv_cache.cpp:69-84 (codes [D, P, Hkv], scales [D/64, P, Hkv]), plus a batch dimension.
void orc_kv_append(const uint16_t* k, const uint16_t* v, const int32_t* positions, int32_t T,
                   int32_t B, int32_t Hkv, int32_t D, int32_t padded_context, int8_t* k_codes,
                   int8_t* v_codes, uint16_t* k_scales, uint16_t* v_scales) {
    const int32_t groups = D / kQuantGroup;
    const size_t code_seq = static_cast<size_t>(D) * padded_context * Hkv;
    const size_t scale_seq = static_cast<size_t>(groups) * padded_context * Hkv;
    for (int32_t b = 0; b < B; ++b) {
        for (int32_t t = 0; t < T; ++t) {
            const int32_t pos = positions[static_cast<size_t>(b) * T + t];
            for (int32_t h = 0; h < Hkv; ++h) {
                for (int32_t g = 0; g < groups; ++g) {
                    const size_t src =
                        static_cast<size_t>(g) * kQuantGroup +
                        static_cast<size_t>(D) * (h + static_cast<size_t>(Hkv) * (t + static_cast<size_t>(T) * b));
                    const size_t code_off = b * code_seq + static_cast<size_t>(g) * kQuantGroup +
                                            static_cast<size_t>(D) * (pos + static_cast<size_t>(padded_context) * h);
                    const size_t scale_off = b * scale_seq + g +
                                             static_cast<size_t>(groups) * (pos + static_cast<size_t>(padded_context) * h);
                    orc_quantize_group(k + src, kQuantGroup, k_codes + code_off, k_scales + scale_off);
                    orc_quantize_group(v + src, kQuantGroup, v_codes + code_off, v_scales + scale_off);
                }
            }
        }
    }
}

// ---- attention -------------------------------------------------------------------------------

// FP64 ideal attention; restates cpu_gqa_decode/cpu_gqa_cached (tests/ops/test_gqa_attention.cpp:
// 228-282) with the contract of include/ninfer/ops/gqa_attention.h:52-66 (BF16 Q, FP32-decoded
// cache values, score dot products, stable softmax and value reduction in FP64). The visible key
// set generalizes the reference's `key <= positions[t]`
// (src/ops/kernel/gqa_attention_decode_i8.cuh:379-390) to an ancestor mask when `parents` is given.
// `decode(b, h, j, kd, vd)` writes row j of head h of sequence b, in FP64, to kd[0..D) / vd[0..D).
} // extern "C"
namespace {
template <class Decode>
void attention_core(const uint16_t* q, const int32_t* positions, const int32_t* parents, int32_t T,
                    int32_t B, int32_t Hq, int32_t Hkv, int32_t D, double scale, double* out,
                    int32_t threads, const Decode& decode) {
    const int32_t G = Hq / Hkv;

    auto work = [&](int32_t b, int32_t h) {
        const int32_t* pos = positions + static_cast<size_t>(b) * T;
        const int32_t L = pos[0];
        // visible[t][u]
        std::vector<uint8_t> vis(static_cast<size_t>(T) * T, 0);
        for (int32_t t = 0; t < T; ++t) {
            if (parents == nullptr) {
                for (int32_t u = 0; u <= t; ++u) { vis[static_cast<size_t>(t) * T + u] = 1; }
            } else {
                // ancestors-or-self; a parent outside [0, u) ends the walk (tree contract)
                int32_t u = t;
                vis[static_cast<size_t>(t) * T + u] = 1;
                while (true) {
                    const int32_t p = parents[static_cast<size_t>(b) * T + u];
                    if (p < 0 || p >= u) { break; }
                    vis[static_cast<size_t>(t) * T + p] = 1;
                    u = p;
                }
            }
        }
        // decode the visible rows of this head once
        std::vector<int32_t> rows;
        for (int32_t j = 0; j < L; ++j) { rows.push_back(j); }
        for (int32_t u = 0; u < T; ++u) { rows.push_back(pos[u]); }
        const size_t n = rows.size();
        std::vector<double> kd(n * D), vd(n * D);
        for (size_t r = 0; r < n; ++r) { decode(b, h, rows[r], &kd[r * D], &vd[r * D]); }
        // Query rows (t, gi) of this KV head as doubles, transposed to [D][R] so the score loop runs
        // keys outermost (each decoded key row is read once per job) while every dot product keeps
        // its own d = 0..D-1 summation order; likewise the value loop keeps the r = 0..n-1 order of
        // every output element.
        const int32_t R = T * G;
        std::vector<double> qt(static_cast<size_t>(D) * R);
        for (int32_t t = 0; t < T; ++t) {
            for (int32_t gi = 0; gi < G; ++gi) {
                const int32_t qh = h * G + gi;
                const uint16_t* qv = q + static_cast<size_t>(D) * (qh + static_cast<size_t>(Hq) * (t + static_cast<size_t>(T) * b));
                for (int32_t d = 0; d < D; ++d) { qt[static_cast<size_t>(d) * R + t * G + gi] = static_cast<double>(bf16(qv[d])); }
            }
        }
        std::vector<double> sc(static_cast<size_t>(R) * n), dot(R);
        std::vector<double> mx(R, -std::numeric_limits<double>::infinity());
        for (size_t r = 0; r < n; ++r) {
            std::fill(dot.begin(), dot.end(), 0.0);
            const double* kr = &kd[r * D];
            for (int32_t d = 0; d < D; ++d) {
                const double kv = kr[d];
                const double* qd = &qt[static_cast<size_t>(d) * R];
                for (int32_t i = 0; i < R; ++i) { dot[i] += qd[i] * kv; }
            }
            for (int32_t i = 0; i < R; ++i) {
                const int32_t t = i / G;
                const bool visible = r < static_cast<size_t>(L) || vis[static_cast<size_t>(t) * T + (r - L)];
                double& s = sc[static_cast<size_t>(i) * n + r];
                if (!visible) {
                    s = -std::numeric_limits<double>::infinity();
                    continue;
                }
                s = dot[i] * scale;
                mx[i] = std::max(mx[i], s);
            }
        }
        std::vector<double> acc(D);
        for (int32_t i = 0; i < R; ++i) {
            double* si = &sc[static_cast<size_t>(i) * n];
            double den = 0.0;
            for (size_t r = 0; r < n; ++r) {
                si[r] = std::isinf(si[r]) && si[r] < 0 ? 0.0 : std::exp(si[r] - mx[i]);
                den += si[r];
            }
            std::fill(acc.begin(), acc.end(), 0.0);
            for (size_t r = 0; r < n; ++r) {
                const double p = si[r];
                const double* vr = &vd[r * D];
                for (int32_t d = 0; d < D; ++d) { acc[d] += p * vr[d]; }
            }
            const int32_t t = i / G, gi = i % G;
            const int32_t qh = h * G + gi;
            double* o = out + static_cast<size_t>(D) * (qh + static_cast<size_t>(Hq) * (t + static_cast<size_t>(T) * b));
            for (int32_t d = 0; d < D; ++d) { o[d] = acc[d] / den; }
        }
    };

    const int32_t jobs = B * Hkv;
    int32_t nt = threads > 0 ? threads : static_cast<int32_t>(std::thread::hardware_concurrency());
    nt = std::max(1, std::min(nt, jobs));
    if (nt == 1) {
        for (int32_t j = 0; j < jobs; ++j) { work(j / Hkv, j % Hkv); }
        return;
    }
    std::vector<std::thread> pool;
    for (int32_t w = 0; w < nt; ++w) {
        pool.emplace_back([&, w]() {
            for (int32_t j = w; j < jobs; j += nt) { work(j / Hkv, j % Hkv); }
        });
    }
    for (auto& th : pool) { th.join(); }
}

} // namespace
extern "C" {

// INT8-G64 cache: value = FP32(code) * FP32(scale) (src/ops/kernel/gqa_attention_kv_quant.cuh:63-78).
void orc_attention(const uint16_t* q, const int8_t* k_codes, const int8_t* v_codes,
                   const uint16_t* k_scales, const uint16_t* v_scales, const int32_t* positions,
                   const int32_t* parents, int32_t T, int32_t B, int32_t Hq, int32_t Hkv,
                   int32_t D, int32_t padded_context, double scale, double* out, int32_t threads) {
    const int32_t groups = D / kQuantGroup;
    const size_t code_seq = static_cast<size_t>(D) * padded_context * Hkv;
    const size_t scale_seq = static_cast<size_t>(groups) * padded_context * Hkv;
    attention_core(q, positions, parents, T, B, Hq, Hkv, D, scale, out, threads,
                   [&](int32_t b, int32_t h, int32_t j, double* kd, double* vd) {
        for (int32_t g = 0; g < groups; ++g) {
            const size_t so = b * scale_seq + g + static_cast<size_t>(groups) * (j + static_cast<size_t>(padded_context) * h);
            const float ks = orc_f16_bits_to_f32(k_scales[so]);
            const float vs = orc_f16_bits_to_f32(v_scales[so]);
            for (int32_t i = 0; i < kQuantGroup; ++i) {
                const int32_t d = g * kQuantGroup + i;
                const size_t co = b * code_seq + d + static_cast<size_t>(D) * (j + static_cast<size_t>(padded_context) * h);
                kd[d] = static_cast<double>(static_cast<float>(k_codes[co]) * ks);
                vd[d] = static_cast<double>(static_cast<float>(v_codes[co]) * vs);
            }
        }
    });
}

// BF16 cache: the stored values themselves (tests/ops/test_gqa_attention.cpp:768-844 feeds the same
// FP64 oracle the BF16-rounded cache rows).
void orc_attention_bf16(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                        const int32_t* positions, const int32_t* parents, int32_t T, int32_t B,
                        int32_t Hq, int32_t Hkv, int32_t D, int32_t padded_context, double scale,
                        double* out, int32_t threads) {
    const size_t seq = static_cast<size_t>(D) * padded_context * Hkv;
    attention_core(q, positions, parents, T, B, Hq, Hkv, D, scale, out, threads,
                   [&](int32_t b, int32_t h, int32_t j, double* kd, double* vd) {
        const size_t row = b * seq + static_cast<size_t>(D) * (j + static_cast<size_t>(padded_context) * h);
        for (int32_t d = 0; d < D; ++d) {
            kd[d] = static_cast<double>(bf16(k_cache[row + d]));
            vd[d] = static_cast<double>(bf16(v_cache[row + d]));
        }
    });
}

// ---- lm_head: Q6G64_F16S RowSplit linear ----------------------------------------------------------

// Restates unpack_lowbit_code (tests/ops/row_split_pack.h:174-192) for 6-bit codes: the low nibble
// of code i sits in byte i/2 (high half for odd i), its two high bits at bit 2i of the group's high
// bytes, and the 6-bit value is sign-extended.
static int q6_code(const uint8_t* nib, const uint8_t* high, int i) {
    const uint32_t low = (i & 1) ? (nib[i >> 1] >> 4) : (nib[i >> 1] & 0x0fu);
    const uint32_t hi = (high[(2 * i) >> 3] >> ((2 * i) & 7)) & 0x03u;
    const uint32_t u = low | (hi << 4);
    return (u & 0x20u) ? static_cast<int>(u) - 64 : static_cast<int>(u);
}

// include/ninfer/ops/linear.h:17-20: exact decode, naive FP64 dot products.
void orc_linear_q6(const uint8_t* qdata, const uint8_t* qhigh, const uint16_t* scales, int32_t N,
                   int32_t K, const uint16_t* x, int32_t T, double* out, int32_t threads) {
    const int32_t Kp = (K + 127) / 128 * 128;
    const int32_t G = Kp / 64;
    std::vector<double> xf(static_cast<size_t>(K) * T);
    for (size_t i = 0; i < xf.size(); ++i) { xf[i] = static_cast<double>(bf16(x[i])); }
    auto rows = [&](int32_t r0, int32_t r1) {
        std::vector<double> w(K);
        for (int32_t n = r0; n < r1; ++n) {
            for (int32_t k = 0; k < K; ++k) {
                const size_t g = static_cast<size_t>(n) * G + k / 64;
                const int code = q6_code(qdata + g * 32, qhigh + g * 16, k % 64);
                w[k] = static_cast<double>(code) * static_cast<double>(orc_f16_bits_to_f32(scales[g]));
            }
            for (int32_t t = 0; t < T; ++t) {
                const double* xt = xf.data() + static_cast<size_t>(t) * K;
                double acc = 0.0;
                for (int32_t k = 0; k < K; ++k) { acc += w[k] * xt[k]; }
                out[n + static_cast<size_t>(N) * t] = acc;
            }
        }
    };
    int32_t nt = threads > 0 ? threads : static_cast<int32_t>(std::thread::hardware_concurrency());
    nt = std::max(1, std::min(nt, N));
    std::vector<std::thread> pool;
    for (int32_t w = 0; w < nt; ++w) {
        const int32_t r0 = static_cast<int32_t>(static_cast<int64_t>(N) * w / nt);
        const int32_t r1 = static_cast<int32_t>(static_cast<int64_t>(N) * (w + 1) / nt);
        pool.emplace_back(rows, r0, r1);
    }
    for (auto& th : pool) { th.join(); }
}

// ---- recurrent state of the hybrid layers -----------------------------------------------------

// Restates gdn_ref::forward_recurrent (tests/ops/gdn_ref.h:342-410) for one sequence, with the
// q/k normalization of normalize_qk_for_fused_oracle (tests/ops/test_gated_delta_rule.cpp:242-260).
void orc_gdn_recurrent(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* g,
                       const float* beta, const float* state_in, int32_t S, int32_t Hqk,
                       int32_t Hv, int32_t T, double scale, int32_t normalize_qk, double* out,
                       double* state_out, double* snapshots) {
    // q/k as the floats the recurrence consumes
    auto qk_rows = [&](const uint16_t* src) {
        std::vector<float> rows(static_cast<size_t>(S) * Hqk * T);
        for (size_t i = 0; i < rows.size(); ++i) { rows[i] = bf16(src[i]); }
        if (normalize_qk) {
            for (size_t r = 0; r < static_cast<size_t>(Hqk) * T; ++r) {
                float* base = rows.data() + r * S;
                double sumsq = 0.0;
                for (int32_t d = 0; d < S; ++d) { sumsq += static_cast<double>(base[d]) * static_cast<double>(base[d]); }
                const double inv = 1.0 / std::sqrt(sumsq + 1.0e-6);
                for (int32_t d = 0; d < S; ++d) { base[d] = static_cast<float>(static_cast<double>(base[d]) * inv); }
            }
        }
        return rows;
    };
    const std::vector<float> qf = qk_rows(q);
    const std::vector<float> kf = qk_rows(k);
    const size_t SS = static_cast<size_t>(S) * S;
    std::vector<double> st(SS), delta(S);
    for (int32_t h = 0; h < Hv; ++h) {
        const int32_t qh = h / (Hv / Hqk);
        for (size_t i = 0; i < SS; ++i) { st[i] = static_cast<double>(state_in[h * SS + i]); }
        for (int32_t t = 0; t < T; ++t) {
            const float* qt = qf.data() + (static_cast<size_t>(t) * Hqk + qh) * S;
            const float* kt = kf.data() + (static_cast<size_t>(t) * Hqk + qh) * S;
            const uint16_t* vt = v + (static_cast<size_t>(t) * Hv + h) * S;
            const double alpha = std::exp(static_cast<double>(g[static_cast<size_t>(t) * Hv + h]));
            const double b = static_cast<double>(beta[static_cast<size_t>(t) * Hv + h]);
            for (int32_t r = 0; r < S; ++r) {
                double* row = st.data() + static_cast<size_t>(r) * S;
                double partial = 0.0;
                for (int32_t c = 0; c < S; ++c) {
                    row[c] *= alpha;
                    partial += row[c] * static_cast<double>(kt[c]);
                }
                delta[r] = b * (static_cast<double>(bf16(vt[r])) - partial);
            }
            for (int32_t r = 0; r < S; ++r) {
                double* row = st.data() + static_cast<size_t>(r) * S;
                for (int32_t c = 0; c < S; ++c) { row[c] += delta[r] * static_cast<double>(kt[c]); }
            }
            double* ot = out + (static_cast<size_t>(t) * Hv + h) * S;
            for (int32_t r = 0; r < S; ++r) {
                const double* row = st.data() + static_cast<size_t>(r) * S;
                double partial = 0.0;
                for (int32_t c = 0; c < S; ++c) { partial += row[c] * static_cast<double>(qt[c]); }
                ot[r] = partial * scale;
            }
            if (snapshots != nullptr) {
                double* snap = snapshots + (static_cast<size_t>(t) * Hv + h) * SS;
                for (size_t i = 0; i < SS; ++i) { snap[i] = st[i]; }
            }
        }
        for (size_t i = 0; i < SS; ++i) { state_out[h * SS + i] = st[i]; }
    }
}

// Restates cpu_prefill_ref (tests/ops/test_causal_conv1d_silu.cpp:48-75): tap j of channel c at
// weight[j*C + c], window value s of channel c at state[s*C + c].
void orc_causal_conv1d_silu(const uint16_t* x, const uint16_t* weight, const uint16_t* state,
                            int32_t C, int32_t T, double* out, uint16_t* windows) {
    const size_t Cs = static_cast<size_t>(C);
    auto u = [&](int32_t c, int32_t t) -> uint16_t { // t >= -3
        return t < 0 ? state[static_cast<size_t>(3 + t) * Cs + c] : x[static_cast<size_t>(t) * Cs + c];
    };
    for (int32_t t = 0; t < T; ++t) {
        for (int32_t c = 0; c < C; ++c) {
            double acc = 0.0;
            for (int32_t j = 0; j < 4; ++j) {
                acc += static_cast<double>(bf16(weight[static_cast<size_t>(j) * Cs + c])) *
                       static_cast<double>(bf16(u(c, t - 3 + j)));
            }
            out[static_cast<size_t>(t) * Cs + c] = acc / (1.0 + std::exp(-acc));
            if (windows != nullptr) {
                for (int32_t s = 0; s < 3; ++s) {
                    windows[static_cast<size_t>(t) * 3 * Cs + static_cast<size_t>(s) * Cs + c] = u(c, t - 2 + s);
                }
            }
        }
    }
}

// ---- argmax ----------------------------------------------------------------------------------

// include/ninfer/ops/argmax.h:11-21: out[t] = min argmax_{v < valid_rows} float(logits[v,t]).
void orc_argmax(const uint16_t* logits, int32_t physical_rows, int32_t columns, int32_t valid_rows,
                int32_t* out) {
    for (int32_t c = 0; c < columns; ++c) {
        const uint16_t* col = logits + static_cast<size_t>(c) * physical_rows;
        int32_t best = 0;
        float bv = bf16(col[0]);
        for (int32_t v = 1; v < valid_rows; ++v) {
            const float x = bf16(col[v]);
            if (x > bv) {
                bv = x;
                best = v;
            }
        }
        out[c] = best;
    }
}

// ---- speculative acceptance (Mode R) -----------------------------------------------------------

// src/ops/kernel/speculative_round.cuh:19-28.
void orc_prepare_verify_inputs(int32_t token, const int32_t* drafts, int32_t length, int32_t K,
                               int32_t* verify_ids, int32_t* positions) {
    for (int32_t i = 0; i <= K; ++i) {
        verify_ids[i] = i == 0 ? token : drafts[i - 1];
        positions[i] = length + i;
    }
}

// src/ops/kernel/mtp_round.cuh (contract include/ninfer/ops/mtp_round.h:10-17): the shifted
// verify ids, then `token` at slot `accepted`; slot K keeps its previous value unless accepted == K.
void orc_mtp_prepare_alignment_ids(const int32_t* verify_ids, int32_t T, int32_t token, int32_t accepted,
                                   int32_t* alignment_ids) {
    for (int32_t i = 0; i + 1 < T; ++i) { alignment_ids[i] = verify_ids[i + 1]; }
    if (accepted >= 0 && accepted < T) { alignment_ids[accepted] = token; }
}

// Penalty: src/ops/kernel/sampling_device.cuh:137-149 (overlay = drafts[0..c-1]).
static float adjusted_logit(float raw, int32_t v, const orc_sampling_config& c,
                            const int32_t* token_counts, const int32_t* overlay, int32_t overlay_len) {
    float x = raw;
    if (c.presence_penalty == 0.0f && c.frequency_penalty == 0.0f) { return x; }
    int32_t cnt = token_counts != nullptr ? token_counts[v] : 0;
    for (int32_t j = 0; j < overlay_len; ++j) {
        if (overlay[j] == v) { ++cnt; }
    }
    if (cnt > 0) { x -= c.presence_penalty; }
    if (c.frequency_penalty != 0.0f) { x -= c.frequency_penalty * static_cast<float>(cnt); }
    return x;
}

// cap: src/ops/kernel/sampling_device.cuh:110-118. Candidates: the `cap` largest sort keys.
// normalize: src/ops/kernel/sampling_device.cuh:190-223, with __expf(x*inv_temp - m) written as
// det_expf(fma(x, inv_temp, -m)) (the contraction nvcc applies to that expression by default).
int32_t orc_truncated_distribution(const uint16_t* column, int32_t token_domain,
                                   const orc_sampling_config* cfg, const int32_t* token_counts,
                                   const int32_t* overlay, int32_t overlay_len, int32_t* cand_idx,
                                   float* prob) {
    int32_t cap = kCandidateCap;
    if (cfg->top_k > 0 && cfg->top_k < cap) { cap = cfg->top_k; }
    if (token_domain < cap) { cap = token_domain; }
    std::vector<uint64_t> keys(static_cast<size_t>(token_domain));
    for (int32_t v = 0; v < token_domain; ++v) {
        keys[v] = sort_key(adjusted_logit(bf16(column[v]), v, *cfg, token_counts, overlay, overlay_len), v);
    }
    std::partial_sort(keys.begin(), keys.begin() + cap, keys.end(), std::greater<uint64_t>());
    float cand_val[kCandidateCap];
    for (int32_t j = 0; j < cap; ++j) {
        cand_val[j] = key_float(keys[j]);
        cand_idx[j] = key_index(keys[j]);
    }
    const float inv_temp = 1.0f / cfg->temperature;
    const float m = cand_val[0] * inv_temp;
    float sum = 0.0f;
    for (int32_t j = 0; j < cap; ++j) {
        const float e = orc_det_expf(std::fma(cand_val[j], inv_temp, -m));
        prob[j] = e;
        sum += e;
    }
    const float e0 = prob[0];
    const float min_p_thresh = (cfg->min_p > 0.0f) ? cfg->min_p * e0 : -1.0f;
    const bool top_p_active = cfg->top_p < 1.0f;
    const float top_p_target = cfg->top_p * sum;
    float cum = 0.0f;
    int32_t support = 0;
    for (int32_t j = 0; j < cap; ++j) {
        if (min_p_thresh >= 0.0f && prob[j] < min_p_thresh) { break; }
        cum += prob[j];
        support = j + 1;
        if (top_p_active && cum >= top_p_target) { break; }
    }
    if (support < 1) { support = 1; }
    float ssum = 0.0f;
    for (int32_t j = 0; j < support; ++j) { ssum += prob[j]; }
    const float inv = 1.0f / ssum;
    for (int32_t j = 0; j < support; ++j) { prob[j] *= inv; }
    return support;
}

// src/ops/kernel/sampling_device.cuh:307-329.
int32_t orc_pick_from_support(const int32_t* cand_idx, const float* prob, int32_t n,
                              int32_t exclude, float u) {
    float mass = 0.0f;
    for (int32_t j = 0; j < n; ++j) {
        if (cand_idx[j] == exclude) { continue; }
        mass += prob[j];
    }
    if (mass <= 0.0f) { return cand_idx[0]; }
    const float goal = u * mass;
    float acc = 0.0f;
    int32_t picked = -1;
    for (int32_t j = 0; j < n; ++j) {
        if (cand_idx[j] == exclude) { continue; }
        acc += prob[j];
        picked = cand_idx[j];
        if (goal < acc) { return picked; }
    }
    return picked;
}

// Commit epilogue: src/ops/kernel/speculative_round.cuh:145-166 (greedy :51-72).
static void commit_round(const int32_t* drafts, int32_t K, int32_t a, int32_t tstar, int32_t L,
                         int32_t* length, int32_t* token, int32_t* sampled_out,
                         int32_t* num_sampled, int32_t* accepted, int64_t* stats) {
    for (int32_t i = 0; i <= K; ++i) { sampled_out[i] = 0; }
    for (int32_t i = 0; i < a; ++i) { sampled_out[i] = drafts[i]; }
    sampled_out[a] = tstar;
    const int32_t produced = a + 1;
    *num_sampled = produced;
    *accepted = a;
    *token = tstar;
    *length = L + produced;
    stats[0] += K;
    stats[1] += a;
    stats[2] += 1;
    for (int32_t i = 0; i < a; ++i) { stats[kStatsPerPositionOffset + i] += 1; }
}

// include/ninfer/ops/speculative_round.h:33-73; greedy branch src/ops/kernel/speculative_round.cuh:
// 51-72; sampling branch :92-166 (column i uses overlay drafts[0..i-1]; accept with
// u(L+i+1, accept) < p_i(d_i); correction from the support excluding d_i with u(L+i+1,
// correction); bonus from column K with u(L+K+1, bonus)).
void orc_speculative_accept(const int32_t* target_tokens, const uint16_t* logits,
                            int32_t physical_rows, const int32_t* drafts, int32_t K,
                            int32_t* length, int32_t* token, int32_t* sampled_out,
                            int32_t* num_sampled, int32_t* accepted, int64_t* stats,
                            int32_t token_domain, const orc_sampling_config* cfg,
                            int32_t* token_counts) {
    const int32_t L = *length;
    if (!(cfg->temperature > 0.0f)) {
        int32_t a = 0;
        while (a < K && target_tokens[a] == drafts[a]) { ++a; }
        commit_round(drafts, K, a, target_tokens[a], L, length, token, sampled_out, num_sampled,
                     accepted, stats);
        return;
    }
    int32_t a = 0;
    int32_t tstar = 0;
    int32_t cand[kCandidateCap];
    float prob[kCandidateCap];
    for (int32_t i = 0; i <= K; ++i) {
        const uint16_t* col = logits + static_cast<size_t>(i) * physical_rows;
        const int32_t n = orc_truncated_distribution(col, token_domain, cfg, token_counts, drafts, i, cand, prob);
        if (i < K) {
            const int32_t d = drafts[i];
            float pd = 0.0f;
            for (int32_t j = 0; j < n; ++j) {
                if (cand[j] == d) {
                    pd = prob[j];
                    break;
                }
            }
            const float u = orc_sampling_uniform(cfg->seed, L + i + 1, 2, 0u);
            if (u < pd) {
                a = i + 1;
                continue;
            }
            const float ur = orc_sampling_uniform(cfg->seed, L + i + 1, 3, 0u);
            tstar = orc_pick_from_support(cand, prob, n, d, ur);
            break;
        }
        const float u = orc_sampling_uniform(cfg->seed, L + K + 1, 4, 0u);
        tstar = orc_pick_from_support(cand, prob, n, -1, u);
    }
    commit_round(drafts, K, a, tstar, L, length, token, sampled_out, num_sampled, accepted, stats);
    if (token_counts != nullptr) {
        for (int32_t i = 0; i <= a; ++i) { token_counts[sampled_out[i]] += 1; }
    }
}

// ---- general acceptance (Mode F; extension, parity unpinned by the reference) ------------------

static uint32_t fixed_u24(float u) {
    float s = std::nearbyint(u * 16777216.0f);
    s = std::max(0.0f, std::min(16777216.0f, s));
    return static_cast<uint32_t>(s);
}

int32_t orc_general_column(const uint16_t* column, int32_t token_domain,
                           const orc_general_config* cfg, uint64_t* weights, uint8_t* in_nucleus,
                           uint64_t* nucleus_mass, uint64_t* total_mass) {
    float xmax = bf16(column[0]);
    for (int32_t v = 1; v < token_domain; ++v) { xmax = std::max(xmax, bf16(column[v])); }
    const float inv_temp = 1.0f / cfg->temperature;
    const float m = xmax * inv_temp;
    uint64_t z = 0;
    for (int32_t v = 0; v < token_domain; ++v) {
        const float w = orc_det_expf(std::fma(bf16(column[v]), inv_temp, -m));
        const float wf = std::nearbyint(w * 1099511627776.0f); // 2^40
        weights[v] = static_cast<uint64_t>(wf);
        z += weights[v];
    }
    *total_mass = z;
    std::vector<uint8_t> member(static_cast<size_t>(token_domain), 1);
    int32_t count = token_domain;
    uint64_t zs = z;
    if (cfg->top_p < 1.0f) {
        const uint64_t p24 = fixed_u24(cfg->top_p);
        const unsigned __int128 prod = static_cast<unsigned __int128>(z) * p24;
        const uint64_t target = static_cast<uint64_t>(prod >> 24);
        std::vector<uint64_t> keys(static_cast<size_t>(token_domain));
        for (int32_t v = 0; v < token_domain; ++v) { keys[v] = sort_key(bf16(column[v]), v); }
        std::sort(keys.begin(), keys.end(), std::greater<uint64_t>());
        std::fill(member.begin(), member.end(), 0);
        uint64_t cum = 0;
        count = 0;
        for (int32_t j = 0; j < token_domain; ++j) {
            const int32_t v = key_index(keys[j]);
            member[v] = 1;
            cum += weights[v];
            ++count;
            if (cum >= target) { break; }
        }
        zs = cum;
    }
    if (in_nucleus != nullptr) { std::memcpy(in_nucleus, member.data(), member.size()); }
    for (int32_t v = 0; v < token_domain; ++v) {
        if (!member[v]) { weights[v] = 0; }
    }
    *nucleus_mass = zs;
    return count;
}

// Inverse-CDF pick over token ids in ascending order: the first v whose running sum exceeds
// floor(U * mass / 2^24); falls back to the last v with nonzero mass.
static int32_t pick_fixed(const std::vector<unsigned __int128>& mass, unsigned __int128 total, uint32_t u24) {
    const unsigned __int128 goal = (total * u24) >> 24;
    unsigned __int128 acc = 0;
    int32_t last = 0;
    for (size_t v = 0; v < mass.size(); ++v) {
        if (mass[v] == 0) { continue; }
        acc += mass[v];
        last = static_cast<int32_t>(v);
        if (goal < acc) { return last; }
    }
    return last;
}

void orc_general_accept(const uint16_t* target_logits, const uint16_t* draft_logits,
                        int32_t physical_rows, const int32_t* drafts, int32_t K,
                        int32_t token_domain, const orc_general_config* cfg,
                        const float* u_accept, float u_residual, int32_t* length, int32_t* token,
                        int32_t* sampled_out, int32_t* num_sampled, int32_t* accepted,
                        int64_t* stats) {
    const int32_t L = *length;
    const size_t V = static_cast<size_t>(token_domain);
    std::vector<uint64_t> wp(V), wq(V);
    int32_t a = 0;
    int32_t tstar = 0;
    for (int32_t i = 0; i <= K; ++i) {
        uint64_t zp = 0, zp_all = 0;
        orc_general_column(target_logits + static_cast<size_t>(i) * physical_rows, token_domain, cfg,
                           wp.data(), nullptr, &zp, &zp_all);
        if (i == K) {
            std::vector<unsigned __int128> mass(V);
            for (size_t v = 0; v < V; ++v) { mass[v] = wp[v]; }
            tstar = pick_fixed(mass, zp, fixed_u24(u_accept[K]));
            break;
        }
        uint64_t zq = 0, zq_all = 0;
        orc_general_column(draft_logits + static_cast<size_t>(i) * physical_rows, token_domain, cfg,
                           wq.data(), nullptr, &zq, &zq_all);
        const int32_t d = drafts[i];
        const unsigned __int128 lhs = static_cast<unsigned __int128>(fixed_u24(u_accept[i])) * wq[d] * zp;
        const unsigned __int128 rhs = (static_cast<unsigned __int128>(wp[d]) * zq) << 24;
        if (lhs < rhs) {
            a = i + 1;
            continue;
        }
        // residual max(0, p - q) over the common denominator zp*zq, scaled down by 2^40
        std::vector<unsigned __int128> mass(V);
        unsigned __int128 total = 0;
        for (size_t v = 0; v < V; ++v) {
            const unsigned __int128 pv = static_cast<unsigned __int128>(wp[v]) * zq;
            const unsigned __int128 qv = static_cast<unsigned __int128>(wq[v]) * zp;
            mass[v] = pv > qv ? (pv - qv) >> 40 : 0;
            total += mass[v];
        }
        if (total == 0) {
            for (size_t v = 0; v < V; ++v) { mass[v] = wp[v]; }
            total = zp;
        }
        tstar = pick_fixed(mass, total, fixed_u24(u_residual));
        break;
    }
    commit_round(drafts, K, a, tstar, L, length, token, sampled_out, num_sampled, accepted, stats);
}

// ---- commit / rollback / compaction ------------------------------------------------------------

void orc_kv_commit_prefix(const uint16_t* k, const uint16_t* v, const int32_t* positions,
                          int32_t T, int32_t commit_count, int32_t Hkv, int32_t D,
                          int32_t padded_context, int8_t* k_codes, int8_t* v_codes,
                          uint16_t* k_scales, uint16_t* v_scales) {
    (void)T;
    orc_kv_append(k, v, positions, commit_count, 1, Hkv, D, padded_context, k_codes, v_codes,
                  k_scales, v_scales);
    // orc_kv_append indexes the source by its own T; commit_count columns of a T-column tensor share
    // the same leading layout because the batch dimension is 1.
}

void orc_kv_rollback(const int32_t* positions, int32_t T, int32_t keep_count, int32_t Hkv,
                     int32_t D, int32_t padded_context, int8_t* k_codes, int8_t* v_codes,
                     uint16_t* k_scales, uint16_t* v_scales) {
    const int32_t groups = D / kQuantGroup;
    for (int32_t i = keep_count; i < T; ++i) {
        const int32_t pos = positions[i];
        for (int32_t h = 0; h < Hkv; ++h) {
            const size_t co = static_cast<size_t>(D) * (pos + static_cast<size_t>(padded_context) * h);
            std::memset(k_codes + co, 0, D);
            std::memset(v_codes + co, 0, D);
            const size_t so = static_cast<size_t>(groups) * (pos + static_cast<size_t>(padded_context) * h);
            for (int32_t g = 0; g < groups; ++g) {
                k_scales[so + g] = 0;
                v_scales[so + g] = 0;
            }
        }
    }
}

void orc_kv_compact_path(int32_t base, const int32_t* path, int32_t count, int32_t Hkv, int32_t D,
                         int32_t padded_context, int8_t* k_codes, int8_t* v_codes,
                         uint16_t* k_scales, uint16_t* v_scales) {
    const int32_t groups = D / kQuantGroup;
    for (int32_t j = 0; j < count; ++j) {
        const int32_t src = base + path[j];
        const int32_t dst = base + j;
        if (src == dst) { continue; }
        for (int32_t h = 0; h < Hkv; ++h) {
            const size_t cs = static_cast<size_t>(D) * (src + static_cast<size_t>(padded_context) * h);
            const size_t cd = static_cast<size_t>(D) * (dst + static_cast<size_t>(padded_context) * h);
            std::memmove(k_codes + cd, k_codes + cs, D);
            std::memmove(v_codes + cd, v_codes + cs, D);
            const size_t ss = static_cast<size_t>(groups) * (src + static_cast<size_t>(padded_context) * h);
            const size_t sd = static_cast<size_t>(groups) * (dst + static_cast<size_t>(padded_context) * h);
            for (int32_t g = 0; g < groups; ++g) {
                k_scales[sd + g] = k_scales[ss + g];
                v_scales[sd + g] = v_scales[ss + g];
            }
        }
    }
}

// ---- tree verification ---------------------------------------------------------------------------

int32_t orc_tree_longest_path(const int32_t* parents, const int32_t* node_tokens,
                              const int32_t* target_tokens, int32_t nodes, int32_t* path) {
    std::vector<int32_t> depth(static_cast<size_t>(nodes), -1);
    depth[0] = 0;
    int32_t best = 0;
    for (int32_t u = 1; u < nodes; ++u) {
        const int32_t p = parents[u];
        if (p < 0 || p >= u || depth[p] < 0) { continue; }
        if (node_tokens[u] != target_tokens[p]) { continue; }
        depth[u] = depth[p] + 1;
        if (depth[u] > depth[best]) { best = u; }
    }
    const int32_t len = depth[best] + 1;
    int32_t u = best;
    for (int32_t j = len - 1; j >= 0; --j) {
        path[j] = u;
        u = parents[u];
    }
    return len;
}

} // extern "C"
