// Deterministic sampler primitives shared by the gfx950 acceptance kernels.
//
// Bit-exactness across CPU and GPU needs every float operation pinned: this header is compiled
// with FP contraction disabled, every fused multiply-add is an explicit fmaf, division is the
// correctly rounded HIP default, and the exponential is the project's own (not the device libm).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "sampler_internal.h"

#pragma clang fp contract(off)

namespace nmi {

// Deterministic exp: Cody-Waite reduction with ln2 split into 0x3f317200 + 0x35bfbe8e, degree-7
// Taylor polynomial on |r| <= ln2/2 (Horner, explicit fma), 2^k applied in two normal-range steps.
// The same algorithm runs in the CPU oracle, so results are bit-identical.
//
// det_exp_poly is its reduction and polynomial for x in [-103.972..., 88.722...]: e^x ~ p * 2^k.
__device__ __forceinline__ float det_exp_poly(float x, int* k_out) {
    const float k = __builtin_rintf(x * 1.44269502162933349609375f);
    float r = __builtin_fmaf(k, -0.693145751953125f, x);
    r = __builtin_fmaf(k, -1.428606765330187045e-06f, r);
    float p = 1.9841270114e-04f;
    p = __builtin_fmaf(p, r, 1.3888889225e-03f);
    p = __builtin_fmaf(p, r, 8.3333337680e-03f);
    p = __builtin_fmaf(p, r, 4.1666667908e-02f);
    p = __builtin_fmaf(p, r, 1.6666667163e-01f);
    p = __builtin_fmaf(p, r, 5.0000000000e-01f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    *k_out = static_cast<int>(k);
    return p;
}

__device__ __forceinline__ bool det_exp_in_range(float x) {
    return x >= -103.97208404541015625f && x <= 88.72283935546875f;
}

__device__ __forceinline__ float det_expf(float x) {
    if (!(x == x)) { return x; }
    if (x > 88.72283935546875f) { return __builtin_inff(); }
    if (x < -103.97208404541015625f) { return 0.0f; }
    int ki;
    const float p = det_exp_poly(x, &ki);
    const int k1 = ki / 2;
    const int k2 = ki - k1;
    const float s1 = __uint_as_float(static_cast<uint32_t>(k1 + 127) << 23);
    const float s2 = __uint_as_float(static_cast<uint32_t>(k2 + 127) << 23);
    return (p * s1) * s2;
}

// SplitMix64 and the counter-based uniform (src/ops/kernel/sampling_device.cuh:53-73).
__device__ __forceinline__ uint64_t splitmix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

__device__ __forceinline__ float sampling_uniform(uint64_t seed, int32_t position, int32_t purpose,
                                                  uint32_t sub) {
    uint64_t key = seed;
    key = splitmix64(key ^ (static_cast<uint64_t>(static_cast<uint32_t>(position)) * 0xD1B54A32D192ED03ull));
    key = splitmix64(key ^ (static_cast<uint64_t>(static_cast<uint32_t>(purpose)) << 21) ^
                     (static_cast<uint64_t>(sub) * 0x2545F4914F6CDD1Dull));
    const uint32_t bits = static_cast<uint32_t>(key >> 40);
    return static_cast<float>(bits) * (1.0f / 16777216.0f);
}

// Ordered candidate key: value in the high word (-0 canonicalized to +0), 0xffffffff - id in the
// low word, larger = better (src/ops/kernel/sampling_device.cuh:85-108).
__device__ __forceinline__ uint32_t ordered_float(float v) {
    if (v == 0.0f) { v = 0.0f; }
    const uint32_t bits = __float_as_uint(v);
    return (bits & 0x80000000u) ? ~bits : (bits ^ 0x80000000u);
}

__device__ __forceinline__ uint64_t sort_key(float v, int32_t idx) {
    return (static_cast<uint64_t>(ordered_float(v)) << 32) |
           static_cast<uint32_t>(0xffffffffu - static_cast<uint32_t>(idx));
}

__device__ __forceinline__ float key_float(uint64_t key) {
    const uint32_t o = static_cast<uint32_t>(key >> 32);
    return __uint_as_float((o & 0x80000000u) ? (o ^ 0x80000000u) : ~o);
}

__device__ __forceinline__ int32_t key_index(uint64_t key) {
    return static_cast<int32_t>(0xffffffffu - static_cast<uint32_t>(key));
}

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int mask) {
    const int lo = __shfl_xor(static_cast<int>(v & 0xffffffffu), mask, 64);
    const int hi = __shfl_xor(static_cast<int>(v >> 32), mask, 64);
    return (static_cast<uint64_t>(static_cast<uint32_t>(hi)) << 32) | static_cast<uint32_t>(lo);
}

// One DPP step of the wave-wide maximum: the value of the lane that CTRL selects (0, the smallest
// key, where that lane lies outside the row or is masked off).
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint64_t dpp_max_u64(uint64_t v) {
    const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v & 0xffffffffu), CTRL, ROW_MASK, 0xf, false));
    const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v >> 32), CTRL, ROW_MASK, 0xf, false));
    const uint64_t o = (static_cast<uint64_t>(hi) << 32) | lo;
    return o > v ? o : v;
}

// Wave-wide maximum (row shifts 1, 2, 4, 8, then row broadcasts 15 and 31: lane 63 holds it, and
// every lane reads it back). The whole wave must be active.
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
    v = dpp_max_u64<0x111, 0xf>(v);
    v = dpp_max_u64<0x112, 0xf>(v);
    v = dpp_max_u64<0x114, 0xf>(v);
    v = dpp_max_u64<0x118, 0xf>(v);
    v = dpp_max_u64<0x142, 0xa>(v);
    v = dpp_max_u64<0x143, 0xc>(v);
    const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v & 0xffffffffu), 63));
    const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v >> 32), 63));
    return (static_cast<uint64_t>(hi) << 32) | lo;
}

} // namespace nmi
