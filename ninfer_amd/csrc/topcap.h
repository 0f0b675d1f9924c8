// Exact top-cap candidate selection shared by the stochastic acceptance kernels and the fused
// lm_head: wave-level selection over unique 64-bit ordered keys, the candidate cap and the
// penalty-adjusted logit (reference src/ops/kernel/sampling_device.cuh:110-149).
#pragma once

#include "sampler_common.h"

#pragma clang fp contract(off)

namespace nmi {

__device__ __forceinline__ int candidate_cap(const nmi_sampling_config& cfg, int32_t vocab) {
    int cap = kCandidateCap; // src/ops/kernel/sampling_device.cuh:110-118
    if (cfg.top_k > 0 && cfg.top_k < cap) { cap = cfg.top_k; }
    if (vocab < cap) { cap = vocab; }
    return cap;
}

// src/ops/kernel/sampling_device.cuh:137-149; overlay = drafts[0..col-1].
__device__ __forceinline__ float adjusted_logit(float raw, int v, const nmi_sampling_config& c,
                                                const int32_t* overlay, int overlay_len) {
    float x = raw;
    if (c.presence_penalty == 0.0f && c.frequency_penalty == 0.0f) { return x; }
    int cnt = c.token_counts != nullptr ? c.token_counts[v] : 0;
    for (int j = 0; j < overlay_len; ++j) {
        if (overlay[j] == v) { ++cnt; }
    }
    if (cnt > 0) { x = x - c.presence_penalty; }
    if (c.frequency_penalty != 0.0f) { x = x - c.frequency_penalty * static_cast<float>(cnt); }
    return x;
}

// ---- exact top-cap selection over unique 64-bit keys (0 = empty slot) -----------------------------
//
// A wave never extracts its keys one by one. A threshold T with at least cap keys >= T is found
// first, with ballots only: MSB-first bit selection over the high words (ordered values) of a few
// representative keys, the lane maxima or list heads. The keys >= T (a few dozen for real logits)
// are compacted into LDS, and each one's rank is the number of candidates above it, so rank r goes
// to out[r]. When more than 64 keys reach T (heavy ties), the exact cap-th largest key is found by a
// 64-bit bit selection over every key and the ranking repeats with exactly cap candidates.

__device__ __forceinline__ uint32_t key_high(uint64_t k) { return static_cast<uint32_t>(k >> 32); }

// Lanes below this one that are set in `mask`.
__device__ __forceinline__ int lanes_below(uint64_t mask) {
    return static_cast<int>(__builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mask >> 32),
                                                      __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask), 0u)));
}

// Orders one wave's LDS writes before its later reads of the same slots by other lanes.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// A threshold on the high words of the wave's M values per lane (0 = no value): the largest t
// whose low 16 bits are zero with at least cap values whose high word is >= t (the cap-th largest
// high word with its low half cleared; the high words of BF16 logits have no low half). 0 when
// fewer than cap values exist.
template <int M>
__device__ __forceinline__ uint32_t wave_cap_high(const uint32_t (&hi)[M], int cap) {
    uint32_t t = 0;
#pragma unroll 1
    for (int bit = 31; bit >= 16; --bit) {
        const uint32_t c = t | (1u << bit);
        int n = 0;
#pragma unroll
        for (int m = 0; m < M; ++m) { n += __popcll(__ballot(hi[m] >= c)); }
        if (n >= cap) { t = c; }
    }
    return t;
}

// The exact cap-th largest key among the wave's N keys per lane (0 when fewer than cap exist).
template <int N>
__device__ __forceinline__ uint64_t wave_cap_key(const uint64_t (&k)[N], int cap) {
    uint64_t t = 0;
#pragma unroll 1
    for (int bit = 63; bit >= 0; --bit) {
        const uint64_t c = t | (1ull << bit);
        int n = 0;
#pragma unroll
        for (int e = 0; e < N; ++e) { n += __popcll(__ballot(k[e] >= c)); }
        if (n >= cap) { t = c; }
    }
    return t;
}

// Ranks the candidates {k[e] != 0, k[e] >= T} if there are at most 64 of them: the cap largest
// go to out[0..cap) in descending order, 0-padded. cand: 64 slots of wave-private LDS.
template <int N>
__device__ __forceinline__ bool wave_rank_top(const uint64_t (&k)[N], uint64_t T, int cap, uint64_t* cand,
                                              uint64_t* out) {
    const int lane = threadIdx.x & 63;
    int total = 0;
#pragma unroll
    for (int e = 0; e < N; ++e) { total += __popcll(__ballot(k[e] != 0 && k[e] >= T)); }
    if (total > 64) { return false; }
    int base = 0;
#pragma unroll
    for (int e = 0; e < N; ++e) {
        const bool sel = k[e] != 0 && k[e] >= T;
        const uint64_t mask = __ballot(sel);
        if (sel) { cand[base + lanes_below(mask)] = k[e]; }
        base += __popcll(mask);
    }
    wave_lds_sync();
    if (lane < total) {
        const uint64_t key = cand[lane];
        int r = 0;
        // eight LDS reads in flight per step (the 64 slots are the wave's own; those at or past
        // total are not counted)
#pragma unroll 1
        for (int j0 = 0; j0 < total; j0 += 8) {
            uint64_t cj[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) { cj[u] = cand[(j0 + u) & 63]; }
#pragma unroll
            for (int u = 0; u < 8; ++u) { r += (j0 + u < total && cj[u] > key) ? 1 : 0; }
        }
        if (r < cap) { out[r] = key; }
    } else if (lane < cap) {
        out[lane] = 0;
    }
    wave_lds_sync();
    return true;
}

// Top cap of the wave's N keys per lane; `heads` are one or more keys per lane that include every
// lane's (or list's) largest key, so at least cap keys reach the threshold derived from them.
template <int N, int M>
__device__ __forceinline__ void wave_top_cap(const uint64_t (&k)[N], const uint64_t (&heads)[M], int cap,
                                             uint64_t* cand, uint64_t* out) {
    uint32_t hi[M];
#pragma unroll
    for (int m = 0; m < M; ++m) { hi[m] = key_high(heads[m]); }
    const uint64_t T = static_cast<uint64_t>(wave_cap_high(hi, cap)) << 32;
    if (!wave_rank_top(k, T, cap, cand, out)) { wave_rank_top(k, wave_cap_key(k, cap), cap, cand, out); }
}

} // namespace nmi
