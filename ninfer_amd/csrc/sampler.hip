// On-GPU acceptance for the MTP verify step (gfx950): argmax, verify-input preparation, greedy and
// reference-stochastic ("Mode R", top-20 candidate cap) speculative acceptance, accepted-hidden
// selection and greedy tree acceptance.
//
// Reference semantics: include/ninfer/ops/{argmax,sampling,speculative_round}.h and
// src/ops/kernel/{argmax,speculative_round,sampling_device}.cuh. The stochastic route keeps the
// reference's two-launch shape (per-tile candidates, then merge + accept with a last-block
// hand-off) but replaces the CUB block merge sort with wave-level extraction over 64-bit ordered
// keys, and __expf with the deterministic det_expf shared with the CPU oracle.
#include "common.h"
#include "device_utils.h"
#include "sampler_internal.h"
#include "sampler_common.h"
#include "topcap.h"

#pragma clang fp contract(off)

namespace nmi {
namespace {

// ---- wave top-k over 64-bit keys ------------------------------------------------------------------

template <int N>
__device__ __forceinline__ void cas_desc(uint64_t (&k)[N], int i, int j) {
    const uint64_t a = k[i];
    const uint64_t b = k[j];
    const bool sw = b > a;
    k[i] = sw ? b : a;
    k[j] = sw ? a : b;
}

// Bitonic sort, descending, fully unrolled (N a power of two).
template <int N>
__device__ __forceinline__ void sort_desc(uint64_t (&k)[N]) {
#pragma unroll
    for (int size = 2; size <= N; size <<= 1) {
#pragma unroll
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
#pragma unroll
            for (int i = 0; i < N; ++i) {
                const int j = i ^ stride;
                if (j > i) {
                    if ((i & size) == 0) {
                        cas_desc(k, i, j);
                    } else {
                        cas_desc(k, j, i);
                    }
                }
            }
        }
    }
}

// Writes the wave's `cap` largest keys (descending, 0-padded) to out[0..cap). Keys are unique
// except the 0 pad, so exactly one lane owns each extracted nonzero key.
template <int N>
__device__ __forceinline__ void wave_topk(uint64_t (&k)[N], int cap, uint64_t* out) {
    sort_desc(k);
    const int lane = threadIdx.x & 63;
    for (int r = 0; r < cap; ++r) {
        const uint64_t best = wave_max_u64(k[0]);
        if (lane == 0) { out[r] = best; }
        if (best != 0 && k[0] == best) {
#pragma unroll
            for (int i = 0; i + 1 < N; ++i) { k[i] = k[i + 1]; }
            k[N - 1] = 0;
        }
    }
}

// ---- argmax ---------------------------------------------------------------------------------------

typedef unsigned short us2 __attribute__((ext_vector_type(2)));

// Two BF16 values -> their 16-bit ordered keys (larger key = larger value; NaN ordered as by bits,
// -0 one below +0): negative halves are inverted, non-negative ones get the sign bit set.
__device__ __forceinline__ us2 ordered16x2(uint32_t w) {
    const uint32_t neg = (w >> 15) & 0x00010001u;
    return __builtin_bit_cast(us2, w ^ (0x80008000u | (neg * 0x7fffu)));
}

// Largest ordered key among the 8 BF16 values of one 16-byte load.
__device__ __forceinline__ uint32_t max_ordered8(const i4& raw) {
    us2 m = __builtin_elementwise_max(ordered16x2(static_cast<uint32_t>(raw[0])), ordered16x2(static_cast<uint32_t>(raw[1])));
    m = __builtin_elementwise_max(m, __builtin_elementwise_max(ordered16x2(static_cast<uint32_t>(raw[2])),
                                                               ordered16x2(static_cast<uint32_t>(raw[3]))));
    return m[0] > m[1] ? m[0] : m[1];
}

__device__ __forceinline__ uint16_t bf16_at(const i4& raw, int e) {
    const uint32_t w = static_cast<uint32_t>(raw[e >> 1]);
    return static_cast<uint16_t>((e & 1) ? (w >> 16) : (w & 0xffffu));
}

// One 1024-thread block per column. Pass 1 keeps, per thread, the largest 16-bit ordered key of
// its 16-byte loads (packed max, 2 values per instruction) and the first load that reached it;
// the winning element and its full key (value, then lowest id; -0 equals +0) are resolved from that
// one load afterwards. A thread whose largest value is a zero rescans its loads for the first
// zero of either sign.
__global__ __launch_bounds__(1024) void argmax_kernel(const uint16_t* logits, int32_t* out,
                                                      int32_t physical_rows, int32_t valid_rows,
                                                      int64_t column_stride) {
    const int col = blockIdx.x;
    const uint16_t* x = logits + static_cast<int64_t>(col) * column_stride;
    uint64_t best = 0;
    const bool aligned = (reinterpret_cast<uintptr_t>(x) & 15u) == 0;
    const int vec = aligned ? valid_rows / 8 : 0;
    const int step = static_cast<int>(blockDim.x);
    constexpr int kArgmaxUnroll = 8; // independent 16-byte loads in flight per thread
    uint32_t top = 0;
    int top_load = -1;
    for (int i0 = threadIdx.x; i0 < vec; i0 += kArgmaxUnroll * step) {
        i4 raw[kArgmaxUnroll];
#pragma unroll
        for (int u = 0; u < kArgmaxUnroll; ++u) {
            const int i = i0 + u * step;
            raw[u] = i < vec ? *reinterpret_cast<const i4*>(x + 8 * i) : i4{0, 0, 0, 0};
        }
#pragma unroll
        for (int u = 0; u < kArgmaxUnroll; ++u) {
            const int i = i0 + u * step;
            const uint32_t m = max_ordered8(raw[u]);
            const bool take = i < vec && (m > top || top_load < 0);
            top = take ? m : top;
            top_load = take ? i : top_load;
        }
    }
    if (top_load >= 0) {
        if (top == 0x8000u || top == 0x7fffu) {
            // Largest value is a zero: the first zero of either sign among this thread's loads.
            for (int i = threadIdx.x; i < vec; i += step) {
                const i4 raw = *reinterpret_cast<const i4*>(x + 8 * i);
                int e0 = -1;
#pragma unroll
                for (int e = 7; e >= 0; --e) { e0 = (bf16_at(raw, e) & 0x7fffu) == 0 ? e : e0; }
                if (e0 >= 0) {
                    best = sort_key(0.0f, 8 * i + e0);
                    break;
                }
            }
        } else {
            const i4 raw = *reinterpret_cast<const i4*>(x + 8 * top_load);
            int e0 = 7;
#pragma unroll
            for (int e = 7; e >= 0; --e) {
                const uint16_t h = bf16_at(raw, e);
                const uint32_t o = (h & 0x8000u) ? (~h & 0xffffu) : (h | 0x8000u);
                e0 = o == top ? e : e0;
            }
            best = sort_key(bf16_to_f32(bf16_at(raw, e0)), 8 * top_load + e0);
        }
    }
    for (int v = 8 * vec + threadIdx.x; v < valid_rows; v += blockDim.x) {
        const uint64_t key = sort_key(bf16_to_f32(x[v]), v);
        best = key > best ? key : best;
    }
    best = wave_max_u64(best);
    __shared__ uint64_t wbest[16];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    if (lane == 0) { wbest[wave] = best; }
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t b = 0;
        for (int w = 0; w < static_cast<int>(blockDim.x / 64); ++w) { b = wbest[w] > b ? wbest[w] : b; }
        out[col] = key_index(b);
    }
    (void)physical_rows;
}

// Multi-workgroup argmax: one 256-thread workgroup per (tile of kArgmaxTile rows, column), one
// 16-byte load per thread (measured on MI355X at [248320, 4]: 2,048-row tiles, 488 workgroups, take
// the greedy acceptance from 8.4 to 6.5 us; 16,384-row tiles leave most CUs idle). The tile's best key (value as an ordered float with -0 = +0,
// then the lowest row) is folded into out[col] by a compare-and-swap loop on the row index, which
// compares against the key of the row out[col] holds at that moment (the reference's tiled atomic
// route, src/ops/kernel/argmax.cuh:96-129). The reference zeroes out first with a memset
// (src/ops/launcher/argmax.cu); here nothing needs initializing: a value outside [0, valid_rows)
// counts as no candidate, and a row inside it is a real candidate whose key the argmax beats or
// equals, so the loop ends at the argmax whatever out held before the call.
constexpr int kArgmaxLoads = 1;                  // 16-byte loads per thread
constexpr int kArgmaxTile = 256 * 8 * kArgmaxLoads;

__global__ __launch_bounds__(256) void argmax_tile_kernel(const uint16_t* logits, int32_t* out,
                                                          int32_t valid_rows, int64_t column_stride) {
    const int col = blockIdx.y;
    const uint16_t* x = logits + static_cast<int64_t>(col) * column_stride;
    const int base = blockIdx.x * kArgmaxTile + threadIdx.x * 8;
    int32_t* slot = out + col;
    // The column's current holder and its key, read by thread 0 while the tile's loads are in
    // flight. out only ever moves to a strictly larger key, so a holder read early that already
    // beats the tile still does; a stale one makes the compare-and-swap below fail and retry.
    int cur = -1;
    uint64_t ck = 0;
    const auto read_holder = [&] {
        if (threadIdx.x == 0) {
            cur = __hip_atomic_load(slot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            ck = (cur >= 0 && cur < valid_rows) ? sort_key(bf16_to_f32(x[cur]), cur) : 0ull;
        }
    };
    uint64_t best = 0;
    if ((reinterpret_cast<uintptr_t>(x) & 15u) == 0) {
        i4 raw[kArgmaxLoads];
#pragma unroll
        for (int u = 0; u < kArgmaxLoads; ++u) {
            const int r0 = base + u * 256 * 8;
            raw[u] = r0 + 8 <= valid_rows ? *reinterpret_cast<const i4*>(x + r0) : i4{0, 0, 0, 0};
        }
        read_holder();
#pragma unroll
        for (int u = 0; u < kArgmaxLoads; ++u) {
            const int r0 = base + u * 256 * 8;
            if (r0 + 8 <= valid_rows) {
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const uint64_t k = sort_key(bf16_to_f32(bf16_at(raw[u], e)), r0 + e);
                    best = k > best ? k : best;
                }
            } else {
                for (int v = r0; v < valid_rows && v < r0 + 8; ++v) {
                    const uint64_t k = sort_key(bf16_to_f32(x[v]), v);
                    best = k > best ? k : best;
                }
            }
        }
    } else {
        read_holder();
        for (int u = 0; u < kArgmaxLoads; ++u) {
            for (int e = 0; e < 8; ++e) {
                const int v = base + u * 256 * 8 + e;
                if (v < valid_rows) {
                    const uint64_t k = sort_key(bf16_to_f32(x[v]), v);
                    best = k > best ? k : best;
                }
            }
        }
    }
    best = wave_max_u64(best);
    __shared__ uint64_t wbest[4];
    if ((threadIdx.x & 63) == 0) { wbest[threadIdx.x >> 6] = best; }
    __syncthreads();
    if (threadIdx.x != 0) { return; }
    best = wbest[0];
#pragma unroll
    for (int w = 1; w < 4; ++w) { best = wbest[w] > best ? wbest[w] : best; }
    if (best == 0) { return; } // no row of this tile is below valid_rows
    const int mine = key_index(best);
    while (true) {
        if (ck >= best) { break; } // keys are unique per row: the holder is at least as good
        const int seen = atomicCAS(slot, cur, mine);
        if (seen == cur) { break; }
        cur = seen;
        ck = (cur >= 0 && cur < valid_rows) ? sort_key(bf16_to_f32(x[cur]), cur) : 0ull;
    }
}

// ---- verify inputs ---------------------------------------------------------------------------------

// src/ops/kernel/speculative_round.cuh:19-28, per sequence b.
__global__ void prepare_verify_inputs_kernel(const int32_t* token, const int32_t* drafts,
                                             const int32_t* length, int32_t* verify_ids,
                                             int32_t* positions, int32_t K) {
    const int b = blockIdx.x;
    for (int i = threadIdx.x; i <= K; i += blockDim.x) {
        verify_ids[b * (K + 1) + i] = i == 0 ? token[b] : drafts[b * K + i - 1];
        positions[b * (K + 1) + i] = length[b] + i;
    }
}

__device__ int pick_from_support(const int32_t* cand_idx, const float* prob, int n, int exclude, float u) {
    float mass = 0.0f; // src/ops/kernel/sampling_device.cuh:307-329
    for (int j = 0; j < n; ++j) {
        if (cand_idx[j] == exclude) { continue; }
        mass = mass + prob[j];
    }
    if (mass <= 0.0f) { return cand_idx[0]; }
    const float goal = u * mass;
    float acc = 0.0f;
    int picked = -1;
    for (int j = 0; j < n; ++j) {
        if (cand_idx[j] == exclude) { continue; }
        acc = acc + prob[j];
        picked = cand_idx[j];
        if (goal < acc) { return picked; }
    }
    return picked;
}

// ---- Mode R launch 1: per-tile top-cap candidates ------------------------------------------------

__global__ __launch_bounds__(256) void spec_tile_topk_kernel(SpecArgs a) {
    const int tile = blockIdx.x;
    const int col = blockIdx.y;
    const int b = blockIdx.z;
    const nmi_sampling_config cfg = a.config[b];
    if (!(cfg.temperature > 0.0f)) { return; }
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int cap = candidate_cap(cfg, a.token_domain);
    const uint16_t* x = a.logits + static_cast<int64_t>(b) * a.logits_seq_stride + static_cast<int64_t>(col) * a.physical_rows;
    const int32_t* drafts = a.drafts + static_cast<int64_t>(b) * a.K;
    const int base = tile * kTileTokens + wave * 1024 + lane * 16;
    uint64_t keys[16];
    const bool vec_ok = base + 16 <= a.token_domain && ((reinterpret_cast<uintptr_t>(x + base) & 15u) == 0);
    if (vec_ok) {
        const i4 r0 = *reinterpret_cast<const i4*>(x + base);
        const i4 r1 = *reinterpret_cast<const i4*>(x + base + 8);
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const uint32_t w = static_cast<uint32_t>(e < 8 ? r0[e >> 1] : r1[(e - 8) >> 1]);
            const uint16_t bits = static_cast<uint16_t>((e & 1) ? (w >> 16) : (w & 0xffffu));
            const float v = adjusted_logit(bf16_to_f32(bits), base + e, cfg, drafts, col);
            keys[e] = sort_key(v, base + e);
        }
    } else {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int v = base + e;
            keys[e] = v < a.token_domain ? sort_key(adjusted_logit(bf16_to_f32(x[v]), v, cfg, drafts, col), v) : 0ull;
        }
    }
    __shared__ uint64_t cand[4][64];
    __shared__ uint64_t wtop[4][kCandidateCap];
    __shared__ uint64_t btop[kCandidateCap];
    uint64_t head[1] = {keys[0]};
#pragma unroll
    for (int e = 1; e < 16; ++e) { head[0] = keys[e] > head[0] ? keys[e] : head[0]; }
    wave_top_cap(keys, head, cap, cand[wave], wtop[wave]);
    if (threadIdx.x < cap) { btop[threadIdx.x] = 0; }
    __syncthreads();
    // Block merge: key i of wave w's descending list ranks i + (keys of the other lists above it).
    if (lane < cap) {
        const uint64_t key = wtop[wave][lane];
        if (key != 0) {
            int r = lane;
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                if (w == wave) { continue; }
                for (int j = 0; j < cap; ++j) { r += wtop[w][j] > key ? 1 : 0; }
            }
            if (r < cap) { btop[r] = key; }
        }
    }
    __syncthreads();
    if (threadIdx.x < cap) {
        uint64_t* dst = a.partial + ((static_cast<int64_t>(b) * a.columns + col) * a.ntiles + tile) * kCandidateCap;
        dst[threadIdx.x] = btop[threadIdx.x];
    }
}

// ---- Mode R launch 2: per-sequence merge, distributions and the sequential accept -----------------

// Key j of a candidate list (descending, 0-padded; slots past cap are never read).
__device__ __forceinline__ uint64_t list_key(const i4& v, int half) {
    return (static_cast<uint64_t>(static_cast<uint32_t>(v[2 * half + 1])) << 32) | static_cast<uint32_t>(v[2 * half]);
}

// The cap largest keys of up to 64 * LISTS descending lists (lane j holds lists j, j + 64, ...) into
// out[0..cap), descending and 0-padded. The threshold T from the list heads bounds the answer from
// below (cap heads reach it), so only keys >= T matter; a list's keys >= T form a prefix, and the
// first kPrefix of every list are read first. When no list has more than kPrefix keys >= T (the
// usual case: the top candidates spread over many lists), the prefixes are ranked directly;
// otherwise every key of every list is loaded and ranked.
template <int LISTS>
__device__ __forceinline__ void merge_sorted_lists(const uint64_t* part, int nlists, int cap, uint64_t* cand,
                                                   uint64_t* out) {
    constexpr int kPrefix = 4;
    const int lane = threadIdx.x & 63;
    uint64_t k[LISTS * kPrefix];
    uint64_t heads[LISTS];
    uint32_t hi[LISTS];
#pragma unroll
    for (int h = 0; h < LISTS; ++h) {
        const int j = lane + 64 * h;
        if (j < nlists) {
            const i4* src = reinterpret_cast<const i4*>(part + static_cast<int64_t>(j) * kCandidateCap);
            const i4 v0 = src[0];
            const i4 v1 = src[1];
            k[h * kPrefix + 0] = list_key(v0, 0);
            k[h * kPrefix + 1] = list_key(v0, 1);
            k[h * kPrefix + 2] = list_key(v1, 0);
            k[h * kPrefix + 3] = list_key(v1, 1);
        } else {
#pragma unroll
            for (int e = 0; e < kPrefix; ++e) { k[h * kPrefix + e] = 0; }
        }
#pragma unroll
        for (int e = 0; e < kPrefix; ++e) {
            if (e >= cap) { k[h * kPrefix + e] = 0; } // slots past cap were never written
        }
        heads[h] = k[h * kPrefix];
        hi[h] = key_high(heads[h]);
    }
    const uint64_t T = static_cast<uint64_t>(wave_cap_high(hi, cap)) << 32;
    bool deep = false;
#pragma unroll
    for (int h = 0; h < LISTS; ++h) {
        const uint64_t last = k[h * kPrefix + kPrefix - 1];
        deep = deep || (kPrefix < cap && last != 0 && last >= T);
    }
    if (!__any(deep) && wave_rank_top(k, T, cap, cand, out)) { return; }
    uint64_t lk[LISTS * kCandidateCap];
#pragma unroll
    for (int h = 0; h < LISTS; ++h) {
        const int j = lane + 64 * h;
        if (j < nlists) {
            const i4* src = reinterpret_cast<const i4*>(part + static_cast<int64_t>(j) * kCandidateCap);
#pragma unroll
            for (int q = 0; q < kCandidateCap / 2; ++q) {
                const i4 v = src[q];
                lk[h * kCandidateCap + 2 * q] = list_key(v, 0);
                lk[h * kCandidateCap + 2 * q + 1] = list_key(v, 1);
            }
        } else {
#pragma unroll
            for (int q = 0; q < kCandidateCap; ++q) { lk[h * kCandidateCap + q] = 0; }
        }
#pragma unroll
        for (int q = 0; q < kCandidateCap; ++q) {
            if (q >= cap) { lk[h * kCandidateCap + q] = 0; }
        }
    }
    wave_top_cap(lk, heads, cap, cand, out);
}


// One workgroup per sequence; wave w merges columns w, w + 4, ... (lane j holds lists j, j + 64, ...,
// LISTS per lane), builds each column's truncated distribution in LDS, then thread 0 runs the accept.
// The lists are the per-tile candidates of spec_tile_topk_kernel, or (target_tokens null) the
// per-workgroup candidates of the fused lm_head, whose keys of a greedy sequence are the raw logits:
// the greedy target of a column is then the largest list head.
template <int LISTS>
__global__ __launch_bounds__(256) void spec_merge_accept_kernel(SpecArgs a) {
    const int b = blockIdx.x;
    const nmi_sampling_config cfg = a.config[b];
    const int K = a.K;
    const int32_t* drafts = a.drafts + static_cast<int64_t>(b) * K;
    int32_t* length = a.length + b;
    int32_t* token = a.token + b;
    int32_t* sampled_out = a.sampled_out + static_cast<int64_t>(b) * (K + 1);
    int32_t* num_sampled = a.num_sampled + b;
    int32_t* accepted = a.accepted + b;
    int64_t* stats = a.stats + static_cast<int64_t>(b) * a.stats_stride;

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    if (!(cfg.temperature > 0.0f)) {
        // Greedy: src/ops/kernel/speculative_round.cuh:51-72.
        __shared__ int32_t g_target[kMaxColumns];
        const int32_t* target = a.target_tokens + static_cast<int64_t>(b) * (K + 1);
        if (a.target_tokens == nullptr) {
            for (int col = wave; col <= K; col += 4) {
                const uint64_t* part = a.partial + (static_cast<int64_t>(b) * a.columns + col) * a.ntiles * kCandidateCap;
                uint64_t h = 0;
#pragma unroll
                for (int q = 0; q < LISTS; ++q) {
                    const int j = lane + 64 * q;
                    const uint64_t v = j < a.ntiles ? part[static_cast<int64_t>(j) * kCandidateCap] : 0ull;
                    h = v > h ? v : h;
                }
                h = wave_max_u64(h);
                if (lane == 0) { g_target[col] = key_index(h); }
            }
            __syncthreads();
            target = g_target;
        }
        // One wave: every input is loaded at once, the accepted prefix is the first mismatch
        // (ballot), and the lanes write the round's commit (src/ops/kernel/speculative_round.cuh:
        // 145-166: drafts [0, a) then the target token, zero padded; length advances by a + 1;
        // statistics) in parallel, from the values read here.
        if (wave == 0) {
            static_assert(kMaxColumns <= 64 && kStatsPerPositionOffset + kMaxColumns <= 64, "one wave per sequence");
            const int32_t tg = lane <= K ? target[lane] : 0;
            const int32_t dr = lane < K ? drafts[lane] : 0;
            const int64_t st = lane < a.stats_stride ? stats[lane] : 0;
            const int32_t len0 = *length;
            const uint64_t mism = __ballot(lane < K && tg != dr);
            const int acc = mism != 0ull ? __ffsll(static_cast<long long>(mism)) - 1 : K;
            const int32_t tstar = __shfl(tg, acc, 64);
            if (lane <= K) { sampled_out[lane] = lane < acc ? dr : (lane == acc ? tstar : 0); }
            if (lane == 0) {
                *num_sampled = acc + 1;
                *accepted = acc;
                *token = tstar;
                *length = len0 + acc + 1;
            }
            const int64_t add = lane == 0 ? K : lane == 1 ? acc : lane == 2 ? 1
                                : (lane >= kStatsPerPositionOffset && lane - kStatsPerPositionOffset < acc) ? 1 : 0;
            if (lane < a.stats_stride && add != 0) { stats[lane] = st + add; }
        }
        return;
    }

    const int cap = candidate_cap(cfg, a.token_domain);
    // The commit's inputs, loaded while the candidate lists merge.
    __shared__ int32_t s_dr[kMaxColumns];
    __shared__ int64_t s_st[64];
    __shared__ int32_t s_len;
    __shared__ int32_t s_res[2]; // accepted drafts, sampled token
    if (static_cast<int>(threadIdx.x) < K) { s_dr[threadIdx.x] = drafts[threadIdx.x]; }
    if (static_cast<int>(threadIdx.x) < 64 && static_cast<int>(threadIdx.x) < a.stats_stride) { s_st[threadIdx.x] = stats[threadIdx.x]; }
    if (threadIdx.x == 0) { s_len = *length; }
    __shared__ uint64_t cand[4][64];
    __shared__ uint64_t top[4][kCandidateCap];
    __shared__ float e_sh[4][kCandidateCap];
    __shared__ int32_t d_idx[kMaxColumns][kCandidateCap];
    __shared__ float d_prob[kMaxColumns][kCandidateCap];
    __shared__ int32_t d_n[kMaxColumns];
    const float inv_temp = 1.0f / cfg.temperature;
    for (int col = wave; col <= K; col += 4) {
        const uint64_t* part = a.partial + (static_cast<int64_t>(b) * a.columns + col) * a.ntiles * kCandidateCap;
        merge_sorted_lists<LISTS>(part, a.ntiles, cap, cand[wave], top[wave]);
        // src/ops/kernel/sampling_device.cuh:190-223 with det_expf(fma(x, inv_temp, -m)).
        const float m = key_float(top[wave][0]) * inv_temp;
        if (lane < cap) {
            const uint64_t key = top[wave][lane];
            d_idx[col][lane] = key_index(key);
            e_sh[wave][lane] = det_expf(__builtin_fmaf(key_float(key), inv_temp, -m));
        }
        wave_lds_sync();
        if (lane == 0) {
            const float* e = e_sh[wave];
            float sum = 0.0f;
            for (int j = 0; j < cap; ++j) { sum = sum + e[j]; }
            const float e0 = e[0];
            const float min_p_thresh = (cfg.min_p > 0.0f) ? cfg.min_p * e0 : -1.0f;
            const bool top_p_active = cfg.top_p < 1.0f;
            const float top_p_target = cfg.top_p * sum;
            float cum = 0.0f;
            int support = 0;
            for (int j = 0; j < cap; ++j) {
                if (min_p_thresh >= 0.0f && e[j] < min_p_thresh) { break; }
                cum = cum + e[j];
                support = j + 1;
                if (top_p_active && cum >= top_p_target) { break; }
            }
            if (support < 1) { support = 1; }
            float ssum = 0.0f;
            for (int j = 0; j < support; ++j) { ssum = ssum + e[j]; }
            const float inv = 1.0f / ssum;
            for (int j = 0; j < support; ++j) { d_prob[col][j] = e[j] * inv; }
            d_n[col] = support;
        }
        wave_lds_sync();
    }
    __syncthreads();
    if (wave != 0) { return; }
    const int L = s_len;
    if (lane == 0) {
    // Sequential accept: src/ops/kernel/speculative_round.cuh:337-366.
    int acc = 0;
    int tstar = 0;
    for (int i = 0; i <= K; ++i) {
        const int n = d_n[i];
        const int32_t* cidx = d_idx[i];
        const float* cprob = d_prob[i];
        if (i < K) {
            const int dtok = s_dr[i];
            float pd = 0.0f;
            for (int j = 0; j < n; ++j) {
                if (cidx[j] == dtok) {
                    pd = cprob[j];
                    break;
                }
            }
            const float u = sampling_uniform(cfg.seed, L + i + 1, kPurposeAccept, 0u);
            if (u < pd) {
                acc = i + 1;
                continue;
            }
            const float ur = sampling_uniform(cfg.seed, L + i + 1, kPurposeCorrection, 0u);
            tstar = pick_from_support(cidx, cprob, n, dtok, ur);
            break;
        }
        const float u = sampling_uniform(cfg.seed, L + K + 1, kPurposeBonus, 0u);
        tstar = pick_from_support(cidx, cprob, n, -1, u);
    }
    s_res[0] = acc;
    s_res[1] = tstar;
    }
    wave_lds_sync();
    // The round's commit (src/ops/kernel/speculative_round.cuh:145-166) by the lanes, from the
    // values read at entry.
    const int acc = s_res[0];
    const int32_t tstar = s_res[1];
    const int32_t out = lane < acc ? s_dr[lane] : (lane == acc ? tstar : 0);
    if (lane <= K) { sampled_out[lane] = out; }
    if (lane == 0) {
        *num_sampled = acc + 1;
        *accepted = acc;
        *token = tstar;
        *length = L + acc + 1;
    }
    const int64_t add = lane == 0 ? K : lane == 1 ? acc : lane == 2 ? 1
                        : (lane >= kStatsPerPositionOffset && lane - kStatsPerPositionOffset < acc) ? 1 : 0;
    if (lane < a.stats_stride && add != 0) { stats[lane] = s_st[lane] + add; }
    if (cfg.token_counts != nullptr && lane <= acc) { atomicAdd(&cfg.token_counts[out], 1); }
}

// ---- MTP alignment ids (include/ninfer/ops/mtp_round.h:10-20) ------------------------------------
// alignment_ids[i] = verify_ids[i + 1] (i < K), then alignment_ids[accepted] = token; slot K keeps
// its previous value unless accepted == K. An accepted count outside [0, K] writes no token.
__global__ void mtp_alignment_ids_kernel(const int32_t* verify_ids, const int32_t* token,
                                         const int32_t* accepted, int32_t* alignment_ids, int32_t T) {
    const int i = threadIdx.x;
    const int acc = *accepted;
    if (i + 1 < T) { alignment_ids[i] = i == acc ? *token : verify_ids[i + 1]; }
    if (i == T - 1 && acc == T - 1) { alignment_ids[i] = *token; }
}

// ---- accepted hidden (include/ninfer/ops/speculative_round.h:76-87) -------------------------------
__global__ void select_hidden_kernel(const uint16_t* hidden, const int32_t* accepted, uint16_t* out,
                                     int32_t rows, int32_t cols) {
    const int row = blockIdx.x * blockDim.x + threadIdx.x;
    if (row >= rows) { return; }
    const int c = *accepted;
    if (c < 0 || c >= cols) { return; }
    out[row] = hidden[static_cast<int64_t>(c) * rows + row];
}

// ---- greedy tree acceptance ------------------------------------------------------------------------
// Node u > 0 is accepted iff its parent is accepted and node_tokens[u] == target_tokens[parent];
// the deepest accepted node wins (lowest index on ties).
// One wave per tree: the lanes load the tree (parents, node tokens, targets), the length and the
// statistics in one round trip; lane 0 walks the depths over LDS (node u needs its parent's depth,
// so the walk stays sequential); the lanes then write the path, the sampled tokens and the
// statistics.
__global__ __launch_bounds__(64) void tree_accept_kernel(const int32_t* parents, const int32_t* node_tokens,
                                                         const int32_t* target_tokens, int32_t N, int32_t* path,
                                                         int32_t* path_len, int32_t* length, int32_t* token,
                                                         int32_t* sampled_out, int32_t* num_sampled, int32_t* accepted,
                                                         int64_t* stats, int32_t stats_stride) {
    __shared__ int32_t spar[kMaxTreeNodes];
    __shared__ int32_t stok[kMaxTreeNodes];
    __shared__ int32_t stgt[kMaxTreeNodes];
    __shared__ int32_t spath[kMaxTreeNodes];
    __shared__ int32_t sdepth[kMaxTreeNodes];
    __shared__ int32_t sres[2]; // best node, path length
    static_assert(kMaxTreeNodes <= 64 && kStatsPerPositionOffset + kMaxTreeNodes <= 64, "one wave per tree");
    const int b = blockIdx.x;
    const int lane = static_cast<int>(threadIdx.x);
    const int32_t* par = parents + static_cast<int64_t>(b) * N;
    const int32_t* tok = node_tokens + static_cast<int64_t>(b) * N;
    const int32_t* tgt = target_tokens + static_cast<int64_t>(b) * N;
    int32_t* pth = path + static_cast<int64_t>(b) * N;
    int32_t* so = sampled_out + static_cast<int64_t>(b) * N;
    int64_t* st = stats + static_cast<int64_t>(b) * stats_stride;
    if (lane < N) {
        spar[lane] = par[lane];
        stok[lane] = tok[lane];
        stgt[lane] = tgt[lane];
    }
    const int64_t st_old = lane < stats_stride ? st[lane] : 0;
    const int32_t len_old = length[b];
    __syncthreads();
    if (lane == 0) {
        int32_t* depth = sdepth;
        depth[0] = 0;
        int best = 0;
        int best_depth = 0;
        for (int u = 1; u < N; ++u) {
            depth[u] = -1;
            const int p = spar[u];
            if (p < 0 || p >= u || depth[p] < 0) { continue; }
            if (stok[u] != stgt[p]) { continue; }
            depth[u] = depth[p] + 1;
            if (depth[u] > best_depth) {
                best = u;
                best_depth = depth[u];
            }
        }
        const int len = best_depth + 1;
        int u = best;
        for (int j = len - 1; j >= 0; --j) {
            spath[j] = u;
            u = spar[u];
        }
        sres[0] = best;
        sres[1] = len;
    }
    __syncthreads();
    const int best = sres[0];
    const int len = sres[1];
    const int acc = len - 1;
    if (lane < N) {
        pth[lane] = lane < len ? spath[lane] : 0;
        so[lane] = lane < acc ? stok[spath[lane + 1]] : (lane == acc ? stgt[best] : 0);
    }
    if (lane == 0) {
        path_len[b] = len;
        num_sampled[b] = acc + 1;
        accepted[b] = acc;
        token[b] = stgt[best];
        length[b] = len_old + acc + 1;
    }
    // stats: [0] += N - 1 drafted nodes, [1] += accepted, [2] += rounds, [4 + j] += 1 for j < acc
    const int64_t add = lane == 0 ? N - 1 : lane == 1 ? acc : lane == 2 ? 1
                        : (lane >= kStatsPerPositionOffset && lane - kStatsPerPositionOffset < acc) ? 1 : 0;
    if (lane < stats_stride && add != 0) { st[lane] = st_old + add; }
}

} // namespace

SpecPlan plan_spec(int32_t token_domain, int32_t columns, int32_t batch) {
    SpecPlan p;
    p.ntiles = (token_domain + kTileTokens - 1) / kTileTokens;
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t at = off;
        off = (off + bytes + 255) & ~static_cast<size_t>(255);
        return at;
    };
    const size_t cols = static_cast<size_t>(columns) * batch;
    p.partial_offset = take(cols * p.ntiles * kCandidateCap * sizeof(uint64_t));
    p.bytes = off;
    return p;
}

void launch_argmax(const uint16_t* logits, int32_t* out, int32_t physical_rows, int32_t valid_rows,
                   int32_t columns, hipStream_t stream) {
    const int tiles = (valid_rows + kArgmaxTile - 1) / kArgmaxTile;
    if (tiles < 2) {
        hipLaunchKernelGGL(argmax_kernel, dim3(columns), dim3(1024), 0, stream, logits, out,
                           physical_rows, valid_rows, static_cast<int64_t>(physical_rows));
        check_launch("argmax_kernel");
        return;
    }
    hipLaunchKernelGGL(argmax_tile_kernel, dim3(tiles, columns), dim3(256), 0, stream, logits, out, valid_rows,
                       static_cast<int64_t>(physical_rows));
    check_launch("argmax_tile_kernel");
}

void launch_prepare_verify_inputs(const int32_t* token, const int32_t* drafts, const int32_t* length,
                                  int32_t* verify_ids, int32_t* positions, int32_t K, int32_t B,
                                  hipStream_t stream) {
    hipLaunchKernelGGL(prepare_verify_inputs_kernel, dim3(B), dim3(64), 0, stream, token, drafts,
                       length, verify_ids, positions, K);
    check_launch("prepare_verify_inputs_kernel");
}

void launch_spec_accept(const SpecArgs& args, int32_t batch, hipStream_t stream) {
    hipLaunchKernelGGL(spec_tile_topk_kernel, dim3(args.ntiles, args.K + 1, batch), dim3(256), 0,
                       stream, args);
    check_launch("spec_tile_topk_kernel");
    hipLaunchKernelGGL(spec_merge_accept_kernel<2>, dim3(batch), dim3(256), 0, stream, args);
    check_launch("spec_merge_accept_kernel");
}

void launch_spec_merge_accept_wide(const SpecArgs& args, int32_t batch, hipStream_t stream) {
    hipLaunchKernelGGL(spec_merge_accept_kernel<4>, dim3(batch), dim3(256), 0, stream, args);
    check_launch("spec_merge_accept_kernel");
}

void launch_mtp_alignment_ids(const int32_t* verify_ids, const int32_t* token, const int32_t* accepted,
                              int32_t* alignment_ids, int32_t T, hipStream_t stream) {
    hipLaunchKernelGGL(mtp_alignment_ids_kernel, dim3(1), dim3(64), 0, stream, verify_ids, token, accepted,
                       alignment_ids, T);
    check_launch("mtp_alignment_ids_kernel");
}

void launch_select_hidden(const uint16_t* hidden, const int32_t* accepted, uint16_t* out,
                          int32_t rows, int32_t cols, hipStream_t stream) {
    hipLaunchKernelGGL(select_hidden_kernel, dim3((rows + 255) / 256), dim3(256), 0, stream, hidden,
                       accepted, out, rows, cols);
    check_launch("select_hidden_kernel");
}

void launch_tree_accept(const int32_t* parents, const int32_t* node_tokens,
                        const int32_t* target_tokens, int32_t N, int32_t B, int32_t* path,
                        int32_t* path_len, int32_t* length, int32_t* token, int32_t* sampled_out,
                        int32_t* num_sampled, int32_t* accepted, int64_t* stats,
                        int32_t stats_stride, hipStream_t stream) {
    hipLaunchKernelGGL(tree_accept_kernel, dim3(B), dim3(64), 0, stream, parents, node_tokens,
                       target_tokens, N, path, path_len, length, token, sampled_out, num_sampled,
                       accepted, stats, stats_stride);
    check_launch("tree_accept_kernel");
}

} // namespace nmi
