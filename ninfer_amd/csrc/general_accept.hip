// General speculative acceptance ("Mode F", no reference counterpart) on gfx950.
//
// Semantics (bit-exact with the CPU oracle's orc_general_accept): for every target column i
// (0..K) and draft column i (0..K-1) the distribution is the full-vocabulary softmax at the
// configured temperature in 2^40 fixed point, W_v = rint(det_expf(fma(x_v, 1/T, -xmax/T)) * 2^40),
// truncated by top-p to the shortest prefix in (value desc, id asc) order whose mass reaches
// floor(z * p24 / 2^24) (p24 = rint(top_p * 2^24)). Draft i is accepted iff
// u24(u_accept[i]) * q_i(d_i) < p_i(d_i), compared exactly in 128 bits over the common denominator.
// At the first rejection the token is drawn from the normalized residual max(0, p_i - q_i)
// (weights (W^p_v z_q - W^q_v z_p) >> 40, falling back to p_i when the residual is empty) with
// u_residual; after K acceptances it is drawn from p_K with u_accept[K]. Draws are inverse-CDF over
// token ids in ascending order.
//
// Every quantity is an integer except W, which depends only on a token's BF16 value, so the
// nucleus is found without sorting: a coarse histogram (high byte of the 16-bit ordered value) of
// counts and masses, then a fine histogram inside the crossing coarse bin, then the rank of the
// last included token among equal values (ids ascending). The nucleus collapses to one 64-bit
// key threshold: token v is a member iff sort_key(x_v, v) >= kstar.
//
// Launches (histogram passes over tiles of 4096 tokens, draw passes over tiles of 1024; all
// columns and sequences in one grid each):
//   1 gen_max      tile maxima; zero the coarse histograms and the column fine counts
//   2 gen_coarse   per-token weights -> coarse counts and masses (replicated LDS histograms, then
//                  global atomics); block 0 of a sequence gathers the drafts' accept-test inputs
//   3 gen_fine     per tile: total mass, top-p target and crossing coarse bin (every block; block 0
//                  writes the column descriptor), then counts of the 256 values inside that bin
//   4 gen_nucleus  per column: crossing value, rank cut, kstar and nucleus mass
//   5 gen_totals   per draw tile: accept decision (recomputed per block), masses of the draw
//   6 gen_pick     per sequence: locate the draw, commit the round
#include "common.h"
#include "device_utils.h"
#include "general_internal.h"
#include "sampler_common.h"

#pragma clang fp contract(off)

namespace nmi {
namespace {

typedef unsigned __int128 u128;

constexpr int kThreads = 256;
constexpr int kPerThread = kGenTile / kThreads; // 16 consecutive tokens per thread in rescans
constexpr int kDrawPerThread = kGenDrawTile / kThreads; // 4 tokens per thread in the draw passes
constexpr int kMaxDrawTilesPerThread = (kGenMaxTiles * kGenTile / kGenDrawTile) / kThreads; // V <= 2^20

struct ColDesc {
    float m;          // xmax / T
    float inv_temp;   // 1 / T
    int32_t c1;       // crossing coarse bin
    int32_t nucleus;  // top-p truncates
    uint64_t cum1;    // mass above the crossing coarse bin
    uint64_t target;  // floor(z * p24 / 2^24)
    uint64_t z;       // full mass
    uint64_t zs;      // nucleus mass
    uint64_t kstar;   // members: sort_key(x_v, v) >= kstar
    uint64_t pad;
};
static_assert(sizeof(ColDesc) == kGenDescBytes, "descriptor size");

struct GenArgs {
    const uint16_t* logits;
    const uint16_t* draft_logits;
    const int32_t* drafts;
    const float* u_accept;
    const float* u_residual;
    int32_t* length;
    int32_t* token;
    int32_t* sampled_out;
    int32_t* num_sampled;
    int32_t* accepted;
    int64_t* stats;
    const nmi_general_config* config;
    int64_t logit_col;   // elements between target columns
    int64_t logit_seq;   // elements between sequences
    int64_t draft_col;
    int64_t draft_seq;
    int32_t stats_stride;
    int32_t V;
    int32_t K;
    int32_t ncols;
    int32_t ntiles;
    int32_t ndraw; // draw tiles of kGenDrawTile tokens
    float* tile_max;
    uint64_t* cmass;
    uint32_t* ccount;
    ColDesc* desc;
    uint32_t* fine;
    uint32_t* fine_total;
    uint64_t* tile_res;
    uint64_t* tile_p;
    struct DraftEntry* dtab;
};

// Inputs of draft i's accept test, gathered once per round by gen_coarse so that no later launch
// waits on drafts -> logits: the BF16 bits of target column i and draft column i at token d_i
// (xpq = xp | xq << 16, zero outside the token domain) and d_i itself (-1 outside the domain).
struct DraftEntry {
    uint32_t xpq;
    int32_t d;
};
static_assert(sizeof(DraftEntry) == kGenDraftEntryBytes, "draft entry size");
constexpr int kMaxCols = 2 * kMaxColumns; // 2K + 1 <= 31 descriptors per sequence

__device__ __forceinline__ const uint16_t* column_ptr(const GenArgs& a, int b, int c) {
    if (c <= a.K) { return a.logits + b * a.logit_seq + c * a.logit_col; }
    return a.draft_logits + b * a.draft_seq + (c - a.K - 1) * a.draft_col;
}

__device__ __forceinline__ uint32_t fixed_u24(float u) {
    float s = __builtin_rintf(u * 16777216.0f);
    s = fmaxf(0.0f, fminf(16777216.0f, s));
    return static_cast<uint32_t>(s);
}

// W = rint(det_expf(y) * 2^40), y = fma(x, 1/T, -xmax/T). Inside det_expf's range the two scaling
// steps and the 2^40 collapse into one exact ldexp: p * 2^k is exact when normal, and times 2^40 it
// stays exact or overflows to inf in both forms; when p * 2^k is subnormal, both forms give a value
// below 2^-85, which rounds to 0. Outside the range (NaN, overflow, underflow) det_expf itself runs.
__device__ __forceinline__ uint64_t gen_weight(float x, float inv_temp, float m) {
    const float y = __builtin_fmaf(x, inv_temp, -m);
    float w;
    if (det_exp_in_range(y)) {
        int k;
        const float p = det_exp_poly(y, &k);
        w = __builtin_ldexpf(p, k + 40);
    } else {
        w = det_expf(y) * 1099511627776.0f; // 2^40
    }
    return static_cast<uint64_t>(__builtin_rintf(w));
}

// 16-bit ordered value of a BF16 token (the high half of the ordered-float key).
__device__ __forceinline__ uint32_t ordered16(float x) { return ordered_float(x) >> 16; }

__device__ __forceinline__ float value_of_ordered16(uint32_t o) {
    const uint32_t bits = (o & 0x8000u) ? (o ^ 0x8000u) : (~o & 0xffffu);
    return bf16_to_f32(static_cast<uint16_t>(bits));
}

// Block-wide inclusive scan over 256 threads: a DPP scan per wave, then the wave totals through
// LDS (sh: at least kThreads / 64 entries). Integer sums, so any order gives the same bits.
template <typename T>
__device__ T block_scan(T v, T* sh) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    v = wave_inclusive_scan(v);
    if (lane == 63) { sh[wave] = v; }
    __syncthreads();
    T add = 0;
    for (int w = 0; w < wave; ++w) { add += sh[w]; }
    __syncthreads();
    return v + add;
}

// The 16 tokens [v0, v0 + 16) of a column as floats (tokens >= V read as -inf), loaded with two
// 16-byte loads when the run is whole and aligned.
__device__ __forceinline__ void load16(const uint16_t* col, int v0, int V, float (&x)[16]) {
    if (v0 + 16 <= V && (reinterpret_cast<uintptr_t>(col + v0) & 15u) == 0) {
        const i4 r0 = *reinterpret_cast<const i4*>(col + v0);
        const i4 r1 = *reinterpret_cast<const i4*>(col + v0 + 8);
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const uint32_t w = static_cast<uint32_t>(e < 8 ? r0[e >> 1] : r1[(e - 8) >> 1]);
            x[e] = bf16_to_f32(static_cast<uint16_t>((e & 1) ? (w >> 16) : (w & 0xffffu)));
        }
    } else {
        uint16_t raw[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) { raw[e] = v0 + e < V ? col[v0 + e] : static_cast<uint16_t>(0xff80u); }
#pragma unroll
        for (int e = 0; e < 16; ++e) { x[e] = bf16_to_f32(raw[e]); }
    }
}

// The 4 tokens [v0, v0 + 4) of a column as floats (tokens >= V read as -inf).
__device__ __forceinline__ void load4(const uint16_t* col, int v0, int V, float (&x)[4]) {
    if (v0 + 4 <= V && (reinterpret_cast<uintptr_t>(col + v0) & 7u) == 0) {
        const uint2 r = *reinterpret_cast<const uint2*>(col + v0);
        x[0] = bf16_to_f32(static_cast<uint16_t>(r.x & 0xffffu));
        x[1] = bf16_to_f32(static_cast<uint16_t>(r.x >> 16));
        x[2] = bf16_to_f32(static_cast<uint16_t>(r.y & 0xffffu));
        x[3] = bf16_to_f32(static_cast<uint16_t>(r.y >> 16));
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) { x[e] = bf16_to_f32(v0 + e < V ? col[v0 + e] : static_cast<uint16_t>(0xff80u)); }
    }
}

// Smallest thread index with `pred`, or kThreads: a ballot per wave, then the four waves' firsts
// through LDS (sh: kThreads / 64 entries).
__device__ int block_first(bool pred, int* sh) {
    const unsigned long long m = __ballot(pred);
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) { sh[wave] = m != 0ull ? 64 * wave + __ffsll(static_cast<long long>(m)) - 1 : kThreads; }
    __syncthreads();
    const int r = min(min(sh[0], sh[1]), min(sh[2], sh[3]));
    __syncthreads();
    return r;
}

__device__ float block_max(float v, float* sh) {
    v = wave_max(v);
    if ((threadIdx.x & 63) == 0) { sh[threadIdx.x >> 6] = v; }
    __syncthreads();
    const float r = fmaxf(fmaxf(sh[0], sh[1]), fmaxf(sh[2], sh[3]));
    __syncthreads();
    return r;
}

__device__ __forceinline__ bool member(const ColDesc& d, float x, int v) {
    return sort_key(x, v) >= d.kstar;
}

__device__ __forceinline__ uint64_t member_weight(const ColDesc& d, float x, int v) {
    return member(d, x, v) ? gen_weight(x, d.inv_temp, d.m) : 0ull;
}

// ---- 1: tile maxima ----------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void gen_max_kernel(GenArgs a) {
    __shared__ float red[kThreads / 64];
    const int t = blockIdx.x, c = blockIdx.y, b = blockIdx.z;
    const uint16_t* col = column_ptr(a, b, c);
    float x[16];
    load16(col, t * kGenTile + kPerThread * static_cast<int>(threadIdx.x), a.V, x);
    float mx = -INFINITY;
#pragma unroll
    for (int e = 0; e < 16; ++e) { mx = fmaxf(mx, x[e]); }
    mx = block_max(mx, red);
    const int64_t cb = static_cast<int64_t>(b) * a.ncols + c;
    if (threadIdx.x == 0) { a.tile_max[cb * a.ntiles + t] = mx; }
    if (t == 0) {
        a.cmass[cb * kGenBins + threadIdx.x] = 0;
        a.ccount[cb * kGenBins + threadIdx.x] = 0;
        a.fine_total[cb * kGenBins + threadIdx.x] = 0;
    }
}

__device__ void column_scale(const GenArgs& a, int64_t cb, float* red, float* m, float* inv_temp) {
    float mx = -INFINITY;
    for (int i = threadIdx.x; i < a.ntiles; i += kThreads) { mx = fmaxf(mx, a.tile_max[cb * a.ntiles + i]); }
    mx = block_max(mx, red);
    *inv_temp = 1.0f / a.config->temperature;
    *m = mx * *inv_temp;
}

// ---- 2: coarse histogram of counts and masses ----------------------------------------------------
// Lanes of a wave mostly fall into a few bins, so lane l adds into replica l % kCoarseReplicas; the
// replica stride of kGenBins + 1 words puts the replicas of one bin in different LDS banks.
// A replica word packs a bin's count (bits 52 and up) over its mass (bits 0-51), so each token costs
// one LDS atomic: a replica sees at most kGenTile / kCoarseReplicas = 256 tokens of a tile, whose
// weights (each at most 2^40 plus the rounding of fma(xmax, 1/T, -xmax/T)) sum below 2^49.
constexpr int kCoarseReplicas = 16;
constexpr int kReplicaStride = kGenBins + 1;
constexpr int kCountShift = 52;
static_assert(kGenTile / kCoarseReplicas <= 256, "packed replica words: count and mass fields");

__global__ __launch_bounds__(kThreads) void gen_coarse_kernel(GenArgs a) {
    __shared__ uint64_t cm[kCoarseReplicas * kReplicaStride];
    __shared__ float red[kThreads / 64];
    const int t = blockIdx.x, c = blockIdx.y, b = blockIdx.z;
    const int64_t cb = static_cast<int64_t>(b) * a.ncols + c;
    if (t == 0 && c == 0 && static_cast<int>(threadIdx.x) < a.K) {
        const int i = threadIdx.x;
        const int d = a.drafts[b * a.K + i];
        const bool in_domain = d >= 0 && d < a.V;
        const uint32_t xp = in_domain ? column_ptr(a, b, i)[d] : 0u;
        const uint32_t xq = in_domain ? column_ptr(a, b, a.K + 1 + i)[d] : 0u;
        a.dtab[static_cast<int64_t>(b) * a.K + i] = DraftEntry{xp | (xq << 16), in_domain ? d : -1};
    }
    for (int i = threadIdx.x; i < kCoarseReplicas * kReplicaStride; i += kThreads) { cm[i] = 0; }
    // The tile's tokens load while the column maximum is reduced.
    const int v0 = t * kGenTile + kPerThread * static_cast<int>(threadIdx.x);
    float x[16];
    load16(column_ptr(a, b, c), v0, a.V, x);
    float m, inv_temp;
    column_scale(a, cb, red, &m, &inv_temp); // synchronizes the block
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        if (v0 + e < a.V) {
            const uint32_t slot = (threadIdx.x % kCoarseReplicas) * kReplicaStride + (ordered16(x[e]) >> 8);
            const uint64_t add = (1ull << kCountShift) + gen_weight(x[e], inv_temp, m);
            atomicAdd(reinterpret_cast<unsigned long long*>(&cm[slot]), static_cast<unsigned long long>(add));
        }
    }
    __syncthreads();
    uint32_t ct = 0;
    uint64_t ms = 0;
#pragma unroll
    for (int r = 0; r < kCoarseReplicas; ++r) {
        const uint64_t w = cm[r * kReplicaStride + threadIdx.x];
        ct += static_cast<uint32_t>(w >> kCountShift);
        ms += w & ((1ull << kCountShift) - 1);
    }
    if (ct != 0) {
        atomicAdd(&a.ccount[cb * kGenBins + threadIdx.x], ct);
        atomicAdd(reinterpret_cast<unsigned long long*>(&a.cmass[cb * kGenBins + threadIdx.x]),
                  static_cast<unsigned long long>(ms));
    }
}

// ---- 3: crossing coarse bin (every block of the column finds it), then the fine counts inside it,
// per tile. Block t == 0 writes the column's descriptor: total mass, top-p target, crossing bin.
__global__ __launch_bounds__(kThreads) void gen_fine_kernel(GenArgs a) {
    __shared__ uint32_t cnt[kGenBins];
    __shared__ uint64_t sh[kThreads];
    __shared__ float red[kThreads / 64];
    __shared__ int first[kThreads / 64];
    __shared__ uint64_t total;
    const int t = blockIdx.x, c = blockIdx.y, b = blockIdx.z;
    const int64_t cb = static_cast<int64_t>(b) * a.ncols + c;
    const int v0 = t * kGenTile + kPerThread * static_cast<int>(threadIdx.x);
    float x[16];
    load16(column_ptr(a, b, c), v0, a.V, x); // issued before the histogram arrives
    const int bin = kGenBins - 1 - static_cast<int>(threadIdx.x); // descending value order
    const uint32_t count = a.ccount[cb * kGenBins + bin];
    const uint64_t mass = a.cmass[cb * kGenBins + bin];
    const float top_p = a.config->top_p;
    const uint64_t incl = block_scan<uint64_t>(mass, sh);
    if (threadIdx.x == kThreads - 1) { total = incl; }
    __syncthreads();
    const uint64_t Z = total;
    ColDesc d{};
    if (t == 0) {
        column_scale(a, cb, red, &d.m, &d.inv_temp);
        d.z = Z;
    }
    if (!(top_p < 1.0f)) {
        if (t == 0 && threadIdx.x == 0) {
            d.c1 = -1;
            d.nucleus = 0;
            d.zs = Z;
            d.kstar = 0;
            a.desc[cb] = d;
        }
        return;
    }
    const uint64_t target = static_cast<uint64_t>((static_cast<u128>(Z) * fixed_u24(top_p)) >> 24);
    const int f = block_first(count != 0 && incl >= target, first);
    if (t == 0 && static_cast<int>(threadIdx.x) == f) {
        d.c1 = bin;
        d.nucleus = 1;
        d.cum1 = incl - mass;
        d.target = target;
        a.desc[cb] = d;
    }
    if (f >= kThreads) { return; }
    const int c1 = kGenBins - 1 - f;
    cnt[threadIdx.x] = 0;
    __syncthreads();
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        const uint32_t o = ordered16(x[e]);
        if (v0 + e < a.V && static_cast<int>(o >> 8) == c1) { atomicAdd(&cnt[o & 0xffu], 1u); }
    }
    __syncthreads();
    a.fine[(cb * a.ntiles + t) * kGenBins + threadIdx.x] = cnt[threadIdx.x];
    if (cnt[threadIdx.x] != 0) { atomicAdd(&a.fine_total[cb * kGenBins + threadIdx.x], cnt[threadIdx.x]); }
}

// ---- 5: crossing value, rank cut among equal values, kstar --------------------------------------
__global__ __launch_bounds__(kThreads) void gen_nucleus_kernel(GenArgs a) {
    __shared__ uint64_t sh[kThreads];
    __shared__ int first[kThreads / 64];
    __shared__ uint64_t bcast[4];
    const int c = blockIdx.x, b = blockIdx.y;
    const int64_t cb = static_cast<int64_t>(b) * a.ncols + c;
    ColDesc d = a.desc[cb];
    if (!d.nucleus) { return; }
    if (threadIdx.x == 0) { bcast[0] = 1; bcast[1] = d.z; bcast[2] = static_cast<uint64_t>(d.c1) << 8; bcast[3] = 1; }
    __syncthreads();
    // Fine bin f = 255 - tid (descending value order).
    const uint32_t f = kGenBins - 1 - threadIdx.x;
    const uint64_t count = a.fine_total[cb * kGenBins + f];
    const uint32_t o16 = (static_cast<uint32_t>(d.c1) << 8) | f;
    const float x = value_of_ordered16(o16);
    const uint64_t w = gen_weight(x, d.inv_temp, d.m);
    const uint64_t mass = count * w;
    const uint64_t incl = block_scan<uint64_t>(mass, sh);
    const int fs = block_first(count != 0 && d.cum1 + incl >= d.target, first);
    if (static_cast<int>(threadIdx.x) == fs) {
        const uint64_t before = d.cum1 + incl - mass;
        // smallest j >= 1 with before + j * w >= target (w > 0 at the crossing)
        uint64_t j = d.target > before ? (d.target - before + w - 1) / w : 0;
        j = j < 1 ? 1 : (j > count ? count : j);
        bcast[0] = j;
        bcast[1] = before + j * w;
        bcast[2] = o16;
    }
    __syncthreads();
    const uint64_t j = bcast[0];
    const uint32_t vstar = static_cast<uint32_t>(bcast[2]);
    // Tile holding the j-th token of value vstar (ids ascending).
    const uint32_t fstar = vstar & 0xffu;
    uint64_t tc = 0;
    if (static_cast<int>(threadIdx.x) < a.ntiles) { tc = a.fine[(cb * a.ntiles + threadIdx.x) * kGenBins + fstar]; }
    const uint64_t tincl = block_scan<uint64_t>(tc, sh);
    const int ts = block_first(static_cast<int>(threadIdx.x) < a.ntiles && tincl >= j, first);
    if (static_cast<int>(threadIdx.x) == ts) { bcast[3] = j - (tincl - tc); } // 1-based rank in tile
    __syncthreads();
    const uint64_t rank = bcast[3];
    // Rescan that tile: thread i owns tokens [16 i, 16 i + 16) of it.
    const uint16_t* col = column_ptr(a, b, c);
    const int v0 = ts * kGenTile + kPerThread * static_cast<int>(threadIdx.x);
    float xs[16];
    load16(col, v0, a.V, xs);
    uint64_t mine = 0;
#pragma unroll
    for (int k = 0; k < kPerThread; ++k) {
        if (v0 + k < a.V && ordered16(xs[k]) == vstar) { ++mine; }
    }
    const uint64_t mincl = block_scan<uint64_t>(mine, sh);
    if (mine != 0 && mincl >= rank && mincl - mine < rank) {
        uint64_t need = rank - (mincl - mine);
        for (int k = 0; k < kPerThread; ++k) {
            const int v = v0 + k;
            if (v < a.V && ordered16(xs[k]) == vstar && --need == 0) {
                d.kstar = sort_key(value_of_ordered16(vstar), v);
                d.zs = bcast[1];
                a.desc[cb] = d;
                break;
            }
        }
    }
}

// Accept decisions of sequence b (identical in every block that evaluates them), from the
// sequence's descriptors in LDS (sd) and thread i's draft entry e and accept uniform ua: thread
// i < K tests draft i, and the first failing draft is the rejection. Returns a; sets *rejected to the
// rejected column (or -1 when all K drafts are accepted).
__device__ int decide(const GenArgs& a, const ColDesc* sd, const DraftEntry& e, float ua, int* rejected, int* sh) {
    bool fail = false;
    const int i = static_cast<int>(threadIdx.x);
    if (i < a.K) {
        const ColDesc& p = sd[i];
        const ColDesc& q = sd[a.K + 1 + i];
        // A draft id outside the token domain has no mass under either distribution: rejected.
        const bool in_domain = e.d >= 0;
        const float xp = in_domain ? bf16_to_f32(static_cast<uint16_t>(e.xpq & 0xffffu)) : 0.0f;
        const float xq = in_domain ? bf16_to_f32(static_cast<uint16_t>(e.xpq >> 16)) : 0.0f;
        const uint64_t wp = in_domain ? member_weight(p, xp, e.d) : 0ull;
        const uint64_t wq = in_domain ? member_weight(q, xq, e.d) : 0ull;
        const u128 lhs = static_cast<u128>(fixed_u24(ua)) * wq * p.zs;
        const u128 rhs = (static_cast<u128>(wp) * q.zs) << 24;
        fail = !(lhs < rhs);
    }
    const int f = block_first(fail, sh);
    *rejected = f < a.K ? f : -1;
    return f < a.K ? f : a.K;
}

// The sequence's descriptors into LDS and thread i's draft entry and accept uniform (one round trip
// for everything decide() reads).
__device__ __forceinline__ void load_decision_inputs(const GenArgs& a, int b, ColDesc* sd, DraftEntry* e, float* ua) {
    const int i = static_cast<int>(threadIdx.x);
    *e = DraftEntry{0u, -1};
    *ua = 0.0f;
    if (i < a.K) {
        *e = a.dtab[static_cast<int64_t>(b) * a.K + i];
        *ua = a.u_accept[b * (a.K + 1) + i];
    }
    if (i < a.ncols) { sd[i] = a.desc[static_cast<int64_t>(b) * a.ncols + i]; }
}

// Draw weights of token v: residual (column pair i) or p (column i); both from one read.
struct DrawMass {
    uint64_t res;
    uint64_t p;
};

__device__ __forceinline__ DrawMass draw_mass_x(int rejected, const ColDesc& p, const ColDesc& q, float xp,
                                                float xq, int v) {
    DrawMass r;
    r.p = member_weight(p, xp, v);
    r.res = 0;
    if (rejected >= 0) {
        const uint64_t wq = member_weight(q, xq, v);
        const u128 pv = static_cast<u128>(r.p) * q.zs;
        const u128 qv = static_cast<u128>(wq) * p.zs;
        r.res = pv > qv ? static_cast<uint64_t>((pv - qv) >> 40) : 0ull;
    }
    return r;
}

// ---- 6: per-tile masses of the draw --------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void gen_totals_kernel(GenArgs a) {
    __shared__ u128 shr[kThreads / 64];
    __shared__ uint64_t shp[kThreads / 64];
    __shared__ int first[kThreads / 64];
    __shared__ ColDesc sd[kMaxCols];
    const int t = blockIdx.x, b = blockIdx.y;
    DraftEntry e;
    float ua;
    load_decision_inputs(a, b, sd, &e, &ua);
    __syncthreads();
    int rejected;
    const int acc = decide(a, sd, e, ua, &rejected, first);
    const int col_p = rejected >= 0 ? rejected : a.K;
    const ColDesc p = sd[col_p];
    const ColDesc q = rejected >= 0 ? sd[a.K + 1 + rejected] : p;
    (void)acc;
    u128 res = 0;
    uint64_t pm = 0;
    const int v0 = t * kGenDrawTile + kDrawPerThread * static_cast<int>(threadIdx.x);
    float xp[kDrawPerThread], xq[kDrawPerThread] = {};
    load4(column_ptr(a, b, col_p), v0, a.V, xp);
    if (rejected >= 0) { load4(column_ptr(a, b, a.K + 1 + rejected), v0, a.V, xq); }
#pragma unroll
    for (int k = 0; k < kDrawPerThread; ++k) {
        if (v0 + k < a.V) {
            const DrawMass dm = draw_mass_x(rejected, p, q, xp[k], xq[k], v0 + k);
            res += dm.res;
            pm += dm.p;
        }
    }
    const u128 rtot = block_scan<u128>(res, shr);
    const uint64_t ptot = block_scan<uint64_t>(pm, shp);
    if (threadIdx.x == kThreads - 1) {
        a.tile_res[(static_cast<int64_t>(b) * a.ndraw + t) * 2] = static_cast<uint64_t>(rtot);
        a.tile_res[(static_cast<int64_t>(b) * a.ndraw + t) * 2 + 1] = static_cast<uint64_t>(rtot >> 64);
        a.tile_p[static_cast<int64_t>(b) * a.ndraw + t] = ptot;
    }
}

// ---- 7: locate the draw (first id whose running mass exceeds floor(total * u24 / 2^24), else the
// last id with mass) and commit the round --------------------------------------------------------
__global__ __launch_bounds__(kThreads) void gen_pick_kernel(GenArgs a) {
    __shared__ u128 sh[kThreads / 64];
    __shared__ int first[kThreads / 64];
    __shared__ int last_tile;
    __shared__ int result;
    __shared__ u128 tile_before;
    __shared__ int crossing_tile;
    __shared__ ColDesc sd[kMaxCols];
    __shared__ int32_t sdrafts[kMaxColumns];
    __shared__ int64_t sstats[4 + kMaxColumns];
    __shared__ int32_t slength;
    const int b = blockIdx.x;
    const int tid = static_cast<int>(threadIdx.x);
    // Thread tid owns draw tiles [tid * tpt, tid * tpt + tpt) (ids ascending across threads).
    const int tpt = (a.ndraw + kThreads - 1) / kThreads;
    const int tile0 = tid * tpt;
    // Everything this block reads except the crossing tile's tokens, requested at once.
    DraftEntry e;
    float ua;
    load_decision_inputs(a, b, sd, &e, &ua);
    u128 rt[kMaxDrawTilesPerThread];
    uint64_t pt[kMaxDrawTilesPerThread];
#pragma unroll
    for (int j = 0; j < kMaxDrawTilesPerThread; ++j) {
        rt[j] = 0;
        pt[j] = 0;
        if (j < tpt && tile0 + j < a.ndraw) {
            const int64_t ti = static_cast<int64_t>(b) * a.ndraw + tile0 + j;
            rt[j] = (static_cast<u128>(a.tile_res[ti * 2 + 1]) << 64) | a.tile_res[ti * 2];
            pt[j] = a.tile_p[ti];
        }
    }
    if (tid < a.K) { sdrafts[tid] = a.drafts[b * a.K + tid]; }
    if (tid < 4 + a.K) { sstats[tid] = a.stats[static_cast<int64_t>(b) * a.stats_stride + tid]; }
    if (tid == 0) { slength = a.length[b]; }
    const float u_res = a.u_residual[b];
    const float u_bonus = a.u_accept[b * (a.K + 1) + a.K];
    __syncthreads();
    int rejected;
    const int acc = decide(a, sd, e, ua, &rejected, first);
    const int col_p = rejected >= 0 ? rejected : a.K;
    const ColDesc p = sd[col_p];
    const ColDesc q = rejected >= 0 ? sd[a.K + 1 + rejected] : p;
    // Totals of the chosen weights (residual, or p when there is no residual mass). The residual
    // masses are non-negative, so their total is nonzero iff some tile's is (a block-wide OR).
    u128 rsum = 0;
#pragma unroll
    for (int j = 0; j < kMaxDrawTilesPerThread; ++j) { rsum += rt[j]; }
    const bool use_res = __syncthreads_or(rejected >= 0 && rsum != 0) != 0;
    u128 tt[kMaxDrawTilesPerThread];
    u128 tsum = 0;
#pragma unroll
    for (int j = 0; j < kMaxDrawTilesPerThread; ++j) {
        tt[j] = use_res ? rt[j] : static_cast<u128>(pt[j]);
        tsum += tt[j];
    }
    const u128 incl = block_scan<u128>(tsum, sh);
    __shared__ u128 total;
    if (tid == kThreads - 1) { total = incl; }
    __syncthreads();
    const float u = rejected >= 0 ? u_res : u_bonus;
    const u128 goal = (total * fixed_u24(u)) >> 24;
    // The first tile whose running mass exceeds goal lies in the first thread whose inclusive sum
    // does (a tile that moves the running mass past goal has nonzero mass).
    const int owner = block_first(tsum != 0 && incl > goal, first);
    const bool crossing = owner < kThreads;
    if (tid == 0) {
        last_tile = -1;
        crossing_tile = 0;
    }
    __syncthreads();
    if (crossing && tid == owner) {
        u128 run = incl - tsum;
        for (int j = 0; j < tpt; ++j) {
            if (tt[j] != 0 && run + tt[j] > goal) {
                crossing_tile = tile0 + j;
                tile_before = run;
                break;
            }
            run += tt[j];
        }
    }
    if (!crossing) {
        // goal >= total: the draw is the last id with nonzero mass.
        int lt = -1;
        for (int j = 0; j < tpt; ++j) { if (tt[j] != 0) { lt = tile0 + j; } }
        if (lt >= 0) { atomicMax(&last_tile, lt); }
    }
    if (tid == 0) { result = -1; }
    __syncthreads();
    const int ts = crossing ? crossing_tile : max(last_tile, 0);
    // Rescan the tile: thread i owns tokens [4 i, 4 i + 4) of it.
    const int v0 = ts * kGenDrawTile + kDrawPerThread * tid;
    float xp[kDrawPerThread], xq[kDrawPerThread] = {};
    load4(column_ptr(a, b, col_p), v0, a.V, xp);
    if (rejected >= 0) { load4(column_ptr(a, b, a.K + 1 + rejected), v0, a.V, xq); }
    uint64_t w[kDrawPerThread];
    u128 mine = 0;
#pragma unroll
    for (int k = 0; k < kDrawPerThread; ++k) {
        const int v = v0 + k;
        w[k] = 0;
        if (v < a.V) {
            const DrawMass dm = draw_mass_x(rejected, p, q, xp[k], xq[k], v);
            w[k] = use_res ? dm.res : dm.p;
        }
        mine += w[k];
    }
    const u128 mincl = block_scan<u128>(mine, sh) + (crossing ? tile_before : u128(0));
    if (crossing) {
        if (mine != 0 && mincl > goal && mincl - mine <= goal) {
            u128 run = mincl - mine;
            for (int k = 0; k < kDrawPerThread; ++k) {
                if (w[k] == 0) { continue; }
                run += w[k];
                if (goal < run) {
                    result = v0 + k;
                    break;
                }
            }
        }
    } else {
        int lastk = -1;
        for (int k = 0; k < kDrawPerThread; ++k) { if (w[k] != 0) { lastk = k; } }
        if (lastk >= 0) { atomicMax(&result, v0 + lastk); }
    }
    __syncthreads();
    // Commit the round (the reference's commit, src/ops/kernel/speculative_round.cuh:145-166), from
    // the values read at entry: stores only.
    const int tstar = result < 0 ? 0 : result;
    if (tid <= a.K) { a.sampled_out[b * (a.K + 1) + tid] = tid < acc ? sdrafts[tid] : (tid == acc ? tstar : 0); }
    if (tid < 4 + a.K) {
        const int64_t add = tid == 0 ? a.K : tid == 1 ? acc : tid == 2 ? 1 : (tid >= kStatsPerPositionOffset && tid - kStatsPerPositionOffset < acc) ? 1 : 0;
        if (add != 0) { a.stats[static_cast<int64_t>(b) * a.stats_stride + tid] = sstats[tid] + add; }
    }
    if (tid == 0) {
        a.num_sampled[b] = acc + 1;
        a.accepted[b] = acc;
        a.token[b] = tstar;
        a.length[b] = slength + acc + 1;
    }
}

} // namespace

GenPlan plan_general(int32_t token_domain, int32_t K, int32_t B) {
    GenPlan p;
    p.ncols = 2 * K + 1;
    p.ntiles = (token_domain + kGenTile - 1) / kGenTile;
    p.ndraw = (token_domain + kGenDrawTile - 1) / kGenDrawTile;
    const auto align = [](size_t x) { return (x + 255) & ~static_cast<size_t>(255); };
    size_t at = 0;
    const size_t cols = static_cast<size_t>(B) * p.ncols;
    p.tile_max_offset = at;
    at = align(at + cols * p.ntiles * sizeof(float));
    p.cmass_offset = at;
    at = align(at + cols * kGenBins * sizeof(uint64_t));
    p.ccount_offset = at;
    at = align(at + cols * kGenBins * sizeof(uint32_t));
    p.desc_offset = at;
    at = align(at + cols * kGenDescBytes);
    p.fine_offset = at;
    at = align(at + cols * p.ntiles * kGenBins * sizeof(uint32_t));
    p.fine_total_offset = at;
    at = align(at + cols * kGenBins * sizeof(uint32_t));
    p.tile_res_offset = at;
    at = align(at + static_cast<size_t>(B) * p.ndraw * 2 * sizeof(uint64_t));
    p.tile_p_offset = at;
    at = align(at + static_cast<size_t>(B) * p.ndraw * sizeof(uint64_t));
    p.dtab_offset = at;
    at = align(at + static_cast<size_t>(B) * K * kGenDraftEntryBytes);
    p.bytes = at;
    return p;
}

void launch_general_accept(const GenLaunch& l, const GenPlan& plan, void* workspace, hipStream_t stream) {
    char* ws = static_cast<char*>(workspace);
    GenArgs a{};
    a.logits = l.logits;
    a.draft_logits = l.draft_logits;
    a.drafts = l.drafts;
    a.u_accept = l.u_accept;
    a.u_residual = l.u_residual;
    a.length = l.length;
    a.token = l.token;
    a.sampled_out = l.sampled_out;
    a.num_sampled = l.num_sampled;
    a.accepted = l.accepted;
    a.stats = l.stats;
    a.config = l.config;
    a.logit_col = l.logit_col;
    a.logit_seq = l.logit_seq;
    a.draft_col = l.draft_col;
    a.draft_seq = l.draft_seq;
    a.stats_stride = l.stats_stride;
    a.V = l.token_domain;
    a.K = l.K;
    a.ncols = plan.ncols;
    a.ntiles = plan.ntiles;
    a.ndraw = plan.ndraw;
    a.tile_max = reinterpret_cast<float*>(ws + plan.tile_max_offset);
    a.cmass = reinterpret_cast<uint64_t*>(ws + plan.cmass_offset);
    a.ccount = reinterpret_cast<uint32_t*>(ws + plan.ccount_offset);
    a.desc = reinterpret_cast<ColDesc*>(ws + plan.desc_offset);
    a.fine = reinterpret_cast<uint32_t*>(ws + plan.fine_offset);
    a.fine_total = reinterpret_cast<uint32_t*>(ws + plan.fine_total_offset);
    a.tile_res = reinterpret_cast<uint64_t*>(ws + plan.tile_res_offset);
    a.tile_p = reinterpret_cast<uint64_t*>(ws + plan.tile_p_offset);
    a.dtab = reinterpret_cast<DraftEntry*>(ws + plan.dtab_offset);
    const dim3 tiles(plan.ntiles, plan.ncols, l.B);
    const dim3 cols(plan.ncols, l.B);
    hipLaunchKernelGGL(gen_max_kernel, tiles, dim3(kThreads), 0, stream, a);
    check_launch("gen_max_kernel");
    hipLaunchKernelGGL(gen_coarse_kernel, tiles, dim3(kThreads), 0, stream, a);
    check_launch("gen_coarse_kernel");
    hipLaunchKernelGGL(gen_fine_kernel, tiles, dim3(kThreads), 0, stream, a);
    check_launch("gen_fine_kernel");
    hipLaunchKernelGGL(gen_nucleus_kernel, cols, dim3(kThreads), 0, stream, a);
    check_launch("gen_nucleus_kernel");
    hipLaunchKernelGGL(gen_totals_kernel, dim3(plan.ndraw, l.B), dim3(kThreads), 0, stream, a);
    check_launch("gen_totals_kernel");
    hipLaunchKernelGGL(gen_pick_kernel, dim3(l.B), dim3(kThreads), 0, stream, a);
    check_launch("gen_pick_kernel");
}

} // namespace nmi
