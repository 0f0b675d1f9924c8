// Q6G64_F16S RowSplit linear (the lm_head of the verify step) and its fused argmax, gfx950.
//
// Contract (reference include/ninfer/ops/linear.h:10-27): out[n,t] = BF16(sum_k W[n,k] x[k,t]) with
// W exactly decoded, code * FP16 scale per group of 64 along K. Storage (reference test packer
// tests/ops/row_split_pack.h:143-195): per row, groups of 64 codes; the nibble plane holds 32 B per
// group (code i in byte i/2, low nibble for even i), the high plane 16 B per group (bits 2i, 2i+1 of
// the group's little-endian bit stream), the scale plane one FP16 per group; a code is the
// sign-extended 6-bit value. The fused form (the reference's deferred FUT-F03 `linear_argmax`,
// docs/maintainer/qwen3.6-35b-a3b-dflash-op-checklist.md:985-1001) returns, per column, the lowest
// row attaining the maximum BF16 logit among rows [0, valid_rows), without writing the logits.
//
// One persistent workgroup per CU; each wave streams 16-row tiles of the weight by LDS-DMA (a
// two-stage ring of 8-group chunks: 4 KB of nibbles, 2 KB of high bits, 256 B of scales) and runs
// v_mfma_f32_16x16x32_f16 with x staged once per workgroup in LDS. A lane decodes 16 codes of one
// row from one 8-byte nibble read and one 4-byte high read: each FP16 pair is built by bit
// operations as 0x6400 | (code + 32) = 1056 + code, then one packed subtraction of 1056 leaves the
// code itself, exactly, in the pairing (e, e + 4) of 8 codes. x is stored in LDS in the same order
// as FP16, each column scaled by a power of two that puts its largest magnitude in [2^14, 2^15),
// so every BF16 value of x is exact in FP16. The MFMA sums exact products in FP32 per group; the
// group result times its FP16 scale is accumulated in FP32, and the column factor is undone
// exactly at the end, so only FP32 summation rounds (the reference's tensor-core route rounds W to
// BF16 first).
#include "common.h"
#include "device_utils.h"
#include "lds_dma.h"
#include "linear_internal.h"
#include "topcap.h"

#include <algorithm>

namespace nmi {
namespace {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));

constexpr int kTileRows = 16;
constexpr int kXPad = 64;     // bytes between x columns in LDS (spreads the columns over the banks)
constexpr int kOutOfRange = 0x40000000; // a DMA source offset past every plane: reads zero

// One streamed chunk of a 16-row tile: CG groups (64 codes each) of every row. LDS stage: nibble
// rows (CG * 32 B), high rows (CG * 16 B), then scales (CG * 2 B per row) in one full-wave 4-byte
// DMA slot of 256 B. A row of R bytes holds R / 16 pieces of 16 B; piece p of row r sits at slot
// p ^ sw(r), sw(r) = (r / (256 / R)) % (R / 16): rows whose bank phase coincides get distinct
// slots, so the 16 lanes of one column of rows read conflict-free.
template <int CG>
struct Chunk {
    static constexpr int kNibRow = CG * 32;
    static constexpr int kHighRow = CG * 16;
    static constexpr int kScaleRow = CG * 2;
    static constexpr int kNib = kTileRows * kNibRow;
    static constexpr int kHigh = kTileRows * kHighRow;
    static constexpr int kStage = kNib + kHigh + 256;
    static constexpr int kNibDma = kNib / 1024;
    static constexpr int kHighDma = kHigh / 1024;
    static constexpr int kDma = kNibDma + kHighDma + 1;
    static_assert(kNib % 1024 == 0 && kHigh % 1024 == 0 && kTileRows * kScaleRow <= 256, "chunk geometry");
};

template <int R>
__device__ __forceinline__ int swz(int row) { return (row / (256 / R)) % (R / 16); }

__device__ __forceinline__ size_t x_lds_bytes(int TP, int Kp) { return static_cast<size_t>(TP) * (Kp * 2 + kXPad); }

// v << S (S > 0) or v >> -S as one full-rate 64-bit VALU shift (the compiler otherwise splits a
// 64-bit shift by a constant into two 32-bit operations).
template <int S>
__device__ __forceinline__ uint64_t shift64(uint64_t v) {
    uint64_t r;
    if constexpr (S == 0) {
        r = v;
    } else if constexpr (S > 0) {
        asm("v_lshlrev_b64 %0, %1, %2" : "=v"(r) : "i"(S), "v"(v));
    } else {
        asm("v_lshrrev_b64 %0, %1, %2" : "=v"(r) : "i"(-S), "v"(v));
    }
    return r;
}

// 16 codes (elements 16b .. 16b + 15 of a group) -> two MFMA A operands of 8 FP16 codes each, in
// the order (e0, e4, e1, e5, e2, e6, e3, e7) of each 8-code half.
//
// Word p of a half holds elements p and p + 4: the nibble plane gives them at bits 4p and 4p + 16
// and the high pairs (spread to bytes 0 and 2 by one permute) at bits 2p and 2p + 16. Both halves
// shift together as one 64-bit value (bits that cross the 32-bit boundary land outside the fields
// kept). Per word, two 3-input bit operations: t = M1 ? nibbles : high bits, then
// w = A ? (t ^ B) : B with A = the 6 code bits of each FP16 and B = 0x6400 | bit 5, which keeps the
// code bits, flips bit 5 ((code & 63) ^ 32 = code + 32) and sets the exponent of 1024.
template <int P>
__device__ __forceinline__ void decode_words(uint64_t nib, uint64_t hs, uint32_t kMaskA, uint32_t kConstB, h2 (&c0)[4],
                                             h2 (&c1)[4]) {
    constexpr uint32_t kNibMask = 0x000f000fu;
    const h2 bias = {static_cast<_Float16>(1056.0f), static_cast<_Float16>(1056.0f)};
    const uint64_t ns = shift64<-4 * P>(nib);
    const uint64_t hsh = shift64<4 - 2 * P>(hs);
    const uint32_t t0 = __builtin_amdgcn_bitop3_b32(kNibMask, static_cast<uint32_t>(ns), static_cast<uint32_t>(hsh), 0xCA);
    const uint32_t t1 = __builtin_amdgcn_bitop3_b32(kNibMask, static_cast<uint32_t>(ns >> 32), static_cast<uint32_t>(hsh >> 32), 0xCA);
    const uint32_t w0 = __builtin_amdgcn_bitop3_b32(t0, kMaskA, kConstB, 0x6A);
    const uint32_t w1 = __builtin_amdgcn_bitop3_b32(t1, kMaskA, kConstB, 0x6A);
    c0[P] = __builtin_bit_cast(h2, w0) - bias; // 1056 + code - 1056: exact
    c1[P] = __builtin_bit_cast(h2, w1) - bias;
}

__device__ __forceinline__ void decode16(uint64_t nib, uint32_t hi, uint32_t kMaskA, uint32_t kConstB, h8& a0, h8& a1) {
    const uint32_t hs0 = __builtin_amdgcn_perm(0u, hi, 0x0c010c00u); // high bytes 0, 1 -> bytes 0, 2
    const uint32_t hs1 = __builtin_amdgcn_perm(0u, hi, 0x0c030c02u);
    const uint64_t hs = (static_cast<uint64_t>(hs1) << 32) | hs0;
    h2 c0[4], c1[4];
    decode_words<0>(nib, hs, kMaskA, kConstB, c0, c1);
    decode_words<1>(nib, hs, kMaskA, kConstB, c0, c1);
    decode_words<2>(nib, hs, kMaskA, kConstB, c0, c1);
    decode_words<3>(nib, hs, kMaskA, kConstB, c0, c1);
    a0 = __builtin_bit_cast(h8, c0);
    a1 = __builtin_bit_cast(h8, c1);
}

// 64-bit argmax key of one BF16 logit: ordered value (larger = greater as a float, -0 = +0), then the
// lower row. 0 is below every real key.
__device__ __forceinline__ uint64_t logit_key(uint16_t b, int row) {
    if (b == 0x8000u) { b = 0; }
    const uint32_t ord = (b & 0x8000u) ? (~static_cast<uint32_t>(b) & 0xffffu) : (static_cast<uint32_t>(b) | 0x8000u);
    return (static_cast<uint64_t>(ord) << 32) | (0xffffffffu - static_cast<uint32_t>(row));
}

__device__ __forceinline__ uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }

__device__ __forceinline__ uint64_t shfl_u64(uint64_t v, int src) {
    const uint32_t lo = __shfl(static_cast<uint32_t>(v), src, 64);
    const uint32_t hi = __shfl(static_cast<uint32_t>(v >> 32), src, 64);
    return (static_cast<uint64_t>(hi) << 32) | lo;
}

// ---- top-cap form: every lane keeps the kCandidateCap largest keys it has seen, descending ----------

// x enters the descending list if it beats the last entry (a uniform skip when no lane's does).
__device__ __forceinline__ void list_insert(uint64_t (&l)[kCandidateCap], uint64_t x) {
    if (!__any(x > l[kCandidateCap - 1])) { return; }
#pragma unroll
    for (int i = 0; i < kCandidateCap; ++i) {
        const bool up = x > l[i];
        const uint64_t keep = up ? x : l[i];
        x = up ? l[i] : x;
        l[i] = keep;
    }
}

// Lists per column per wave: with TP < 16 the keys of a finished tile are first spread so that each
// lane owns one column (64 / TP lanes per column, TP / 4 rows each); with TP = 16 a lane keeps the
// 4 rows of its own MFMA column.
template <int TP>
constexpr int lists_per_column() { return TP == 16 ? 4 : 64 / TP; }

template <int W>
constexpr size_t topcap_lds_bytes() {
    return static_cast<size_t>(W) * 64 * kCandidateCap * 8 + static_cast<size_t>(W) * (64 + kCandidateCap) * 8;
}

// Per-lane DMA source offsets within a tile (fixed for the kernel). Nibble DMA d covers rows
// 4d .. 4d+3 (16 lanes x 16 B per row); LDS slot s of row r holds piece s ^ r. High DMA d covers
// rows 8d .. 8d+7 (8 lanes per row); slot s of row r holds piece s ^ (r / 2 % 8). Scales: lane ->
// (row lane / 4, 4-byte piece lane % 4).
template <int CG>
struct LinDma {
    int n[Chunk<CG>::kNibDma];
    int h[Chunk<CG>::kHighDma];
    int s;
};

template <int CG>
__device__ __forceinline__ LinDma<CG> make_lin_dma(int lane, int G) {
    using C = Chunk<CG>;
    LinDma<CG> d;
#pragma unroll
    for (int q = 0; q < C::kNibDma; ++q) {
        constexpr int P = C::kNibRow / 16;
        const int row = (1024 / C::kNibRow) * q + lane / P;
        const int slot = lane % P;
        d.n[q] = row * (G * 32) + 16 * (slot ^ swz<C::kNibRow>(row));
    }
#pragma unroll
    for (int q = 0; q < C::kHighDma; ++q) {
        constexpr int P = C::kHighRow / 16;
        const int row = (1024 / C::kHighRow) * q + lane / P;
        const int slot = lane % P;
        d.h[q] = row * (G * 16) + 16 * (slot ^ swz<C::kHighRow>(row));
    }
    constexpr int SL = C::kScaleRow / 4; // 4-byte scale words per row
    d.s = lane < kTileRows * SL ? (lane / SL) * (G * 2) + 4 * (lane % SL) : kOutOfRange;
    return d;
}

struct Planes {
    __amdgpu_buffer_rsrc_t n, h, s;
};

// The whole source offset rides in the range-checked voffset (soffset is not checked), so rows past
// N and groups past G at the end of a plane read as zero instead of past the allocation.
// KEEP_PARTIAL: the high and scale planes, of which a chunk reads part of each 128-byte line (64 and
// 8 bytes per row at 4 groups), load with the default cache policy, so the later chunks of a row
// find the rest of the line in L2 instead of fetching it again (the K-outer form reads a row's
// chunks one block apart); the nibble rows are whole lines and stay non-temporal.
template <int CG, bool KEEP_PARTIAL = false>
__device__ __forceinline__ void issue_item(NMI_AS3 char* st, const Planes& pl, const LinDma<CG>& d, int tile, int chunk,
                                           int G) {
    using C = Chunk<CG>;
    const int r0 = tile * kTileRows;
    const int o_n = r0 * (G * 32) + chunk * C::kNibRow;
    const int o_h = r0 * (G * 16) + chunk * C::kHighRow;
    const int o_s = r0 * (G * 2) + chunk * C::kScaleRow;
#pragma unroll
    for (int q = 0; q < C::kNibDma; ++q) { dma16_nt(pl.n, st + q * 1024, d.n[q] + o_n, 0); }
    if constexpr (KEEP_PARTIAL) {
#pragma unroll
        for (int q = 0; q < C::kHighDma; ++q) { dma16(pl.h, st + C::kNib + q * 1024, d.h[q] + o_h, 0); }
        dma4s(pl.s, st + C::kNib + C::kHigh, d.s + o_s, 0);
    } else {
#pragma unroll
        for (int q = 0; q < C::kHighDma; ++q) { dma16_nt(pl.h, st + C::kNib + q * 1024, d.h[q] + o_h, 0); }
        dma4s_nt(pl.s, st + C::kNib + C::kHigh, d.s + o_s, 0);
    }
}

template <int TP, int W, int CG, bool HEAD>
__global__ __launch_bounds__(64 * W) void linear_q6_kernel(LinearArgs a) {
    using CH = Chunk<CG>;
    extern __shared__ __attribute__((aligned(16))) char dsmem[];
    NMI_AS3 char* smem = (NMI_AS3 char*)dsmem;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int G = a.G;
    const int xstride = a.Kp * 2 + kXPad;
    NMI_AS3 char* xl = smem;
    NMI_AS3 uint32_t* cmax = (NMI_AS3 uint32_t*)(smem + x_lds_bytes(TP, a.Kp)); // per column: max |x| (BF16 bits)
    NMI_AS3 float* cfac = (NMI_AS3 float*)(cmax + TP);                         // per column: power-of-two factor
    const size_t ring0 = (x_lds_bytes(TP, a.Kp) + static_cast<size_t>(TP) * 8 + 15) & ~static_cast<size_t>(15);
    NMI_AS3 char* ring = smem + ring0 + static_cast<size_t>(wave) * 2 * CH::kStage;

    const int gw = blockIdx.x * W + wave; // wave index of the launch
    const int nch = (G + CG - 1) / CG;
    const int ntw = gw < a.ntiles ? (a.ntiles - gw + a.waves - 1) / a.waves : 0;
    const int items = ntw * nch;
    const Planes pl{raw_buffer(a.qdata, a.nib_bytes), raw_buffer(a.qhigh, a.high_bytes), raw_buffer(a.scales, a.scale_bytes)};
    const LinDma<CG> dl = make_lin_dma<CG>(lane, G);
    const int c = lane & 15;  // MFMA column (x column) of this lane
    const int b = lane >> 4;  // 16-code block of a group / accumulator row block

    // (tile, chunk) of item j and of item j + 2 (the next DMA), advanced by one item per iteration
    int tile = gw, chunk = 0;
    int tile2 = gw, chunk2 = 0;
    auto advance = [&](int& t, int& ch) {
        if (++ch == nch) {
            ch = 0;
            t += a.waves;
        }
    };
    // the first two chunks stream in while x is staged (the ring and x do not overlap)
    if (items > 0) { issue_item<CG>(ring, pl, dl, tile2, chunk2, G); }
    advance(tile2, chunk2);
    if (items > 1) { issue_item<CG>(ring + CH::kStage, pl, dl, tile2, chunk2, G); }
    advance(tile2, chunk2);
    // ---- x of this pass -> LDS as FP16, each 8-element block stored as (e0, e4, e1, e5, e2, e6, e3,
    // e7); columns past the pass and elements past K are zero. Two passes over x (it is small):
    // the column maxima, then the scaled values.
    const int kb = a.Kp / 8;
    const bool vec = (a.K & 7) == 0;
    auto load8 = [&](int t, int k0, uint16_t (&v)[8]) {
        if (t < a.tp && vec && k0 + 8 <= a.K) {
            const i4 raw = *reinterpret_cast<const i4*>(a.x + k0 + static_cast<int64_t>(a.K) * (a.t0 + t));
#pragma unroll
            for (int e = 0; e < 8; ++e) { v[e] = static_cast<uint16_t>(static_cast<uint32_t>(raw[e >> 1]) >> (16 * (e & 1))); }
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                v[e] = (t < a.tp && k0 + e < a.K) ? a.x[k0 + e + static_cast<int64_t>(a.K) * (a.t0 + t)] : 0;
            }
        }
    };
    if (threadIdx.x < TP) { cmax[threadIdx.x] = 0; }
    __syncthreads();
    for (int i = threadIdx.x; i < TP * kb; i += 64 * W) {
        const int t = i / kb;
        uint16_t v[8];
        load8(t, (i - t * kb) * 8, v);
        uint32_t m = 0;
#pragma unroll
        for (int e = 0; e < 8; ++e) { m = max(m, static_cast<uint32_t>(v[e] & 0x7fffu)); } // |x| orders as its bits
        if (m != 0) { atomicMax((uint32_t*)&cmax[t], m); }
    }
    __syncthreads();
    if (threadIdx.x < TP) {
        // factor = 2^(14 - floor(log2 max|x|)): max|x| lands in [2^14, 2^15) and every BF16 value of the
        // column is exact in FP16 down to 2^-28 of the maximum (clamped so the factor stays finite).
        const uint32_t m = cmax[threadIdx.x];
        float f = 1.0f;
        if (m != 0 && m < 0x7f80u) { f = ldexpf(1.0f, 14 - max(static_cast<int>(m >> 7) - 127, -100)); }
        cfac[threadIdx.x] = f;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < TP * kb; i += 64 * W) {
        const int t = i / kb;
        const int blk = i - t * kb;
        uint16_t v[8];
        load8(t, blk * 8, v);
        const float f = cfac[t];
        h2 pk[4];
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            pk[p] = h2{static_cast<_Float16>(bf16_to_f32(v[p]) * f), static_cast<_Float16>(bf16_to_f32(v[p + 4]) * f)};
        }
        *(NMI_AS3 i4*)(xl + t * xstride + blk * 16) = __builtin_bit_cast(i4, pk);
    }
    __syncthreads();

    // x column of this lane's MFMA column: lanes past the pass's columns alias a real one (their
    // results are never stored), so every lane reads LDS unconditionally
    const NMI_AS3 char* xcol = xl + (c & (TP - 1)) * xstride + 2 * b * 16;
    const float cinv = 1.0f / cfac[c & (TP - 1)]; // a power of two: exact
    const uint32_t kMaskA = 0x003f003fu;  // the 6 code bits of each FP16 half
    const uint32_t kConstB = 0x64206420u; // exponent of 1024 and bit 5 (the flip) of each half

    float tot[4] = {0.f, 0.f, 0.f, 0.f};
    uint64_t best = 0;
    // top-cap form: the sequence and in-sequence column of this lane's MFMA column, and whether its
    // keys carry penalties (stochastic sequences with a nonzero presence or frequency penalty; the
    // keys of a greedy sequence are the raw logits, so its list head is the argmax)
    uint64_t lst[kCandidateCap];
    int hseq = 0, hcol = 0;
    bool hpen = false;
    if constexpr (HEAD) {
#pragma unroll
        for (int q = 0; q < kCandidateCap; ++q) { lst[q] = 0; }
        if (c < a.tp) {
            const int t = a.t0 + c;
            hseq = t / a.cols_per_seq;
            hcol = t - hseq * a.cols_per_seq;
            const nmi_sampling_config& cf = a.config[hseq];
            hpen = cf.temperature > 0.0f && (cf.presence_penalty != 0.0f || cf.frequency_penalty != 0.0f);
        }
    }
#pragma unroll 1
    for (int j = 0; j < items; ++j) {
        NMI_AS3 char* st = ring + (j & 1) * CH::kStage;
        if (j + 1 < items) {
            __builtin_amdgcn_s_waitcnt((CH::kDma & 0xf) | ((CH::kDma >> 4) << 14) | (0x7 << 4) | (0xf << 8));
        } else {
            __builtin_amdgcn_s_waitcnt((0x7 << 4) | (0xf << 8));
        }
        // chunk j -> registers, then the stage takes chunk j + 2
        uint64_t nib[CG];
        uint32_t hig[CG];
        uint32_t sc[4][CG / 2];
        const int r = c; // A-operand row of this lane
#pragma unroll
        for (int gl = 0; gl < CG; ++gl) {
            nib[gl] = *(const NMI_AS3 uint64_t*)(st + r * CH::kNibRow + 16 * ((2 * gl + (b >> 1)) ^ swz<CH::kNibRow>(r)) +
                                                 8 * (b & 1));
            hig[gl] = *(const NMI_AS3 uint32_t*)(st + CH::kNib + r * CH::kHighRow + 16 * (gl ^ swz<CH::kHighRow>(r)) + 4 * b);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
            for (int q = 0; q < CG / 2; ++q) {
                sc[i][q] = *(const NMI_AS3 uint32_t*)(st + CH::kNib + CH::kHigh + (4 * b + i) * CH::kScaleRow + 4 * q);
            }
        }
        if (j + 2 < items) {
            __builtin_amdgcn_s_waitcnt(0xc07f); // lgkmcnt(0): the stage is free
            issue_item<CG>(st, pl, dl, tile2, chunk2, G);
        }
        advance(tile2, chunk2);
        auto group = [&](int gl) {
            const NMI_AS3 char* xp = xcol + (chunk * CG + gl) * 128;
            const i4 x0 = *(const NMI_AS3 i4*)xp;
            const i4 x1 = *(const NMI_AS3 i4*)(xp + 16);
            h8 a0, a1;
            decode16(nib[gl], hig[gl], kMaskA, kConstB, a0, a1);
            f4 acc = {0.f, 0.f, 0.f, 0.f};
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, __builtin_bit_cast(h8, x0), acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, __builtin_bit_cast(h8, x1), acc, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t w = sc[i][gl >> 1];
                const float s = f16_bits_to_f32(static_cast<uint16_t>((gl & 1) ? (w >> 16) : (w & 0xffffu)));
                tot[i] = fmaf(s, acc[i], tot[i]);
            }
        };
        if (chunk * CG + CG <= G) {
            // a full chunk: straight-line code the scheduler can interleave across groups
#pragma unroll
            for (int gl = 0; gl < CG; ++gl) { group(gl); }
        } else {
            const int ng = G - chunk * CG;
#pragma unroll
            for (int gl = 0; gl < CG; ++gl) {
                if (gl < ng) { group(gl); }
            }
        }
        if (chunk == nch - 1) {
            // tile done: lane holds rows 4b + i, column c
            const int r0 = tile * kTileRows;
            uint64_t kk[4] = {0, 0, 0, 0};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = r0 + 4 * b + i;
                const uint16_t bfv = f32_to_bf16_bits(tot[i] * cinv);
                if (a.out != nullptr && c < a.tp && row < a.N) {
                    a.out[row + static_cast<int64_t>(a.N) * (a.t0 + c)] = bfv;
                }
                if (row < a.valid_rows) { best = max_u64(best, logit_key(bfv, row)); }
                if constexpr (HEAD) {
                    // rows past valid_rows (the token domain) never reach the penalty lookup: the
                    // counts array covers the domain only
                    const bool live = c < a.tp && row < a.valid_rows;
                    float v = bf16_to_f32(bfv);
                    if (hpen && live) {
                        v = adjusted_logit(v, row, a.config[hseq], a.drafts + static_cast<int64_t>(hseq) * (a.cols_per_seq - 1),
                                           hcol);
                    }
                    kk[i] = live ? sort_key(v, row) : 0ull;
                }
                tot[i] = 0.0f;
            }
            if constexpr (HEAD) {
                if constexpr (TP == 16) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) { list_insert(lst, kk[i]); }
                } else {
                    // lane -> (column lane / (64 / TP), rows s, s + 64 / TP, ... of the tile), s = lane % (64 / TP);
                    // row r of column col sits in lane col + 16 * (r / 4), register r % 4
                    constexpr int LPC = 64 / TP;
                    constexpr int RPL = TP / 4;
                    const int col = lane / LPC;
                    const int s0 = lane % LPC;
#pragma unroll
                    for (int e = 0; e < RPL; ++e) {
                        const int r = s0 + LPC * e;
                        const int src = col + 16 * (r >> 2);
                        uint64_t v = 0;
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            const uint64_t g = shfl_u64(kk[q], src);
                            v = q == (r & 3) ? g : v;
                        }
                        list_insert(lst, v);
                    }
                }
            }
        }
        advance(tile, chunk);
    }
    if (a.keys != nullptr) {
        best = max_u64(best, shfl_xor_u64(best, 16));
        best = max_u64(best, shfl_xor_u64(best, 32));
        if (lane < a.tp) { a.keys[static_cast<int64_t>(a.t0 + lane) * a.waves + gw] = best; }
    }
    if constexpr (HEAD) {
        // Workgroup top-cap per column: every lane's list goes to LDS (x and the ring are done with),
        // then wave w merges the W * lists_per_column lists of columns w, w + W, ...
        constexpr int LPC = lists_per_column<TP>();
        constexpr int NL = W * LPC;
        constexpr int LPL = (NL + 63) / 64;
        static_assert(LPL <= 2, "top-cap merge holds at most two lists per lane");
        __syncthreads();
        NMI_AS3 uint64_t* lists = (NMI_AS3 uint64_t*)smem;
#pragma unroll
        for (int q = 0; q < kCandidateCap; ++q) { lists[(wave * 64 + lane) * kCandidateCap + q] = lst[q]; }
        uint64_t* wcand = (uint64_t*)(lists + W * 64 * kCandidateCap + wave * 64);
        uint64_t* wout = (uint64_t*)(lists + W * 64 * kCandidateCap + W * 64 + wave * kCandidateCap);
        __syncthreads();
        for (int lc = wave; lc < a.tp; lc += W) {
            uint64_t k[LPL * kCandidateCap];
            uint64_t heads[LPL];
#pragma unroll
            for (int h = 0; h < LPL; ++h) {
                const int q = lane + 64 * h;
                const int w = q / LPC;
                const int sl = q % LPC;
                const int src = TP == 16 ? lc + 16 * sl : lc * LPC + sl;
                const bool ok = q < NL;
#pragma unroll
                for (int e = 0; e < kCandidateCap; ++e) {
                    k[h * kCandidateCap + e] = ok ? lists[(w * 64 + src) * kCandidateCap + e] : 0ull;
                }
                heads[h] = k[h * kCandidateCap];
            }
            wave_top_cap(k, heads, kCandidateCap, wcand, wout);
            if (lane < kCandidateCap) {
                a.cand[(static_cast<int64_t>(a.t0 + lc) * gridDim.x + blockIdx.x) * kCandidateCap + lane] = wout[lane];
            }
            wave_lds_sync();
        }
    }
}

// ---- wide form: more than 16 columns, 32 or 64 per pass over the weight ---------------------------
//
// The column passes above re-stream the whole weight once per 4, 8 or 16 columns (x of 16 columns
// at K = 5120 already fills the LDS). Here K is the outer loop: x moves through the LDS in blocks of
// 256 (4 groups) for all 16 * NCB columns, and each wave keeps FP32 totals for its MAXT tiles x
// 16 * NCB columns in registers while it streams those tiles' 4-group chunks of the block. A lane
// decodes its 16 codes of a group once and feeds NCB pairs of MFMAs (one per 16-column block).
// Each x block carries its own power-of-two column factors (its largest |x| lands in
// [2^14, 2^15), so its BF16 values are exact in FP16); a block's per-group sums, weighted by their
// scales, are rescaled by the factor's exact inverse into the totals. A workgroup runs ROUNDS
// rounds over K, each for MAXT further tiles per wave, so 64 columns (128 totals per 8 tiles, more
// than a lane has at two waves per SIMD) take 4 tiles per wave and two rounds: each code is decoded
// once for all 64 columns. The epilogue of a round writes BF16 logits, folds argmax keys, or per
// column merges the round's rows into the workgroup's kCandidateCap largest keys (top-cap form).
constexpr int kWideWaves = 8;
constexpr int kWideCG = 4;          // groups per streamed chunk and per x block (256 elements of K)
constexpr int kWideStages = 2;      // chunk stages per wave: kWideStages chunks in flight while one computes
constexpr int kXBlockCol = kWideCG * 128; // bytes of one column of an x block (FP16)
constexpr int kWideTilesPerWave = 8; // tiles per wave over all rounds (every form: the same grid)

// The two forms: 32 columns, 8 tiles per wave in one round, x blocks consumed in pairs (four
// buffers: the pair in use and the next pair); 64 columns, 4 tiles per wave per round, x blocks one
// after another (three buffers, the most that fit beside the chunk stages at 64 columns).
template <int NCB>
struct WideForm {
    static constexpr int kTiles = NCB == 2 ? 8 : 4;
    static constexpr int kRounds = kWideTilesPerWave / kTiles;
    static constexpr bool kPairs = NCB == 2;
    static constexpr int kXBuffers = kPairs ? 4 : 3;
};

template <int NCB>
constexpr size_t wide_x_bytes() { return static_cast<size_t>(WideForm<NCB>::kXBuffers) * 16 * NCB * (kXBlockCol + 4); } // x blocks + factors

template <int NCB>
constexpr size_t wide_lds_bytes() {
    constexpr size_t main = wide_x_bytes<NCB>() + static_cast<size_t>(kWideWaves) * kWideStages * Chunk<kWideCG>::kStage;
    // top-cap epilogue: the workgroup's BF16 logits of every column for one round, then the selection scratch
    constexpr size_t keys = static_cast<size_t>(16 * NCB) * kWideWaves * WideForm<NCB>::kTiles * kTileRows * 2 +
                            static_cast<size_t>(kWideWaves) * (64 + kCandidateCap) * 8;
    return main > keys ? main : keys;
}

// One item's per-group sums, weighted by the group scales: a lane decodes its 16 codes of each
// group once and feeds NCB pairs of MFMAs (one per 16-column block of the x block xk).
template <int NCB>
__device__ __forceinline__ void group_sums(const uint64_t (&nib)[kWideCG], const uint32_t (&hig)[kWideCG],
                                           const uint32_t (&sc)[4][kWideCG / 2], int ng, const NMI_AS3 char* xk, int c,
                                           int b, float (&bacc)[NCB][4]) {
    const uint32_t kMaskA = 0x003f003fu;
    const uint32_t kConstB = 0x64206420u;
#pragma unroll
    for (int gl = 0; gl < kWideCG; ++gl) {
        if (gl < ng) {
            h8 a0, a1;
            decode16(nib[gl], hig[gl], kMaskA, kConstB, a0, a1);
            const int q0 = 8 * gl + 2 * b;
#pragma unroll
            for (int cb = 0; cb < NCB; ++cb) {
                const NMI_AS3 char* xc = xk + (c + 16 * cb) * kXBlockCol;
                const i4 x0 = *(const NMI_AS3 i4*)(xc + 16 * (q0 ^ c));
                const i4 x1 = *(const NMI_AS3 i4*)(xc + 16 * ((q0 + 1) ^ c));
                f4 acc = {0.f, 0.f, 0.f, 0.f};
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, __builtin_bit_cast(h8, x0), acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, __builtin_bit_cast(h8, x1), acc, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const uint32_t w = sc[r][gl >> 1];
                    const float sv = f16_bits_to_f32(static_cast<uint16_t>((gl & 1) ? (w >> 16) : (w & 0xffffu)));
                    bacc[cb][r] = fmaf(sv, acc[r], bacc[cb][r]);
                }
            }
        }
    }
}

template <int NCB>
__global__ __launch_bounds__(64 * kWideWaves) void linear_q6_wide_kernel(LinearArgs a) {
    constexpr int W = kWideWaves;
    constexpr int CG = kWideCG;
    constexpr int MAXT = WideForm<NCB>::kTiles;
    constexpr int ROUNDS = WideForm<NCB>::kRounds;
    constexpr int NC = 16 * NCB;      // columns of the pass
    constexpr int TPC = 64 * W / NC;  // x staging threads per column (consecutive lanes of one wave)
    constexpr int EPT = CG * 64 / TPC; // x elements of a block per staging thread
    constexpr int NX = EPT / 8;       // 16-byte x loads per staging thread
    constexpr int S = kWideStages;
    static_assert(MAXT % S == 0 && MAXT > S && TPC <= 64, "wide geometry");
    using CH = Chunk<CG>;
    extern __shared__ __attribute__((aligned(16))) char dsmem[];
    NMI_AS3 char* smem = (NMI_AS3 char*)dsmem;
    constexpr int XB = WideForm<NCB>::kXBuffers;
    NMI_AS3 float* finv = (NMI_AS3 float*)(smem + XB * NC * kXBlockCol); // [XB][NC] 1 / column factor
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    NMI_AS3 char* ring = smem + wide_x_bytes<NCB>() + wave * S * CH::kStage;
    const int G = a.G;
    const int nkb = (G + CG - 1) / CG;
    const int gw = blockIdx.x * W + wave;
    const int nwaves = gridDim.x * W;
    const Planes pl{raw_buffer(a.qdata, a.nib_bytes), raw_buffer(a.qhigh, a.high_bytes), raw_buffer(a.scales, a.scale_bytes)};
    const LinDma<CG> dl = make_lin_dma<CG>(lane, G);
    const int c = lane & 15; // MFMA column within a 16-column block
    const int b = lane >> 4; // 16-code block of a group / accumulator row block

    // x staging: thread -> (column scol, K slice spart of a block). One 16-byte buffer load per piece
    // whatever the column or K (past K or past the pass's columns the offset leaves the range and
    // reads zero), so every lane issues exactly NX loads.
    const int scol = threadIdx.x / TPC;
    const int spart = threadIdx.x - scol * TPC;
    // The pass's own columns only (at most 8192 x 64 BF16 values), so the out-of-range offset lies
    // far past the resource whatever T is.
    const __amdgpu_buffer_rsrc_t xr_src = raw_buffer(a.x + static_cast<int64_t>(a.K) * a.t0, static_cast<int64_t>(a.K) * a.tp * 2);
    i4 xr[NX];
    auto xload = [&](int kb) {
#pragma unroll
        for (int n = 0; n < NX; ++n) {
            const int k = kb * CG * 64 + spart * EPT + 8 * n;
            const int off = (scol < a.tp && k < a.K) ? 2 * (a.K * scol + k) : kOutOfRange;
            xr[n] = __builtin_bit_cast(i4, __builtin_amdgcn_raw_buffer_load_b128(xr_src, off, 0, 0));
        }
    };
    // Column factor over the TPC lanes of the column, then the pieces as FP16 in the pairing
    // (e0, e4, e1, e5, e2, e6, e3, e7); piece q of column col sits at 16-byte slot q ^ (col % 16).
    auto xstage = [&](int buf) {
        uint32_t m = 0;
#pragma unroll
        for (int n = 0; n < NX; ++n) {
#pragma unroll
            for (int h = 0; h < 4; ++h) {
                const uint32_t w = static_cast<uint32_t>(xr[n][h]);
                m = max(m, max(w & 0x7fffu, (w >> 16) & 0x7fffu));
            }
        }
#pragma unroll
        for (int s = 1; s < TPC; s <<= 1) { m = max(m, static_cast<uint32_t>(__shfl_xor(static_cast<int>(m), s, 64))); }
        float f = 1.0f;
        if (m != 0 && m < 0x7f80u) { f = ldexpf(1.0f, 14 - max(static_cast<int>(m >> 7) - 127, -100)); }
        NMI_AS3 char* dst = smem + buf * NC * kXBlockCol + scol * kXBlockCol;
#pragma unroll
        for (int n = 0; n < NX; ++n) {
            uint16_t v[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) { v[e] = static_cast<uint16_t>(static_cast<uint32_t>(xr[n][e >> 1]) >> (16 * (e & 1))); }
            h2 pk[4];
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                pk[p] = h2{static_cast<_Float16>(bf16_to_f32(v[p]) * f), static_cast<_Float16>(bf16_to_f32(v[p + 4]) * f)};
            }
            const int q = spart * NX + n;
            *(NMI_AS3 i4*)(dst + 16 * (q ^ (scol & 15))) = __builtin_bit_cast(i4, pk);
        }
        if (spart == 0) { finv[buf * NC + scol] = 1.0f / f; } // a power of two: exact
    };

    // waits for item j: the S - 1 younger items stay in flight, and the x loads while they are younger
    constexpr int kYoung = (S - 1) * CH::kDma;
    constexpr int kWaitItem = (kYoung & 0xf) | ((kYoung >> 4) << 14) | (0x7 << 4) | (0xf << 8);
    constexpr int kWaitItemX = ((kYoung + NX) & 0xf) | (((kYoung + NX) >> 4) << 14) | (0x7 << 4) | (0xf << 8);
    constexpr int RPW = MAXT * kTileRows; // rows per wave, column and round
    NMI_AS3 uint16_t* lg = (NMI_AS3 uint16_t*)smem;

#pragma unroll 1
    for (int round = 0; round < ROUNDS; ++round) {
        // This round's tiles of the wave: gw + (round * MAXT + j) * nwaves, j < MAXT.
        const int tile0 = gw + round * MAXT * nwaves;
        float tot[MAXT][NCB][4];
#pragma unroll
        for (int i = 0; i < MAXT; ++i) {
#pragma unroll
            for (int cb = 0; cb < NCB; ++cb) {
#pragma unroll
                for (int r = 0; r < 4; ++r) { tot[i][cb][r] = 0.0f; }
            }
        }
        if constexpr (WideForm<NCB>::kPairs) {
        // Blocks go in pairs: item j of pair p streams chunk 2p + (j & 1) of tile tile0 + (j / 2) *
        // nwaves, so a tile's two chunks of the pair are consecutive items and the 128-byte lines of
        // its high plane (64 bytes per chunk) are used whole while they are in L2. x block kb lives
        // in buffer kb % 4: pair p computes on blocks 2p and 2p + 1 while blocks 2p + 2 and 2p + 3
        // are staged. Slots past the last tile and blocks past the last one still issue their DMAs
        // (they read zero or bytes that are never used), so every wait below is one fixed count.
        constexpr int J = 2 * MAXT; // items per pair
        static_assert(J > 2 * S, "both x blocks of the next pair land inside the pair");
        auto issue = [&](NMI_AS3 char* st, int pp, int j) {
            issue_item<CG, true>(st, pl, dl, tile0 + (j >> 1) * nwaves, 2 * pp + (j & 1), G);
        };
        const int npairs = (nkb + 1) / 2;
        auto clamp_block = [&](int kb) { return kb < nkb ? kb : nkb - 1; };
        xload(0);
#pragma unroll
        for (int j = 0; j < S; ++j) { issue(ring + j * CH::kStage, 0, j); }
        __builtin_amdgcn_s_waitcnt(((S * CH::kDma) & 0xf) | (((S * CH::kDma) >> 4) << 14) | (0x7 << 4) | (0xf << 8));
        xstage(0);
        xload(clamp_block(1));
        __builtin_amdgcn_s_waitcnt(0); // once per round: block 1 lands behind the first items
        xstage(1);
#pragma unroll 1
        for (int pp = 0; pp < npairs; ++pp) {
            __syncthreads(); // blocks 2p, 2p + 1 are in LDS; every wave is done with blocks 2p - 2, 2p - 1
            // x loads of block 2p + 2: issued after items 0 .. S - 1, staged at item S; those of block
            // 2p + 3: issued at item S after items .. 2S - 1, staged at item 2S
            xload(clamp_block(2 * pp + 2));
            float fi[2][NCB];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
#pragma unroll
                for (int cb = 0; cb < NCB; ++cb) { fi[h][cb] = finv[((2 * pp + h) & (XB - 1)) * NC + c + 16 * cb]; }
            }
#pragma unroll
            for (int j = 0; j < J; ++j) {
                const int i = j >> 1;
                const int h = j & 1;
                const int kb = 2 * pp + h;
                NMI_AS3 char* st = ring + (j % S) * CH::kStage;
                if (j < S || (j > S && j < 2 * S)) {
                    __builtin_amdgcn_s_waitcnt(kWaitItemX);
                } else {
                    __builtin_amdgcn_s_waitcnt(kWaitItem);
                }
                if (j == S) {
                    xstage((2 * pp + 2) & (XB - 1));
                    xload(clamp_block(2 * pp + 3));
                }
                if (j == 2 * S) { xstage((2 * pp + 3) & (XB - 1)); }
                const NMI_AS3 char* xk = smem + (kb & (XB - 1)) * NC * kXBlockCol;
                const int ng = min(CG, G - kb * CG); // <= 0 for the block past the last
                float bacc[NCB][4];
#pragma unroll
                for (int cb = 0; cb < NCB; ++cb) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) { bacc[cb][r] = 0.0f; }
                }
                uint64_t nib[CG];
                uint32_t hig[CG];
                uint32_t sc[4][CG / 2];
#pragma unroll
                for (int gl = 0; gl < CG; ++gl) {
                    nib[gl] = *(const NMI_AS3 uint64_t*)(st + c * CH::kNibRow + 16 * ((2 * gl + (b >> 1)) ^ swz<CH::kNibRow>(c)) +
                                                         8 * (b & 1));
                    hig[gl] = *(const NMI_AS3 uint32_t*)(st + CH::kNib + c * CH::kHighRow + 16 * (gl ^ swz<CH::kHighRow>(c)) + 4 * b);
                }
#pragma unroll
                for (int r = 0; r < 4; ++r) {
#pragma unroll
                    for (int q = 0; q < CG / 2; ++q) {
                        sc[r][q] = *(const NMI_AS3 uint32_t*)(st + CH::kNib + CH::kHigh + (4 * b + r) * CH::kScaleRow + 4 * q);
                    }
                }
                __builtin_amdgcn_s_waitcnt(0xc07f); // lgkmcnt(0): the stage is free
                if (j + S < J) {
                    issue(st, pp, j + S);
                } else {
                    issue(st, pp + 1, j + S - J);
                }
                group_sums<NCB>(nib, hig, sc, ng, xk, c, b, bacc);
                if (ng > 0) {
#pragma unroll
                    for (int cb = 0; cb < NCB; ++cb) {
#pragma unroll
                        for (int r = 0; r < 4; ++r) { tot[i][cb][r] = fmaf(bacc[cb][r], fi[h][cb], tot[i][cb][r]); }
                    }
                }
            }
        }
        } else {
        // Blocks go one after another: item j of block kb streams chunk kb of tile tile0 + j * nwaves.
        // x block kb lives in buffer kb % XB: block kb computes while block kb + 1 sits staged, and
        // block kb + 2 is loaded at the block's start and staged at item S, once its loads have
        // landed. Slots past the last tile and the block past the last one still issue their DMAs
        // (they read zero or bytes that are never used), so every wait below is one fixed count.
        auto issue = [&](NMI_AS3 char* st, int kb, int j) { issue_item<CG, true>(st, pl, dl, tile0 + j * nwaves, kb, G); };
        auto clamp_block = [&](int kb) { return kb < nkb ? kb : nkb - 1; };
        xload(0);
#pragma unroll
        for (int j = 0; j < S; ++j) { issue(ring + j * CH::kStage, 0, j); }
        __builtin_amdgcn_s_waitcnt(((S * CH::kDma) & 0xf) | (((S * CH::kDma) >> 4) << 14) | (0x7 << 4) | (0xf << 8));
        xstage(0);
        xload(clamp_block(1));
        __builtin_amdgcn_s_waitcnt(0); // once per round: block 1 lands behind the first items
        xstage(1);

        int buf = 0;      // kb % XB
        int buf_next = 2; // (kb + 2) % XB
#pragma unroll 1
        for (int kb = 0; kb < nkb; ++kb) {
            __syncthreads(); // blocks kb and kb + 1 are in LDS; every wave is done with block kb - 1
            xload(clamp_block(kb + 2));
            float fi[NCB];
#pragma unroll
            for (int cb = 0; cb < NCB; ++cb) { fi[cb] = finv[buf * NC + c + 16 * cb]; }
            const NMI_AS3 char* xk = smem + buf * NC * kXBlockCol;
            const int ng = min(CG, G - kb * CG);
#pragma unroll
            for (int j = 0; j < MAXT; ++j) {
                NMI_AS3 char* st = ring + (j % S) * CH::kStage;
                if (j < S) {
                    __builtin_amdgcn_s_waitcnt(kWaitItemX);
                } else {
                    __builtin_amdgcn_s_waitcnt(kWaitItem);
                }
                if (j == S) { xstage(buf_next); }
                float bacc[NCB][4];
#pragma unroll
                for (int cb = 0; cb < NCB; ++cb) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) { bacc[cb][r] = 0.0f; }
                }
                uint64_t nib[CG];
                uint32_t hig[CG];
                uint32_t sc[4][CG / 2];
#pragma unroll
                for (int gl = 0; gl < CG; ++gl) {
                    nib[gl] = *(const NMI_AS3 uint64_t*)(st + c * CH::kNibRow + 16 * ((2 * gl + (b >> 1)) ^ swz<CH::kNibRow>(c)) +
                                                         8 * (b & 1));
                    hig[gl] = *(const NMI_AS3 uint32_t*)(st + CH::kNib + c * CH::kHighRow + 16 * (gl ^ swz<CH::kHighRow>(c)) + 4 * b);
                }
#pragma unroll
                for (int r = 0; r < 4; ++r) {
#pragma unroll
                    for (int q = 0; q < CG / 2; ++q) {
                        sc[r][q] = *(const NMI_AS3 uint32_t*)(st + CH::kNib + CH::kHigh + (4 * b + r) * CH::kScaleRow + 4 * q);
                    }
                }
                __builtin_amdgcn_s_waitcnt(0xc07f); // lgkmcnt(0): the stage is free
                if (j + S < MAXT) {
                    issue(st, kb, j + S);
                } else {
                    issue(st, kb + 1, j + S - MAXT);
                }
                group_sums<NCB>(nib, hig, sc, ng, xk, c, b, bacc);
#pragma unroll
                for (int cb = 0; cb < NCB; ++cb) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) { tot[j][cb][r] = fmaf(bacc[cb][r], fi[cb], tot[j][cb][r]); }
                }
            }
            buf = buf == XB - 1 ? 0 : buf + 1;
            buf_next = buf_next == XB - 1 ? 0 : buf_next + 1;
        }
        }
        __builtin_amdgcn_s_waitcnt(0); // the DMAs of the items past the last block
        __syncthreads();               // LDS is free for the epilogue

        // ---- epilogue of the round: lane holds rows 4b + r of tile tile0 + i * nwaves for columns
        // c + 16 cb. The top-cap form first puts the round's BF16 logits in LDS ([column][wave][tile
        // slot][16 rows]).
        uint64_t best[NCB]; // argmax keys of the round
#pragma unroll
        for (int cb = 0; cb < NCB; ++cb) { best[cb] = 0; }
#pragma unroll
        for (int i = 0; i < MAXT; ++i) {
            const int r0 = (tile0 + i * nwaves) * kTileRows + 4 * b;
#pragma unroll
            for (int cb = 0; cb < NCB; ++cb) {
                const int col = c + 16 * cb;
                uint16_t bf[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    bf[r] = f32_to_bf16_bits(tot[i][cb][r]);
                    if (a.keys != nullptr && r0 + r < a.valid_rows) { best[cb] = max_u64(best[cb], logit_key(bf[r], r0 + r)); }
                }
                const uint2 packed{static_cast<uint32_t>(bf[0]) | (static_cast<uint32_t>(bf[1]) << 16),
                                   static_cast<uint32_t>(bf[2]) | (static_cast<uint32_t>(bf[3]) << 16)};
                if (a.cand != nullptr) {
                    *(NMI_AS3 i2*)(lg + (col * W + wave) * RPW + i * kTileRows + 4 * b) =
                        i2{static_cast<int>(packed.x), static_cast<int>(packed.y)};
                }
                if (a.out != nullptr && col < a.tp) {
                    uint16_t* o = a.out + static_cast<int64_t>(a.N) * (a.t0 + col) + r0;
                    if (r0 + 4 <= a.N && (a.N & 3) == 0) { // 8-byte aligned
                        *reinterpret_cast<uint2*>(o) = packed;
                    } else {
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            if (r0 + r < a.N) { o[r] = bf[r]; }
                        }
                    }
                }
            }
        }
        if (a.keys != nullptr) {
            // the wave's key per column over the rounds so far: folded into its own slot (the
            // earlier round's value is this lane's own store)
#pragma unroll
            for (int cb = 0; cb < NCB; ++cb) {
                uint64_t v = max_u64(best[cb], shfl_xor_u64(best[cb], 16));
                v = max_u64(v, shfl_xor_u64(v, 32));
                if (lane < 16 && c + 16 * cb < a.tp) {
                    uint64_t* kslot = a.keys + static_cast<int64_t>(a.t0 + c + 16 * cb) * nwaves + gw;
                    *kslot = round > 0 ? max_u64(v, *kslot) : v;
                }
            }
        }
        if (a.cand != nullptr) {
            // Top-cap form: wave w takes columns w, w + W, ...: the round's W * RPW keys of the
            // column (penalty-adjusted logits of rows below valid_rows), KPL per lane, plus the
            // workgroup's list from the earlier rounds (one key per lane below kCandidateCap, read
            // back from its own candidate slot), then the kCandidateCap largest.
            constexpr int KPL = W * RPW / 64; // keys per lane
            uint64_t* wcand = (uint64_t*)(smem + NC * W * RPW * 2 + wave * 64 * 8);
            uint64_t* wout = (uint64_t*)(smem + NC * W * RPW * 2 + W * 64 * 8 + wave * kCandidateCap * 8);
            __syncthreads();
#pragma unroll 1
            for (int lc = wave; lc < a.tp; lc += W) {
                const int t = a.t0 + lc;
                const int hseq = t / a.cols_per_seq;
                const int hcol = t - hseq * a.cols_per_seq;
                const nmi_sampling_config& cf = a.config[hseq];
                const bool hpen = cf.temperature > 0.0f && (cf.presence_penalty != 0.0f || cf.frequency_penalty != 0.0f);
                uint64_t* slot_out = a.cand + (static_cast<int64_t>(t) * gridDim.x + blockIdx.x) * kCandidateCap;
                uint64_t k[KPL + 1];
#pragma unroll
                for (int e = 0; e < KPL; ++e) {
                    const int slot = (e % (RPW / 64)) * 64 + lane; // row slot within the origin wave
                    const int wv = e / (RPW / 64);                 // origin wave
                    const int row = ((blockIdx.x * W + wv) + (round * MAXT + slot / kTileRows) * nwaves) * kTileRows +
                                    slot % kTileRows;
                    k[e] = 0;
                    if (row < a.valid_rows) { // the penalty counts cover the token domain only
                        float v = bf16_to_f32(lg[(lc * W + wv) * RPW + slot]);
                        if (hpen) { v = adjusted_logit(v, row, cf, a.drafts + static_cast<int64_t>(hseq) * (a.cols_per_seq - 1), hcol); }
                        k[e] = sort_key(v, row);
                    }
                }
                // this wave wrote the slot in the earlier round (same column, same lanes)
                k[KPL] = round > 0 && lane < kCandidateCap ? slot_out[lane] : 0ull;
                // the lane maxima bound the threshold: the cap largest of them leave a few dozen
                // candidates, where all keys per lane as heads cost one ballot per key and bit
                uint64_t head[1] = {k[0]};
#pragma unroll
                for (int e = 1; e <= KPL; ++e) { head[0] = max_u64(head[0], k[e]); }
                wave_top_cap(k, head, kCandidateCap, wcand, wout);
                if (lane < kCandidateCap) { slot_out[lane] = wout[lane]; }
                wave_lds_sync();
            }
        }
        __syncthreads(); // the next round's x and chunk stages reuse the LDS
    }
}

// One workgroup per column: the largest partial key -> the row.
__global__ __launch_bounds__(256) void linear_argmax_reduce_kernel(const uint64_t* keys, int32_t waves, int32_t* out) {
    const int t = blockIdx.x;
    uint64_t best = 0;
    for (int i = threadIdx.x; i < waves; i += 256) { best = max_u64(best, keys[static_cast<int64_t>(t) * waves + i]); }
#pragma unroll
    for (int m = 32; m > 0; m >>= 1) { best = max_u64(best, shfl_xor_u64(best, m)); }
    __shared__ uint64_t wb[4];
    if ((threadIdx.x & 63) == 0) { wb[threadIdx.x >> 6] = best; }
    __syncthreads();
    if (threadIdx.x == 0) {
        best = max_u64(max_u64(wb[0], wb[1]), max_u64(wb[2], wb[3]));
        out[t] = static_cast<int32_t>(0xffffffffu - static_cast<uint32_t>(best));
    }
}

size_t lds_bytes(int TP, int W, int CG, int Kp) {
    const size_t x = static_cast<size_t>(TP) * (Kp * 2 + kXPad) + static_cast<size_t>(TP) * 8;
    const size_t stage = CG == 8 ? Chunk<8>::kStage : Chunk<4>::kStage;
    return ((x + 15) & ~static_cast<size_t>(15)) + static_cast<size_t>(W) * 2 * stage;
}

} // namespace

// Built instances (columns per pass, waves per workgroup, groups per chunk), in order of preference
// (measured on MI355X: 8 waves with 8-group chunks stream best; 4-group chunks free the LDS that
// 16 columns of x need; fewer columns per pass re-stream the weight). The first whose LDS map fits
// is taken, starting from the column class of T.
struct LinearInstance {
    int tp, waves, cg;
};
constexpr LinearInstance kInstances[] = {
    {16, 8, 4}, {16, 4, 4},                                    // T > 8
    {8, 8, 8}, {8, 8, 4}, {8, 4, 8}, {8, 4, 4},                // T in 5..8 (T > 8 when x is too large)
    {4, 8, 8}, {4, 16, 4}, {4, 8, 4}, {4, 4, 4},               // T <= 4 (and the last resort)
};
constexpr int kInstanceCount = sizeof(kInstances) / sizeof(kInstances[0]);

LinearPlan plan_linear(int32_t N, int32_t Kp, int32_t T, bool top_cap, int32_t K) {
    const int32_t ntiles = (N + kTileRows - 1) / kTileRows;
    constexpr size_t kLds = 160 * 1024;
    const int32_t wide_grid = (ntiles + kWideWaves * kWideTilesPerWave - 1) / (kWideWaves * kWideTilesPerWave);
    if (T > 16 && K % 8 == 0 && wide_grid <= kLinearGrid) {
        // one pass over the weight per 32 columns (T <= 32) or per 64 columns in two rounds (above)
        LinearPlan p{};
        p.wide = true;
        p.tp = T > 32 ? 64 : 32;
        p.waves = kWideWaves;
        p.cg = kWideCG;
        p.lds = p.tp == 64 ? wide_lds_bytes<4>() : wide_lds_bytes<2>();
        p.passes = (T + p.tp - 1) / p.tp;
        p.grid = wide_grid;
        return p;
    }
    const int first = T <= 4 ? 6 : (T <= 8 ? 2 : 0);
    LinearPlan p{};
    for (int i = first; i < kInstanceCount; ++i) {
        if (top_cap && kInstances[i].waves > 8) { continue; } // the top-cap merge holds <= 2 lists per lane
        p.tp = kInstances[i].tp;
        p.waves = kInstances[i].waves;
        p.cg = kInstances[i].cg;
        p.lds = lds_bytes(p.tp, p.waves, p.cg, Kp);
        if (p.lds <= kLds) { break; }
    }
    p.passes = (T + p.tp - 1) / p.tp;
    // Waves get equal tile counts: the fewest workgroups (at most one per CU) for which every wave
    // holds ceil(ntiles / (256 * waves)) tiles, instead of all 256 with a partial last round.
    const int32_t per_wave = (ntiles + kLinearGrid * p.waves - 1) / (kLinearGrid * p.waves);
    const int32_t waves_needed = (ntiles + per_wave - 1) / per_wave;
    p.grid = std::max<int32_t>(1, std::min<int32_t>(kLinearGrid, (waves_needed + p.waves - 1) / p.waves));
    return p;
}

size_t linear_argmax_workspace_bytes(int32_t T) {
    return static_cast<size_t>(T) * kLinearGrid * kLinearMaxWaves * sizeof(uint64_t);
}

size_t linear_topcap_workspace_bytes(int32_t T) {
    return static_cast<size_t>(T) * kLinearGrid * kCandidateCap * sizeof(uint64_t);
}

template <int TP, int W, int CG, bool HEAD>
void launch_kernel(const LinearArgs& a, const LinearPlan& p, hipStream_t stream) {
    static const bool lds_raised = [] {
        NMI_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(&linear_q6_kernel<TP, W, CG, HEAD>),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
        return true;
    }();
    (void)lds_raised;
    size_t lds = p.lds;
    if constexpr (HEAD) { lds = std::max(lds, topcap_lds_bytes<W>()); }
    hipLaunchKernelGGL((linear_q6_kernel<TP, W, CG, HEAD>), dim3(p.grid), dim3(64 * W), lds, stream, a);
}

template <int TP, int W, int CG>
void launch_instance(const LinearArgs& a, const LinearPlan& p, hipStream_t stream) {
    if constexpr (W <= 8) {
        if (a.cand != nullptr) {
            launch_kernel<TP, W, CG, true>(a, p, stream);
            return;
        }
    } else {
        if (a.cand != nullptr) { throw Unsupported("linear: no top-cap instance with more than 8 waves"); }
    }
    launch_kernel<TP, W, CG, false>(a, p, stream);
}

template <int NCB>
void launch_wide(const LinearArgs& a, const LinearPlan& p, hipStream_t stream) {
    static const bool lds_raised = [] {
        NMI_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(&linear_q6_wide_kernel<NCB>),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
        return true;
    }();
    (void)lds_raised;
    hipLaunchKernelGGL((linear_q6_wide_kernel<NCB>), dim3(p.grid), dim3(64 * kWideWaves), wide_lds_bytes<NCB>(), stream, a);
    check_launch("linear_q6_wide_kernel");
}

void launch_linear_q6(LinearArgs a, const LinearPlan& p, hipStream_t stream) {
    a.ntiles = (a.N + kTileRows - 1) / kTileRows;
    a.waves = p.grid * p.waves;
    if (p.wide) {
        for (int32_t pass = 0; pass < p.passes; ++pass) {
            a.t0 = pass * p.tp;
            a.tp = std::min(p.tp, a.T - a.t0);
            if (p.tp == 64) {
                launch_wide<4>(a, p, stream);
            } else {
                launch_wide<2>(a, p, stream);
            }
        }
        return;
    }
    for (int32_t pass = 0; pass < p.passes; ++pass) {
        a.t0 = pass * p.tp;
        a.tp = std::min(p.tp, a.T - a.t0);
#define NMI_LINEAR_CASE(TP, W, CG)                                                                            \
    if (p.tp == TP && p.waves == W && p.cg == CG) {                                                           \
        launch_instance<TP, W, CG>(a, p, stream);                                                             \
        check_launch("linear_q6_kernel");                                                                     \
        continue;                                                                                             \
    }
        NMI_LINEAR_CASE(16, 8, 4)
        NMI_LINEAR_CASE(16, 4, 4)
        NMI_LINEAR_CASE(8, 8, 8)
        NMI_LINEAR_CASE(8, 8, 4)
        NMI_LINEAR_CASE(8, 4, 8)
        NMI_LINEAR_CASE(8, 4, 4)
        NMI_LINEAR_CASE(4, 16, 4)
        NMI_LINEAR_CASE(4, 8, 8)
        NMI_LINEAR_CASE(4, 8, 4)
        NMI_LINEAR_CASE(4, 4, 4)
#undef NMI_LINEAR_CASE
        throw Unsupported("linear: no built kernel instance for this plan");
    }
}

void launch_linear_argmax_reduce(const uint64_t* keys, int32_t T, int32_t waves, int32_t* out, hipStream_t stream) {
    hipLaunchKernelGGL(linear_argmax_reduce_kernel, dim3(T), dim3(256), 0, stream, keys, waves, out);
    check_launch("linear_argmax_reduce_kernel");
}

} // namespace nmi
