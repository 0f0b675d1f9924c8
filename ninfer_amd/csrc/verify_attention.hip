// Verify attention for the MTP speculative-decoding step on gfx950.
//
// Semantics (reference include/ninfer/ops/gqa_attention.h:52-91): for sequence b, query token t
// and query head qh (KV head h = qh / G), attend over cache rows [0, positions[0]) plus the new
// rows positions[u] (positions are sequential) with u visible from t (u <= t causal; u an
// ancestor-or-self of t for trees), reading INT8-G64 codes with FP16 scales. A1 first quantizes
// the new K/V columns into their rows (the split owning them writes them, as the reference's
// decode kernel does, src/ops/kernel/gqa_attention_decode_i8.cuh:168-209). Split-K over keys with
// an online softmax per split and a log-sum-exp merge (reference reducer
// src/ops/kernel/gqa_attention_decode.cuh:144-227).
//
// MI355X design:
//  * One workgroup = 4 waves = one (sequence, row chunk, KV head, key split); 2 workgroups per CU.
//    Each wave streams 32-key chunks (chunk w, w+4, ...). A chunk (K codes, V codes, FP16 scales)
//    moves HBM -> LDS by asynchronous buffer_load ... lds DMA into a per-wave two-stage ring with
//    a lookahead of two chunks; every code DMA instruction reads 1 KB of whole 128-byte rows.
//    The loop is software-pipelined: chunk j+1 is read from LDS and its QK^T issued while chunk
//    j's softmax and PV run.
//  * QK^T runs as S^T = K' * Q^T on v_mfma_f32_16x16x32_f16: K' = FP16(code * scale) (one packed
//    multiply per pair after an exact SDWA int8 -> FP16 convert) is the A operand, Q (BF16 -> FP16
//    exact after a per-row power-of-two rescale) the B operand. K rows sit in LDS with their
//    16-byte pieces XOR-swizzled by row, so the A-operand ds_read_b128 is conflict-free.
//  * PV runs as O^T = V'^T * P^T on the same instruction. The S^T accumulator layout (lane = query
//    row, 4 keys per 16-key tile) is exactly the B-operand layout of P^T, so probabilities never
//    leave registers. V rows land in LDS in their natural layout; each lane reads 8 bytes of 8 keys
//    (dims 8c..8c+7) and transposes in registers with SDWA converts. Row sums come from one more
//    MFMA with an all-ones A operand.
//  * The softmax keeps a lazy reference maximum: probabilities are FP16 exp2(s - m + 8) and m
//    moves (rescaling O) only when a score exceeds it by 2^7, so most chunks skip the rescale.
//  * GQA x q_len rows (5 x 4 = 20 for the 40/8 geometry) are padded to two 16-row MFMA tiles.
//    33..80 rows (a 16-node tree at group 5) take five tiles in one workgroup at one wave per
//    SIMD, so every key is streamed once (several 32-row chunks would each stream all keys): the
//    Q operands sit in LDS and the tiles run one after another on each chunk's converted K', V'.
#include "common.h"
#include "device_utils.h"
#include "ops_internal.h"

#include <algorithm>
#include <cmath>
#include <type_traits>
#include <utility>

#include "lds_dma.h"

namespace nmi {
namespace {

constexpr int kWaves = 4;
constexpr int kChunk = 32;
constexpr int kStride = kChunk * kWaves; // keys between one wave's consecutive chunks

// Geometry of one head dimension D (128 or 256): one 32-key stage of one KV head in LDS and the
// workgroup's LDS map.
template <int D>
struct Geo {
    static constexpr int GQ = D / 64;                  // INT8-G64 quant groups per row
    static constexpr int PIECES = D / 16;              // 16-byte pieces of a code row
    static constexpr int QPIECES = D / 8;              // 16-byte pieces of a BF16 Q row
    static constexpr int kStageK = 0;                  // K codes: 32 rows x D B, piece p of row r at slot p ^ (r % PIECES)
    static constexpr int kStageV = 32 * D;             // V codes: 32 rows x D B, natural order
    static constexpr int kStageKS = 64 * D;            // K scales: 256 B (D=128: 64 keys x 2 FP16, keys 32-63 unused;
                                                       //           D=256: 32 keys x 4 FP16)
    static constexpr int kStageVS = 64 * D + 256;      // V scales, same shape
    static constexpr int kStageBytes = 64 * D + 512;   // 8,704 B / 16,896 B
    static constexpr int kScaleKeyBytes = 2 * GQ;      // scale bytes of one key
    static constexpr int kDmaPerChunk = D / 16 + 2;    // code DMAs of 1 KB each + one per scale plane
    static constexpr int kRingBytes = kWaves * 2 * kStageBytes; // two stages per wave
    static constexpr int kNewStage = kRingBytes;       // A1: new rows quantized in-kernel (Q tile before)
    static constexpr int kPosLds = kNewStage + kStageBytes; // positions[0 .. T), T <= 32
    static constexpr int kWideK = kPosLds + 128;       // a wave met a K scale of 512 or more
    static constexpr int kSmemBytes = kPosLds + 144;   // D=128: 78,480 B (two workgroups per CU); D=256: 152,208 B
};
static_assert(Geo<128>::kStageBytes == 8704 && Geo<128>::kSmemBytes == 78480, "D=128 LDS map");
// Probabilities are FP16 exp2(score - m + 8); the reference maximum m moves only when a score
// exceeds it by more than 2^7, so P <= 2^15 stays inside FP16 and most chunks skip the rescale.
constexpr float kPOffset = 8.0f;
constexpr float kLazyTau = 7.0f;
constexpr int kQOutOfRange = 0x40000000; // a Q DMA offset past every Q buffer: the DMA writes zeros

// s_waitcnt immediates (gfx9 encoding: vmcnt[3:0] + vmcnt[15:14], expcnt[6:4], lgkmcnt[11:8]).
constexpr int waitcnt_vm(int n) { return (n & 0xf) | ((n >> 4) << 14) | (0x7 << 4) | (0xf << 8); }
constexpr int kWaitLgkm0 = 0xc07f;

// Wait until one chunk's DMA has landed; with `next_in_flight` the following chunk's stays
// outstanding (DMAs of one wave complete in issue order).
template <int D>
__device__ __forceinline__ void wait_chunk(bool next_in_flight) {
    if (next_in_flight) {
        __builtin_amdgcn_s_waitcnt(waitcnt_vm(Geo<D>::kDmaPerChunk));
    } else {
        __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    }
}

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));

// A partial O plane holds FP16 values: the merges load the 32-bit word holding element i and take
// its half later (i & 1), so a batch of loads stays in flight (converting each value inside its
// guarded load makes the compiler wait for that load before the next one).
__device__ __forceinline__ uint32_t partial_o_word(const uint16_t* base, int64_t i) {
    return reinterpret_cast<const uint32_t*>(base)[i >> 1];
}
__device__ __forceinline__ float partial_o_half(uint32_t w, int64_t i) {
    return f16_bits_to_f32(static_cast<uint16_t>(w >> (16 * static_cast<uint32_t>(i & 1))));
}
__device__ __forceinline__ float partial_o_at(const uint16_t* base, int64_t i) {
    return partial_o_half(partial_o_word(base, i), i);
}
typedef __bf16 bf8 __attribute__((ext_vector_type(8)));

struct AttnArgs {
    const uint16_t* q;
    const uint16_t* k_new; // fused A1 append (single row chunk only): BF16 [D, Hkv, T, B]
    const uint16_t* v_new;
    const int32_t* positions;
    const int32_t* parents;
    int8_t* kc;
    int8_t* vc;
    uint16_t* ks;
    uint16_t* vs;
    uint16_t* kb; // BF16 cache planes (BF16 kernel only)
    uint16_t* vb;
    uint16_t* part_o; // FP16 bits [row chunk][KV head][split_slots][rows][D], each row divided by its sum
    float* part_ml;   // [row chunk][KV head][split_slots][rows][2]
    int32_t* seq_table; // B > 1: per sequence (first slot, split count), written by the partial launch
    int64_t code_seq;
    int64_t scale_seq;
    int32_t P;
    int32_t T;
    int32_t Hq;
    int32_t Hkv;
    int32_t G;
    int32_t tokens_per_chunk;
    int32_t row_chunks;
    int32_t nsplit;      // B == 1: key splits (host plan)
    int32_t kps;         // B == 1: keys per split (host plan)
    int32_t B;
    int32_t split_slots; // partial slots per (row chunk, KV head)
    int32_t split_budget; // B > 1: most splits the batch's keys are cut into per (row chunk, KV head)
    int32_t max_keys; // envelope max_visible_keys (<= max_context <= P): clamps device positions
    float scale_log2; // softmax scale * log2(e)
};

// Keys per split of a batch-1 plan chosen on the device from the actual window, over the `launched`
// splits of each of `cols` (row chunk, KV head) units the grid holds: the reference's device-side
// active-split policy (src/ops/launcher/gqa_attention_decode.cu:16-20), with this build's host
// rules (at least 256 keys, a multiple of 128, no power-of-two stride of 1,024 keys or more, and
// one workgroup per CU where 1-1.75 would leave doubly loaded CUs). Used when the envelope is much
// wider than the windows it admits, as for a graph replayed over many rounds: a plan sized for
// the envelope's end would leave most splits empty and stream each window through a few.
__device__ __forceinline__ int b1_device_kps(int window, int launched, int cols) {
    constexpr int kCus = kAttnTargetWorkgroups / 2;
    const auto up128 = [](int x) { return (x + 127) / 128 * 128; };
    const auto off_pow2 = [](int k) { return (k >= 1024 && (k & (k - 1)) == 0) ? k + 128 : k; };
    const int w = max(window, 1);
    int kps = off_pow2(max(kAttnMinKeysPerSplit, up128((w + launched - 1) / launched)));
    const int n = (w + kps - 1) / kps;
    if (cols * n > kCus && cols * n * 4 < kCus * 7 && cols <= kCus) {
        const int per_col = kCus / cols;
        const int k1 = off_pow2(max(kAttnMinKeysPerSplit, up128((w + per_col - 1) / per_col)));
        const int n1 = (w + k1 - 1) / k1;
        if (n1 <= launched && (cols * n1 + kCus - 1) / kCus * k1 < (cols * n + kCus - 1) / kCus * kps) { kps = k1; }
    }
    return kps;
}

// ---- split plan of a batch -----------------------------------------------------------------------
// B == 1 keeps the host plan, so the first chunk DMAs need not wait for the positions. For B > 1 the
// sequences' windows W_i (keys visible to their last token, from the device positions) are cut into
// splits of kps keys (a multiple of 128, at least kAttnMinKeysPerSplit): sequence i owns
// n_i = max(1, ceil(W_i / kps)) consecutive partial slots of its (row chunk, KV head), and kps is the
// smallest value with sum n_i <= split_budget, so ragged contexts fill the resident workgroups
// evenly. With budget <= B every sequence gets one split.
struct SplitRange {
    int b;     // owning sequence (-1: none)
    int first; // its first slot
    int count; // its number of splits
    int kps;
};

__device__ __forceinline__ int seq_window(const int32_t* positions, int T, int max_keys, int i) {
    return max(0, min(positions[static_cast<int64_t>(i) * T + T - 1] + 1, max_keys));
}

// Wave-wide integer sum by DPP (row shifts 1, 2, 4, 8, then row broadcasts 15 and 31; lane 63
// holds the total, which every lane reads back). The whole wave must be active.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ int dpp_from_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, ROW_MASK, 0xf, false);
}

__device__ __forceinline__ int wave_sum_i(int v) {
    v += dpp_from_i<0x111, 0xf>(v);
    v += dpp_from_i<0x112, 0xf>(v);
    v += dpp_from_i<0x114, 0xf>(v);
    v += dpp_from_i<0x118, 0xf>(v);
    v += dpp_from_i<0x142, 0xa>(v);
    v += dpp_from_i<0x143, 0xc>(v);
    return __builtin_amdgcn_readlane(v, 63);
}

// max(1, ceil(w / kps)) in 32-bit arithmetic (w >= 0, kps >= 128).
__device__ __forceinline__ int splits_of(int w, unsigned kps) {
    return max(1, static_cast<int>((static_cast<unsigned>(w) + kps - 1u) / kps));
}

// The batch's windows as the split plan reads them: each lane holds the window of sequence `lane`
// in a register, so the search below repeats no memory load for batches of up to 64 sequences;
// later rounds of 64 reload theirs.
struct BatchWindows {
    const int32_t* positions;
    int T, B, max_keys;
    int w0; // window of sequence `lane` (0 past the batch)

    __device__ __forceinline__ int at(int base, int lane) const {
        if (base == 0) { return w0; }
        const int i = base + lane;
        return i < B ? seq_window(positions, T, max_keys, i) : 0;
    }
};

__device__ __forceinline__ BatchWindows batch_windows(const int32_t* positions, int T, int B, int max_keys) {
    const int lane = threadIdx.x & 63;
    return BatchWindows{positions, T, B, max_keys, lane < B ? seq_window(positions, T, max_keys, lane) : 0};
}

// sum over the batch of max(1, ceil(W_i / kps)) (whole wave).
__device__ int batch_split_count(const BatchWindows& bw, unsigned kps) {
    const int lane = threadIdx.x & 63;
    int n = 0;
    for (int base = 0; base < bw.B; base += 64) {
        const int w = bw.at(base, lane);
        if (base + lane < bw.B) { n += splits_of(w, kps); }
    }
    return wave_sum_i(n);
}

// Keys per split of the batch (whole wave; every lane returns the same).
__device__ unsigned batch_kps(const BatchWindows& bw, int budget) {
    const int lane = threadIdx.x & 63;
    const int B = bw.B;
    unsigned long long total = 0;
    int wmax = 0;
    for (int base = 0; base < B; base += 64) {
        const int w = bw.at(base, lane);
        total += static_cast<unsigned>(w);
        wmax = max(wmax, w);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        total += __shfl_xor(total, off, 64);
        wmax = max(wmax, __shfl_xor(wmax, off, 64));
    }
    const auto up128 = [](unsigned long long x) { return ((x + 127ull) / 128ull) * 128ull; };
    unsigned long long kps;
    if (budget <= B) {
        kps = up128(static_cast<unsigned long long>(max(wmax, 1)));
    } else {
        // count(k) >= total / k, so lo is a lower bound; count(hi) <= total / hi + B <= budget.
        unsigned long long lo = up128((total + budget - 1) / budget);
        unsigned long long hi = up128((total + (budget - B) - 1) / (budget - B));
        lo = lo < kAttnMinKeysPerSplit ? kAttnMinKeysPerSplit : lo;
        hi = hi < lo ? lo : hi;
        while (lo < hi) {
            const unsigned long long mid = lo + ((hi - lo) / 256ull) * 128ull;
            if (batch_split_count(bw, static_cast<unsigned>(mid)) <= budget) {
                hi = mid;
            } else {
                lo = mid + 128ull;
            }
        }
        kps = lo;
    }
    kps = kps < kAttnMinKeysPerSplit ? kAttnMinKeysPerSplit : kps;
    kps = (kps >= 1024 && (kps & (kps - 1)) == 0) ? kps + 128 : kps; // as the host plan: no power-of-two stride
    kps = kps > 0x7FFFFF80ull ? 0x7FFFFF80ull : kps;
    return static_cast<unsigned>(kps);
}

// The sequence owning partial slot `slot` (b = -1 past the last split), whole wave. With `table`,
// also stores every sequence's (first slot, split count) there, for the merge.
__device__ SplitRange batch_split_range(const int32_t* positions, int T, int B, int max_keys, int budget, int slot,
                                        int32_t* table) {
    const int lane = threadIdx.x & 63;
    const BatchWindows bw = batch_windows(positions, T, B, max_keys);
    const unsigned kps = batch_kps(bw, budget);
    SplitRange r{-1, 0, 0, static_cast<int>(kps)};
    int run = 0;
    for (int base = 0; base < B; base += 64) {
        const int i = base + lane;
        const int w = bw.at(base, lane);
        const int n = i < B ? splits_of(w, kps) : 0;
        const int incl = wave_inclusive_scan(n);
        const int excl = run + incl - n;
        if (table != nullptr && i < B) {
            table[2 * i] = excl;
            table[2 * i + 1] = n;
        }
        const unsigned long long m = __ballot(i < B && slot >= excl && slot < excl + n);
        if (m != 0ull && r.b < 0) {
            const int src = __ffsll(static_cast<long long>(m)) - 1;
            r.b = base + src;
            r.first = __shfl(excl, src, 64);
            r.count = __shfl(n, src, 64);
            if (table == nullptr) { return r; }
        }
        run += __builtin_amdgcn_readlane(incl, 63);
    }
    return r;
}

// Visibility of new node u (0 <= u < T) from query token t, as a bitmask over u.
// The ancestor walk follows parents[u] only while it lies in [0, u) (the tree contract; the greedy
// tree acceptance treats any other parent the same way), so every read stays inside the T-entry
// parents row and a malformed tree cannot make a later node visible.
__device__ __forceinline__ uint32_t new_key_mask(const int32_t* parents, int32_t t) {
    if (parents == nullptr) { return t >= 31 ? 0xffffffffu : ((2u << t) - 1u); }
    uint32_t m = 1u << t;
    int32_t u = t;
#pragma unroll 1
    for (int guard = 0; guard < 32; ++guard) {
        const int32_t p = parents[u];
        if (p < 0 || p >= u) { break; }
        m |= 1u << p;
        u = p;
    }
    return m;
}

// 8 INT8 codes (two dwords) -> 8 FP16 values, exactly.
__device__ __forceinline__ h8 cvt_codes8(int lo, int hi) {
    const uint32_t w[4] = {
        i8_bytes_to_f16x2<0, 1>(static_cast<uint32_t>(lo)),
        i8_bytes_to_f16x2<2, 3>(static_cast<uint32_t>(lo)),
        i8_bytes_to_f16x2<0, 1>(static_cast<uint32_t>(hi)),
        i8_bytes_to_f16x2<2, 3>(static_cast<uint32_t>(hi)),
    };
    return __builtin_bit_cast(h8, w);
}

__device__ __forceinline__ h8 scale_h8(h8 x, h2 s) {
    h2 p[4];
    __builtin_memcpy(p, &x, sizeof(p));
#pragma unroll
    for (int i = 0; i < 4; ++i) { p[i] *= s; }
    return __builtin_bit_cast(h8, p);
}

// Byte (T & 3) of word (T >> 2) from key slots 2w and 2w+1 -> packed FP16 pair (V transpose).
template <int T, typename V>
__device__ __forceinline__ uint32_t v_pair(const V& a, const V& b) {
    return i8x2_to_f16x2<T & 3>(static_cast<uint32_t>(a[T >> 2]), static_cast<uint32_t>(b[T >> 2]));
}

// Buffer resources of one (sequence, KV head): raw byte buffers, so DMA offsets are 32-bit.
struct HeadBuffers {
    __amdgpu_buffer_rsrc_t k, v, ks, vs;
};

// Per-lane DMA source offsets, fixed for the whole kernel. One 1 KB code DMA covers 1024 / D rows;
// lane -> (row lane / PIECES, slot lane % PIECES). K slot s of row r holds piece s ^ (r % PIECES),
// and r % PIECES depends on the DMA's index when a DMA covers fewer than PIECES rows (D = 256:
// 4 rows per DMA, 16 pieces), so K keeps one offset per DMA index modulo kvar(D).
struct DmaLanes {
    int k[4];
    int v;
    int sc; // scale word lane
};

template <int D>
constexpr int kvar() { return Geo<D>::PIECES / (1024 / D) > 1 ? Geo<D>::PIECES / (1024 / D) : 1; }

template <int D>
__device__ __forceinline__ DmaLanes make_dma_lanes(int lane) {
    constexpr int P = Geo<D>::PIECES;
    constexpr int ROWS = 1024 / D;
    const int row = lane / P;
    const int slot = lane % P;
    DmaLanes dl{};
#pragma unroll
    for (int q = 0; q < kvar<D>(); ++q) { dl.k[q] = row * D + 16 * (slot ^ ((ROWS * q + row) % P)); }
    dl.v = row * D + 16 * slot;
    dl.sc = lane * 4;
    return dl;
}

// Issue the DMA of one 32-key chunk (c0 + 32 <= P) into `st`: 4 K blocks, 4 V blocks and the K and
// V scale words of keys c0..c0+63 (the upper 32 are not used; the chunk offset of the scales sits in
// the range-checked voffset, so words past the head's last row read as zero). Block offsets of the
// codes go through soffset, which moves only the source address; the LDS address is M0 + 16 * lane
// (4 * lane for scales). Both scale loads run on the full wave: lane-divergent descriptors would
// turn one DMA into a waterfall loop.
// ONCE: every key of the launch is read by one workgroup (one row chunk), so the code DMAs take the
// non-temporal policy (the scale DMAs keep the default: measured faster).
template <int D, bool ONCE>
__device__ __forceinline__ void issue_chunk(NMI_AS3 char* st, const HeadBuffers& hb, const DmaLanes& dl,
                                            int c0, int lane) {
    using G = Geo<D>;
    constexpr int NDMA = D / 32; // 1 KB code DMAs per plane
    // c0 is wave-uniform; lane 0's copy puts the DMA soffset in an SGPR (a VGPR soffset would make
    // the compiler wrap every DMA in a readfirstlane loop).
    const int so = __builtin_amdgcn_readfirstlane(c0) * D;
    if constexpr (ONCE) {
#pragma unroll
        for (int r8 = 0; r8 < NDMA; ++r8) { dma16_nt(hb.k, st + G::kStageK + r8 * 1024, dl.k[r8 % kvar<D>()], so + r8 * 1024); }
#pragma unroll
        for (int r8 = 0; r8 < NDMA; ++r8) { dma16_nt(hb.v, st + G::kStageV + r8 * 1024, dl.v, so + r8 * 1024); }
    } else {
#pragma unroll
        for (int r8 = 0; r8 < NDMA; ++r8) { dma16(hb.k, st + G::kStageK + r8 * 1024, dl.k[r8 % kvar<D>()], so + r8 * 1024); }
#pragma unroll
        for (int r8 = 0; r8 < NDMA; ++r8) { dma16(hb.v, st + G::kStageV + r8 * 1024, dl.v, so + r8 * 1024); }
    }
    const int vso = dl.sc + c0 * G::kScaleKeyBytes;
    dma4(hb.ks, st + G::kStageKS, vso);
    dma4(hb.vs, st + G::kStageVS, vso);
}

// One chunk in registers: K codes in A-operand order, the K scale words of key 16kt + c, the V
// scale words of keys 4g..4g+3 and 16+4g..16+4g+3, and D/16 bytes (dims (D/16)c ..) of the lane's
// 8 V rows.
template <int D>
struct ChunkRegs {
    static constexpr int GQ = D / 64;
    using VRow = std::conditional_t<D == 128, i2, i4>; // the lane's bytes of one V row
    using KSc = std::conditional_t<D == 128, uint32_t, i2>; // one key's K scales
    i4 kr[2][GQ];
    KSc ksc[2];
    i4 vsw[2][D / 128];
    VRow vr[8];
};

template <int D>
__device__ __forceinline__ void read_chunk(const NMI_AS3 char* st, ChunkRegs<D>& r, int lane, int c, int g) {
    using G = Geo<D>;
    using CR = ChunkRegs<D>;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
        for (int gq = 0; gq < G::GQ; ++gq) {
            // A operand: key 16kt + c, dims 64gq + 16g .. +15 = piece 4gq + g of row 16kt + c.
            const int slot = (4 * gq + g) ^ ((16 * kt + c) % G::PIECES);
            r.kr[kt][gq] = *(const NMI_AS3 i4*)(st + G::kStageK + (16 * kt + c) * D + 16 * slot);
        }
        r.ksc[kt] = *(const NMI_AS3 typename CR::KSc*)(st + G::kStageKS + G::kScaleKeyBytes * (16 * kt + c));
    }
#pragma unroll
    for (int h = 0; h < D / 128; ++h) {
        // 4 keys' scales: 16 B (D = 128) or 32 B (D = 256).
        r.vsw[0][h] = *(const NMI_AS3 i4*)(st + G::kStageVS + 4 * G::kScaleKeyBytes * g + 16 * h);
        r.vsw[1][h] = *(const NMI_AS3 i4*)(st + G::kStageVS + G::kScaleKeyBytes * (16 + 4 * g) + 16 * h);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int row = j < 4 ? 4 * g + j : 16 + 4 * g + (j - 4);
        r.vr[j] = *(const NMI_AS3 typename CR::VRow*)(st + G::kStageV + row * D + (D / 16) * c);
    }
}

// ---- FP32-range decode ----------------------------------------------------------------------
//
// The MFMA operands are FP16(code * scale), exact for every scale below 512 (FP16 exponent field
// below 24: |code * scale| <= 127 * 515.8 < 65,504). The reference decodes cached K/V in FP32
// (include/ninfer/ops/gqa_attention.h:30) and INT8-G64 scales reach 65,504. A larger V scale makes
// V' overflow, and an overflowing V' always leaves O non-finite (p * inf, or 0 * inf = NaN), which
// the merge sees. A larger K scale may instead give a score of -inf, which would drop its key
// silently, so every lane ORs the exponent bits 14 and 13 of its K scale words into a flag (two VALU
// per chunk, from registers the chunk has in any case), and a workgroup whose waves saw such a
// scale marks its partial rows (row sum -1). The merge recomputes a marked or non-finite split's
// partial exactly in FP32 (verify_attn_exact_split below).
template <int D>
__device__ __forceinline__ uint32_t wide_k_bits(const ChunkRegs<D>& r) {
    if constexpr (D == 128) {
        const uint32_t a = r.ksc[0];
        const uint32_t b = r.ksc[1];
        return (a & (a << 1)) | (b & (b << 1));
    } else {
        uint32_t f = 0u;
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
            for (int w = 0; w < 2; ++w) {
                const uint32_t x = static_cast<uint32_t>(r.ksc[kt][w]);
                f |= x & (x << 1);
            }
        }
        return f;
    }
}

// Which keys of a chunk a row may see: keys below vis_all are visible to every row; key
// new_base + u (u < 32, key < key_end) is visible to the row's token if bit u of its mask is set.
// V scales of keys at or past key_end count as zero (those rows may hold stale bytes).
struct KeyRange {
    int vis_all;
    int new_base;
    int key_end;
};

// Online-softmax state of one wave: NT tiles of 16 rows.
template <int NT, int D>
struct RowState {
    h8 q[NT][D / 64][2]; // B operand of Q^T: rows 16nt + c, dims 64gq + 16g + 8s + e
    float rowmul[NT];    // softmax scale * log2(e) / Q power-of-two factor
    float rowthr[NT];    // kLazyTau / rowmul: the lazy-rescale threshold in raw score units
    uint32_t nmask[NT];
    float m[NT];         // reference maximum in raw score units
    f4 O[NT][D / 16];    // O^T tiles: tile t row 4g+e is dim (D/16)(4g+e) + t
    f4 l[NT];            // row sums, equal in all four entries (ones x P^T)
};

// FP16 scale `gq` of one key's scale word(s), broadcast to both halves of a pair.
__device__ __forceinline__ uint32_t scale_pair(uint32_t w, int gq) {
    return __builtin_amdgcn_perm(w, w, gq ? 0x03020302u : 0x01000100u);
}
__device__ __forceinline__ uint32_t scale_pair(const i2& w, int gq) {
    const uint32_t x = static_cast<uint32_t>(w[gq >> 1]);
    return __builtin_amdgcn_perm(x, x, (gq & 1) ? 0x03020302u : 0x01000100u);
}

// S^T = K' Q^T with K' = FP16(code * scale) as the A operand (key 16kt + c).
template <int NT, int D>
__device__ __forceinline__ void qk_chunk(const ChunkRegs<D>& r, const RowState<NT, D>& s, f4 (&sacc)[2][NT]) {
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
        for (int gq = 0; gq < D / 64; ++gq) {
            const uint32_t sp = scale_pair(r.ksc[kt], gq);
            const h2 s2 = __builtin_bit_cast(h2, sp);
            const h8 a0 = scale_h8(cvt_codes8(r.kr[kt][gq][0], r.kr[kt][gq][1]), s2);
            const h8 a1 = scale_h8(cvt_codes8(r.kr[kt][gq][2], r.kr[kt][gq][3]), s2);
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                const f4 acc = gq == 0 ? f4{0.f, 0.f, 0.f, 0.f} : sacc[kt][nt];
                sacc[kt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, s.q[nt][gq][0], acc, 0, 0, 0);
                sacc[kt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, s.q[nt][gq][1], sacc[kt][nt], 0, 0, 0);
            }
        }
    }
}

// Maximum of a lane's 8 scores over the 4 lanes that share its row (lanes c, c+16, c+32, c+48).
// IEEE maximum (NaN-propagating) runs as v_maximum3_f32 on gfx950, without the canonicalizing
// moves fmaxf needs for operands read back from MFMA accumulators; a NaN score makes the row's
// output NaN under either maximum.
__device__ __forceinline__ float fmax_ieee(float a, float b) { return __builtin_elementwise_maximum(a, b); }

__device__ __forceinline__ float score_max(const float (&sv)[8]) {
    float v = fmax_ieee(fmax_ieee(fmax_ieee(sv[0], sv[1]), fmax_ieee(sv[2], sv[3])),
                        fmax_ieee(fmax_ieee(sv[4], sv[5]), fmax_ieee(sv[6], sv[7])));
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmax_ieee(__uint_as_float(r[0]), __uint_as_float(r[1]));
    r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmax_ieee(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Online softmax of one chunk; the S^T accumulator layout is the B-operand layout of P^T. `masked`
// is uniform across the wave. State is anything with m, rowmul, rowthr, nmask, O[NT][D/16] and
// l; the probabilities come out as FP32 exp2(score * rowmul - m * rowmul + kPOffset).
template <int NT, int D, typename State>
__device__ __forceinline__ void softmax_probs(const f4 (&sacc)[2][NT], int c0, bool masked, State& s,
                                              const KeyRange& kr, int g, float (&p)[NT][8]) {
    // Phases over all tiles (scores, maxima, one rescale branch, probabilities), so the tiles'
    // dependent steps interleave.
    float sv[NT][8];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
            for (int e = 0; e < 4; ++e) { sv[nt][4 * kt + e] = sacc[kt][nt][e]; }
        }
    }
    if (masked) {
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                // Branch-free: bitwise operators, and a shift count that is always in range.
                const int key = c0 + 16 * (i >> 2) + 4 * g + (i & 3);
                const int u = key - kr.new_base;
                const bool bit = ((s.nmask[nt] >> (u & 31)) & 1u) != 0u;
                const bool vis = (key < kr.vis_all) | ((key < kr.key_end) & (static_cast<unsigned>(u) < 32u) & bit);
                sv[nt][i] = vis ? sv[nt][i] : -INFINITY;
            }
        }
    }
    float cmax[NT];
    bool need_any = false;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        cmax[nt] = score_max(sv[nt]);
        need_any |= cmax[nt] > s.m[nt] + s.rowthr[nt];
    }
    if (__any(need_any)) {
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const bool need = cmax[nt] > s.m[nt] + s.rowthr[nt];
            const float mn = need ? cmax[nt] : s.m[nt];
            const float alpha = need ? __builtin_amdgcn_exp2f((s.m[nt] - mn) * s.rowmul[nt]) : 1.0f;
#pragma unroll
            for (int t = 0; t < D / 16; ++t) { s.O[nt][t] *= alpha; }
            s.l[nt] *= alpha;
            s.m[nt] = mn;
        }
    }
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        const float bias = s.m[nt] == -INFINITY ? 0.0f : fmaf(-s.m[nt], s.rowmul[nt], kPOffset);
#pragma unroll
        for (int i = 0; i < 8; ++i) { p[nt][i] = __builtin_amdgcn_exp2f(fmaf(sv[nt][i], s.rowmul[nt], bias)); }
    }
}

template <int NT, int D>
__device__ __forceinline__ void softmax_chunk(const f4 (&sacc)[2][NT], int c0, bool masked, RowState<NT, D>& s,
                                              const KeyRange& kr, int g, h8 (&pop)[NT]) {
    float p[NT][8];
    softmax_probs<NT, D>(sacc, c0, masked, s, kr, g, p);
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
#pragma unroll
        for (int i = 0; i < 8; ++i) { pop[nt][i] = static_cast<_Float16>(p[nt][i]); }
    }
}

// The FP16 V scales of the lane's group for its 8 keys (4g + j and 16 + 4g + j), as 4 key pairs.
// D = 128: the lane's dims 8c..8c+7 lie in group c >> 3, and a key's scales are one word.
// D = 256: dims 16c..16c+15 lie in group c >> 2, and a key's scales are two words.
template <int D>
__device__ __forceinline__ void v_scale_pairs(const i4 (&vsw)[2][D / 128], int c, h2 (&vsp)[4]) {
    if constexpr (D == 128) {
        const uint32_t vsel = (c >> 3) ? 0x07060302u : 0x05040100u; // FP16 half of this lane's group
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            vsp[2 * half] = __builtin_bit_cast(h2, __builtin_amdgcn_perm(static_cast<uint32_t>(vsw[half][0][1]), static_cast<uint32_t>(vsw[half][0][0]), vsel));
            vsp[2 * half + 1] = __builtin_bit_cast(h2, __builtin_amdgcn_perm(static_cast<uint32_t>(vsw[half][0][3]), static_cast<uint32_t>(vsw[half][0][2]), vsel));
        }
    } else {
        const int grp = c >> 2;                               // FP16 index of the group in a key's 4
        const uint32_t vsel = (grp & 1) ? 0x07060302u : 0x05040100u;
        const int w = grp >> 1;                               // word of the key holding it
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            // keys j and j + 1 of this half: words [2j + w] of the 32 bytes (two i4)
#pragma unroll
            for (int p2 = 0; p2 < 2; ++p2) {
                const uint32_t a = static_cast<uint32_t>(vsw[half][p2][w]);      // key 2 p2
                const uint32_t b = static_cast<uint32_t>(vsw[half][p2][2 + w]);  // key 2 p2 + 1
                vsp[2 * half + p2] = __builtin_bit_cast(h2, __builtin_amdgcn_perm(b, a, vsel));
            }
        }
    }
}

// O^T += V'^T P^T with V' = FP16(code * scale); l += ones x P^T. Keys at or past key_end of a
// masked chunk get a zero V scale.
template <int NT, int D>
__device__ __forceinline__ void pv_chunk(const h8 (&pop)[NT], const typename ChunkRegs<D>::VRow (&vr)[8],
                                         const i4 (&vsw)[2][D / 128], int c0, bool masked, RowState<NT, D>& s,
                                         const KeyRange& kr, int c, int g) {
    h2 vsp[4];
    v_scale_pairs<D>(vsw, c, vsp);
    if (masked) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int key = c0 + (j < 4 ? 4 * g + j : 16 + 4 * g + (j - 4));
            if (key >= kr.key_end) { vsp[j >> 1][j & 1] = static_cast<_Float16>(0.0f); }
        }
    }
#define NMI_PV_TILE(TT)                                                                            \
    {                                                                                              \
        h2 pr[4];                                                                                  \
        _Pragma("unroll") for (int w = 0; w < 4; ++w) {                                            \
            pr[w] = __builtin_bit_cast(h2, v_pair<TT>(vr[2 * w], vr[2 * w + 1])) * vsp[w];         \
        }                                                                                          \
        const h8 va = __builtin_bit_cast(h8, pr);                                                  \
        _Pragma("unroll") for (int nt = 0; nt < NT; ++nt) {                                        \
            s.O[nt][TT] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pop[nt], s.O[nt][TT], 0, 0, 0); \
        }                                                                                          \
    }
    NMI_PV_TILE(0)
    NMI_PV_TILE(1)
    NMI_PV_TILE(2)
    NMI_PV_TILE(3)
    NMI_PV_TILE(4)
    NMI_PV_TILE(5)
    NMI_PV_TILE(6)
    NMI_PV_TILE(7)
    if constexpr (D == 256) {
        NMI_PV_TILE(8)
        NMI_PV_TILE(9)
        NMI_PV_TILE(10)
        NMI_PV_TILE(11)
        NMI_PV_TILE(12)
        NMI_PV_TILE(13)
        NMI_PV_TILE(14)
        NMI_PV_TILE(15)
    }
#undef NMI_PV_TILE
    const h8 ones = {1, 1, 1, 1, 1, 1, 1, 1};
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) { s.l[nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones, pop[nt], s.l[nt], 0, 0, 0); }
}

template <int NT, int D>
__device__ __forceinline__ void compute_chunk(const ChunkRegs<D>& r, int c0, bool masked, RowState<NT, D>& s,
                                              const KeyRange& kr, int c, int g) {
    f4 sacc[2][NT];
    qk_chunk<NT, D>(r, s, sacc);
    h8 pop[NT];
    softmax_chunk<NT, D>(sacc, c0, masked, s, kr, g, pop);
    pv_chunk<NT, D>(pop, r.vr, r.vsw, c0, masked, s, kr, c, g);
}

// acc *= alpha on an MFMA accumulator kept in AGPRs: each element is read, multiplied and written
// back in place. Written with the multiply in VGPRs instead, the compiler homes the five-tile
// accumulators in VGPRs and copies all of them out of AGPRs at every loop iteration (~180 moves
// per chunk), although the lazy rescale itself rarely runs.
__device__ __forceinline__ void scale_acc(f4& acc, float alpha) {
    float x[4] = {acc[0], acc[1], acc[2], acc[3]};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        float t;
        asm("v_accvgpr_read_b32 %1, %0\n\tv_mul_f32 %1, %1, %2\n\tv_accvgpr_write_b32 %0, %1"
            : "+a"(x[e]), "=&v"(t)
            : "v"(alpha));
    }
    acc = f4{x[0], x[1], x[2], x[3]};
}

template <int TT, int D>
__device__ __forceinline__ void v_operand(const typename ChunkRegs<D>::VRow (&vr)[8], const h2 (&vsp)[4], h8 (&va)[D / 16]) {
    h2 pr[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) { pr[w] = __builtin_bit_cast(h2, v_pair<TT>(vr[2 * w], vr[2 * w + 1])) * vsp[w]; }
    va[TT] = __builtin_bit_cast(h8, pr);
}

template <int D, int... TT>
__device__ __forceinline__ void v_operands(const typename ChunkRegs<D>::VRow (&vr)[8], const h2 (&vsp)[4], h8 (&va)[D / 16],
                                           std::integer_sequence<int, TT...>) {
    (v_operand<TT, D>(vr, vsp, va), ...);
}

// The five-tile form (80 rows): the chunk's K' and V'^T operands are converted once, and each phase
// (QK^T, the score maxima, the lazy rescale, the probabilities and PV) runs over all tiles before
// the next, so the one wave on its SIMD has independent work between dependent steps and a single
// rescale branch. Per row the arithmetic is the one compute_chunk does.
template <int NT, int D, bool MASKED>
__device__ __forceinline__ void compute_chunk_tiles(const ChunkRegs<D>& r, int c0, RowState<NT, D>& s,
                                                    const KeyRange& kr, int c, int g, const NMI_AS3 char* qop) {
    const int lane = threadIdx.x & 63;
    h8 ka[2][D / 64][2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
        for (int gq = 0; gq < D / 64; ++gq) {
            const h2 s2 = __builtin_bit_cast(h2, scale_pair(r.ksc[kt], gq));
            ka[kt][gq][0] = scale_h8(cvt_codes8(r.kr[kt][gq][0], r.kr[kt][gq][1]), s2);
            ka[kt][gq][1] = scale_h8(cvt_codes8(r.kr[kt][gq][2], r.kr[kt][gq][3]), s2);
        }
    }
    float sv[NT][8];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        f4 sacc[2];
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
            for (int gq = 0; gq < D / 64; ++gq) {
                const f4 acc = gq == 0 ? f4{0.f, 0.f, 0.f, 0.f} : sacc[kt];
                const h8 q0 = *(const NMI_AS3 h8*)(qop + ((nt * (D / 64) + gq) * 2) * 1024 + 16 * lane);
                const h8 q1 = *(const NMI_AS3 h8*)(qop + ((nt * (D / 64) + gq) * 2 + 1) * 1024 + 16 * lane);
                sacc[kt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka[kt][gq][0], q0, acc, 0, 0, 0);
                sacc[kt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka[kt][gq][1], q1, sacc[kt], 0, 0, 0);
            }
        }
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
            for (int e = 0; e < 4; ++e) { sv[nt][4 * kt + e] = sacc[kt][e]; }
        }
    }
    h2 vsp[4];
    v_scale_pairs<D>(r.vsw, c, vsp);
    if constexpr (MASKED) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int key = c0 + (j < 4 ? 4 * g + j : 16 + 4 * g + (j - 4));
            if (key >= kr.key_end) { vsp[j >> 1][j & 1] = static_cast<_Float16>(0.0f); }
        }
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int key = c0 + 16 * (i >> 2) + 4 * g + (i & 3);
                const int u = key - kr.new_base;
                const bool bit = ((s.nmask[nt] >> (u & 31)) & 1u) != 0u;
                const bool vis = (key < kr.vis_all) | ((key < kr.key_end) & (static_cast<unsigned>(u) < 32u) & bit);
                sv[nt][i] = vis ? sv[nt][i] : -INFINITY;
            }
        }
    }
    h8 va[D / 16];
    v_operands<D>(r.vr, vsp, va, std::make_integer_sequence<int, D / 16>{});
    float cmax[NT];
    bool need_any = false;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        cmax[nt] = score_max(sv[nt]);
        need_any |= cmax[nt] > s.m[nt] + s.rowthr[nt];
    }
    if (__any(need_any)) {
        // scale_acc reads accumulators that MFMAs wrote: 16 wait states of margin for the MFMA
        // write -> VALU read hazard, whatever the compiler placed before this rare block.
        asm volatile("s_nop 7\n\ts_nop 7");
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const bool need = cmax[nt] > s.m[nt] + s.rowthr[nt];
            const float mn = need ? cmax[nt] : s.m[nt];
            const float alpha = need ? __builtin_amdgcn_exp2f((s.m[nt] - mn) * s.rowmul[nt]) : 1.0f;
#pragma unroll
            for (int t = 0; t < D / 16; ++t) { scale_acc(s.O[nt][t], alpha); }
            scale_acc(s.l[nt], alpha);
            s.m[nt] = mn;
        }
    }
    const h8 ones = {1, 1, 1, 1, 1, 1, 1, 1};
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        const float bias = s.m[nt] == -INFINITY ? 0.0f : fmaf(-s.m[nt], s.rowmul[nt], kPOffset);
        h8 pop;
#pragma unroll
        for (int i = 0; i < 8; ++i) { pop[i] = static_cast<_Float16>(__builtin_amdgcn_exp2f(fmaf(sv[nt][i], s.rowmul[nt], bias))); }
#pragma unroll
        for (int t = 0; t < D / 16; ++t) { s.O[nt][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va[t], pop, s.O[nt][t], 0, 0, 0); }
        s.l[nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones, pop, s.l[nt], 0, 0, 0);
    }
}

// Quantize one new token row of one KV head (one wave: lane owns dim lane + 64 i of group i of K and
// V; reference contract include/ninfer/ops/gqa_attention.h:25-30) into the cache and into key slot
// u of the LDS stage `st`, in the layout the chunk DMA produces.
template <int D>
__device__ __forceinline__ void append_row(const uint16_t* ksrc, const uint16_t* vsrc, int8_t* kdst,
                                           int8_t* vdst, uint16_t* ksdst, uint16_t* vsdst,
                                           NMI_AS3 char* st, int u, int lane) {
    using G = Geo<D>;
    constexpr int GQ = G::GQ;
    float x[2 * GQ];
#pragma unroll
    for (int i = 0; i < GQ; ++i) {
        x[i] = bf16_to_f32(ksrc[64 * i + lane]);
        x[GQ + i] = bf16_to_f32(vsrc[64 * i + lane]);
    }
    uint16_t sbits[2 * GQ];
    int8_t code[2 * GQ];
#pragma unroll
    for (int i = 0; i < 2 * GQ; ++i) {
        const float amax = wave_max(fabsf(x[i]));
        sbits[i] = f32_to_f16_bits(amax > 0.0f ? amax / 127.0f : 0.0f);
        const float sc = f16_bits_to_f32(sbits[i]);
        const float inv = sc > 0.0f ? 1.0f / sc : 0.0f;
        float rr = inv != 0.0f ? rintf(x[i] * inv) : 0.0f;
        rr = fminf(127.0f, fmaxf(-127.0f, rr));
        code[i] = static_cast<int8_t>(rr);
    }
#pragma unroll
    for (int i = 0; i < GQ; ++i) {
        kdst[64 * i + lane] = code[i];
        vdst[64 * i + lane] = code[GQ + i];
    }
    if (lane == 0) {
#pragma unroll
        for (int i = 0; i < GQ; i += 2) {
            const uint32_t kw = static_cast<uint32_t>(sbits[i]) | (static_cast<uint32_t>(sbits[i + 1]) << 16);
            const uint32_t vw = static_cast<uint32_t>(sbits[GQ + i]) | (static_cast<uint32_t>(sbits[GQ + i + 1]) << 16);
            *reinterpret_cast<uint32_t*>(ksdst + i) = kw;
            *reinterpret_cast<uint32_t*>(vsdst + i) = vw;
            *(NMI_AS3 uint32_t*)(st + G::kStageKS + G::kScaleKeyBytes * u + 2 * i) = kw;
            *(NMI_AS3 uint32_t*)(st + G::kStageVS + G::kScaleKeyBytes * u + 2 * i) = vw;
        }
    }
    // Swizzled K row u: dim d sits in piece d >> 4 at slot (d >> 4) ^ (u % PIECES).
    const int krow = G::kStageK + u * D + (lane & 15);
#pragma unroll
    for (int i = 0; i < GQ; ++i) {
        st[krow + 16 * ((4 * i + (lane >> 4)) ^ (u % G::PIECES))] = static_cast<char>(code[i]);
        st[G::kStageV + u * D + 64 * i + lane] = static_cast<char>(code[GQ + i]);
    }
}

// Merge the four waves' (m, l, O) through LDS (reusing the staging area) and write the
// workgroup's partial: out_o [rows][D] (rows < R), O / l in FP16 (a weighted mean of V' values, so
// finite wherever V' is), and out_ml [rows][2] (log2-domain max, row sum l) in FP32.
// Rows go through LDS 32 at a time (two 16-row tiles per batch). The combine is branch-free (a wave
// that saw no visible key has m = -inf, weight 0 and zero accumulators) and every LDS read of a row
// is issued before its first use. CACHED: ordinary stores instead of non-temporal ones.
template <int NT, int D, bool CACHED, typename State>
__device__ __forceinline__ void write_partial(const State& s, char* smem, int R, int wave, int c, int g,
                                              uint16_t* out_o, float* out_ml, bool kmark = false) {
    constexpr int kRowStride = D + 4;                       // floats; rows stay 16-byte aligned
    float* sm_o = reinterpret_cast<float*>(smem);           // [kWaves][32][kRowStride]
    float* sm_m = sm_o + kWaves * 32 * kRowStride;          // [32][kWaves]: one 16-byte read per row
    float* sm_l = sm_m + kWaves * 32;                       // [32][kWaves]
    constexpr int NB = (NT + 1) / 2;
    constexpr int UPR = D / 4;                              // f4 units of one row
    constexpr int RPP = 256 / UPR;                          // rows per pass of the 256 threads
    // The thread index is laundered here, so the unit mapping below is computed at this point
    // instead of being kept live across the whole kernel (at two workgroups per CU the compiler
    // otherwise spills a lane offset and reloads it from scratch here).
    int tid = static_cast<int>(threadIdx.x);
    asm volatile("" : "+v"(tid));
    const int d4 = 4 * (tid & (UPR - 1));
    const int r0 = tid / UPR;
#pragma unroll
    for (int jb = 0; jb < NB; ++jb) {
        if (jb > 0) { __syncthreads(); } // the previous batch's rows have been read
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int nt = 2 * jb + u;
            if (nt >= NT) { continue; }
            const int r = 16 * u + c; // row within the batch
            if (g == 0) {
                // log2-domain maximum of this wave's partial; O and l both carry the 2^kPOffset factor.
                sm_m[r * kWaves + wave] = s.m[nt] == -INFINITY ? -INFINITY : s.m[nt] * s.rowmul[nt];
                sm_l[r * kWaves + wave] = s.l[nt][0];
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                // O^T tile t row (4g + e) is dim (D/16)(4g + e) + t: D/16 consecutive dims per (lane, e).
                float* dst = sm_o + (wave * 32 + r) * kRowStride + (D / 16) * (4 * g + e);
#pragma unroll
                for (int q4 = 0; q4 < D / 64; ++q4) {
                    *reinterpret_cast<f4*>(dst + 4 * q4) =
                        f4{s.O[nt][4 * q4][e], s.O[nt][4 * q4 + 1][e], s.O[nt][4 * q4 + 2][e], s.O[nt][4 * q4 + 3][e]};
                }
            }
        }
        __syncthreads();
        const int rb = 32 * jb;
        const int rows = min(32, R - rb);
        constexpr int KR = 32 / RPP; // rows per thread and batch
        // Every LDS read of the batch first (rows past the last valid one re-read it), then the
        // combine, then the guarded stores.
        f4 mv[KR], lv[KR], ow[KR][kWaves];
#pragma unroll
        for (int k = 0; k < KR; ++k) {
            const int r = min(r0 + RPP * k, rows - 1);
            mv[k] = *reinterpret_cast<const f4*>(sm_m + r * kWaves);
            lv[k] = *reinterpret_cast<const f4*>(sm_l + r * kWaves);
#pragma unroll
            for (int w = 0; w < kWaves; ++w) { ow[k][w] = *reinterpret_cast<const f4*>(sm_o + (w * 32 + r) * kRowStride + d4); }
        }
#pragma unroll
        for (int k = 0; k < KR; ++k) {
            const int r = r0 + RPP * k;
            const float M = fmaxf(fmaxf(mv[k][0], mv[k][1]), fmaxf(mv[k][2], mv[k][3]));
            f4 o = {0.f, 0.f, 0.f, 0.f};
            float lsum = 0.0f;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) {
                const float wgt = mv[k][w] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mv[k][w] - M);
                o += wgt * ow[k][w];
                lsum = fmaf(lv[k][w], wgt, lsum);
            }
            if (r >= rows) { continue; }
            const int row = rb + r;
            const float inv = lsum > 0.0f ? __builtin_amdgcn_rcpf(lsum) : 0.0f;
            const u2 oh = {static_cast<uint32_t>(f32_to_f16_bits(o[0] * inv)) | (static_cast<uint32_t>(f32_to_f16_bits(o[1] * inv)) << 16),
                           static_cast<uint32_t>(f32_to_f16_bits(o[2] * inv)) | (static_cast<uint32_t>(f32_to_f16_bits(o[3] * inv)) << 16)};
            if (kmark) { lsum = -1.0f; } // a K scale of 512 or more: the merge recomputes this split
            // Read once, by the merge: non-temporal unless the plan routes long splits' partials
            // through the caches.
            if constexpr (CACHED) {
                *reinterpret_cast<u2*>(out_o + row * D + d4) = oh;
                if (d4 == 0) {
                    out_ml[2 * row] = M;
                    out_ml[2 * row + 1] = lsum;
                }
            } else {
                __builtin_nontemporal_store(oh, reinterpret_cast<u2*>(out_o + row * D + d4));
                if (d4 == 0) {
                    __builtin_nontemporal_store(M, out_ml + 2 * row);
                    __builtin_nontemporal_store(lsum, out_ml + 2 * row + 1);
                }
            }
        }
    }
}

// D = 128: 78 KB of LDS and at most 256 registers, two workgroups per CU. D = 256: 152 KB of LDS,
// one workgroup (one wave per SIMD) per CU, which leaves 512 registers per lane for the doubled
// accumulators and chunk registers. NT = 5 (D = 128): 80 query rows (a 16-node tree at group 5)
// in one workgroup, so every key is streamed once; one wave per SIMD, the Q tile in LDS of its own.
// One partial of the INT8 kernel: the keys [k0, kend) of sequence b (k0 a multiple of 128) for KV
// head h and this workgroup's row chunk, into partial slot `slot`.
template <int NT, int D, bool ONCE, bool CACHED, bool DEV = false>
__device__ __forceinline__ void partial_segment(const AttnArgs& a, char* smem, int b, int k0, int kend, int slot, int h) {
    constexpr int G = D / 64; // quant groups per row
    using GE = Geo<D>;
    constexpr int RMAX = NT == 5 ? kAttnWideRows : kAttnRowsPerTile; // rows per partial slot
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int c = lane & 15;
    const int g = lane >> 4;
    const int rc = blockIdx.z;

    const int64_t head_code = static_cast<int64_t>(b) * a.code_seq + static_cast<int64_t>(h) * a.P * D;
    const int64_t head_scale = static_cast<int64_t>(b) * a.scale_seq + static_cast<int64_t>(h) * a.P * G;
    int8_t* kbase = a.kc + head_code;
    int8_t* vbase = a.vc + head_code;
    uint16_t* ksbase = a.ks + head_scale;
    uint16_t* vsbase = a.vs + head_scale;
    const HeadBuffers hb{raw_buffer(kbase, static_cast<int64_t>(a.P) * D), raw_buffer(vbase, static_cast<int64_t>(a.P) * D),
                         raw_buffer(ksbase, static_cast<int64_t>(a.P) * 2 * G), raw_buffer(vsbase, static_cast<int64_t>(a.P) * 2 * G)};
    const DmaLanes dl = make_dma_lanes<D>(lane);
    NMI_AS3 char* ring = (NMI_AS3 char*)smem + wave * 2 * GE::kStageBytes;

    // Q tile (rows r = tl * G + gi of this workgroup, 256 B each) moves HBM -> LDS by DMA before
    // any chunk DMA is queued, into the new-row stage area (free until an owner builds that stage).
    // Wave 0 waits for it with an exact vmcnt that leaves the chunk DMAs in flight.
    const int t0 = rc * a.tokens_per_chunk;
    const int Tc = min(a.tokens_per_chunk, a.T - t0);
    const int R = Tc * a.G;
    NMI_AS3 char* qtile = (NMI_AS3 char*)smem + (NT == 5 ? GE::kSmemBytes : GE::kNewStage);
    NMI_AS3 int32_t* pos_lds = (NMI_AS3 int32_t*)((NMI_AS3 char*)smem + GE::kPosLds);
    const int32_t* pos = a.positions + static_cast<int64_t>(b) * a.T;
    if (threadIdx.x == 0) { *(NMI_AS3 int32_t*)((NMI_AS3 char*)smem + GE::kWideK) = 0; }
    if (wave == 0) {
        // Positions travel the same way (a vector load here would wait behind every chunk DMA).
        if (lane < a.T) { __builtin_amdgcn_global_load_lds((const NMI_AS1 void*)(pos + lane), (NMI_AS3 void*)pos_lds, 4, 0, 0); }
        constexpr int QP = GE::QPIECES;  // 16-byte pieces of a Q row
        constexpr int RPD = 64 / QP;     // Q rows per 1 KB DMA
        // All 16 * NT rows the tiles read: rows past R take an offset past the buffer and land as
        // zeros, so the tiles need no masking of their Q operands.
        const __amdgpu_buffer_rsrc_t qr =
            raw_buffer(a.q + static_cast<int64_t>(D) * (h * a.G + static_cast<int64_t>(a.Hq) * a.T * b),
                       static_cast<int64_t>(a.T) * a.Hq * D * 2);
#pragma unroll
        for (int k = 0; RPD * k < 16 * NT; ++k) {
            const int row = RPD * k + lane / QP;
            const int tl = row / a.G;
            const int gi = row - tl * a.G;
            // Slot (lane % QP) of the row holds piece (slot - row) % QP: rows rotate across the LDS
            // banks, so the 16 lanes that read one column of rows do not conflict.
            const int piece = ((lane % QP) - row) & (QP - 1);
            const int off = row < R ? 2 * (D * (gi + a.Hq * (t0 + tl)) + 8 * piece) : kQOutOfRange;
            dma16(qr, qtile + k * 1024, off, 0);
        }
    }

    // The first two chunks do not depend on the positions. A chunk that turns out to lie past the
    // split's range is simply never read (it stays inside the padded cache, and the waits below
    // fall back to vmcnt(0) when the next chunk is unused). The first chunk's DMA starts right away;
    // the second waits until Q has landed, so Q is not queued behind every wave's two chunks at
    // launch (measured on MI355X: C2 14.60 -> 13.92 us per layer, C3, C4 and C5 unchanged).
    // Chunks at or past the envelope hold no key any position can see, so they are not fetched (the
    // last split of a plan usually ends past the envelope: at C2, keys 7,684-7,935). A batch-1 plan
    // split on the device (the DEV instance) learns its range from the positions, so it fetches
    // nothing before them.
    constexpr bool dev = DEV;
    int first = k0 + kChunk * wave;
    const bool issued0 = !dev && first + kChunk <= a.P && first < a.max_keys;
    if (issued0) { issue_chunk<D, ONCE>(ring, hb, dl, first, lane); }
    if (wave == 0) {
        if (issued0) {
            __builtin_amdgcn_s_waitcnt(waitcnt_vm(GE::kDmaPerChunk));
        } else {
            __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
        }
    }
    // A bare barrier: the DMA'd Q and positions are in LDS once wave 0's wait returns, and a full
    // __syncthreads() would also wait for the chunk DMAs.
    __builtin_amdgcn_s_barrier();
    if constexpr (dev) {
        // this split's keys of the device window: `slot` of the a.nsplit launched splits
        const int win = min(max(__builtin_amdgcn_readfirstlane(pos_lds[a.T - 1]) + 1, 0), a.max_keys);
        const int kpsd = b1_device_kps(win, a.nsplit, a.Hkv * a.row_chunks);
        k0 = slot * kpsd;
        kend = k0 + kpsd;
        first = k0 + kChunk * wave;
        if (first + kChunk <= a.P && first < a.max_keys) { issue_chunk<D, ONCE>(ring, hb, dl, first, lane); }
    }
    if (first + kStride + kChunk <= a.P && first + kStride < a.max_keys) {
        issue_chunk<D, ONCE>(ring + GE::kStageBytes, hb, dl, first + kStride, lane);
    }
    i4 qraw[NT][G][2];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        const int r = 16 * nt + c;
#pragma unroll
        for (int gq = 0; gq < G; ++gq) {
#pragma unroll
            for (int hs = 0; hs < 2; ++hs) {
                const int piece = 8 * gq + 2 * g + hs; // dims 8 * piece .. + 7
                const i4 v = *(const NMI_AS3 i4*)(qtile + (NT == 5 ? r : (r & 31)) * (2 * D) + 16 * ((piece + r) & (GE::QPIECES - 1)));
                qraw[nt][gq][hs] = v;
            }
        }
    }

    const int32_t* par = a.parents ? a.parents + static_cast<int64_t>(b) * a.T : nullptr;
    const int pos_first = __builtin_amdgcn_readfirstlane(pos_lds[0]);
    const int pos_last = __builtin_amdgcn_readfirstlane(pos_lds[a.T - 1]);

    // ---- Q operand (B operand of S^T = K' Q^T) from the raw rows.
    RowState<NT, D> s;
    const float thr_unit = kLazyTau / a.scale_log2; // the lazy threshold of a row whose factor is 1
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        const int r = 16 * nt + c;
        const bool valid = r < R;
        const int t = t0 + (valid ? r / a.G : 0);
        float x[G][2][8];
        float amax = 0.0f;
#pragma unroll
        for (int gq = 0; gq < G; ++gq) {
#pragma unroll
            for (int hs = 0; hs < 2; ++hs) {
                const i4 raw = qraw[nt][gq][hs];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int w = raw[e >> 1];
                    const uint16_t bits = static_cast<uint16_t>((e & 1) ? (static_cast<uint32_t>(w) >> 16) : (static_cast<uint32_t>(w) & 0xffffu));
                    x[gq][hs][e] = bf16_to_f32(bits);
                    amax = fmaxf(amax, fabsf(x[gq][hs][e]));
                }
            }
        }
        amax = group4_max(amax);
        // factor = 2^(14 - floor(log2(amax))) puts max|q| in [2^14, 2^15): FP16 holds every BF16
        // value of the row exactly down to 2^-28 of its maximum. The exponent is clamped so the
        // factor and the lazy threshold stay finite for rows of tiny values.
        int fexp = 0; // factor = 2^fexp
        if (amax > 0.0f && amax < INFINITY) {
            fexp = 14 - max(static_cast<int>((__float_as_uint(amax) >> 23) & 0xff) - 127, -100);
        }
        const float factor = ldexpf(1.0f, fexp);
#pragma unroll
        for (int gq = 0; gq < G; ++gq) {
#pragma unroll
            for (int hs = 0; hs < 2; ++hs) {
#pragma unroll
                for (int e = 0; e < 8; ++e) { s.q[nt][gq][hs][e] = static_cast<_Float16>(x[gq][hs][e] * factor); }
            }
        }
        // scale_log2 / factor and kLazyTau / rowmul, as exact power-of-two scalings (no divides on
        // the path to the first chunk).
        s.rowmul[nt] = ldexpf(a.scale_log2, -fexp);
        s.rowthr[nt] = ldexpf(thr_unit, fexp);
        s.nmask[nt] = valid ? new_key_mask(par, t) : 0u;
        s.m[nt] = -INFINITY;
        s.l[nt] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t8 = 0; t8 < D / 16; ++t8) { s.O[nt][t8] = f4{0.f, 0.f, 0.f, 0.f}; }
    }
    if constexpr (NT == 5) {
        // The five tiles' Q operands (the same in every wave) move to LDS, over the raw Q rows once
        // every wave has read them, and are read back per tile: 80 fewer registers per lane.
        __syncthreads();
        if (wave == 0) {
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
#pragma unroll
                for (int gq = 0; gq < G; ++gq) {
#pragma unroll
                    for (int hs = 0; hs < 2; ++hs) { *(NMI_AS3 h8*)(qtile + ((nt * G + gq) * 2 + hs) * 1024 + 16 * lane) = s.q[nt][gq][hs]; }
                }
            }
        }
        __syncthreads();
    }

    const int window = min(pos_last + 1, a.max_keys);
    const int L = max(0, min(pos_first, window));
    const int k1 = min(kend, window);
    const bool fused = a.k_new != nullptr;
    // With the fused append the cache rows >= L are written by this launch: splits stream only the
    // history below L, and the split holding L attends to the new rows from its own registers.
    const int hend = fused ? min(k1, L) : k1;
    const bool owner = fused && L >= k0 && L < kend && L < window;
    const int64_t pidx = (static_cast<int64_t>(rc) * a.Hkv + h) * a.split_slots + slot;
    uint16_t* out_o = a.part_o + pidx * (RMAX * D);
    float* out_ml = a.part_ml + pidx * (2 * RMAX);


    if (k0 >= hend && !owner) {
        __builtin_amdgcn_s_waitcnt(0);
        if (threadIdx.x < RMAX) {
            out_ml[2 * threadIdx.x] = -INFINITY;
            out_ml[2 * threadIdx.x + 1] = 0.0f;
        }
        return;
    }

    // ---- fused A1 append: the owner quantizes the T new rows into the cache and into its new-row
    // stage; wave 0 attends to them before its history chunks.
    uint32_t kwide = 0u; // exponent bits 14 and 13 of the K scales seen (FP32-range test)
    if (owner) {
        NMI_AS3 char* ns = (NMI_AS3 char*)smem + GE::kNewStage;
        __syncthreads(); // every wave has read its Q rows from this area
        for (int i = threadIdx.x; i < GE::kStageBytes / 16; i += blockDim.x) { *(NMI_AS3 i4*)(ns + 16 * i) = i4{0, 0, 0, 0}; }
        __syncthreads();
        for (int t = wave; t < a.T; t += kWaves) {
            const int p = pos_lds[t];
            if (p < 0 || p >= a.P) { continue; }
            const int64_t src = static_cast<int64_t>(D) * (h + static_cast<int64_t>(a.Hkv) * (t + static_cast<int64_t>(a.T) * b));
            append_row<D>(a.k_new + src, a.v_new + src, kbase + static_cast<int64_t>(p) * D, vbase + static_cast<int64_t>(p) * D,
                       ksbase + static_cast<int64_t>(p) * G, vsbase + static_cast<int64_t>(p) * G, ns, t, lane);
        }
        __syncthreads();
        if (wave == 0) {
            ChunkRegs<D> r;
            read_chunk<D>(ns, r, lane, c, g);
            kwide |= wide_k_bits<D>(r);
            const KeyRange nk{L, L, min(window, L + a.T)};
            if constexpr (NT == 5) {
                compute_chunk_tiles<NT, D, true>(r, L, s, nk, c, g, qtile);
            } else {
                compute_chunk<NT, D>(r, L, true, s, nk, c, g);
            }
        }
    }

    // ---- history chunks, software-pipelined: while chunk j's softmax and PV run, chunk j+1 is
    // read from LDS and its QK^T issued, and chunks j+2, j+3 are in flight as DMA. D = 256 and the
    // five-tile form hold one chunk in registers at a time (the DMA lookahead stays two chunks).
    const KeyRange hk{min(L, k1), L, hend};
    if constexpr (D == 256 || NT == 5) {
        int stage = 0;
#pragma unroll 1
        for (int cj = first; cj < hend; cj += kStride) {
            NMI_AS3 char* st = ring + stage * GE::kStageBytes;
            wait_chunk<D>(cj + kStride < hend); // chunk cj landed; the next one may stay in flight
            ChunkRegs<D> r;
            read_chunk<D>(st, r, lane, c, g);
            kwide |= wide_k_bits<D>(r);
            if (cj + 2 * kStride < hend) {
                __builtin_amdgcn_s_waitcnt(kWaitLgkm0); // chunk cj sits in registers: reuse its stage
                issue_chunk<D, ONCE>(st, hb, dl, cj + 2 * kStride, lane);
            }
            if constexpr (NT == 5) {
                // The masked and unmasked forms are separate code paths: one merged path would
                // carry the scores through AGPRs across the mask (40 more moves per chunk).
                if (cj + kChunk > hk.vis_all) {
                    compute_chunk_tiles<NT, D, true>(r, cj, s, hk, c, g, qtile);
                } else {
                    compute_chunk_tiles<NT, D, false>(r, cj, s, hk, c, g, qtile);
                }
            } else {
                compute_chunk<NT, D>(r, cj, cj + kChunk > hk.vis_all, s, hk, c, g);
            }
            stage ^= 1;
        }
    } else if (first < hend) {
        int stage = 0;
        int cj = first;
        ChunkRegs<D> r;
        wait_chunk<D>(first + kStride < hend);
        read_chunk<D>(ring, r, lane, c, g);
        if (first + 2 * kStride < hend) {
            __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
            issue_chunk<D, ONCE>(ring, hb, dl, first + 2 * kStride, lane);
        }
        f4 sacc[2][NT];
        kwide |= wide_k_bits<D>(r);
        qk_chunk<NT, D>(r, s, sacc);
        typename ChunkRegs<D>::VRow vcur[8];
        i4 vswcur[2][D / 128];
#pragma unroll
        for (int j = 0; j < 8; ++j) { vcur[j] = r.vr[j]; }
#pragma unroll
        for (int h = 0; h < D / 128; ++h) {
            vswcur[0][h] = r.vsw[0][h];
            vswcur[1][h] = r.vsw[1][h];
        }
        stage = 1;
#pragma unroll 1
        for (; cj < hend; cj += kStride) {
            // Issue priority alternates per chunk (phase offset by the workgroup index), so waves
            // sharing a SIMD take turns by progress instead of the oldest one always issuing first
            // (MI355X, C3, four paired runs: -1.0 to -2.5 us per layer; C2 unchanged).
            if ((((cj - first) / kStride) + blockIdx.x + blockIdx.y) & 1) {
                __builtin_amdgcn_s_setprio(3);
            } else {
                __builtin_amdgcn_s_setprio(0);
            }
            const int cn = cj + kStride; // next chunk (if < hend, its DMA was issued two steps ago)
            NMI_AS3 char* stn = ring + stage * GE::kStageBytes;
            // Chunk j+1's DMA done (j+2's may stay outstanding). Reading a stage past the end is
            // harmless: those registers are never used.
            wait_chunk<D>(cn + kStride < hend);
            ChunkRegs<D> rn;
            read_chunk<D>(stn, rn, lane, c, g);
            h8 pop[NT];
            softmax_chunk<NT, D>(sacc, cj, cj + kChunk > hk.vis_all, s, hk, g, pop);
            if (cn + 2 * kStride < hend) {
                __builtin_amdgcn_s_waitcnt(kWaitLgkm0); // chunk j+1 sits in registers: reuse its stage
                issue_chunk<D, ONCE>(stn, hb, dl, cn + 2 * kStride, lane);
            }
            stage ^= 1;
            f4 sn[2][NT];
            if (cn < hend) { // the last chunk has no successor (a stage past the end holds anything)
                kwide |= wide_k_bits<D>(rn);
                qk_chunk<NT, D>(rn, s, sn);
            }
            pv_chunk<NT, D>(pop, vcur, vswcur, cj, cj + kChunk > hk.vis_all, s, hk, c, g);
#pragma unroll
            for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) { sacc[kt][nt] = sn[kt][nt]; }
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) { vcur[j] = rn.vr[j]; }
#pragma unroll
            for (int h = 0; h < D / 128; ++h) {
                vswcur[0][h] = rn.vsw[0][h];
                vswcur[1][h] = rn.vsw[1][h];
            }
        }
    }

    NMI_AS3 int32_t* kwide_word = (NMI_AS3 int32_t*)((NMI_AS3 char*)smem + GE::kWideK);
    if (__any((kwide & 0x40004000u) != 0u) && lane == 0) { *kwide_word = 1; }

    // ---- merge the four waves through LDS (reusing the staging ring), then write the partial.
    __builtin_amdgcn_s_waitcnt(0); // no DMA may land in the ring after this point
    __syncthreads();
    static_assert(kWaves * 32 * (D + 4 + 2) * 4 <= GE::kSmemBytes, "wave merge exceeds the LDS map");
    write_partial<NT, D, CACHED>(s, smem, R, wave, c, g, out_o, out_ml, *kwide_word != 0);
}

// CACHED: the batch-1 partials go out with ordinary (cached) stores; an instance of its own, launched
// only for the plans that ask for it (kAttnCachedPartialKeys).
// DEV: a batch-1 plan split on the device (b1_device_kps of the window; up to two row tiles).
template <int NT, int D, bool ONCE, bool CACHED = false, bool DEV = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(D == 128 && NT <= 2 ? 2 : 1, D == 128 && NT <= 2 ? 2 : 1))) void verify_attn_partial_kernel(AttnArgs a) {
    using GE = Geo<D>;
    constexpr int RMAX = NT == 5 ? kAttnWideRows : kAttnRowsPerTile; // rows per partial slot
    static_assert(NT <= 2 || (NT == 5 && D == 128), "row tiles per wave");
    __shared__ __attribute__((aligned(16))) char smem[NT == 5 ? GE::kSmemBytes + RMAX * 2 * D : GE::kSmemBytes];
    // B = 1 (up to two row tiles) has a code path of its own, in which the sequence and slot are
    // compile-time facts (measured on MI355X: C2 13.9 -> 13.5 us per layer). The five-tile form
    // keeps one path: a second copy raises its register pressure into spills.
    if constexpr (NT <= 2) {
        if (a.B == 1) {
            // grid (KV head, split, row chunk): the dispatch order runs over the splits of every
            // head together, so the splits past a device window shorter than the envelope plan (the
            // last ones) are the workgroups that share a CU, not live splits of the last heads
            const int split = blockIdx.y;
            const int k0 = split * a.kps;
            partial_segment<NT, D, ONCE, CACHED, DEV>(a, smem, 0, k0, k0 + a.kps, split, blockIdx.x);
            return;
        }
        // Slot 0 of row chunk 0, KV head 0 also records the sequences' ranges for the merge.
        const bool recorder = blockIdx.x == 0 && blockIdx.y == 0 && blockIdx.z == 0;
        const SplitRange sr = batch_split_range(a.positions, a.T, a.B, a.max_keys, a.split_budget, blockIdx.x,
                                                recorder ? a.seq_table : nullptr);
        if (sr.b < 0) { return; } // a slot past the batch's last split: no partial
        const int k0 = (static_cast<int>(blockIdx.x) - sr.first) * sr.kps;
        partial_segment<NT, D, ONCE, false>(a, smem, sr.b, k0, k0 + sr.kps, blockIdx.x, blockIdx.y);
    } else {
        int b = 0;
        int k0 = blockIdx.x * a.kps;
        int kend = k0 + a.kps;
        if (a.B > 1) {
            const bool recorder = blockIdx.x == 0 && blockIdx.y == 0 && blockIdx.z == 0;
            const SplitRange sr = batch_split_range(a.positions, a.T, a.B, a.max_keys, a.split_budget, blockIdx.x,
                                                    recorder ? a.seq_table : nullptr);
            if (sr.b < 0) { return; }
            b = sr.b;
            k0 = (static_cast<int>(blockIdx.x) - sr.first) * sr.kps;
            kend = k0 + sr.kps;
        }
        partial_segment<NT, D, ONCE, false>(a, smem, b, k0, kend, blockIdx.x, blockIdx.y);
    }
}


// ---- BF16 KV cache -------------------------------------------------------------------------------
//
// Same split-K structure. A stage holds 32 keys of BF16 K (row r's 16-byte piece p at slot
// p ^ (r % PB)) and V (natural order), no scales; QK^T and PV run on v_mfma_f32_16x16x32_bf16 with
// the cache values and BF16 Q exactly as stored. P goes to the MFMA as two BF16 terms
// (hi = BF16(p), lo = BF16(p - hi)), so the product keeps ~16 significant bits of P. At head_dim
// 128 the split that owns the new rows copies them into the cache and into a stage of its own
// (BF16 caches have no codec); at head_dim 256, or when several row chunks read the new rows, a
// launch of their own copies them before this kernel.
template <int D>
struct GeoB {
    static constexpr int PB = D / 8;                // 16-byte pieces of a BF16 row
    static constexpr int kStageK = 0;
    static constexpr int kStageV = 64 * D;          // 32 rows x 2D B
    static constexpr int kStageBytes = 128 * D;     // 16 KB / 32 KB
    static constexpr int STAGES = D == 128 ? 2 : 1; // stages per wave (LDS budget)
    static constexpr int kDmaPerChunk = D / 8;      // 1 KB DMAs: D/16 per plane
    static constexpr int kRingBytes = kWaves * STAGES * kStageBytes;
    static constexpr int kQTile = kRingBytes;       // Q tile: 32 rows x 2D B
    static constexpr int kPosLds = kQTile + 64 * D;
    // D = 128: the new rows of A1 (32 rows of K and V) get a stage of their own; D = 256 has no room
    // for one, and its A1 copies the new rows into the cache in a launch of their own.
    static constexpr bool kFusedAppend = D == 128;
    static constexpr int kNewStage = kPosLds + 128;
    static constexpr int kSmemBytes = kFusedAppend ? kNewStage + kStageBytes : kPosLds + 128; // 155,776 B / 147,584 B
};

// Lane -> (row lane / PB, slot lane % PB) of each 1 KB DMA (512 / D rows); K slot s of row r holds
// piece s ^ (r % PB), so the K source offset depends on the DMA index (one XOR per DMA).
struct DmaLanesB {
    int row; // row within one DMA
    int slot;
    int v;
};

template <int D>
__device__ __forceinline__ DmaLanesB make_dma_lanes_b(int lane) {
    constexpr int PB = GeoB<D>::PB;
    DmaLanesB dl;
    dl.row = lane / PB;
    dl.slot = lane % PB;
    dl.v = dl.row * 2 * D + 16 * dl.slot;
    return dl;
}

// K rows of chunk c0 into the stage's K plane (D/16 DMAs); ONCE as for issue_chunk.
template <int D, bool ONCE>
__device__ __forceinline__ void issue_k_b(NMI_AS3 char* st, __amdgpu_buffer_rsrc_t rk, const DmaLanesB& dl, int c0) {
    using G = GeoB<D>;
    constexpr int ROWS = 512 / D; // rows per 1 KB DMA
    const int so = __builtin_amdgcn_readfirstlane(c0) * 2 * D; // wave-uniform, in an SGPR
#pragma unroll
    for (int r = 0; r < D / 16; ++r) {
        const int koff = dl.row * 2 * D + 16 * (dl.slot ^ ((ROWS * r + dl.row) % G::PB));
        if constexpr (ONCE) {
            dma16_nt(rk, st + G::kStageK + r * 1024, koff, so + r * 1024);
        } else {
            dma16(rk, st + G::kStageK + r * 1024, koff, so + r * 1024);
        }
    }
}

// V rows of chunk c0 into the stage's V plane (D/16 DMAs).
template <int D, bool ONCE>
__device__ __forceinline__ void issue_v_b(NMI_AS3 char* st, __amdgpu_buffer_rsrc_t rv, const DmaLanesB& dl, int c0) {
    using G = GeoB<D>;
    const int so = __builtin_amdgcn_readfirstlane(c0) * 2 * D; // wave-uniform, in an SGPR
#pragma unroll
    for (int r = 0; r < D / 16; ++r) {
        if constexpr (ONCE) {
            dma16_nt(rv, st + G::kStageV + r * 1024, dl.v, so + r * 1024);
        } else {
            dma16(rv, st + G::kStageV + r * 1024, dl.v, so + r * 1024);
        }
    }
}

template <int D, bool ONCE>
__device__ __forceinline__ void issue_chunk_b(NMI_AS3 char* st, __amdgpu_buffer_rsrc_t rk, __amdgpu_buffer_rsrc_t rv,
                                              const DmaLanesB& dl, int c0) {
    issue_k_b<D, ONCE>(st, rk, dl, c0);
    issue_v_b<D, ONCE>(st, rv, dl, c0);
}

template <int D>
struct ChunkRegsB {
    i4 kb[2][D / 32];   // A operand of S^T: key 16kt + c, dims 32ks + 8g .. +7
    i4 vr[8][D / 128];  // the lane's dims (D/16)c .. of V rows 4g + j and 16 + 4g + j
};

template <int D>
__device__ __forceinline__ void read_k_b(const NMI_AS3 char* st, ChunkRegsB<D>& r, int c, int g) {
    using G = GeoB<D>;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
        for (int ks = 0; ks < D / 32; ++ks) {
            const int row = 16 * kt + c;
            const int slot = (4 * ks + g) ^ (row % G::PB);
            r.kb[kt][ks] = *(const NMI_AS3 i4*)(st + G::kStageK + row * 2 * D + 16 * slot);
        }
    }
}

template <int D>
__device__ __forceinline__ void read_v_b(const NMI_AS3 char* st, ChunkRegsB<D>& r, int c, int g) {
    using G = GeoB<D>;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int row = j < 4 ? 4 * g + j : 16 + 4 * g + (j - 4);
#pragma unroll
        for (int h = 0; h < D / 128; ++h) {
            r.vr[j][h] = *(const NMI_AS3 i4*)(st + G::kStageV + row * 2 * D + (D / 8) * c + 16 * h);
        }
    }
}

// Q stays in LDS (the B operand of Q^T, rows 16nt + c, dims 32ks + 8g + e, is read per chunk).
template <int NT, int D>
struct RowStateB {
    float rowmul[NT];   // softmax scale * log2(e)
    float rowthr[NT];
    uint32_t nmask[NT];
    float m[NT];
    f4 O[NT][D / 16];   // O^T tiles: tile t row 4g+e is dim (D/16)(4g+e) + t
    f4 l[NT];
};

// Q^T operand for k-step ks of tile nt from the LDS Q tile (rows >= R read as zero).
template <int D>
__device__ __forceinline__ bf8 q_operand_b(const NMI_AS3 char* qtile, int nt, int ks, int c, int g, int R) {
    const int r = 16 * nt + c;
    const int piece = 4 * ks + g;
    const i4 v = *(const NMI_AS3 i4*)(qtile + (r & 31) * (2 * D) + 16 * ((piece + r) & (D / 8 - 1)));
    return __builtin_bit_cast(bf8, r < R ? v : i4{0, 0, 0, 0});
}

template <int NT, int D>
__device__ __forceinline__ void qk_chunk_b(const ChunkRegsB<D>& r, const NMI_AS3 char* qtile, int c, int g, int R,
                                           f4 (&sacc)[2][NT]) {
#pragma unroll
    for (int ks = 0; ks < D / 32; ++ks) {
        bf8 qv[NT];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) { qv[nt] = q_operand_b<D>(qtile, nt, ks, c, g, R); }
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
            const bf8 a = __builtin_bit_cast(bf8, r.kb[kt][ks]);
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                const f4 acc = ks == 0 ? f4{0.f, 0.f, 0.f, 0.f} : sacc[kt][nt];
                sacc[kt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qv[nt], acc, 0, 0, 0);
            }
        }
    }
}

// BF16 element t of the lane's slice of a V row.
template <int D>
__device__ __forceinline__ uint32_t v_word_b(const i4 (&row)[D / 128], int t) {
    return static_cast<uint32_t>(row[t >> 3][(t >> 1) & 3]);
}

// O^T += V^T (P_hi + P_lo)^T and l += ones x (P_hi + P_lo)^T. V values of keys at or past key_end
// in a masked chunk are replaced by zero (those rows may hold anything).
template <int NT, int D>
__device__ __forceinline__ void pv_chunk_b(const float (&p)[NT][8], const ChunkRegsB<D>& r, int c0, bool masked,
                                           RowStateB<NT, D>& s, const KeyRange& kr, int g) {
    bf8 phi[NT], plo[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const __bf16 hi = static_cast<__bf16>(p[nt][i]);
            phi[nt][i] = hi;
            plo[nt][i] = static_cast<__bf16>(p[nt][i] - static_cast<float>(hi));
        }
    }
    uint32_t keep = 0xffu; // bit j: key j of the lane's 8 is below key_end
    if (masked) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int key = c0 + (j < 4 ? 4 * g + j : 16 + 4 * g + (j - 4));
            keep &= key < kr.key_end ? 0xffu : ~(1u << j);
        }
    }
#pragma unroll
    for (int t = 0; t < D / 16; ++t) {
        uint32_t w[4];
        const uint32_t sel = (t & 1) ? 0x07060302u : 0x05040100u;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t lo = (keep >> (2 * q)) & 1u ? v_word_b<D>(r.vr[2 * q], t) : 0u;
            const uint32_t hi = (keep >> (2 * q + 1)) & 1u ? v_word_b<D>(r.vr[2 * q + 1], t) : 0u;
            w[q] = __builtin_amdgcn_perm(hi, lo, sel);
        }
        const bf8 va = __builtin_bit_cast(bf8, w);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            s.O[nt][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, phi[nt], s.O[nt][t], 0, 0, 0);
            s.O[nt][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, plo[nt], s.O[nt][t], 0, 0, 0);
        }
    }
    bf8 ones;
#pragma unroll
    for (int i = 0; i < 8; ++i) { ones[i] = static_cast<__bf16>(1.0f); }
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        s.l[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, phi[nt], s.l[nt], 0, 0, 0);
        s.l[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, plo[nt], s.l[nt], 0, 0, 0);
    }
}

template <int NT, int D, bool ONCE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void verify_attn_partial_bf16_kernel(AttnArgs a) {
    using GB = GeoB<D>;
    __shared__ __attribute__((aligned(16))) char smem[GB::kSmemBytes];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int c = lane & 15;
    const int g = lane >> 4;
    // B = 1: grid (KV head, split, row chunk), as in the INT8 kernel; batches: (slot, KV head, row chunk)
    const int h = a.B == 1 ? blockIdx.x : blockIdx.y;
    const int rc = blockIdx.z;
    int b = 0;
    int split = a.B == 1 ? blockIdx.y : blockIdx.x;
    int kps = a.kps;
    int slot0 = 0;
    if (a.B > 1) {
        // Slot 0 of row chunk 0, KV head 0 also records the sequences' ranges for the merge.
        const bool recorder = blockIdx.x == 0 && h == 0 && rc == 0;
        const SplitRange sr = batch_split_range(a.positions, a.T, a.B, a.max_keys, a.split_budget, blockIdx.x,
                                                recorder ? a.seq_table : nullptr);
        if (sr.b < 0) { return; } // a slot past the batch's last split: no partial
        b = sr.b;
        split = blockIdx.x - sr.first;
        kps = sr.kps;
        slot0 = sr.first;
    }
    const int k0 = split * kps;

    const int64_t head = static_cast<int64_t>(b) * a.code_seq + static_cast<int64_t>(h) * a.P * D;
    const __amdgpu_buffer_rsrc_t rk = raw_buffer(a.kb + head, static_cast<int64_t>(a.P) * D * 2);
    const __amdgpu_buffer_rsrc_t rv = raw_buffer(a.vb + head, static_cast<int64_t>(a.P) * D * 2);
    const DmaLanesB dl = make_dma_lanes_b<D>(lane);
    NMI_AS3 char* ring = (NMI_AS3 char*)smem + wave * GB::STAGES * GB::kStageBytes;

    // Q tile (rows r = tl * G + gi, 2D bytes each, piece p at slot (p + r) % QP) and positions by
    // LDS DMA before the chunk DMAs, as in the INT8 kernel.
    const int t0 = rc * a.tokens_per_chunk;
    const int Tc = min(a.tokens_per_chunk, a.T - t0);
    const int R = Tc * a.G;
    NMI_AS3 char* qtile = (NMI_AS3 char*)smem + GB::kQTile;
    NMI_AS3 int32_t* pos_lds = (NMI_AS3 int32_t*)((NMI_AS3 char*)smem + GB::kPosLds);
    const int32_t* pos = a.positions + static_cast<int64_t>(b) * a.T;
    if (wave == 0) {
        if (lane < a.T) { __builtin_amdgcn_global_load_lds((const NMI_AS1 void*)(pos + lane), (NMI_AS3 void*)pos_lds, 4, 0, 0); }
        constexpr int QP = D / 8;
        constexpr int RPD = 64 / QP;
#pragma unroll 1
        for (int k = 0; RPD * k < R; ++k) {
            const int row = RPD * k + lane / QP;
            if (row < R) {
                const int tl = row / a.G;
                const int gi = row - tl * a.G;
                const int piece = ((lane % QP) - row) & (QP - 1);
                const uint16_t* src = a.q + static_cast<int64_t>(D) * (h * a.G + gi + static_cast<int64_t>(a.Hq) * (t0 + tl + static_cast<int64_t>(a.T) * b)) + 8 * piece;
                __builtin_amdgcn_global_load_lds((const NMI_AS1 void*)src, (NMI_AS3 void*)(qtile + k * 1024), 16, 0, 0);
            }
        }
    }
    const int first = k0 + kChunk * wave;
    if (first + kChunk <= a.P) { issue_chunk_b<D, ONCE>(ring, rk, rv, dl, first); }
    if (GB::STAGES == 2 && first + kStride + kChunk <= a.P) { issue_chunk_b<D, ONCE>(ring + GB::kStageBytes, rk, rv, dl, first + kStride); }
    if (wave == 0) {
        if (GB::STAGES == 2 && first + kStride + kChunk <= a.P) {
            __builtin_amdgcn_s_waitcnt(waitcnt_vm(2 * GB::kDmaPerChunk));
        } else if (first + kChunk <= a.P) {
            __builtin_amdgcn_s_waitcnt(waitcnt_vm(GB::kDmaPerChunk));
        } else {
            __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
        }
    }
    __builtin_amdgcn_s_barrier();

    // ---- per-row state (Q is used as stored: BF16 is exact for the BF16 MFMA).
    RowStateB<NT, D> s;
    const int32_t* par = a.parents ? a.parents + static_cast<int64_t>(b) * a.T : nullptr;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        const int r = 16 * nt + c;
        const bool valid = r < R;
        const int t = t0 + (valid ? r / a.G : 0);
        s.rowmul[nt] = a.scale_log2;
        s.rowthr[nt] = kLazyTau / s.rowmul[nt];
        s.nmask[nt] = valid ? new_key_mask(par, t) : 0u;
        s.m[nt] = -INFINITY;
        s.l[nt] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t8 = 0; t8 < D / 16; ++t8) { s.O[nt][t8] = f4{0.f, 0.f, 0.f, 0.f}; }
    }

    const int pos_first = __builtin_amdgcn_readfirstlane(pos_lds[0]);
    const int pos_last = __builtin_amdgcn_readfirstlane(pos_lds[a.T - 1]);
    const int window = min(pos_last + 1, a.max_keys);
    const int L = max(0, min(pos_first, window));
    const int k1 = min(k0 + kps, window);
    // With the fused append (D = 128) the new rows are copied into the cache by this launch: splits
    // stream only the history below L, and the split holding L attends to the new rows from a stage
    // built from the inputs. Otherwise they are already in the cache.
    const bool fused = GB::kFusedAppend && a.k_new != nullptr;
    const int hend = fused ? min(k1, L) : k1;
    const bool owner = fused && L >= k0 && L < k0 + kps && L < window;
    const int64_t pidx = (static_cast<int64_t>(rc) * a.Hkv + h) * a.split_slots + slot0 + split;
    uint16_t* out_o = a.part_o + pidx * (32 * D);
    float* out_ml = a.part_ml + pidx * 64;
    if (k0 >= hend && !owner) {
        __builtin_amdgcn_s_waitcnt(0);
        if (threadIdx.x < 32) {
            out_ml[2 * threadIdx.x] = -INFINITY;
            out_ml[2 * threadIdx.x + 1] = 0.0f;
        }
        return;
    }

    if constexpr (GB::kFusedAppend) {
        if (owner) {
            // Every thread copies 16-byte pieces of the T new K/V rows into cache rows pos[t] and
            // into the stage (K piece p of row r at slot p ^ (r % PB), V in natural order; rows
            // without a new token, or whose position lies outside the cache, stay zero).
            NMI_AS3 char* ns = (NMI_AS3 char*)smem + GB::kNewStage;
            constexpr int PB = GB::PB;
            for (int i = threadIdx.x; i < 32 * PB; i += blockDim.x) {
                const int r = i / PB;
                const int pc = i - r * PB;
                i4 kv = {0, 0, 0, 0};
                i4 vv = {0, 0, 0, 0};
                const int pr = r < a.T ? pos_lds[r] : -1;
                if (pr >= 0 && pr < a.P) {
                    const int64_t src = static_cast<int64_t>(D) * (h + static_cast<int64_t>(a.Hkv) * (r + static_cast<int64_t>(a.T) * b)) + 8 * pc;
                    kv = *reinterpret_cast<const i4*>(a.k_new + src);
                    vv = *reinterpret_cast<const i4*>(a.v_new + src);
                    *reinterpret_cast<i4*>(a.kb + head + static_cast<int64_t>(pr) * D + 8 * pc) = kv;
                    *reinterpret_cast<i4*>(a.vb + head + static_cast<int64_t>(pr) * D + 8 * pc) = vv;
                }
                *(NMI_AS3 i4*)(ns + GB::kStageK + r * 2 * D + 16 * (pc ^ (r % PB))) = kv;
                *(NMI_AS3 i4*)(ns + GB::kStageV + r * 2 * D + 16 * pc) = vv;
            }
            __syncthreads();
            if (wave == 0) {
                ChunkRegsB<D> r;
                read_k_b<D>(ns, r, c, g);
                read_v_b<D>(ns, r, c, g);
                const KeyRange nk{L, L, min(window, L + a.T)};
                f4 sacc[2][NT];
                qk_chunk_b<NT, D>(r, qtile, c, g, R, sacc);
                float p[NT][8];
                softmax_probs<NT, D>(sacc, L, true, s, nk, g, p);
                pv_chunk_b<NT, D>(p, r, L, true, s, nk, g);
            }
        }
    }

    const KeyRange hk{min(L, hend), L, hend};
    if constexpr (GB::STAGES == 2) {
        // ---- chunks: read one into registers, put the DMA of the chunk two steps ahead into its
        // stage, then compute it.
        int stage = 0;
#pragma unroll 1
        for (int cj = first; cj < hend; cj += kStride) {
            NMI_AS3 char* st = ring + stage * GB::kStageBytes;
            if (cj + kStride < hend) {
                __builtin_amdgcn_s_waitcnt(waitcnt_vm(GB::kDmaPerChunk));
            } else {
                __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
            }
            ChunkRegsB<D> r;
            read_k_b<D>(st, r, c, g);
            read_v_b<D>(st, r, c, g);
            const int cn = cj + 2 * kStride;
            if (cn < hend) {
                __builtin_amdgcn_s_waitcnt(kWaitLgkm0); // chunk cj sits in registers: reuse its stage
                issue_chunk_b<D, ONCE>(st, rk, rv, dl, cn);
            }
            f4 sacc[2][NT];
            qk_chunk_b<NT, D>(r, qtile, c, g, R, sacc);
            float p[NT][8];
            const bool masked = cj + kChunk > hk.vis_all;
            softmax_probs<NT, D>(sacc, cj, masked, s, hk, g, p);
            pv_chunk_b<NT, D>(p, r, cj, masked, s, hk, g);
            stage ^= 1;
        }
    } else {
        // ---- one stage per wave: the K plane is refilled with the next chunk's keys as soon as
        // they sit in registers, the V plane after the softmax, so K and V registers are never
        // live together. DMAs complete in issue order (K(cj), V(cj), K(cn), V(cn)).
        NMI_AS3 char* st = ring;
#pragma unroll 1
        for (int cj = first; cj < hend; cj += kStride) {
            const int cn = cj + kStride;
            __builtin_amdgcn_s_waitcnt(waitcnt_vm(GB::kDmaPerChunk / 2)); // K(cj) landed
            ChunkRegsB<D> r;
            read_k_b<D>(st, r, c, g);
            if (cn < hend) {
                __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
                issue_k_b<D, ONCE>(st, rk, dl, cn);
            }
            f4 sacc[2][NT];
            qk_chunk_b<NT, D>(r, qtile, c, g, R, sacc);
            float p[NT][8];
            const bool masked = cj + kChunk > hk.vis_all;
            softmax_probs<NT, D>(sacc, cj, masked, s, hk, g, p);
            if (cn < hend) {
                __builtin_amdgcn_s_waitcnt(waitcnt_vm(GB::kDmaPerChunk / 2)); // V(cj) landed
            } else {
                __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
            }
            read_v_b<D>(st, r, c, g);
            if (cn < hend) {
                __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
                issue_v_b<D, ONCE>(st, rv, dl, cn);
            }
            pv_chunk_b<NT, D>(p, r, cj, masked, s, hk, g);
        }
    }

    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    static_assert(kWaves * 32 * (D + 4 + 2) * 4 <= GB::kSmemBytes, "wave merge exceeds the LDS map");
    write_partial<NT, D, false>(s, smem, R, wave, c, g, out_o, out_ml);
}

struct MergeArgs {
    const uint16_t* part_o; // FP16 O / l

    const float* part_ml;
    void* out;
    int32_t T;
    int32_t Hq;
    int32_t Hkv;
    int32_t G;
    int32_t tokens_per_chunk;
    int32_t row_chunks;
    int32_t nsplit;
    int32_t out_f32;
    const int32_t* seq_table;
    int32_t B;
    int32_t split_slots;
    int32_t rows_per_slot; // rows of one partial slot (32, or 80 for the 5-tile tree form)
    // Exact recompute of a split (FP32-range decode; INT8 caches only): the partial kernel's inputs.
    const uint16_t* q;
    const int32_t* positions;
    const int32_t* parents;
    const int8_t* kc;
    const int8_t* vc;
    const uint16_t* ks;
    const uint16_t* vs;
    int64_t code_seq;
    int64_t scale_seq;
    int32_t P;
    int32_t kps;          // B == 1: keys per split
    int32_t max_keys;
    int32_t split_budget; // B > 1: the device batch plan's budget
    int32_t fused;        // the partial launch wrote the new rows itself (its split holding L took them)
    float scale_log2;
};

constexpr int kMergeThreads = 256;
constexpr int kMergeDims = 32;                               // output dims per block
constexpr int kMergeGroups = kMergeThreads / kMergeDims;     // split groups per block
constexpr int kMergePre = 8;                                 // 64 splits loaded up front
constexpr int kMergeB1Dims = 32; // output dims per batch-1 merge block (C2 on MI355X: 12.1 us per layer; 64: 12.35, 16: 12.47)
constexpr int kMergeMaxSplits = 2048;

// ---- exact recompute of a split (FP32-range decode) -------------------------------------------
//
// A split whose partial the fast path could not hold (marked by the partial kernel for a K scale of
// 512 or more, or non-finite: a V scale that large) is recomputed here for one query row and one
// 32-dim slice, with the reference's decode FP32(code) * scale (include/ninfer/ops/gqa_attention.h:30)
// and FP32 arithmetic, over exactly the keys the partial kernel gave that split: [k0, min(kend,
// window)), below L when the launch wrote the new rows itself, plus the new rows [L, L + T) for the
// split holding L. A key at or past L is visible to token t when bit (key - L) of t's mask is set
// (causal or ancestor mask). Whole workgroup of 256 threads, one key per thread per block of 256.
// m is the log2-domain maximum; l and o carry the partial kernel's 2^kPOffset factor.
constexpr int kExactLds = 256 + 256 + 8 * 32 + 16; // + D floats of the query row

template <int D>
__device__ void exact_split(const MergeArgs& a, int b, int t, int qh, int k0, int kend, int d0, float* xs,
                            float& m_out, float& l_out, float& o_out) {
    constexpr int G = D / 64;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    float* xq = xs;                    // [D] query row * scale * log2(e)
    float* xp = xs + D;                // [256] probabilities of the block's keys
    float* xo = xs + D + 256;          // [8][32] slice sums per key part
    float* xr = xs + D + 256 + 8 * 32; // [16] reductions
    const int h = qh / a.G;
    const int32_t* pos = a.positions + static_cast<int64_t>(b) * a.T;
    const int pos_first = pos[0];
    const int pos_last = pos[a.T - 1];
    const int window = max(0, min(pos_last + 1, a.max_keys));
    const int L = max(0, min(pos_first, window));
    const int k1 = min(kend, window);
    const int hend = a.fused ? min(k1, L) : k1;
    const bool owner = a.fused && L >= k0 && L < kend && L < window;
    const int n1 = max(0, hend - k0);
    const int n2 = owner ? max(0, min(window, L + a.T) - L) : 0;
    const uint32_t nmask = new_key_mask(a.parents ? a.parents + static_cast<int64_t>(b) * a.T : nullptr, t);
    const int8_t* kbase = a.kc + static_cast<int64_t>(b) * a.code_seq + static_cast<int64_t>(h) * a.P * D;
    const int8_t* vbase = a.vc + static_cast<int64_t>(b) * a.code_seq + static_cast<int64_t>(h) * a.P * D;
    const uint16_t* ksb = a.ks + static_cast<int64_t>(b) * a.scale_seq + static_cast<int64_t>(h) * a.P * G;
    const uint16_t* vsb = a.vs + static_cast<int64_t>(b) * a.scale_seq + static_cast<int64_t>(h) * a.P * G;
    __syncthreads(); // the caller's use of xs is over
    if (tid < D) { xq[tid] = bf16_to_f32(a.q[static_cast<int64_t>(D) * (qh + static_cast<int64_t>(a.Hq) * (t + static_cast<int64_t>(a.T) * b)) + tid]) * a.scale_log2; }
    __syncthreads();
    float M = -INFINITY; // uniform
    float Ls = 0.0f;     // uniform
    float Od = 0.0f;     // threads tid < 32: dim d0 + tid
    const auto key_of = [&](int i) { return i < n1 ? k0 + i : L + (i - n1); };
    for (int base = 0; base < n1 + n2; base += 256) {
        const int i = base + tid;
        float sk = -INFINITY;
        if (i < n1 + n2) {
            const int k = key_of(i);
            const bool vis = k < L || (static_cast<unsigned>(k - L) < 32u && ((nmask >> (k - L)) & 1u) != 0u);
            if (vis) {
                float acc = 0.0f;
#pragma unroll
                for (int gq = 0; gq < G; ++gq) {
                    const float sc = f16_bits_to_f32(ksb[static_cast<int64_t>(k) * G + gq]);
                    float part = 0.0f;
                    for (int d = 0; d < 64; ++d) {
                        part = fmaf(xq[64 * gq + d], static_cast<float>(kbase[static_cast<int64_t>(k) * D + 64 * gq + d]) * sc, part);
                    }
                    acc += part;
                }
                sk = acc;
            }
        }
        float bm = wave_max(sk);
        if (lane == 0) { xr[wave] = bm; }
        __syncthreads();
        bm = fmaxf(fmaxf(xr[0], xr[1]), fmaxf(xr[2], xr[3]));
        const float Mn = fmaxf(M, bm);
        const float alpha = (M == -INFINITY || Mn == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(M - Mn);
        const float pk = (sk == -INFINITY || Mn == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(sk - Mn + kPOffset);
        xp[tid] = pk;
        float bs = wave_sum(pk);
        __syncthreads(); // xr read by every thread, xp written
        if (lane == 0) { xr[4 + wave] = bs; }
        // O slice: thread (dim tid % 32, key part tid / 32) sums its 32 keys of the block
        const int dim = tid & 31;
        const int part = tid >> 5;
        const int dg = (d0 + dim) / 64;
        float acc = 0.0f;
        for (int j = 0; j < 32; ++j) {
            const int ii = base + 32 * part + j;
            const float pj = xp[32 * part + j];
            if (pj != 0.0f) {
                const int k = key_of(ii);
                const float v = static_cast<float>(vbase[static_cast<int64_t>(k) * D + d0 + dim]) * f16_bits_to_f32(vsb[static_cast<int64_t>(k) * G + dg]);
                acc = fmaf(pj, v, acc);
            }
        }
        xo[32 * part + dim] = acc;
        __syncthreads();
        bs = (xr[4] + xr[5]) + (xr[6] + xr[7]);
        if (tid < 32) {
            float s = 0.0f;
#pragma unroll
            for (int q8 = 0; q8 < 8; ++q8) { s += xo[32 * q8 + tid]; }
            Od = fmaf(Od, alpha, s);
        }
        Ls = fmaf(Ls, alpha, bs);
        M = Mn;
        __syncthreads(); // xp, xo and xr are reused by the next block
    }
    m_out = M;
    l_out = Ls;
    o_out = Od;
}

// The merge of one output row's 32-dim slice over its splits in split order (running log-sum-exp),
// recomputing each split the fast path could not hold. Whole workgroup; writes the output.
// DEV: the partial launch split the batch-1 window on the device (b1_device_kps).
template <int D, int RPS, bool DEV = false>
__device__ void merge_row_exact(const MergeArgs& a, int b, int t, int qh, int d0, float* xs) {
    const int tid = threadIdx.x;
    const int h = qh / a.G;
    const int gi = qh - h * a.G;
    const int rc = t / a.tokens_per_chunk;
    const int r = (t - rc * a.tokens_per_chunk) * a.G + gi;
    const int rps = RPS > 0 ? RPS : a.rows_per_slot;
    int first = 0;
    int count = a.nsplit;
    int kps = a.kps;
    int* xi = reinterpret_cast<int*>(xs + D + 256 + 8 * 32);
    if constexpr (DEV) {
        const int win = min(max(a.positions[a.T - 1] + 1, 0), a.max_keys);
        kps = b1_device_kps(win, a.nsplit, a.Hkv * a.row_chunks);
    }
    if (a.B > 1) {
        first = a.seq_table[2 * b];
        count = a.seq_table[2 * b + 1];
        __syncthreads();
        if (tid < 64) {
            const int kb = static_cast<int>(batch_kps(batch_windows(a.positions, a.T, a.B, a.max_keys), a.split_budget));
            if (tid == 0) { xi[8] = kb; }
        }
        __syncthreads();
        kps = xi[8];
    }
    const int64_t slot0 = (static_cast<int64_t>(rc) * a.Hkv + h) * a.split_slots;
    float M = -INFINITY;
    float Ls = 0.0f;
    float Od = 0.0f;
    for (int j = 0; j < count; ++j) {
        const int64_t slot = slot0 + first + j;
        float ms = a.part_ml[slot * (2 * rps) + 2 * r];
        float ls = a.part_ml[slot * (2 * rps) + 2 * r + 1];
        float od = tid < 32 ? partial_o_at(a.part_o, slot * (static_cast<int64_t>(rps) * D) + static_cast<int64_t>(r) * D + d0 + tid) : 0.0f;
        const bool nonfin = tid < 32 && ls > 0.0f && !__builtin_isfinite(od);
        __syncthreads();
        if (tid < 64) {
            const bool any = __any(nonfin);
            if (tid == 0) { xi[9] = any ? 1 : 0; }
        }
        __syncthreads();
        const bool redo = a.kc != nullptr && (ls < 0.0f || !__builtin_isfinite(ls) || xi[9] != 0);
        if (redo) {
            exact_split<D>(a, b, t, qh, j * kps, j * kps + kps, d0, xs, ms, ls, od);
        } else {
            od *= ls; // the stored O / l back to O
        }
        if (ls > 0.0f) {
            const float Mn = fmaxf(M, ms);
            const float al = M == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(M - Mn);
            const float be = __builtin_amdgcn_exp2f(ms - Mn);
            Od = fmaf(Od, al, od * be);
            Ls = fmaf(Ls, al, ls * be);
            M = Mn;
        }
    }
    if (tid < 32) {
        const float val = Ls > 0.0f ? Od / Ls : 0.0f;
        const int64_t oi = static_cast<int64_t>(D) * (qh + static_cast<int64_t>(a.Hq) * (t + static_cast<int64_t>(a.T) * b)) + d0 + tid;
        if (a.out_f32) {
            static_cast<float*>(a.out)[oi] = val;
        } else {
            static_cast<uint16_t*>(a.out)[oi] = f32_to_bf16_bits(val);
        }
    }
}

// Log-sum-exp merge over splits (reference src/ops/kernel/gqa_attention_decode.cuh:144-227,
// including "every split empty => 0"). Block (row, dim slice): (b, t, qh) x 32 dims. Thread
// (group sg, dim) owns splits sg, sg + 8, ...; the first 64 splits' partial values and every
// split's (m, l) are requested before any reduction, so the block waits for memory about once.
// The partials are written and read with non-temporal hints (each is read exactly once): 15.08 ->
// 14.87 us per C2 layer on MI355X.
template <int D, int RPS, bool DEV = false, int DIMS = kMergeB1Dims>
__global__ __launch_bounds__(kMergeThreads) void verify_attn_merge_kernel(MergeArgs a) {
    constexpr int kGroups = kMergeThreads / DIMS; // split groups per block
    constexpr int kPre = 64 / kGroups;             // the first 64 splits' values loaded up front
    // Ordinary loads of the partials, whichever way they were written (measured on MI355X against
    // non-temporal loads: C3 with cached partials 98.6 -> 98.2 us, C2 13.39 -> 13.37 us per layer).
    const auto ld = [](const float* p) { return *p; };
    __shared__ float wts[kMergeMaxSplits];
    __shared__ float lw[kMergeMaxSplits];
    __shared__ float red[kMergeThreads / 64];
    __shared__ float part[kGroups][DIMS];
    __shared__ int redo_flag;
    if (threadIdx.x == 0) { redo_flag = 0; }
    // Block x serves KV head x % Hkv (B == 1: batches use verify_attn_merge_rows_kernel). Blocks are
    // dealt to the XCDs round-robin, and the batch-1 partial grid runs KV head fastest, so at 8 KV
    // heads a head's partials and the blocks that merge them share an XCD and its L2.
    const int h = static_cast<int>(blockIdx.x) % a.Hkv;
    const int hrow = static_cast<int>(blockIdx.x) / a.Hkv; // t * G + gi
    const int gi = hrow % a.G;
    const int t = hrow / a.G;
    const int b = 0;
    const int qh = h * a.G + gi;
    const int rc = t / a.tokens_per_chunk;
    const int r = (t - rc * a.tokens_per_chunk) * a.G + gi;
    const int nsplit = a.nsplit; // B == 1 (batches use verify_attn_merge_rows_kernel)
    const int64_t slot0 = (static_cast<int64_t>(rc) * a.Hkv + h) * a.split_slots;
    constexpr int rps = RPS; // rows per partial slot (the launch's plan.rows_per_slot)
    const float* ml = a.part_ml + slot0 * (2 * rps);
    const uint16_t* po = a.part_o + slot0 * (rps * D);
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int sg = tid / DIMS;
    const int d = blockIdx.y * DIMS + (tid - sg * DIMS);

    uint32_t pre[kPre]; // FP16 words, converted at use
#pragma unroll
    for (int k = 0; k < kPre; ++k) {
        const int s = sg + kGroups * k;
        pre[k] = s < nsplit ? partial_o_word(po, static_cast<int64_t>(s) * rps * D + r * D + d) : 0u;
    }
    float M = -INFINITY;
    bool redo = false; // a split the fast path could not hold (marked, or non-finite)
    for (int s = tid; s < nsplit; s += kMergeThreads) {
        const float ls = ld(ml + s * (2 * rps) + 2 * r + 1);
        const float ms = ld(ml + s * (2 * rps) + 2 * r);
        redo |= ls < 0.0f || !__builtin_isfinite(ls);
        wts[s] = ls > 0.0f ? ms : -INFINITY;
        lw[s] = ls;
        M = fmaxf(M, wts[s]);
    }
    M = wave_max(M);
    if (lane == 0) { red[wave] = M; }
    __syncthreads();
    M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    float lsum = 0.0f;
    for (int s = tid; s < nsplit; s += kMergeThreads) {
        const float w = (M != -INFINITY && wts[s] != -INFINITY) ? __builtin_amdgcn_exp2f(wts[s] - M) : 0.0f;
        wts[s] = w * lw[s]; // the weight of the split's O / l
        lsum = fmaf(lw[s], w, lsum);
    }
    lsum = wave_sum(lsum);
    if (lane == 0) { red[wave] = lsum; }
    __syncthreads();
    lsum = (red[0] + red[1]) + (red[2] + red[3]);

    // A split with zero weight (no visible key) never wrote its partial rows: skip it rather than
    // multiply whatever the workspace holds by zero.
    float o = 0.0f;
    if (lsum > 0.0f) {
#pragma unroll
        for (int k = 0; k < kPre; ++k) {
            const int s = sg + kGroups * k;
            if (s < nsplit) {
                const float v = partial_o_half(pre[k], d);
                redo |= wts[s] != 0.0f && !__builtin_isfinite(v);
                o = wts[s] != 0.0f ? fmaf(v, wts[s], o) : o;
            }
        }
#pragma unroll 4
        for (int s = sg + kGroups * kPre; s < nsplit; s += kGroups) {
            const float v = partial_o_at(po, static_cast<int64_t>(s) * rps * D + r * D + d);
            redo |= wts[s] != 0.0f && !__builtin_isfinite(v);
            o = wts[s] != 0.0f ? fmaf(v, wts[s], o) : o;
        }
    }
    part[sg][tid - sg * DIMS] = o;
    if (redo) { redo_flag = 1; }
    __syncthreads();
    if (redo_flag != 0 && a.kc != nullptr) {
        // the split weights are no longer needed: their LDS holds the exact path's scratch
        static_assert(D + kExactLds <= kMergeMaxSplits, "exact-path scratch exceeds the weights' LDS");
        // the exact path serves 32 dims per call
#pragma unroll 1
        for (int h32 = 0; h32 < DIMS / 32; ++h32) { merge_row_exact<D, RPS, DEV>(a, b, t, qh, blockIdx.y * DIMS + 32 * h32, wts); }
        return;
    }
    if (tid < DIMS) {
        float acc = 0.0f;
#pragma unroll
        for (int k = 0; k < kGroups; ++k) { acc += part[k][tid]; }
        const float val = lsum > 0.0f ? acc / lsum : 0.0f;
        const int64_t oi = static_cast<int64_t>(D) * (qh + static_cast<int64_t>(a.Hq) * (t + static_cast<int64_t>(a.T) * b)) + d;
        if (a.out_f32) {
            static_cast<float*>(a.out)[oi] = val;
        } else {
            static_cast<uint16_t*>(a.out)[oi] = f32_to_bf16_bits(val);
        }
    }
}

// Batched form of the merge (B > 1, a few splits per sequence): a block serves 8 output rows
// (b, t, qh) x 32 dims, and each thread merges its (row, dim) over the sequence's splits in split
// order with a running log-sum-exp, eight splits' loads in flight. Same result contract as above.
constexpr int kMergeRowsPerBlock = kMergeThreads / kMergeDims;

template <int D>
__global__ __launch_bounds__(kMergeThreads) void verify_attn_merge_rows_kernel(MergeArgs a) {
    __shared__ int redo_flag;
    const int tid = threadIdx.x;
    if (tid == 0) { redo_flag = 0; }
    __syncthreads();
    const int row_id = min(static_cast<int>(blockIdx.x * kMergeRowsPerBlock + tid / kMergeDims), a.B * a.T * a.Hq - 1); // (b, t, qh)
    const bool row_live = static_cast<int>(blockIdx.x * kMergeRowsPerBlock + tid / kMergeDims) < a.B * a.T * a.Hq;
    const int qh = row_id % a.Hq;
    const int t = (row_id / a.Hq) % a.T;
    const int b = row_id / (a.Hq * a.T);
    const int h = qh / a.G;
    const int gi = qh - h * a.G;
    const int rc = t / a.tokens_per_chunk;
    const int r = (t - rc * a.tokens_per_chunk) * a.G + gi;
    const int d = blockIdx.y * kMergeDims + (tid & (kMergeDims - 1));
    const int first = a.seq_table[2 * b];
    const int nsplit = a.seq_table[2 * b + 1];
    const int64_t slot0 = (static_cast<int64_t>(rc) * a.Hkv + h) * a.split_slots + first;
    const int rps = a.rows_per_slot;
    const float* ml = a.part_ml + slot0 * (2 * rps) + 2 * r;
    const uint16_t* po = a.part_o + slot0 * (rps * D) + r * D + (d & ~1); // whole words: d & 1 picks the half
    float M = -INFINITY;
    float lsum = 0.0f;
    float o = 0.0f;
    bool redo = false; // a split the fast path could not hold (marked, or non-finite)
    constexpr int kBatch = 8;
#pragma unroll 1
    for (int s0 = 0; s0 < nsplit; s0 += kBatch) {
        float2 mlv[kBatch];
        uint32_t ow[kBatch]; // FP16 words, converted at use
#pragma unroll
        for (int k = 0; k < kBatch; ++k) {
            const int s = s0 + k;
            mlv[k] = s < nsplit ? *reinterpret_cast<const float2*>(ml + static_cast<int64_t>(s) * (2 * rps)) : float2{-INFINITY, 0.0f};
            ow[k] = s < nsplit ? partial_o_word(po, static_cast<int64_t>(s) * rps * D + (d & 1)) : 0u;
        }
#pragma unroll
        for (int k = 0; k < kBatch; ++k) {
            const float ov = partial_o_half(ow[k], d);
            redo |= s0 + k < nsplit && (mlv[k].y < 0.0f || !__builtin_isfinite(mlv[k].y) ||
                                        (mlv[k].y > 0.0f && !__builtin_isfinite(ov)));
            // A split with no visible key never wrote its partial rows: skip it.
            if (!(mlv[k].y > 0.0f)) { continue; }
            const float mn = fmaxf(M, mlv[k].x);
            const float alpha = M == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(M - mn);
            const float beta = __builtin_amdgcn_exp2f(mlv[k].x - mn);
            o = fmaf(o, alpha, ov * (mlv[k].y * beta));
            lsum = fmaf(lsum, alpha, mlv[k].y * beta);
            M = mn;
        }
    }
    if (redo && row_live) { redo_flag = 1; }
    __syncthreads();
    if (redo_flag != 0 && a.kc != nullptr) {
        // the workgroup's rows one after another, exactly
        __shared__ float xs[D + kExactLds];
        for (int k = 0; k < kMergeRowsPerBlock; ++k) {
            const int rid = static_cast<int>(blockIdx.x) * kMergeRowsPerBlock + k;
            if (rid >= a.B * a.T * a.Hq) { break; }
            merge_row_exact<D, 0>(a, rid / (a.Hq * a.T), (rid / a.Hq) % a.T, rid % a.Hq, blockIdx.y * kMergeDims, xs);
        }
        return;
    }
    if (!row_live) { return; }
    const float val = lsum > 0.0f ? o / lsum : 0.0f;
    const int64_t oi = static_cast<int64_t>(D) * (qh + static_cast<int64_t>(a.Hq) * (t + static_cast<int64_t>(a.T) * b)) + d;
    if (a.out_f32) {
        static_cast<float*>(a.out)[oi] = val;
    } else {
        static_cast<uint16_t*>(a.out)[oi] = f32_to_bf16_bits(val);
    }
}

// INT8-G64 encoder for A2, the prefix commit and multi-row-chunk A1 (reference contract
// include/ninfer/ops/gqa_attention.h:25-30; device encoder
// src/ops/kernel/gqa_attention_decode_i8.cuh:168-209). Block (t, b, h): one wave per (K|V, group),
// lane i owns element i of the 64-element group.
template <int D>
__global__ __launch_bounds__(256) void kv_quant_append_kernel(const uint16_t* k, const uint16_t* v,
                                                              const int32_t* positions,
                                                              const int32_t* count, CommitBounds cb,
                                                              int32_t T, int32_t Hkv, int32_t P,
                                                              int8_t* kc, int8_t* vc, uint16_t* ks,
                                                              uint16_t* vs, int64_t code_seq,
                                                              int64_t scale_seq) {
    constexpr int G = D / 64;
    const int t = blockIdx.x;
    const int b = blockIdx.y;
    const int h = blockIdx.z;
    if (count != nullptr) {
        const int n = count[b];
        if (n < cb.min_count || n > cb.max_count || t >= n) { return; }
    }
    const int lane = threadIdx.x & 63;
    const int p = positions[static_cast<int64_t>(b) * T + t];
    if (p < 0) { return; }
    const int pos = p & cb.slot_mask;
    if (pos >= P) { return; }
    for (int unit = threadIdx.x >> 6; unit < 2 * G; unit += blockDim.x / 64) {
        const int which = unit / G;
        const int grp = unit - which * G;
        const uint16_t* src = (which ? v : k) + static_cast<int64_t>(D) * (h + static_cast<int64_t>(Hkv) * (t + static_cast<int64_t>(T) * b)) + grp * 64;
        const float x = bf16_to_f32(src[lane]);
        const float amax = wave_max(fabsf(x));
        const uint16_t sbits = f32_to_f16_bits(amax > 0.0f ? amax / 127.0f : 0.0f);
        const float s = f16_bits_to_f32(sbits);
        const float inv = s > 0.0f ? 1.0f / s : 0.0f;
        int8_t code = 0;
        if (inv != 0.0f) {
            float rr = rintf(x * inv);
            rr = fminf(127.0f, fmaxf(-127.0f, rr));
            code = static_cast<int8_t>(rr);
        }
        int8_t* cdst = (which ? vc : kc) + static_cast<int64_t>(b) * code_seq + static_cast<int64_t>(D) * (pos + static_cast<int64_t>(P) * h) + grp * 64;
        cdst[lane] = code;
        if (lane == 0) {
            uint16_t* sdst = (which ? vs : ks) + static_cast<int64_t>(b) * scale_seq + static_cast<int64_t>(G) * (pos + static_cast<int64_t>(P) * h) + grp;
            *sdst = sbits;
        }
    }
}

// BF16 cache append (A2, and A1 on a BF16 cache): column t of sequence b is copied bit for bit into
// row positions[t] (reference gqa_kv_append on a BF16 cache). Block (t, b, h).
__global__ __launch_bounds__(64) void bf16_kv_append_kernel(const uint16_t* k, const uint16_t* v, const int32_t* positions,
                                                            const int32_t* count, CommitBounds cb, int32_t T,
                                                            int32_t Hkv, int32_t P, int32_t D, uint16_t* kb,
                                                            uint16_t* vb, int64_t seq) {
    const int t = blockIdx.x;
    const int b = blockIdx.y;
    const int h = blockIdx.z;
    if (count != nullptr) {
        const int n = count[b];
        if (n < cb.min_count || n > cb.max_count || t >= n) { return; }
    }
    const int p = positions[static_cast<int64_t>(b) * T + t];
    if (p < 0) { return; }
    const int pos = p & cb.slot_mask;
    if (pos >= P) { return; }
    const int64_t src = static_cast<int64_t>(D) * (h + static_cast<int64_t>(Hkv) * (t + static_cast<int64_t>(T) * b));
    const int64_t dst = static_cast<int64_t>(b) * seq + static_cast<int64_t>(D) * (pos + static_cast<int64_t>(P) * h);
    for (int i = threadIdx.x; i < D / 8; i += blockDim.x) {
        *reinterpret_cast<i4*>(kb + dst + 8 * i) = *reinterpret_cast<const i4*>(k + src + 8 * i);
        *reinterpret_cast<i4*>(vb + dst + 8 * i) = *reinterpret_cast<const i4*>(v + src + 8 * i);
    }
}

} // namespace

namespace {

// Splits per (sequence, row chunk, KV head) a batch-1 plan aims for: about 512 workgroups at
// head_dim 128 (two per CU), 256 at head_dim 256 (its LDS map holds one workgroup per CU).
// Rows of one row chunk and the resident workgroups a plan aims at: 32 rows (two 16-row tiles) and
// two workgroups per CU; the wide form takes up to 80 rows (five tiles) in one chunk and one
// workgroup per CU.
struct RowForm {
    bool wide;
    int32_t per_chunk; // tokens per row chunk
    int64_t target;    // resident workgroups
};

// Split lengths of 1,024 keys or more that are powers of two get one more 128-key step: the
// workgroups of a launch stream at one split-length stride from each other, and a power-of-two
// stride in a physically contiguous plane lands their concurrent reads on the same memory channels.
// Measured on MI355X at C3 (4,096 -> 4,224 keys): the layers whose planes were placed contiguously
// ran at 110-125 us against 97-100 us for the others; with 4,224 keys all eight take 97-100 us.
int64_t off_power_of_two(int64_t kps) { return (kps >= 1024 && (kps & (kps - 1)) == 0) ? kps + 128 : kps; }

RowForm row_form(int32_t Hq, int32_t Hkv, int32_t D, int32_t T, bool wide_rows) {
    const int32_t G = Hq / Hkv;
    const bool wide = wide_rows && D == 128 && static_cast<int64_t>(T) * G > kAttnRowsPerTile &&
                      static_cast<int64_t>(T) * G <= kAttnWideRows;
    RowForm f;
    f.wide = wide;
    f.per_chunk = wide ? T : std::min<int32_t>(std::max<int32_t>(1, kAttnRowsPerTile / G), T);
    f.target = (D == 128 && !wide) ? kAttnTargetWorkgroups : kAttnTargetWorkgroups / 2;
    return f;
}

int64_t wanted_splits(int32_t Hq, int32_t Hkv, int32_t D, int32_t T, int32_t B, bool wide_rows) {
    const RowForm f = row_form(Hq, Hkv, D, T, wide_rows);
    const int64_t row_chunks = (T + f.per_chunk - 1) / f.per_chunk;
    const int64_t units = static_cast<int64_t>(Hkv) * B * row_chunks;
    return std::max<int64_t>(1, (f.target + units - 1) / units);
}

} // namespace

SplitPlan plan_attention(int32_t Hq, int32_t Hkv, int32_t D, int32_t T, int32_t B,
                         uint32_t max_visible_keys, bool wide_rows) {
    SplitPlan p;
    const RowForm f = row_form(Hq, Hkv, D, T, wide_rows);
    p.G = Hq / Hkv;
    p.tokens_per_chunk = f.per_chunk;
    p.row_chunks = (T + p.tokens_per_chunk - 1) / p.tokens_per_chunk;
    p.rows_per_slot = f.wide ? kAttnWideRows : kAttnRowsPerTile;
    const int64_t want = wanted_splits(Hq, Hkv, D, T, B, wide_rows);
    // B > 1: the device cuts the batch's actual keys into at most split_budget splits per (row
    // chunk, KV head), sized so that every split workgroup is resident at once.
    const int64_t cols = static_cast<int64_t>(Hkv) * p.row_chunks;
    p.split_budget = static_cast<int32_t>(std::max<int64_t>(1, f.target / cols));
    int64_t kps = (static_cast<int64_t>(max_visible_keys) + want - 1) / want;
    kps = ((kps + 127) / 128) * 128;
    kps = std::max<int64_t>(kps, kAttnMinKeysPerSplit);
    kps = off_power_of_two(kps);
    int64_t nsplit = std::max<int64_t>(1, (static_cast<int64_t>(max_visible_keys) + kps - 1) / kps);
    if (B == 1 && f.target == kAttnTargetWorkgroups) {
        // Between one and 1.75 workgroups per CU, the CUs that hold two splits stream twice the
        // keys of the others and set the layer's time. The fewest splits that fit one workgroup
        // per CU are taken instead when their longest CU streams fewer keys (an envelope of 9,732
        // keys at 8 KV heads: 39 splits of 256 keys = 312 workgroups become 26 of 384). Only the
        // two-per-CU forms: their largest plan (wanted_splits() x 256 keys, at least 512
        // workgroups) is never one of these, so attention_workspace_bound() stays exact.
        const int64_t cus = kAttnTargetWorkgroups / 2;
        const int64_t wgs = cols * nsplit;
        const auto deepest = [&](int64_t n, int64_t k) { return (cols * n + cus - 1) / cus * k; };
        if (wgs > cus && wgs * 4 < cus * 7 && cols <= cus) {
            const int64_t per_col = cus / cols;
            int64_t k1 = (static_cast<int64_t>(max_visible_keys) + per_col - 1) / per_col;
            k1 = off_power_of_two(std::max<int64_t>(((k1 + 127) / 128) * 128, kAttnMinKeysPerSplit));
            const int64_t n1 = std::max<int64_t>(1, (static_cast<int64_t>(max_visible_keys) + k1 - 1) / k1);
            if (deepest(n1, k1) < deepest(nsplit, kps)) {
                kps = k1;
                nsplit = n1;
            }
        }
    }
    p.keys_per_split = static_cast<int32_t>(kps);
    p.nsplit = static_cast<int32_t>(nsplit);
    p.split_slots = B == 1 ? p.nsplit : std::max(p.split_budget, B);
    // INT8 caches (the only ones offered the wide form) at head_dim 128 with one row chunk.
    p.cached_partials = B == 1 && wide_rows && D == 128 && !f.wide && p.row_chunks == 1 &&
                        p.keys_per_split >= kAttnCachedPartialKeys;
    const size_t part_units = static_cast<size_t>(cols) * p.split_slots;
    p.part_o_offset = 0;
    const size_t o_bytes = part_units * p.rows_per_slot * static_cast<size_t>(D) * sizeof(uint16_t); // FP16 O / l
    p.part_ml_offset = (o_bytes + 255) & ~static_cast<size_t>(255);
    const size_t ml_bytes = part_units * 2 * p.rows_per_slot * sizeof(float);
    p.seq_table_offset = (p.part_ml_offset + ml_bytes + 255) & ~static_cast<size_t>(255);
    const size_t table_bytes = static_cast<size_t>(B) * 2 * sizeof(int32_t);
    p.bytes = ((p.seq_table_offset + table_bytes + 255) & ~static_cast<size_t>(255));
    return p;
}

void choose_b1_device_plan(SplitPlan& p, int32_t B, uint32_t min_visible_keys, bool int8_cache) {
    // An envelope whose shortest window would leave more than half of the plan's splits empty
    // (a graph replayed from a short context up to a long envelope) splits each window on the
    // device instead. The INT8 batch-1 kernel of one or two row tiles serves it; its speculative
    // first chunks then wait for the positions.
    const int64_t live_at_min = (std::max<int64_t>(min_visible_keys, 1) + p.keys_per_split - 1) / p.keys_per_split;
    p.b1_device_plan = B == 1 && int8_cache && p.rows_per_slot == kAttnRowsPerTile && live_at_min * 2 < p.nsplit;
}

size_t attention_workspace_bound(int32_t Hq, int32_t Hkv, int32_t D, int32_t T) {
    // A batch-1 plan never has more than wanted_splits() splits (at least that many keys per split
    // cover any context), and it reaches that count once every split holds the minimum 256 keys.
    size_t bound = 0;
    for (const bool wide : {false, true}) {
        const int64_t want = wanted_splits(Hq, Hkv, D, T, 1, wide);
        bound = std::max(bound, plan_attention(Hq, Hkv, D, T, 1, static_cast<uint32_t>(want * kAttnMinKeysPerSplit), wide).bytes);
    }
    return bound;
}

void launch_kv_append(const uint16_t* k, const uint16_t* v, const int32_t* positions,
                      const int32_t* count, CommitBounds bounds, int32_t T, const CacheRef& c,
                      hipStream_t stream) {
    dim3 grid(T, c.B, c.Hkv);
    if (c.kb != nullptr) {
        hipLaunchKernelGGL(bf16_kv_append_kernel, grid, dim3(64), 0, stream, k, v, positions, count, bounds, T, c.Hkv,
                           c.P, c.D, c.kb, c.vb, c.code_seq);
        check_launch("bf16_kv_append_kernel");
        return;
    }
    if (c.D == 128) {
        hipLaunchKernelGGL(kv_quant_append_kernel<128>, grid, dim3(256), 0, stream, k, v, positions,
                           count, bounds, T, c.Hkv, c.P, c.kc, c.vc, c.ks, c.vs, c.code_seq, c.scale_seq);
    } else if (c.D == 256) {
        hipLaunchKernelGGL(kv_quant_append_kernel<256>, grid, dim3(256), 0, stream, k, v, positions,
                           count, bounds, T, c.Hkv, c.P, c.kc, c.vc, c.ks, c.vs, c.code_seq, c.scale_seq);
    } else {
        throw Unsupported("kv append: head_dim 128 and 256 are built");
    }
    check_launch("kv_quant_append_kernel");
}

void launch_verify_attention(const uint16_t* q, const uint16_t* k_new, const uint16_t* v_new,
                             const int32_t* positions, const int32_t* parents, int32_t T,
                             int32_t Hq, const CacheRef& c, float scale, uint32_t max_keys,
                             void* workspace, const SplitPlan& plan, void* out, bool out_f32,
                             hipStream_t stream) {
    if (c.D != 128 && c.D != 256) { throw Unsupported("verify attention: head_dim 128 and 256 are built"); }
    if (plan.rows_per_slot != kAttnRowsPerTile && (c.kb != nullptr || c.D != 128 || plan.row_chunks != 1)) {
        throw Unsupported("verify attention: the 80-row form serves INT8 caches of head_dim 128 only");
    }
    if (plan.split_slots > kMergeMaxSplits) { throw Unsupported("verify attention: too many key splits"); }
    if (k_new != nullptr && (plan.row_chunks > 1 || (c.kb != nullptr && c.D != 128))) {
        // Several row-chunk workgroups read the new rows, or a BF16 cache of head_dim 256 (no room
        // for a new-row stage): write them in a launch of their own.
        launch_kv_append(k_new, v_new, positions, nullptr, CommitBounds{}, T, c, stream);
        k_new = nullptr;
        v_new = nullptr;
    }
    char* ws = static_cast<char*>(workspace);
    AttnArgs a{};
    a.q = q;
    a.k_new = k_new;
    a.v_new = v_new;
    a.positions = positions;
    a.parents = parents;
    a.kc = c.kc;
    a.vc = c.vc;
    a.kb = c.kb;
    a.vb = c.vb;
    a.ks = c.ks;
    a.vs = c.vs;
    a.part_o = reinterpret_cast<uint16_t*>(ws + plan.part_o_offset);
    a.part_ml = reinterpret_cast<float*>(ws + plan.part_ml_offset);
    a.seq_table = reinterpret_cast<int32_t*>(ws + plan.seq_table_offset);
    a.code_seq = c.code_seq;
    a.scale_seq = c.scale_seq;
    a.P = c.P;
    a.T = T;
    a.Hq = Hq;
    a.Hkv = c.Hkv;
    a.G = plan.G;
    a.tokens_per_chunk = plan.tokens_per_chunk;
    a.row_chunks = plan.row_chunks;
    a.nsplit = plan.nsplit;
    a.kps = plan.keys_per_split;
    a.B = c.B;
    a.split_slots = plan.split_slots;
    a.split_budget = plan.split_budget;
    a.max_keys = static_cast<int32_t>(max_keys);
    a.scale_log2 = scale * 1.4426950408889634f;
    // One row chunk: every key is read by exactly one workgroup (non-temporal DMAs).
    const bool once = plan.row_chunks == 1;
    const int rows = plan.tokens_per_chunk * plan.G;
    const dim3 grid_split_major(plan.split_slots, c.Hkv, plan.row_chunks);
    // the batch-1 paths (BF16, and INT8 of up to two row tiles) take (KV head, split, row chunk)
    const dim3 grid_b1(c.Hkv, plan.split_slots, plan.row_chunks);
    dim3 grid = grid_split_major;
#define NMI_PARTIAL(KERNEL, NT, D)                                                                             \
    if (once) {                                                                                               \
        hipLaunchKernelGGL((KERNEL<NT, D, true>), grid, dim3(256), 0, stream, a);                            \
    } else {                                                                                                  \
        hipLaunchKernelGGL((KERNEL<NT, D, false>), grid, dim3(256), 0, stream, a);                           \
    }
    // INT8 cache, up to two row tiles: the host plan, or the batch-1 plan split on the device
#define NMI_PARTIAL_I8(NT, D, ONCE, CACHED)                                                                   \
    if (dev) {                                                                                                \
        hipLaunchKernelGGL((verify_attn_partial_kernel<NT, D, ONCE, CACHED, true>), grid, dim3(256), 0, stream, a); \
    } else {                                                                                                  \
        hipLaunchKernelGGL((verify_attn_partial_kernel<NT, D, ONCE, CACHED>), grid, dim3(256), 0, stream, a); \
    }
#define NMI_PARTIAL_I8_ONCE(NT, D)                                                                            \
    if (once) {                                                                                               \
        NMI_PARTIAL_I8(NT, D, true, false)                                                                    \
    } else {                                                                                                  \
        NMI_PARTIAL_I8(NT, D, false, false)                                                                   \
    }
    const bool dev = plan.b1_device_plan;
    if (c.kb != nullptr) {
        if (c.B == 1) { grid = grid_b1; }
        if (c.D == 128) {
            if (rows <= 16) {
                NMI_PARTIAL(verify_attn_partial_bf16_kernel, 1, 128)
            } else {
                NMI_PARTIAL(verify_attn_partial_bf16_kernel, 2, 128)
            }
        } else if (rows <= 16) {
            NMI_PARTIAL(verify_attn_partial_bf16_kernel, 1, 256)
        } else {
            NMI_PARTIAL(verify_attn_partial_bf16_kernel, 2, 256)
        }
    } else if (c.D == 128) {
        if (plan.rows_per_slot != kAttnWideRows && c.B == 1) { grid = grid_b1; }
        if (plan.rows_per_slot == kAttnWideRows) {
            NMI_PARTIAL(verify_attn_partial_kernel, 5, 128)
        } else if (plan.cached_partials && rows <= 16) {
            NMI_PARTIAL_I8(1, 128, true, true)
        } else if (plan.cached_partials) {
            NMI_PARTIAL_I8(2, 128, true, true)
        } else if (rows <= 16) {
            NMI_PARTIAL_I8_ONCE(1, 128)
        } else {
            NMI_PARTIAL_I8_ONCE(2, 128)
        }
    } else {
        if (c.B == 1) { grid = grid_b1; }
        if (rows <= 16) {
            NMI_PARTIAL_I8_ONCE(1, 256)
        } else {
            NMI_PARTIAL_I8_ONCE(2, 256)
        }
    }
#undef NMI_PARTIAL_I8_ONCE
#undef NMI_PARTIAL_I8
#undef NMI_PARTIAL
    check_launch("verify_attn_partial_kernel");

    MergeArgs mg{};
    mg.part_o = a.part_o;
    mg.part_ml = a.part_ml;
    mg.out = out;
    mg.T = T;
    mg.Hq = Hq;
    mg.Hkv = c.Hkv;
    mg.G = plan.G;
    mg.tokens_per_chunk = plan.tokens_per_chunk;
    mg.row_chunks = plan.row_chunks;
    mg.nsplit = plan.nsplit;
    mg.seq_table = a.seq_table;
    mg.B = c.B;
    mg.split_slots = plan.split_slots;
    mg.rows_per_slot = plan.rows_per_slot;
    mg.out_f32 = out_f32 ? 1 : 0;
    mg.q = q;
    mg.positions = positions;
    mg.parents = parents;
    mg.kc = c.kc;
    mg.vc = c.vc;
    mg.ks = c.ks;
    mg.vs = c.vs;
    mg.code_seq = c.code_seq;
    mg.scale_seq = c.scale_seq;
    mg.P = c.P;
    mg.kps = plan.keys_per_split;
    mg.max_keys = static_cast<int32_t>(max_keys);
    mg.split_budget = plan.split_budget;
    mg.fused = k_new != nullptr ? 1 : 0;
    mg.scale_log2 = a.scale_log2;
    const dim3 rows_grid((c.B * T * Hq + kMergeRowsPerBlock - 1) / kMergeRowsPerBlock, c.D / kMergeDims);
    if (c.B > 1 && c.D == 128) {
        hipLaunchKernelGGL(verify_attn_merge_rows_kernel<128>, rows_grid, dim3(kMergeThreads), 0, stream, mg);
    } else if (c.B > 1) {
        hipLaunchKernelGGL(verify_attn_merge_rows_kernel<256>, rows_grid, dim3(kMergeThreads), 0, stream, mg);
    } else if (c.D == 128 && plan.rows_per_slot == kAttnWideRows) {
        hipLaunchKernelGGL((verify_attn_merge_kernel<128, kAttnWideRows>), dim3(c.B * T * Hq, 128 / kMergeB1Dims), dim3(kMergeThreads), 0, stream, mg);
    } else if (c.D == 128 && dev) {
        hipLaunchKernelGGL((verify_attn_merge_kernel<128, kAttnRowsPerTile, true>), dim3(c.B * T * Hq, 128 / kMergeB1Dims), dim3(kMergeThreads), 0, stream, mg);
    } else if (c.D == 128) {
        hipLaunchKernelGGL((verify_attn_merge_kernel<128, kAttnRowsPerTile>), dim3(c.B * T * Hq, 128 / kMergeB1Dims), dim3(kMergeThreads), 0, stream, mg);
    } else if (dev) {
        hipLaunchKernelGGL((verify_attn_merge_kernel<256, kAttnRowsPerTile, true>), dim3(c.B * T * Hq, 256 / kMergeB1Dims), dim3(kMergeThreads), 0, stream, mg);
    } else {
        hipLaunchKernelGGL((verify_attn_merge_kernel<256, kAttnRowsPerTile>), dim3(c.B * T * Hq, 256 / kMergeB1Dims), dim3(kMergeThreads), 0, stream, mg);
    }
    check_launch("verify_attn_merge_kernel");
}

} // namespace nmi
