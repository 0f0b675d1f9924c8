// Verify attention for the MTP speculative-decoding step on gfx950.
//
// Semantics (reference include/ninfer/ops/gqa_attention.h:52-91): for sequence b, query token t
// and query head qh (KV head h = qh / G), attend over cache rows [0, positions[0]) plus the new
// rows positions[u] with u visible from t (u <= t causal; u an ancestor-or-self of t for trees),
// reading INT8-G64 codes with FP16 scales. A1 first quantizes the new K/V columns into their rows
// (the split owning a row writes it, as the reference's decode kernel does,
// src/ops/kernel/gqa_attention_decode_i8.cuh:168-209). Split-K over keys with an online softmax
// per split and a log-sum-exp merge (reference reducer src/ops/kernel/gqa_attention_decode.cuh:
// 144-227).
//
// MI355X design:
//  * One workgroup = 4 waves = one (sequence, row chunk, KV head, key split); 2 workgroups per CU.
//    Each wave streams 32-key chunks (chunk w, w+4, ...). A chunk (K codes, V codes, FP16 scales:
//    8,448 bytes) moves HBM -> LDS by asynchronous global_load_lds DMA into a per-wave two-stage
//    ring with a lookahead of two chunks: 16.5 KB per wave, 132 KB per CU stay in flight while
//    the current chunk is computed, at no VGPR cost.
//  * QK^T runs as S^T = K * Q^T on v_mfma_f32_16x16x32_f16: K codes (exact in FP16) are the A
//    operand, Q (BF16 -> FP16 exact after a per-row power-of-two rescale) the B operand. Each
//    32-dim MFMA step stays inside one 64-wide quant group and each group accumulates separately,
//    so the per-(key, group) FP16 scale is applied exactly in FP32. The K DMA writes LDS in MFMA
//    operand order, so every lane reads its own 16 bytes (conflict-free ds_read_b128).
//  * PV runs as O^T = V^T * P^T on the same instruction. The S^T accumulator layout (lane = query
//    row, 4 keys per 16-key tile) is exactly the B-operand layout of P^T, so probabilities never
//    leave registers. V rows land in LDS in their natural layout; each lane reads 8 bytes of 8 keys
//    (dims 8c..8c+7) and transposes in registers with SDWA converts.
//  * GQA x q_len rows (5 x 4 = 20 for the 40/8 geometry) are padded to two 16-row MFMA tiles.
#include "common.h"
#include "device_utils.h"
#include "ops_internal.h"

#include <algorithm>
#include <cmath>

#define NMI_AS1 __attribute__((address_space(1)))
#define NMI_AS3 __attribute__((address_space(3)))

namespace nmi {
namespace {

constexpr int kWaves = 4;
constexpr int kChunk = 32;
constexpr int kStageK = 0;       // 4 x 1 KB, MFMA operand order
constexpr int kStageV = 4096;    // 32 rows x 128 B, natural order
constexpr int kStageS = 8192;    // 32 K scale words then 32 V scale words
constexpr int kStageBytes = 8448;
constexpr int kSmemBytes = kWaves * 2 * kStageBytes; // 67,584 B; the epilogue merge reuses it

typedef _Float16 h2 __attribute__((ext_vector_type(2)));

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
    float* part_o;  // [unit][nsplit][32][D]
    float* part_ml; // [unit][nsplit][32][2]
    int64_t code_seq;
    int64_t scale_seq;
    int32_t P;
    int32_t T;
    int32_t Hq;
    int32_t Hkv;
    int32_t G;
    int32_t tokens_per_chunk;
    int32_t row_chunks;
    int32_t nsplit;
    int32_t kps;
    int32_t max_keys; // envelope max_visible_keys (<= max_context <= P): clamps device positions
    float scale_log2; // softmax scale * log2(e)
};

// Visibility of new node u (0 <= u < T) from query token t, as a bitmask over u.
__device__ __forceinline__ uint32_t new_key_mask(const int32_t* parents, int32_t t) {
    if (parents == nullptr) { return t >= 31 ? 0xffffffffu : ((2u << t) - 1u); }
    uint32_t m = 0;
    int32_t u = t;
#pragma unroll 1
    for (int guard = 0; guard < 32 && u >= 0 && u < 32; ++guard) {
        m |= 1u << u;
        u = parents[u];
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

// Byte (T & 3) of word (T >> 2) from key slots 2w and 2w+1 -> packed FP16 pair (V transpose).
template <int T>
__device__ __forceinline__ uint32_t v_pair(const i2& a, const i2& b) {
    return i8x2_to_f16x2<T & 3>(static_cast<uint32_t>(a[T >> 2]), static_cast<uint32_t>(b[T >> 2]));
}

__device__ __forceinline__ _Float16 half_bits_at(const i4& v, int idx) {
    const uint32_t word = static_cast<uint32_t>(v[idx >> 1]);
    return __builtin_bit_cast(_Float16, static_cast<uint16_t>((idx & 1) ? (word >> 16) : (word & 0xffffu)));
}

// Issue the DMA of one 32-key chunk (the caller guarantees c0 + 32 <= P) into `stage`.
__device__ __forceinline__ void issue_chunk(NMI_AS3 char* stage, const int8_t* kbase, const int8_t* vbase,
                                            const uint16_t* ksbase, const uint16_t* vsbase, int c0,
                                            int lane) {
    const int c = lane & 15;
    const int g = lane >> 4;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
        for (int gq = 0; gq < 2; ++gq) {
            const int8_t* src = kbase + static_cast<int64_t>(c0 + 16 * kt + c) * 128 + 64 * gq + 16 * g;
            __builtin_amdgcn_global_load_lds((const NMI_AS1 void*)src, (NMI_AS3 void*)(stage + kStageK + (2 * kt + gq) * 1024), 16, 0, 0);
        }
    }
#pragma unroll
    for (int r8 = 0; r8 < 4; ++r8) {
        const int8_t* src = vbase + static_cast<int64_t>(c0 + 8 * r8 + (lane >> 3)) * 128 + 16 * (lane & 7);
        __builtin_amdgcn_global_load_lds((const NMI_AS1 void*)src, (NMI_AS3 void*)(stage + kStageV + r8 * 1024), 16, 0, 0);
    }
    const uint16_t* ssrc = (lane < 32 ? ksbase + static_cast<int64_t>(c0 + lane) * 2 : vsbase + static_cast<int64_t>(c0 + lane - 32) * 2);
    __builtin_amdgcn_global_load_lds((const NMI_AS1 void*)ssrc, (NMI_AS3 void*)(stage + kStageS), 4, 0, 0);
}

// Quantize-append one new token row of one KV head (one wave: lane owns dims lane and lane + 64 of
// K and V), reference contract include/ninfer/ops/gqa_attention.h:25-30.
__device__ __forceinline__ void append_row(const uint16_t* ksrc, const uint16_t* vsrc, int8_t* kdst,
                                           int8_t* vdst, uint16_t* ksdst, uint16_t* vsdst, int lane) {
    const float x[4] = {bf16_to_f32(ksrc[lane]), bf16_to_f32(ksrc[64 + lane]), bf16_to_f32(vsrc[lane]),
                        bf16_to_f32(vsrc[64 + lane])};
    uint16_t sbits[4];
    int8_t code[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float amax = wave_max(fabsf(x[i]));
        sbits[i] = f32_to_f16_bits(amax > 0.0f ? amax / 127.0f : 0.0f);
        const float s = f16_bits_to_f32(sbits[i]);
        const float inv = s > 0.0f ? 1.0f / s : 0.0f;
        float r = inv != 0.0f ? rintf(x[i] * inv) : 0.0f;
        r = fminf(127.0f, fmaxf(-127.0f, r));
        code[i] = static_cast<int8_t>(r);
    }
    kdst[lane] = code[0];
    kdst[64 + lane] = code[1];
    vdst[lane] = code[2];
    vdst[64 + lane] = code[3];
    if (lane == 0) {
        *reinterpret_cast<uint32_t*>(ksdst) = static_cast<uint32_t>(sbits[0]) | (static_cast<uint32_t>(sbits[1]) << 16);
        *reinterpret_cast<uint32_t*>(vsdst) = static_cast<uint32_t>(sbits[2]) | (static_cast<uint32_t>(sbits[3]) << 16);
    }
}

template <int NT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void verify_attn_partial_kernel(AttnArgs a) {
    constexpr int D = 128;
    constexpr int G = 2;       // quant groups per row
    constexpr int DT = D / 16; // O^T tiles of 16 dims
    __shared__ __attribute__((aligned(16))) char smem[kSmemBytes];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int c = lane & 15;
    const int g = lane >> 4;
    const int split = blockIdx.x;
    const int h = blockIdx.y;
    const int b = blockIdx.z / a.row_chunks;
    const int rc = blockIdx.z - b * a.row_chunks;
    const int k0 = split * a.kps;

    const int64_t head_code = static_cast<int64_t>(b) * a.code_seq + static_cast<int64_t>(h) * a.P * D;
    const int64_t head_scale = static_cast<int64_t>(b) * a.scale_seq + static_cast<int64_t>(h) * a.P * G;
    int8_t* kbase = a.kc + head_code;
    int8_t* vbase = a.vc + head_code;
    uint16_t* ksbase = a.ks + head_scale;
    uint16_t* vsbase = a.vs + head_scale;
    NMI_AS3 char* my_stage0 = (NMI_AS3 char*)smem + wave * 2 * kStageBytes;

    // The first chunk does not depend on the positions: start its DMA right away.
    const int first = k0 + kChunk * wave;
    if (first + kChunk <= a.P) { issue_chunk(my_stage0, kbase, vbase, ksbase, vsbase, first, lane); }

    const int32_t* pos = a.positions + static_cast<int64_t>(b) * a.T;
    const int32_t* par = a.parents ? a.parents + static_cast<int64_t>(b) * a.T : nullptr;
    const int window = min(pos[a.T - 1] + 1, a.max_keys);
    const int L = max(0, min(pos[0], window));
    const int t0 = rc * a.tokens_per_chunk;
    const int Tc = min(a.tokens_per_chunk, a.T - t0);
    const int R = Tc * a.G;
    const int k1 = min(k0 + a.kps, window);
    const int64_t unit = (static_cast<int64_t>(b) * a.row_chunks + rc) * a.Hkv + h;
    const int64_t pidx = unit * a.nsplit + split;
    float* out_o = a.part_o + pidx * (32 * D);
    float* out_ml = a.part_ml + pidx * 64;

    // ---- fused A1 append: this split writes the new rows inside [k0, k0 + kps). Only launched
    // with a single row chunk, so no other workgroup reads these rows concurrently.
    if (a.k_new != nullptr) {
        bool owner = false;
        for (int t = 0; t < a.T; ++t) {
            const int p = pos[t];
            const bool mine = p >= k0 && p < k0 + a.kps && p >= 0 && p < a.P;
            owner |= mine;
            if (mine && (t & (kWaves - 1)) == wave) {
                const int64_t src = static_cast<int64_t>(D) * (h + static_cast<int64_t>(a.Hkv) * (t + static_cast<int64_t>(a.T) * b));
                append_row(a.k_new + src, a.v_new + src, kbase + static_cast<int64_t>(p) * D,
                           vbase + static_cast<int64_t>(p) * D, ksbase + static_cast<int64_t>(p) * G,
                           vsbase + static_cast<int64_t>(p) * G, lane);
            }
        }
        if (owner) {
            // Stores visible (and this CU's L1 invalidated) before any DMA of the new rows.
            __threadfence();
            __syncthreads();
            if (first + kChunk <= a.P && first < pos[a.T - 1] + 1 && first + kChunk > pos[0]) {
                issue_chunk(my_stage0, kbase, vbase, ksbase, vsbase, first, lane); // re-fetch
            }
        }
    }

    if (k0 >= k1) {
        __builtin_amdgcn_s_waitcnt(0);
        if (threadIdx.x < 32) {
            out_ml[2 * threadIdx.x] = -INFINITY;
            out_ml[2 * threadIdx.x + 1] = 0.0f;
        }
        return;
    }

    // ---- Q operand: rows r = 16*nt + c; dims d = 64*gq + 16*g + 8*s + e.
    h8 qop[NT][G][2];
    float rowmul[NT];
    uint32_t nmask[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        const int r = 16 * nt + c;
        const bool valid = r < R;
        const int tl = valid ? r / a.G : 0;
        const int gi = valid ? r - tl * a.G : 0;
        const int t = t0 + tl;
        const int qh = h * a.G + gi;
        const uint16_t* qrow = a.q + static_cast<int64_t>(D) * (qh + static_cast<int64_t>(a.Hq) * (t + static_cast<int64_t>(a.T) * b));
        float x[G][2][8];
        float amax = 0.0f;
#pragma unroll
        for (int gq = 0; gq < G; ++gq) {
#pragma unroll
            for (int s = 0; s < 2; ++s) {
                const i4 raw = valid ? *reinterpret_cast<const i4*>(qrow + 64 * gq + 16 * g + 8 * s) : i4{0, 0, 0, 0};
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int w = raw[e >> 1];
                    const uint16_t bits = static_cast<uint16_t>((e & 1) ? (static_cast<uint32_t>(w) >> 16) : (static_cast<uint32_t>(w) & 0xffffu));
                    x[gq][s][e] = bf16_to_f32(bits);
                    amax = fmaxf(amax, fabsf(x[gq][s][e]));
                }
            }
        }
        amax = group4_max(amax);
        // factor = 2^(14 - floor(log2(amax))) puts max|q| in [2^14, 2^15): FP16 holds every BF16
        // value of the row exactly down to 2^-28 of its maximum.
        float factor = 1.0f;
        if (amax > 0.0f && amax < INFINITY) {
            const int ex = static_cast<int>((__float_as_uint(amax) >> 23) & 0xff) - 127;
            factor = ldexpf(1.0f, 14 - ex);
        }
#pragma unroll
        for (int gq = 0; gq < G; ++gq) {
#pragma unroll
            for (int s = 0; s < 2; ++s) {
#pragma unroll
                for (int e = 0; e < 8; ++e) { qop[nt][gq][s][e] = static_cast<_Float16>(x[gq][s][e] * factor); }
            }
        }
        rowmul[nt] = a.scale_log2 / factor;
        nmask[nt] = valid ? new_key_mask(par, t) : 0u;
    }

    float m[NT];
    float l[NT];
    f4 O[NT][DT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        m[nt] = -INFINITY;
        l[nt] = 0.0f;
#pragma unroll
        for (int t = 0; t < DT; ++t) { O[nt][t] = f4{0.f, 0.f, 0.f, 0.f}; }
    }

    const int hist_end = min(L, k1); // keys below this are visible to every row
    const int vgroup = c >> 3;       // quant group of this lane's V dims 8c..8c+7

    // Lookahead of two chunks: while chunk i is computed, chunks i+1 and i+2 are in flight. Chunk
    // i+2 reuses chunk i's stage once chunk i sits in registers.
    constexpr int kStride = kChunk * kWaves;
    if (first + kStride < k1) { issue_chunk(my_stage0 + kStageBytes, kbase, vbase, ksbase, vsbase, first + kStride, lane); }
    int stage = 0;
#pragma unroll 1
    for (int c0 = first; c0 < k1; c0 += kStride) {
        NMI_AS3 char* st = my_stage0 + stage * kStageBytes;
        // Wait for this chunk's 9 DMA instructions; the next chunk's 9 may stay outstanding.
        if (c0 + kStride < k1) {
            __builtin_amdgcn_s_waitcnt(0x0f79); // vmcnt(9)
        } else {
            __builtin_amdgcn_s_waitcnt(0x0f70); // vmcnt(0)
        }
        i4 kr[2][G];
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
            for (int gq = 0; gq < G; ++gq) { kr[kt][gq] = *(NMI_AS3 const i4*)(st + kStageK + (2 * kt + gq) * 1024 + 16 * lane); }
        }
        const i4 ksw0 = *(NMI_AS3 const i4*)(st + kStageS + (4 * g) * 4);
        const i4 ksw1 = *(NMI_AS3 const i4*)(st + kStageS + (16 + 4 * g) * 4);
        const i4 vsw0 = *(NMI_AS3 const i4*)(st + kStageS + 128 + (4 * g) * 4);
        const i4 vsw1 = *(NMI_AS3 const i4*)(st + kStageS + 128 + (16 + 4 * g) * 4);
        i2 vr[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int row = j < 4 ? 4 * g + j : 16 + 4 * g + (j - 4);
            vr[j] = *(NMI_AS3 const i2*)(st + kStageV + row * 128 + 8 * c);
        }
        // Chunk i is in registers once these reads retire; then its stage takes chunk i+2.
        const int c2 = c0 + 2 * kStride;
        if (c2 < k1) {
            __builtin_amdgcn_s_waitcnt(0xc07f); // lgkmcnt(0)
            issue_chunk(st, kbase, vbase, ksbase, vsbase, c2, lane);
        }
        stage ^= 1;

        // ---- S^T = K Q^T per quant group
        f4 sacc[2][NT][G];
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
            for (int gq = 0; gq < G; ++gq) {
                const h8 ka0 = cvt_codes8(kr[kt][gq][0], kr[kt][gq][1]);
                const h8 ka1 = cvt_codes8(kr[kt][gq][2], kr[kt][gq][3]);
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) {
                    f4 acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka0, qop[nt][gq][0], f4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                    sacc[kt][nt][gq] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka1, qop[nt][gq][1], acc, 0, 0, 0);
                }
            }
        }

        const bool full = (c0 + kChunk) <= hist_end;
        h8 pop[NT];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            float sv[2][4];
            float cmax = -INFINITY;
#pragma unroll
            for (int kt = 0; kt < 2; ++kt) {
                const i4& ksw = kt ? ksw1 : ksw0;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float s = static_cast<float>(half_bits_at(ksw, 2 * e)) * sacc[kt][nt][0][e];
                    s = fmaf(static_cast<float>(half_bits_at(ksw, 2 * e + 1)), sacc[kt][nt][1][e], s);
                    s *= rowmul[nt];
                    if (!full) {
                        const int key = c0 + 16 * kt + 4 * g + e;
                        bool vis = key < hist_end;
                        if (!vis && key >= L && key < k1) {
                            const int u = key - L;
                            vis = u < 32 && ((nmask[nt] >> u) & 1u);
                        }
                        s = vis ? s : -INFINITY;
                    }
                    sv[kt][e] = s;
                    cmax = fmaxf(cmax, s);
                }
            }
            cmax = group4_max(cmax);
            const float mnew = fmaxf(m[nt], cmax);
            const bool live = mnew != -INFINITY;
            // Probabilities carry a 2^15 factor (exact in FP16, cancels in O / l) so the PV operand
            // stays in FP16's normal range down to 2^-29 of the row maximum.
            const float mref = mnew - 15.0f;
            float lsum = 0.0f;
#pragma unroll
            for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float pe = live ? __builtin_amdgcn_exp2f(sv[kt][e] - mref) : 0.0f;
                    lsum += pe;
                    pop[nt][4 * kt + e] = static_cast<_Float16>(pe);
                }
            }
            const bool grew = mnew > m[nt];
            if (__any(grew)) {
                const float alpha = grew ? __builtin_amdgcn_exp2f(m[nt] - mnew) : 1.0f;
                l[nt] *= alpha;
#pragma unroll
                for (int t = 0; t < DT; ++t) { O[nt][t] *= alpha; }
            }
            l[nt] += lsum;
            m[nt] = mnew;
        }

        // ---- O^T += V^T P^T. V' = FP16(code * scale): codes convert exactly, one packed multiply
        // rounds the product once. Keys past the range end get a zero scale (their rows may be
        // uninitialized).
        h2 vsp[4];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
#pragma unroll
            for (int h1 = 0; h1 < 2; ++h1) {
                const int j = 2 * w + h1;
                vsp[w][h1] = half_bits_at(j < 4 ? vsw0 : vsw1, 2 * (j & 3) + vgroup);
            }
        }
        if (!full) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int key = c0 + (j < 4 ? 4 * g + j : 16 + 4 * g + (j - 4));
                if (key >= k1) { vsp[j >> 1][j & 1] = static_cast<_Float16>(0.0f); }
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
            O[nt][TT] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pop[nt], O[nt][TT], 0, 0, 0);   \
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
#undef NMI_PV_TILE
    }

    // ---- merge the four waves through LDS (reusing the staging ring), then write the partial.
    __builtin_amdgcn_s_waitcnt(0); // no DMA may land in the ring after this point
    __syncthreads();
    float* sm_o = reinterpret_cast<float*>(smem);      // [kWaves][32][D + 1]
    float* sm_m = sm_o + kWaves * 32 * (D + 1);        // [kWaves][32]
    float* sm_l = sm_m + kWaves * 32;                  // [kWaves][32]
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        const float lt = group4_sum(l[nt]);
        const int r = 16 * nt + c;
        if (g == 0) {
            sm_m[wave * 32 + r] = m[nt];
            sm_l[wave * 32 + r] = lt;
        }
#pragma unroll
        for (int t = 0; t < DT; ++t) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                // O^T tile t row (4g + e) is dim 8*(4g + e) + t.
                sm_o[(wave * 32 + r) * (D + 1) + 8 * (4 * g + e) + t] = O[nt][t][e];
            }
        }
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < R * D; idx += blockDim.x) {
        const int r = idx / D;
        const int d = idx - r * D;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) { M = fmaxf(M, sm_m[w * 32 + r]); }
        float o = 0.0f;
        float lsum = 0.0f;
        if (M != -INFINITY) {
#pragma unroll
            for (int w = 0; w < kWaves; ++w) {
                const float mw = sm_m[w * 32 + r];
                if (mw == -INFINITY) { continue; }
                const float wgt = __builtin_amdgcn_exp2f(mw - M);
                o = fmaf(sm_o[(w * 32 + r) * (D + 1) + d], wgt, o);
                lsum = fmaf(sm_l[w * 32 + r], wgt, lsum);
            }
        }
        out_o[r * D + d] = o;
        if (d == 0) {
            out_ml[2 * r] = M;
            out_ml[2 * r + 1] = lsum;
        }
    }
}

struct MergeArgs {
    const float* part_o;
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
};

constexpr int kMergeThreads = 256;
constexpr int kMergeMaxSplits = 2048;

// Log-sum-exp merge over splits (reference src/ops/kernel/gqa_attention_decode.cuh:144-227,
// including "every split empty => 0"). One block per output row (b, t, qh): the first 32 splits'
// partial rows are requested up front, every split's (m, l) becomes a weight in LDS through block
// reductions, then two thread halves accumulate alternate splits.
template <int D>
__global__ __launch_bounds__(kMergeThreads) void verify_attn_merge_kernel(MergeArgs a) {
    __shared__ float wts[kMergeMaxSplits];
    __shared__ float lw[kMergeMaxSplits];
    __shared__ float red[kMergeThreads / 64];
    __shared__ float half_o[D];
    const int row_id = blockIdx.x; // (b, t, qh)
    const int qh = row_id % a.Hq;
    const int t = (row_id / a.Hq) % a.T;
    const int b = row_id / (a.Hq * a.T);
    const int h = qh / a.G;
    const int gi = qh - h * a.G;
    const int rc = t / a.tokens_per_chunk;
    const int r = (t - rc * a.tokens_per_chunk) * a.G + gi;
    const int64_t unit = (static_cast<int64_t>(b) * a.row_chunks + rc) * a.Hkv + h;
    const float* ml = a.part_ml + unit * a.nsplit * 64;
    const float* po = a.part_o + unit * a.nsplit * (32 * D);
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;

    // Issue the first partial-row loads before any reduction: thread (half, d) owns splits
    // s = half + 2k.
    constexpr int kPre = 16;
    const int half = tid / D;
    const int d = tid - half * D;
    float pre[kPre];
#pragma unroll
    for (int k = 0; k < kPre; ++k) {
        const int s = half + 2 * k;
        pre[k] = s < a.nsplit ? po[static_cast<int64_t>(s) * 32 * D + r * D + d] : 0.0f;
    }
    float M = -INFINITY;
    for (int s = tid; s < a.nsplit; s += kMergeThreads) {
        const float ls = ml[s * 64 + 2 * r + 1];
        const float ms = ml[s * 64 + 2 * r];
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
    for (int s = tid; s < a.nsplit; s += kMergeThreads) {
        const float w = (M != -INFINITY && wts[s] != -INFINITY) ? __builtin_amdgcn_exp2f(wts[s] - M) : 0.0f;
        wts[s] = w;
        lsum = fmaf(lw[s], w, lsum);
    }
    lsum = wave_sum(lsum);
    if (lane == 0) { red[wave] = lsum; }
    __syncthreads();
    lsum = (red[0] + red[1]) + (red[2] + red[3]);

    float o = 0.0f;
    if (lsum > 0.0f) {
#pragma unroll
        for (int k = 0; k < kPre; ++k) {
            const int s = half + 2 * k;
            if (s < a.nsplit) { o = fmaf(pre[k], wts[s], o); }
        }
#pragma unroll 4
        for (int s = half + 2 * kPre; s < a.nsplit; s += 2) {
            o = fmaf(po[static_cast<int64_t>(s) * 32 * D + r * D + d], wts[s], o);
        }
    }
    if (half == 1) { half_o[d] = o; }
    __syncthreads();
    if (half == 0) {
        o += half_o[d];
        const float val = lsum > 0.0f ? o / lsum : 0.0f;
        const int64_t oi = static_cast<int64_t>(D) * (qh + static_cast<int64_t>(a.Hq) * (t + static_cast<int64_t>(a.T) * b)) + d;
        if (a.out_f32) {
            static_cast<float*>(a.out)[oi] = val;
        } else {
            static_cast<uint16_t*>(a.out)[oi] = f32_to_bf16_bits(val);
        }
    }
}

// INT8-G64 encoder for A2, the prefix commit and multi-row-chunk A1 (reference contract
// include/ninfer/ops/gqa_attention.h:25-30; device encoder
// src/ops/kernel/gqa_attention_decode_i8.cuh:168-209). Block (t, b, h): one wave per (K|V, group),
// lane i owns element i of the 64-element group.
template <int D>
__global__ __launch_bounds__(256) void kv_quant_append_kernel(const uint16_t* k, const uint16_t* v,
                                                              const int32_t* positions,
                                                              const int32_t* count, int32_t T,
                                                              int32_t Hkv, int32_t P, int8_t* kc,
                                                              int8_t* vc, uint16_t* ks,
                                                              uint16_t* vs, int64_t code_seq,
                                                              int64_t scale_seq) {
    constexpr int G = D / 64;
    const int t = blockIdx.x;
    const int b = blockIdx.y;
    const int h = blockIdx.z;
    if (count != nullptr && t >= count[b]) { return; }
    const int lane = threadIdx.x & 63;
    const int pos = positions[static_cast<int64_t>(b) * T + t];
    if (pos < 0 || pos >= P) { return; }
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

} // namespace

SplitPlan plan_attention(int32_t Hq, int32_t Hkv, int32_t D, int32_t T, int32_t B,
                         uint32_t max_visible_keys) {
    SplitPlan p;
    p.G = Hq / Hkv;
    p.tokens_per_chunk = std::max<int32_t>(1, kAttnRowsPerTile / p.G);
    p.tokens_per_chunk = std::min(p.tokens_per_chunk, T);
    p.row_chunks = (T + p.tokens_per_chunk - 1) / p.tokens_per_chunk;
    const int64_t units = static_cast<int64_t>(Hkv) * B * p.row_chunks;
    const int64_t want = std::max<int64_t>(1, (kAttnTargetWorkgroups + units - 1) / units);
    int64_t kps = (static_cast<int64_t>(max_visible_keys) + want - 1) / want;
    kps = ((kps + 127) / 128) * 128;
    kps = std::max<int64_t>(kps, kAttnMinKeysPerSplit);
    p.keys_per_split = static_cast<int32_t>(kps);
    p.nsplit = static_cast<int32_t>((static_cast<int64_t>(max_visible_keys) + kps - 1) / kps);
    p.nsplit = std::max(p.nsplit, 1);
    const size_t part_units = static_cast<size_t>(units) * p.nsplit;
    p.part_o_offset = 0;
    const size_t o_bytes = part_units * 32 * static_cast<size_t>(D) * sizeof(float);
    p.part_ml_offset = (o_bytes + 255) & ~static_cast<size_t>(255);
    const size_t ml_bytes = part_units * 64 * sizeof(float);
    p.bytes = ((p.part_ml_offset + ml_bytes + 255) & ~static_cast<size_t>(255));
    return p;
}

void launch_kv_append(const uint16_t* k, const uint16_t* v, const int32_t* positions,
                      const int32_t* count, int32_t T, const CacheRef& c, hipStream_t stream) {
    if (c.D != 128) { throw Unsupported("kv append: only head_dim 128 is built"); }
    dim3 grid(T, c.B, c.Hkv);
    hipLaunchKernelGGL(kv_quant_append_kernel<128>, grid, dim3(256), 0, stream, k, v, positions,
                       count, T, c.Hkv, c.P, c.kc, c.vc, c.ks, c.vs, c.code_seq, c.scale_seq);
    check_launch("kv_quant_append_kernel");
}

void launch_verify_attention(const uint16_t* q, const uint16_t* k_new, const uint16_t* v_new,
                             const int32_t* positions, const int32_t* parents, int32_t T,
                             int32_t Hq, const CacheRef& c, float scale, uint32_t max_keys,
                             void* workspace, const SplitPlan& plan, void* out, bool out_f32,
                             hipStream_t stream) {
    if (c.D != 128) { throw Unsupported("verify attention: only head_dim 128 is built"); }
    if (plan.nsplit > kMergeMaxSplits) { throw Unsupported("verify attention: too many key splits"); }
    if (k_new != nullptr && plan.row_chunks > 1) {
        // Several row-chunk workgroups read the new rows: write them in a launch of their own.
        launch_kv_append(k_new, v_new, positions, nullptr, T, c, stream);
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
    a.ks = c.ks;
    a.vs = c.vs;
    a.part_o = reinterpret_cast<float*>(ws + plan.part_o_offset);
    a.part_ml = reinterpret_cast<float*>(ws + plan.part_ml_offset);
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
    a.max_keys = static_cast<int32_t>(max_keys);
    a.scale_log2 = scale * 1.4426950408889634f;
    const int rows = plan.tokens_per_chunk * plan.G;
    dim3 grid(plan.nsplit, c.Hkv, c.B * plan.row_chunks);
    if (rows <= 16) {
        hipLaunchKernelGGL(verify_attn_partial_kernel<1>, grid, dim3(256), 0, stream, a);
    } else {
        hipLaunchKernelGGL(verify_attn_partial_kernel<2>, grid, dim3(256), 0, stream, a);
    }
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
    mg.out_f32 = out_f32 ? 1 : 0;
    hipLaunchKernelGGL(verify_attn_merge_kernel<128>, dim3(c.B * T * Hq), dim3(kMergeThreads), 0, stream, mg);
    check_launch("verify_attn_merge_kernel");
}

} // namespace nmi
