// Verify attention for the MTP speculative-decoding step on gfx950.
//
// Semantics (reference include/ninfer/ops/gqa_attention.h:52-91): for sequence b, query token t
// and query head qh (KV head h = qh / G), attend over cache rows [0, positions[0]) plus the new
// rows positions[u] with u visible from t (u <= t causal; u an ancestor-or-self of t for trees),
// reading INT8-G64 codes with FP16 scales. Split-K over keys with an online softmax per split and
// a log-sum-exp merge (reference split reducer src/ops/kernel/gqa_attention_decode.cuh:144-227).
//
// MI355X design:
//  * One workgroup = 4 waves = one (sequence, row chunk, KV head, key split). Each wave streams
//    32-key chunks (chunk w, w+4, ...) with 128-bit loads straight into MFMA operand registers,
//    double buffered; no LDS on the hot path.
//  * QK^T runs as S^T = K * Q^T on v_mfma_f32_16x16x32_f16: K codes (exact in FP16) are the A
//    operand (16 keys x 32 dims per step, each 32-dim step inside one 64-wide quant group), Q
//    (BF16 -> FP16 exact after a per-row power-of-two rescale) is the B operand. Each quant group
//    accumulates separately so the per-(key, group) FP16 scale is applied exactly in FP32.
//  * PV runs as O^T = V^T * P^T on the same instruction. The S^T accumulator layout (lane = query
//    row, 4 keys per 16-key tile) is exactly the B-operand layout of P^T, so probabilities never
//    leave registers. V is the A operand with the dimension permutation d = 8*lane16 + tile: each
//    lane loads 8 bytes per key (fully coalesced 128 B rows) and transposes in registers.
//  * GQA x q_len rows (5 x 4 = 20 for the 40/8 geometry) are padded to two 16-row MFMA tiles.
#include "common.h"
#include "device_utils.h"
#include "ops_internal.h"

#include <algorithm>
#include <cmath>

namespace nmi {
namespace {

constexpr int kWaves = 4;
constexpr int kChunk = 32;

struct AttnArgs {
    const uint16_t* q;
    const int32_t* positions;
    const int32_t* parents;
    const int8_t* kc;
    const int8_t* vc;
    const uint16_t* ks;
    const uint16_t* vs;
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

// Byte (t & 3) of word (t >> 2) from key slots 2w and 2w+1 -> packed FP16 pair (V transpose).
template <int T>
__device__ __forceinline__ uint32_t v_pair(const i2& a, const i2& b) {
    return i8x2_to_f16x2<T & 3>(static_cast<uint32_t>(a[T >> 2]), static_cast<uint32_t>(b[T >> 2]));
}

typedef _Float16 h2 __attribute__((ext_vector_type(2)));

// K half of a 32-key chunk: lane (c, g) holds key tile kt's row c0+16kt+c at dims 64gq+16g..+15,
// and the FP16 scales of keys c0+16kt+4g..+3 (both groups, interleaved per key).
template <int D>
struct KRegs {
    i4 k[2][D / 64];
    i4 sc[2];
};
// V half: 8 key slots (4g+j and 16+4g+j) x 8 dims at d = 8c..8c+7, plus the same scale words.
struct VRegs {
    i2 v[8];
    i4 sc[2];
};

template <int D>
__device__ __forceinline__ void load_k(KRegs<D>& r, const int8_t* kbase, const uint16_t* ksbase,
                                       int c0, int c, int g) {
    constexpr int G = D / 64;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
        const int8_t* krow = kbase + static_cast<int64_t>(c0 + 16 * kt + c) * D + 16 * g;
#pragma unroll
        for (int gq = 0; gq < G; ++gq) { r.k[kt][gq] = *reinterpret_cast<const i4*>(krow + 64 * gq); }
        r.sc[kt] = *reinterpret_cast<const i4*>(ksbase + static_cast<int64_t>(c0 + 16 * kt + 4 * g) * G);
    }
}

template <int D>
__device__ __forceinline__ void load_v(VRegs& r, const int8_t* vbase, const uint16_t* vsbase, int c0,
                                       int c, int g) {
    constexpr int G = D / 64;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int key = c0 + (j < 4 ? 4 * g + j : 16 + 4 * g + (j - 4));
        r.v[j] = *reinterpret_cast<const i2*>(vbase + static_cast<int64_t>(key) * D + 8 * c);
    }
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
        r.sc[kt] = *reinterpret_cast<const i4*>(vsbase + static_cast<int64_t>(c0 + 16 * kt + 4 * g) * G);
    }
}

__device__ __forceinline__ _Float16 half_bits_at(const i4& v, int idx) {
    const uint32_t word = static_cast<uint32_t>(v[idx >> 1]);
    return __builtin_bit_cast(_Float16, static_cast<uint16_t>((idx & 1) ? (word >> 16) : (word & 0xffffu)));
}

__device__ __forceinline__ float half_at(const i4& v, int idx) {
    const int word = v[idx >> 1];
    const uint16_t bits = static_cast<uint16_t>((idx & 1) ? (static_cast<uint32_t>(word) >> 16)
                                                          : (static_cast<uint32_t>(word) & 0xffffu));
    return f16_bits_to_f32(bits);
}

template <int D, int NT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void verify_attn_partial_kernel(AttnArgs a) {
    static_assert(D == 128, "head_dim 128 kernel");
    constexpr int G = D / 64;
    constexpr int DT = D / 16; // O^T tiles of 16 dims
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int c = lane & 15;
    const int g = lane >> 4;
    const int split = blockIdx.x;
    const int h = blockIdx.y;
    const int b = blockIdx.z / a.row_chunks;
    const int rc = blockIdx.z - b * a.row_chunks;

    const int32_t* pos = a.positions + static_cast<int64_t>(b) * a.T;
    const int32_t* par = a.parents ? a.parents + static_cast<int64_t>(b) * a.T : nullptr;
    const int window = min(pos[a.T - 1] + 1, a.max_keys);
    const int L = max(0, min(pos[0], window));
    const int t0 = rc * a.tokens_per_chunk;
    const int Tc = min(a.tokens_per_chunk, a.T - t0);
    const int R = Tc * a.G;
    const int k0 = split * a.kps;
    const int k1 = min(k0 + a.kps, window);
    const int64_t unit = (static_cast<int64_t>(b) * a.row_chunks + rc) * a.Hkv + h;
    const int64_t pidx = unit * a.nsplit + split;
    float* out_o = a.part_o + pidx * (32 * D);
    float* out_ml = a.part_ml + pidx * 64;

    if (k0 >= k1) {
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

    const int64_t head_code = (static_cast<int64_t>(b) * a.code_seq) + static_cast<int64_t>(h) * a.P * D;
    const int64_t head_scale = (static_cast<int64_t>(b) * a.scale_seq) + static_cast<int64_t>(h) * a.P * G;
    const int8_t* kbase = a.kc + head_code;
    const int8_t* vbase = a.vc + head_code;
    const uint16_t* ksbase = a.ks + head_scale;
    const uint16_t* vsbase = a.vs + head_scale;

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
    const int vgroup = (8 * c) / 64; // quant group of this lane's V dims (D == 128)

    // Software pipeline with one register set per operand: the next chunk's K is requested as soon
    // as this chunk's QK^T has consumed K, and its V as soon as PV has consumed V.
    KRegs<D> kr;
    VRegs vr;
    int c0 = k0 + kChunk * wave;
    if (c0 < k1) {
        load_k<D>(kr, kbase, ksbase, c0, c, g);
        load_v<D>(vr, vbase, vsbase, c0, c, g);
    }
#pragma unroll 1
    while (c0 < k1) {
        const int c1 = c0 + kChunk * kWaves;
        const bool more = c1 < k1;

        // ---- S^T = K Q^T per quant group
        f4 sacc[2][NT][G];
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
            for (int gq = 0; gq < G; ++gq) {
                const h8 ka0 = cvt_codes8(kr.k[kt][gq][0], kr.k[kt][gq][1]);
                const h8 ka1 = cvt_codes8(kr.k[kt][gq][2], kr.k[kt][gq][3]);
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) {
                    f4 acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka0, qop[nt][gq][0], f4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                    sacc[kt][nt][gq] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka1, qop[nt][gq][1], acc, 0, 0, 0);
                }
            }
        }
        float kscale[2][4][G];
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
#pragma unroll
                for (int gq = 0; gq < G; ++gq) { kscale[kt][e][gq] = static_cast<float>(half_bits_at(kr.sc[kt], G * e + gq)); }
            }
        }
        if (more) { load_k<D>(kr, kbase, ksbase, c1, c, g); }

        const bool full = (c0 + kChunk) <= hist_end;
        h8 pop[NT];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            float sv[2][4];
            float cmax = -INFINITY;
#pragma unroll
            for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float s = 0.0f;
#pragma unroll
                    for (int gq = 0; gq < G; ++gq) { s = fmaf(kscale[kt][e][gq], sacc[kt][nt][gq][e], s); }
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
            const float alpha = live ? __builtin_amdgcn_exp2f(m[nt] - mnew) : 1.0f;
            float lsum = 0.0f;
#pragma unroll
            for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float pe = live ? __builtin_amdgcn_exp2f(sv[kt][e] - mnew) : 0.0f;
                    lsum += pe;
                    pop[nt][4 * kt + e] = static_cast<_Float16>(pe * 32768.0f);
                }
            }
            l[nt] = l[nt] * alpha + lsum;
            m[nt] = mnew;
#pragma unroll
            for (int t = 0; t < DT; ++t) { O[nt][t] *= alpha; }
        }

        // ---- O^T += V^T P^T. V' = FP16(code * scale): codes convert exactly, one packed multiply
        // rounds the product once.
        h2 vsp[4];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
#pragma unroll
            for (int h1 = 0; h1 < 2; ++h1) {
                const int j = 2 * w + h1;
                vsp[w][h1] = half_bits_at(vr.sc[j >> 2], G * (j & 3) + vgroup);
            }
        }
        if (!full) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int key = c0 + (j < 4 ? 4 * g + j : 16 + 4 * g + (j - 4));
                if (key >= k1) { vsp[j >> 1][j & 1] = static_cast<_Float16>(0.0f); }
            }
        }
        static_assert(DT == 8, "V transpose is written for 8 tiles");
#define NMI_PV_TILE(TT)                                                                            \
    {                                                                                              \
        h2 pr[4];                                                                                  \
        _Pragma("unroll") for (int w = 0; w < 4; ++w) {                                            \
            pr[w] = __builtin_bit_cast(h2, v_pair<TT>(vr.v[2 * w], vr.v[2 * w + 1])) * vsp[w];     \
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
        if (more) { load_v<D>(vr, vbase, vsbase, c1, c, g); }
        c0 = c1;
    }

    // ---- merge the four waves through LDS, then write this split's partial.
    __shared__ float sm_o[kWaves][32][D + 1];
    __shared__ float sm_m[kWaves][32];
    __shared__ float sm_l[kWaves][32];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        const float lt = group4_sum(l[nt]);
        const int r = 16 * nt + c;
        if (g == 0) {
            sm_m[wave][r] = m[nt];
            sm_l[wave][r] = lt;
        }
#pragma unroll
        for (int t = 0; t < DT; ++t) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                // O^T tile t row (4g + e) is dim 8*(4g + e) + t.
                sm_o[wave][r][8 * (4 * g + e) + t] = O[nt][t][e];
            }
        }
    }
    for (int r = NT * 16 + threadIdx.x; r < 32; r += blockDim.x) {
        for (int w = 0; w < kWaves; ++w) {
            sm_m[w][r] = -INFINITY;
            sm_l[w][r] = 0.0f;
        }
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < R * D; idx += blockDim.x) {
        const int r = idx / D;
        const int d = idx - r * D;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) { M = fmaxf(M, sm_m[w][r]); }
        float o = 0.0f;
        float lsum = 0.0f;
        if (M != -INFINITY) {
#pragma unroll
            for (int w = 0; w < kWaves; ++w) {
                const float mw = sm_m[w][r];
                if (mw == -INFINITY) { continue; }
                const float wgt = __builtin_amdgcn_exp2f(mw - M);
                o = fmaf(sm_o[w][r][d], wgt, o);
                lsum = fmaf(sm_l[w][r], wgt, lsum);
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
    float out_scale; // undoes the 2^15 probability scaling of the PV operand
    int32_t out_f32;
};

// Log-sum-exp merge over splits (reference src/ops/kernel/gqa_attention_decode.cuh:144-227,
// including "every split empty => 0").
template <int D>
__global__ __launch_bounds__(D) void verify_attn_merge_kernel(MergeArgs a) {
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
    const int d = threadIdx.x;

    float M = -INFINITY;
    for (int s = 0; s < a.nsplit; ++s) {
        if (ml[s * 64 + 2 * r + 1] > 0.0f) { M = fmaxf(M, ml[s * 64 + 2 * r]); }
    }
    float o = 0.0f;
    float lsum = 0.0f;
    if (M != -INFINITY) {
        for (int s = 0; s < a.nsplit; ++s) {
            const float ls = ml[s * 64 + 2 * r + 1];
            if (!(ls > 0.0f)) { continue; }
            const float w = __builtin_amdgcn_exp2f(ml[s * 64 + 2 * r] - M);
            lsum = fmaf(ls, w, lsum);
            o = fmaf(po[static_cast<int64_t>(s) * 32 * D + r * D + d], w, o);
        }
    }
    const float val = lsum > 0.0f ? (o / lsum) * a.out_scale : 0.0f;
    const int64_t oi = static_cast<int64_t>(D) * (qh + static_cast<int64_t>(a.Hq) * (t + static_cast<int64_t>(a.T) * b)) + d;
    if (a.out_f32) {
        static_cast<float*>(a.out)[oi] = val;
    } else {
        static_cast<uint16_t*>(a.out)[oi] = f32_to_bf16_bits(val);
    }
}

// INT8-G64 encoder (reference contract include/ninfer/ops/gqa_attention.h:25-30; device encoder
// src/ops/kernel/gqa_attention_decode_i8.cuh:168-209). One wave per (KV head, K|V, group): lane i
// owns element i of the 64-element group.
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
    if (count != nullptr && t >= count[b]) { return; }
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int pos = positions[static_cast<int64_t>(b) * T + t];
    if (pos < 0 || pos >= P) { return; }
    const int units = Hkv * 2 * G;
    for (int unit = wave; unit < units; unit += blockDim.x / 64) {
        const int h = unit / (2 * G);
        const int rem = unit - h * 2 * G;
        const int which = rem / G;
        const int grp = rem - which * G;
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
    dim3 grid(T, c.B);
    hipLaunchKernelGGL(kv_quant_append_kernel<128>, grid, dim3(256), 0, stream, k, v, positions,
                       count, T, c.Hkv, c.P, c.kc, c.vc, c.ks, c.vs, c.code_seq, c.scale_seq);
    check_launch("kv_quant_append_kernel");
}

void launch_verify_attention(const uint16_t* q, const int32_t* positions, const int32_t* parents,
                             int32_t T, int32_t Hq, const CacheRef& c, float scale,
                             uint32_t max_keys, void* workspace, const SplitPlan& plan, void* out,
                             bool out_f32, hipStream_t stream) {
    if (c.D != 128) { throw Unsupported("verify attention: only head_dim 128 is built"); }
    char* ws = static_cast<char*>(workspace);
    AttnArgs a{};
    a.q = q;
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
        hipLaunchKernelGGL((verify_attn_partial_kernel<128, 1>), grid, dim3(256), 0, stream, a);
    } else {
        hipLaunchKernelGGL((verify_attn_partial_kernel<128, 2>), grid, dim3(256), 0, stream, a);
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
    mg.out_scale = 1.0f / 32768.0f;
    mg.out_f32 = out_f32 ? 1 : 0;
    hipLaunchKernelGGL(verify_attn_merge_kernel<128>, dim3(c.B * T * Hq), dim3(128), 0, stream, mg);
    check_launch("verify_attn_merge_kernel");
}

} // namespace nmi
