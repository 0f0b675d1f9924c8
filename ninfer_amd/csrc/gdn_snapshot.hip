// Recurrent-state ops of the hybrid (Gated DeltaNet) layers on the verify path, with per-token
// snapshot slots, and the device scalar ops that commit a slot after acceptance (gfx950).
//
// Reference contracts: include/ninfer/ops/gated_delta_rule.h:26-71 (recurrence, distinct-state
// and snapshot forms), include/ninfer/ops/causal_conv1d_silu.h:9-42 (width-4 causal depthwise
// convolution + SiLU, snapshot form), include/ninfer/ops/scalar.h:9-33 (device scalar ops). The
// verify round writes the state after each of its T tokens to slot t; after acceptance the slot
// index of the accepted prefix becomes the next round's initial slot
// (tests/ops/test_speculative_round.cpp:356-497), so rejected tokens cost no state copy.
#include "common.h"
#include "gdn_internal.h"

namespace nmi {
namespace {

typedef float f4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float(static_cast<uint32_t>(h) << 16); }

// Round-to-nearest-even FP32 -> BF16 (NaN stays NaN).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    const uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) { return static_cast<uint16_t>((u >> 16) | 0x40u); }
    return static_cast<uint16_t>((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

// The value of the lane that DPP control CTRL selects inside the lane's 16-lane row.
template <int CTRL>
__device__ __forceinline__ float dpp_row(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}

// Sum over the 16 lanes that own one state row (lanes 16i .. 16i+15 of the wave), all in the VALU:
// swap neighbours (quad_perm 1,0,3,2), then pairs (quad_perm 2,3,0,1), then quads (row_half_mirror),
// then half-rows (row_mirror). Each step adds a lane and its partner in either order, so every lane
// of the row ends with the same bits.
__device__ __forceinline__ float row_sum16(float x) {
    x += dpp_row<0xB1>(x);
    x += dpp_row<0x4E>(x);
    x += dpp_row<0x141>(x);
    x += dpp_row<0x140>(x);
    return x;
}

// One workgroup = 16 state rows of one value head; 16 lanes per row, S/16 consecutive columns per
// lane. Row r of head h is S_h[r, :] (the value index r, the key index along the row), stored at
// state + (h * S + r) * S. Every row evolves on its own:
//   row *= alpha; partial = row . k; delta = beta * (v[r] - partial); row += delta * k;
//   out[r] = BF16(scale * row . q)          (include/ninfer/ops/gated_delta_rule.h:26-32)
// The row stays in registers across the T tokens; snapshot slot t receives it after token t.
// The token inputs (k, q of the head's q/k head, v of the 16 rows, g, beta) of up to kGdnTokens
// tokens are staged in LDS first, so the sequential token loop never waits on global memory; their
// loads overlap the dependent initial-slot -> state loads.
constexpr int kGdnTokens = 16;
constexpr int kGdnRows = 16;                   // state rows per workgroup
constexpr int kGdnThreads = 16 * kGdnRows;     // 16 lanes per row

// Snapshot rows are written once and read back at most once, a round later: stream them past the
// caches.
__device__ __forceinline__ void store_snapshot(float* dst, f4v x) { __builtin_nontemporal_store(x, reinterpret_cast<f4v*>(dst)); }

template <int S>
__global__ __launch_bounds__(kGdnThreads) void gdn_recurrent_kernel(GdnArgs a) {
    constexpr int CPL = S / 16; // columns per lane
    __shared__ __attribute__((aligned(16))) float ks[kGdnTokens][S];
    __shared__ __attribute__((aligned(16))) float qs[kGdnTokens][S];
    __shared__ float vs[kGdnTokens][kGdnRows];
    __shared__ float gs[kGdnTokens];
    __shared__ float bs[kGdnTokens];
    const int h = blockIdx.y;
    const int rl = threadIdx.x >> 4; // row within the workgroup
    const int r = blockIdx.x * kGdnRows + rl;
    const int j = threadIdx.x & 15;
    const int qh = h / (a.Hv / a.Hqk);
    const int64_t head_elems = static_cast<int64_t>(S) * S;
    const int64_t row_off = static_cast<int64_t>(h) * head_elems + static_cast<int64_t>(r) * S + j * CPL;

    // Token inputs of the first block: issued before the slot-dependent state loads.
    auto stage = [&](int t0) {
        const int nt = min(kGdnTokens, a.T - t0);
        for (int i = threadIdx.x; i < nt * S; i += kGdnThreads) {
            const int t = i / S;
            const int c = i - t * S;
            const int64_t off = (static_cast<int64_t>(t0 + t) * a.Hqk + qh) * S + c;
            ks[t][c] = bf16_to_f32(a.k[off]);
            qs[t][c] = bf16_to_f32(a.q[off]);
        }
        for (int i = threadIdx.x; i < nt * kGdnRows; i += kGdnThreads) {
            const int t = i / kGdnRows;
            const int rr = i - t * kGdnRows;
            vs[t][rr] = bf16_to_f32(a.v[(static_cast<int64_t>(t0 + t) * a.Hv + h) * S + blockIdx.x * kGdnRows + rr]);
        }
        if (threadIdx.x < nt) {
            const int64_t hv_t = static_cast<int64_t>(t0 + threadIdx.x) * a.Hv + h;
            gs[threadIdx.x] = expf(a.g[hv_t]);
            bs[threadIdx.x] = a.beta[hv_t];
        }
    };
    stage(0);

    const float* src = a.state_in;
    if (a.initial_slot != nullptr) {
        const int slot = *a.initial_slot;
        if (slot < 0 || slot >= a.slots) { return; } // outside [0, Slots): nothing is read or written
        src = a.states + static_cast<int64_t>(slot) * a.Hv * head_elems;
    }
    float row[CPL];
#pragma unroll
    for (int i = 0; i < CPL; i += (CPL >= 4 ? 4 : CPL)) {
        if constexpr (CPL >= 4) {
            const f4v x = *reinterpret_cast<const f4v*>(src + row_off + i);
            row[i] = x[0];
            row[i + 1] = x[1];
            row[i + 2] = x[2];
            row[i + 3] = x[3];
        } else {
#pragma unroll
            for (int e = 0; e < CPL; ++e) { row[e] = src[row_off + e]; }
        }
    }

#pragma unroll 1
    for (int t0 = 0; t0 < a.T; t0 += kGdnTokens) {
        if (t0 > 0) {
            __syncthreads(); // every row is done with the previous block
            stage(t0);
        }
        __syncthreads();
        const int nt = min(kGdnTokens, a.T - t0);
#pragma unroll 1
        for (int tl = 0; tl < nt; ++tl) {
            const int t = t0 + tl;
            float kv[CPL], qv[CPL];
#pragma unroll
            for (int e = 0; e < CPL; ++e) {
                kv[e] = ks[tl][j * CPL + e];
                qv[e] = qs[tl][j * CPL + e];
            }
            if (a.normalize_qk) {
                // x / sqrt(sum(x^2) + 1e-6) over the whole [S] row (gated_delta_rule.h:35-36)
                float kk = 0.0f, qq = 0.0f;
#pragma unroll
                for (int e = 0; e < CPL; ++e) {
                    kk = fmaf(kv[e], kv[e], kk);
                    qq = fmaf(qv[e], qv[e], qq);
                }
                const float kinv = 1.0f / sqrtf(row_sum16(kk) + 1.0e-6f);
                const float qinv = 1.0f / sqrtf(row_sum16(qq) + 1.0e-6f);
#pragma unroll
                for (int e = 0; e < CPL; ++e) {
                    kv[e] *= kinv;
                    qv[e] *= qinv;
                }
            }
            const float alpha = gs[tl];
            const float beta = bs[tl];
            const float vr = vs[tl][rl];
            float partial = 0.0f;
#pragma unroll
            for (int e = 0; e < CPL; ++e) {
                row[e] *= alpha;
                partial = fmaf(row[e], kv[e], partial);
            }
            const float delta = beta * (vr - row_sum16(partial));
            float o = 0.0f;
#pragma unroll
            for (int e = 0; e < CPL; ++e) {
                row[e] = fmaf(delta, kv[e], row[e]);
                o = fmaf(row[e], qv[e], o);
            }
            o = row_sum16(o);
            const int64_t hv_t = static_cast<int64_t>(t) * a.Hv + h;
            if (j == 0) { a.out[hv_t * S + r] = f32_to_bf16(a.scale * o); }
            if (a.initial_slot != nullptr) {
                float* dst = a.states + static_cast<int64_t>(t) * a.Hv * head_elems + row_off;
#pragma unroll
                for (int i = 0; i < CPL; i += (CPL >= 4 ? 4 : CPL)) {
                    if constexpr (CPL >= 4) {
                        store_snapshot(dst + i, f4v{row[i], row[i + 1], row[i + 2], row[i + 3]});
                    } else {
#pragma unroll
                        for (int e = 0; e < CPL; ++e) { dst[e] = row[e]; }
                    }
                }
            }
        }
    }
    if (a.initial_slot == nullptr) {
        float* dst = a.state_out + row_off;
#pragma unroll
        for (int e = 0; e < CPL; ++e) { dst[e] = row[e]; }
    }
}

// One thread per channel c: u = (state window, oldest first) ++ x[c, :];
// out[c, t] = BF16(SiLU(sum_j w[c, j] * u[t - 3 + j])) (include/ninfer/ops/causal_conv1d_silu.h:9-19).
// The window after token t goes to snapshot slot t, or the final window to state_out.
__global__ __launch_bounds__(256) void conv1d_silu_kernel(ConvArgs a) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= a.C) { return; }
    // x of the first kConvTokens tokens is loaded before the slot-dependent window loads.
    constexpr int kConvTokens = 16;
    uint16_t xb[kConvTokens];
#pragma unroll
    for (int i = 0; i < kConvTokens; ++i) { xb[i] = i < a.T ? a.x[static_cast<int64_t>(i) * a.C + c] : 0; }
    const uint16_t* win = a.state_in;
    if (a.initial_slot != nullptr) {
        const int slot = *a.initial_slot;
        if (slot < 0 || slot >= a.slots) { return; }
        win = a.states + static_cast<int64_t>(slot) * 3 * a.C;
    }
    uint16_t u0 = win[c], u1 = win[a.C + c], u2 = win[2 * a.C + c];
    // weight [C, 4] with C fastest: tap j of channel c at j * C + c
    const float w0 = bf16_to_f32(a.weight[c]), w1 = bf16_to_f32(a.weight[a.C + c]);
    const float w2 = bf16_to_f32(a.weight[2 * a.C + c]), w3 = bf16_to_f32(a.weight[3 * a.C + c]);
#pragma unroll 1
    for (int t = 0; t < a.T; ++t) {
        uint16_t xt;
        if (t < kConvTokens) {
#pragma unroll
            for (int i = 0; i < kConvTokens; ++i) {
                if (i == t) { xt = xb[i]; }
            }
        } else {
            xt = a.x[static_cast<int64_t>(t) * a.C + c];
        }
        float acc = w0 * bf16_to_f32(u0);
        acc = fmaf(w1, bf16_to_f32(u1), acc);
        acc = fmaf(w2, bf16_to_f32(u2), acc);
        acc = fmaf(w3, bf16_to_f32(xt), acc);
        a.out[static_cast<int64_t>(t) * a.C + c] = f32_to_bf16(acc / (1.0f + expf(-acc)));
        u0 = u1;
        u1 = u2;
        u2 = xt;
        if (a.initial_slot != nullptr) {
            uint16_t* dst = a.states + static_cast<int64_t>(t) * 3 * a.C;
            dst[c] = u0;
            dst[a.C + c] = u1;
            dst[2 * a.C + c] = u2;
        }
    }
    if (a.initial_slot == nullptr) {
        a.state_out[c] = u0;
        a.state_out[a.C + c] = u1;
        a.state_out[2 * a.C + c] = u2;
    }
}

// include/ninfer/ops/scalar.h:27-30.
__global__ void scalar_kernel(int32_t op, const int32_t* src, int32_t* dst32, long long* dst64, int32_t value) {
    if (threadIdx.x != 0) { return; }
    switch (op) {
    case 0: *dst32 = value; break;
    case 1: *dst32 = *src; break;
    case 2: *dst32 = *dst32 + 1; break;
    default: *dst64 = *dst64 + 1; break;
    }
}

} // namespace

void launch_gdn_recurrent(const GdnArgs& a, int32_t S, hipStream_t stream) {
    const dim3 grid(S / kGdnRows, a.Hv);
    const dim3 block(kGdnThreads);
    switch (S) {
    case 16: hipLaunchKernelGGL(gdn_recurrent_kernel<16>, grid, block, 0, stream, a); break;
    case 32: hipLaunchKernelGGL(gdn_recurrent_kernel<32>, grid, block, 0, stream, a); break;
    case 64: hipLaunchKernelGGL(gdn_recurrent_kernel<64>, grid, block, 0, stream, a); break;
    case 128: hipLaunchKernelGGL(gdn_recurrent_kernel<128>, grid, block, 0, stream, a); break;
    default: throw Unsupported("gated_delta_rule: head dimension must be 16, 32, 64, or 128");
    }
    check_launch("gdn_recurrent_kernel");
}

void launch_conv1d_silu(const ConvArgs& a, hipStream_t stream) {
    const int threads = 256;
    hipLaunchKernelGGL(conv1d_silu_kernel, dim3((a.C + threads - 1) / threads), dim3(threads), 0, stream, a);
    check_launch("conv1d_silu_kernel");
}

void launch_scalar_op(int32_t op, const int32_t* src, int32_t* dst32, long long* dst64, int32_t value,
                      hipStream_t stream) {
    hipLaunchKernelGGL(scalar_kernel, dim3(1), dim3(64), 0, stream, op, src, dst32, dst64, value);
    check_launch("scalar_kernel");
}

} // namespace nmi
