// Launch interface of the Q6G64_F16S RowSplit linear kernels (linear_q6.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "common.h"

namespace nmi {

inline constexpr int kLinearGrid = 256;       // persistent workgroups (one per CU)
inline constexpr int kLinearMaxWaves = 16;    // waves per workgroup
inline constexpr int kLinearMaxPaddedK = 8192;

struct LinearArgs {
    const uint8_t* qdata;   // nibble plane: N x G x 32 B (element i of a group: byte i/2, low nibble if even)
    const uint8_t* qhigh;   // high plane: N x G x 16 B (element i: bits 2i, 2i+1)
    const uint16_t* scales; // FP16 per (row, group): N x G
    const uint16_t* x;      // BF16 [K, T]
    uint16_t* out;          // BF16 [N, T], or null (argmax only)
    uint64_t* keys;         // argmax partial keys [T][waves], or null
    // Top-cap form (the lm_head half of stochastic acceptance): per column, per workgroup, the
    // kCandidateCap largest keys of the penalty-adjusted BF16 logits over rows [0, valid_rows),
    // descending and 0-padded, at cand[(column * grid + workgroup) * kCandidateCap]; null = off.
    uint64_t* cand;
    const nmi_sampling_config* config; // [B] device configs (column t belongs to sequence t / cols_per_seq)
    const int32_t* drafts;             // [cols_per_seq - 1, B]: the penalty overlay of each column
    int32_t cols_per_seq;
    int64_t nib_bytes, high_bytes, scale_bytes;
    int32_t N, K, Kp, G, T;
    int32_t t0, tp;         // this pass: columns [t0, t0 + tp)
    int32_t valid_rows;     // argmax rows [0, valid_rows)
    int32_t ntiles;         // ceil(N / 16)
    int32_t waves;          // total waves of the launch (key stride)
};

// Columns per pass and waves per workgroup for a problem (LDS fit), and the LDS bytes.
struct LinearPlan {
    bool wide;       // K-outer form: 32 or 64 columns per pass (T > 16)
    int32_t tp;      // 4, 8, 16, or 32 / 64 (wide)
    int32_t waves;   // per workgroup
    int32_t cg;      // groups of 64 codes per streamed chunk (4 or 8)
    int32_t grid;    // workgroups
    size_t lds;
    int32_t passes;
};
// K: the unpadded K (the wide form needs K % 8 == 0: x columns start 16-byte aligned).
LinearPlan plan_linear(int32_t N, int32_t Kp, int32_t T, bool top_cap, int32_t K);
size_t linear_argmax_workspace_bytes(int32_t T);
// Candidate-list bytes of the top-cap form for T columns (any plan: at most one list per CU).
size_t linear_topcap_workspace_bytes(int32_t T);

void launch_linear_q6(LinearArgs a, const LinearPlan& p, hipStream_t stream);
void launch_linear_argmax_reduce(const uint64_t* keys, int32_t T, int32_t waves, int32_t* out, hipStream_t stream);

} // namespace nmi
