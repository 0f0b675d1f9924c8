// Host-side interface of the general (Mode F) acceptance kernels (general_accept.hip).
#pragma once

#include "common.h"

namespace nmi {

inline constexpr int32_t kGenTile = 4096;       // tokens per tile (histogram passes)
inline constexpr int32_t kGenDrawTile = 1024;   // tokens per tile of the draw passes
inline constexpr int32_t kGenBins = 256;        // histogram bins per level
inline constexpr int32_t kGenMaxTiles = 256;    // one tile per thread in the per-column scans
inline constexpr int32_t kGenDescBytes = 64;    // per-column nucleus descriptor
inline constexpr int32_t kGenDraftEntryBytes = 8; // per-draft accept-test inputs

// Workspace layout, shared by the size query and the launch.
struct GenPlan {
    int32_t ncols = 0;  // K + 1 target columns then K draft columns
    int32_t ntiles = 0;
    int32_t ndraw = 0;  // draw tiles
    size_t tile_max_offset = 0;
    size_t cmass_offset = 0;
    size_t ccount_offset = 0;
    size_t desc_offset = 0;
    size_t fine_offset = 0;
    size_t fine_total_offset = 0; // per column: fine counts summed over tiles
    size_t tile_res_offset = 0;
    size_t tile_p_offset = 0;
    size_t dtab_offset = 0;   // per draft: BF16 bits of its target/draft logits, its id
    size_t bytes = 0;
};

struct GenLaunch {
    const uint16_t* logits = nullptr;       // BF16 [rows, >=K+1, B]
    const uint16_t* draft_logits = nullptr; // BF16 [rows_d, >=K, B]
    const int32_t* drafts = nullptr;        // I32 [K, B]
    const float* u_accept = nullptr;        // FP32 [K+1, B]
    const float* u_residual = nullptr;      // FP32 [1, B]
    int32_t* length = nullptr;
    int32_t* token = nullptr;
    int32_t* sampled_out = nullptr;         // I32 [K+1, B]
    int32_t* num_sampled = nullptr;
    int32_t* accepted = nullptr;
    int64_t* stats = nullptr;               // I64 [stats_stride, B]
    const nmi_general_config* config = nullptr; // device pointer
    int64_t logit_col = 0;
    int64_t logit_seq = 0;
    int64_t draft_col = 0;
    int64_t draft_seq = 0;
    int32_t stats_stride = 0;
    int32_t token_domain = 0;
    int32_t K = 0;
    int32_t B = 0;
};

GenPlan plan_general(int32_t token_domain, int32_t K, int32_t B);
void launch_general_accept(const GenLaunch& l, const GenPlan& plan, void* workspace, hipStream_t stream);

} // namespace nmi
