// Launch interfaces of the acceptance kernels (sampler.hip, general_accept.hip).
#pragma once

#include "common.h"

namespace nmi {

inline constexpr int kCandidateCap = 20;          // src/ops/common/sampling_workspace.h:30-31
inline constexpr int kStatsPerPositionOffset = 4; // src/ops/kernel/speculative_round.cuh:15
inline constexpr int kPurposeAccept = 2;          // include/ninfer/ops/sampling.h:14-20
inline constexpr int kPurposeCorrection = 3;
inline constexpr int kPurposeBonus = 4;
inline constexpr int kMaxColumns = 16;            // K <= 15 (reference kSamplerMaxColumns)
inline constexpr int kTileTokens = 4096;   // tokens per candidate tile (256 threads x 16)
inline constexpr int kMaxTreeNodes = 32;
inline constexpr int kMergeMaxTiles = 128;   // tile lists one merge wave holds (2 per lane)
inline constexpr int kMergeWideLists = 256;  // lists of the wide merge (4 per lane)

struct SpecPlan {
    int32_t ntiles = 0;
    size_t partial_offset = 0;
    size_t bytes = 0;
};

struct SpecArgs {
    const int32_t* target_tokens; // [K+1, B]; null: greedy targets are the list heads (fused lm_head)
    const uint16_t* logits;       // [physical_rows, columns_total, B]
    const int32_t* drafts;        // [K, B]
    int32_t* length;              // [B]
    int32_t* token;
    int32_t* sampled_out;         // [K+1, B]
    int32_t* num_sampled;
    int32_t* accepted;
    int64_t* stats;               // [stats_stride, B]
    const nmi_sampling_config* config; // [B] device
    uint64_t* partial;            // [B][columns][ntiles][kCandidateCap] per-tile candidates
    int64_t logits_seq_stride;    // elements between sequences
    int32_t physical_rows;
    int32_t token_domain;
    int32_t K;
    int32_t columns;              // K + 1 (workspace columns)
    int32_t ntiles;
    int32_t stats_stride;
};

SpecPlan plan_spec(int32_t token_domain, int32_t columns, int32_t batch);

// Validates the acceptance state and outputs (drafts [K, B], scalars [B], sampled_out [K+1, B],
// stats [>=4+K, B], config) and fills those fields of the kernel arguments; B out.
SpecArgs check_accept_state(const nmi_tensor* drafts, nmi_tensor* length, nmi_tensor* token,
                            nmi_tensor* sampled_out, nmi_tensor* num_sampled, nmi_tensor* accepted,
                            nmi_tensor* stats, const nmi_sampling_config* config, const std::string& op,
                            int32_t& B);

void launch_argmax(const uint16_t* logits, int32_t* out, int32_t physical_rows, int32_t valid_rows,
                   int32_t columns, hipStream_t stream);
void launch_prepare_verify_inputs(const int32_t* token, const int32_t* drafts, const int32_t* length,
                                  int32_t* verify_ids, int32_t* positions, int32_t K, int32_t B,
                                  hipStream_t stream);
void launch_spec_accept(const SpecArgs& args, int32_t batch, hipStream_t stream);
// Merge + accept alone over up to kMergeWideLists candidate lists per column (the fused lm_head's
// per-workgroup lists in args.partial, ntiles = lists per column).
void launch_spec_merge_accept_wide(const SpecArgs& args, int32_t batch, hipStream_t stream);
void launch_mtp_alignment_ids(const int32_t* verify_ids, const int32_t* token, const int32_t* accepted,
                              int32_t* alignment_ids, int32_t T, hipStream_t stream);
void launch_select_hidden(const uint16_t* hidden, const int32_t* accepted, uint16_t* out,
                          int32_t rows, int32_t cols, hipStream_t stream);
void launch_tree_accept(const int32_t* parents, const int32_t* node_tokens,
                        const int32_t* target_tokens, int32_t N, int32_t B, int32_t* path,
                        int32_t* path_len, int32_t* length, int32_t* token, int32_t* sampled_out,
                        int32_t* num_sampled, int32_t* accepted, int64_t* stats,
                        int32_t stats_stride, hipStream_t stream);

} // namespace nmi
