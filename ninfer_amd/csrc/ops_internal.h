// Host-side launch interfaces between the C ABI (validation, capi.cpp) and the kernel files.
#pragma once

#include "common.h"

namespace nmi {

// A validated INT8-G64 cache view (src/core/kv_cache.h:13-24) with an optional batch dimension.
struct CacheRef {
    int8_t* kc = nullptr;
    int8_t* vc = nullptr;
    uint16_t* ks = nullptr; // FP16 bits
    uint16_t* vs = nullptr;
    uint16_t* kb = nullptr; // BF16 cache planes (kc/vc/ks/vs stay null)
    uint16_t* vb = nullptr;
    int64_t code_seq = 0;  // code elements between sequences
    int64_t scale_seq = 0; // scale elements between sequences
    int32_t P = 0;         // padded context
    int32_t Hkv = 0;
    int32_t D = 0;
    int32_t B = 1;
};

// Split-K plan for the verify attention: shared by the workspace query and the launch, like the
// reference's shared layout builder (src/ops/wrapper/gqa_attention.cpp:138-153,229-245).
struct SplitPlan {
    int32_t G = 0;                // query heads per KV head
    int32_t tokens_per_chunk = 0; // tokens whose G rows fit one 32-row MFMA tile pair
    int32_t row_chunks = 0;
    int32_t nsplit = 0;           // key splits per (sequence, row chunk, KV head)
    int32_t keys_per_split = 0;   // multiple of 128 (B == 1)
    int32_t split_slots = 0;      // partial slots per (row chunk, KV head)
    int32_t split_budget = 0;     // B > 1: most splits per (row chunk, KV head) the device cuts the batch into
    int32_t rows_per_slot = 32;   // query rows of one partial slot: 32, or 80 (one row chunk of 5 MFMA tiles)
    bool cached_partials = false; // partials written and read through the caches (long B = 1 splits)
    bool b1_device_plan = false;  // B = 1: the launched splits divide the device window (wide envelopes)
    size_t part_o_offset = 0;
    size_t part_ml_offset = 0;
    size_t seq_table_offset = 0; // B > 1: per sequence (first slot, split count)
    size_t bytes = 0;
};

inline constexpr int32_t kAttnRowsPerTile = 32;
inline constexpr int32_t kAttnWideRows = 80;          // INT8, head_dim 128: up to 80 rows in one row chunk
inline constexpr int32_t kAttnTargetWorkgroups = 512; // 2 per CU on 256 CUs
inline constexpr int32_t kAttnMinKeysPerSplit = 256;
inline constexpr int32_t kAttnMaxTokens = 32;
// B = 1 splits of at least this many keys write their partials with ordinary (cached) stores and the
// merge reads them with ordinary loads; shorter splits use the non-temporal forms. Measured on
// MI355X: C3 (4,096-key splits) 99.3-99.5 -> 98.2-98.3 us per layer; C2 (256-key splits) 13.32-13.35
// us with non-temporal partials against 13.52-13.54 us cached.
inline constexpr int32_t kAttnCachedPartialKeys = 1024;

// wide_rows: the INT8 head_dim-128 cache may serve 33..80 query rows (T x G) in one row chunk of
// five 16-row tiles (one workgroup per CU) instead of several 32-row chunks that each stream every key.
SplitPlan plan_attention(int32_t Hq, int32_t Hkv, int32_t D, int32_t T, int32_t B,
                         uint32_t max_visible_keys, bool wide_rows);

// Marks a batch-1 plan whose splits are chosen on the device from the actual window, when the
// envelope's shortest window would leave more than half of its splits empty (INT8, 32-row slots).
void choose_b1_device_plan(SplitPlan& p, int32_t B, uint32_t min_visible_keys, bool int8_cache);

// The largest plan_attention(Hq, Hkv, D, T, 1, keys, either form).bytes over every envelope (keys >= 1).
size_t attention_workspace_bound(int32_t Hq, int32_t Hkv, int32_t D, int32_t T);

// Size of the per-device static split scratch of nmi_gqa_attention_noalloc. 16 MiB holds every plan
// of one sequence (T <= 32, any context, the registered geometries: at most 5.2 MiB, the 80-row
// form at 40/8 heads and T = 16, 8 KV heads x 32 splits x 80 rows x 128 dims x 2 B of FP16 O / l
// plus the FP32 (m, l) pairs) and of batches up to ~240 sequences at T <= 6 (64 sequences at T = 4:
// 4.1 MiB); larger batches need more and are rejected.
inline constexpr size_t kStaticScratchBytes = size_t{16} << 20;

// The calling device's static scratch (resolved on first use per device); throws Unsupported when
// `need` exceeds kStaticScratchBytes.
void* static_scratch(size_t need, const std::string& op);

// Device-side bounds of a prefix commit: a device count outside [min_count, max_count] writes
// nothing (the reference's launch-resource envelope, kv_cache_append_prefix.cuh), and position p
// lands in row p & slot_mask (every bit for a linear cache, capacity - 1 for a cyclic ring).
struct CommitBounds {
    int32_t min_count = 0;
    int32_t max_count = 0x7FFFFFFF;
    int32_t slot_mask = 0x7FFFFFFF;
};

// Quantize-append (INT8-G64) or copy (BF16): columns t (< count[b] when count != nullptr, and only
// when count[b] is inside the bounds) of k/v BF16 [D, Hkv, T, B] into rows positions[t + T*b].
void launch_kv_append(const uint16_t* k, const uint16_t* v, const int32_t* positions,
                      const int32_t* count, CommitBounds bounds, int32_t T, const CacheRef& cache,
                      hipStream_t stream);

// Split-K verify attention over cache rows; parents == nullptr is the causal mask. With k_new/v_new
// (A1) the new columns are quantized into rows positions[t] first, by the owning split.
void launch_verify_attention(const uint16_t* q, const uint16_t* k_new, const uint16_t* v_new,
                             const int32_t* positions, const int32_t* parents, int32_t T,
                             int32_t Hq, const CacheRef& cache, float scale, uint32_t max_keys,
                             void* workspace, const SplitPlan& plan, void* out, bool out_f32,
                             hipStream_t stream);

// Commit helpers (kv_commit.hip).
void launch_kv_rollback(const int32_t* positions, const int32_t* keep_count, int32_t T,
                        const CacheRef& cache, hipStream_t stream);
void launch_kv_compact_path(const int32_t* base_position, const int32_t* path,
                            const int32_t* path_len, int32_t T, const CacheRef& cache,
                            hipStream_t stream);

} // namespace nmi
