// CPU oracle for the MTP verify step. TEST INFRASTRUCTURE ONLY.
//
// This library is a scalar restatement of the reference semantics that the HIP path is checked
// against. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and
// only as the checker or as the reported CPU baseline; the product library never links it.
//
// Every function cites the reference file:line it restates (paths relative to the reference
// repository root). Functions whose result no reference vector, known-answer test or closed form
// pins are marked "parity unpinned" here and in the design notes.
//
// Conventions: BF16 and FP16 values travel as their raw uint16 bit patterns. Tensor layouts are
// the reference's column-major `ne` order (first index fastest):
//   q        BF16 [D, Hq, T, B]
//   k/v new  BF16 [D, Hkv, T, B]
//   codes    I8   [D, P, Hkv, B]        (P = padded context)
//   scales   FP16 [D/64, P, Hkv, B]
//   logits   BF16 [physical_rows, C, B]
#pragma once

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

// ---- scalar numerics -------------------------------------------------------------------------
uint16_t orc_f32_to_f16_bits(float x);
float orc_f16_bits_to_f32(uint16_t h);
uint16_t orc_f32_to_bf16_bits(float x);
float orc_bf16_bits_to_f32(uint16_t h);
float orc_det_expf(float x);
uint64_t orc_splitmix64(uint64_t x);
float orc_sampling_uniform(uint64_t seed, int32_t position, int32_t purpose, uint32_t sub);
uint64_t orc_sort_key(float v, int32_t idx);

// ---- INT8 group-64 codec ---------------------------------------------------------------------
// One group of `n` (=64) BF16 values -> n codes + one FP16 scale.
void orc_quantize_group(const uint16_t* src_bf16, int32_t n, int8_t* codes, uint16_t* scale_bits);

// Append T new K/V columns into the cache rows positions[t] (per sequence b).
void orc_kv_append(const uint16_t* k, const uint16_t* v, const int32_t* positions, int32_t T,
                   int32_t B, int32_t Hkv, int32_t D, int32_t padded_context, int8_t* k_codes,
                   int8_t* v_codes, uint16_t* k_scales, uint16_t* v_scales);

// ---- attention -------------------------------------------------------------------------------
// FP64 ideal attention over BF16 Q and FP32-decoded cache values. For sequence b, query token t
// sees every history row j < positions[0,b] and the new rows positions[u,b] with u visible from t:
// u <= t (causal, parents == NULL) or u an ancestor-or-self of t (parents[t,b] = parent node index,
// -1 for a root). `threads` <= 0 uses hardware_concurrency.
void orc_attention(const uint16_t* q, const int8_t* k_codes, const int8_t* v_codes,
                   const uint16_t* k_scales, const uint16_t* v_scales, const int32_t* positions,
                   const int32_t* parents, int32_t T, int32_t B, int32_t Hq, int32_t Hkv,
                   int32_t D, int32_t padded_context, double scale, double* out, int32_t threads);

// Same oracle over a BF16 cache: k_cache/v_cache BF16 [B][Hkv][padded_context][D], values used as
// stored (the new rows are expected to be in the planes already).
void orc_attention_bf16(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                        const int32_t* positions, const int32_t* parents, int32_t T, int32_t B,
                        int32_t Hq, int32_t Hkv, int32_t D, int32_t padded_context, double scale,
                        double* out, int32_t threads);

// ---- lm_head: Q6G64_F16S RowSplit linear ----------------------------------------------------------
// out[n + N*t] = sum_k decode(w)[n,k] * bf16(x[k + K*t]) in FP64, decode = sign-extended 6-bit code
// times the group's FP16 scale, exactly. qdata: N x G x 32 B, qhigh: N x G x 16 B, scales: N x G
// FP16, G = align_up(K, 128) / 64. `threads` <= 0 uses hardware_concurrency.
void orc_linear_q6(const uint8_t* qdata, const uint8_t* qhigh, const uint16_t* scales, int32_t N,
                   int32_t K, const uint16_t* x, int32_t T, double* out, int32_t threads);

// ---- recurrent state of the hybrid layers -----------------------------------------------------
// Gated DeltaNet recurrence in FP64 (one sequence). q/k BF16 [S,Hqk,T], v BF16 [S,Hv,T], g/beta
// FP32 [Hv,T], state_in FP32 [S,S,Hv] (row = value index, key index fastest). normalize_qk: q and
// k rows become float(x / sqrt(sum(x^2) + 1e-6)) first. out [S,Hv,T] and state_out [S,S,Hv] in
// FP64; snapshots (may be NULL) receive the state after token t at t * Hv*S*S.
void orc_gdn_recurrent(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* g,
                       const float* beta, const float* state_in, int32_t S, int32_t Hqk,
                       int32_t Hv, int32_t T, double scale, int32_t normalize_qk, double* out,
                       double* state_out, double* snapshots);

// Width-4 causal depthwise convolution + SiLU in FP64. x BF16 [C,T], weight BF16 [C,4], state
// BF16 [C,3] (oldest first). out [C,T] in FP64 (before the BF16 boundary); windows (may be NULL)
// receives the BF16 window after token t at t * 3*C, in the [C,3] layout.
void orc_causal_conv1d_silu(const uint16_t* x, const uint16_t* weight, const uint16_t* state,
                            int32_t C, int32_t T, double* out, uint16_t* windows);

// ---- argmax ----------------------------------------------------------------------------------
void orc_argmax(const uint16_t* logits, int32_t physical_rows, int32_t columns, int32_t valid_rows,
                int32_t* out);

// ---- speculative acceptance (reference semantics, "Mode R") ----------------------------------
typedef struct {
    float temperature;
    int32_t top_k;
    float top_p;
    float min_p;
    float presence_penalty;
    float frequency_penalty;
    uint64_t seed;
} orc_sampling_config;

// State scalars live in the caller's host memory; `token_counts` may be NULL.
void orc_mtp_prepare_alignment_ids(const int32_t* verify_ids, int32_t T, int32_t token, int32_t accepted,
                                   int32_t* alignment_ids);
void orc_prepare_verify_inputs(int32_t token, const int32_t* drafts, int32_t length, int32_t K,
                               int32_t* verify_ids, int32_t* positions);

void orc_speculative_accept(const int32_t* target_tokens, const uint16_t* logits,
                            int32_t physical_rows, const int32_t* drafts, int32_t K,
                            int32_t* length, int32_t* token, int32_t* sampled_out,
                            int32_t* num_sampled, int32_t* accepted, int64_t* stats,
                            int32_t token_domain, const orc_sampling_config* cfg,
                            int32_t* token_counts);

// Truncated distribution of one column (cap <= 20 candidates), exposed for tests.
int32_t orc_truncated_distribution(const uint16_t* column, int32_t token_domain,
                                   const orc_sampling_config* cfg, const int32_t* token_counts,
                                   const int32_t* overlay, int32_t overlay_len, int32_t* cand_idx,
                                   float* prob);
int32_t orc_pick_from_support(const int32_t* cand_idx, const float* prob, int32_t n,
                              int32_t exclude, float u);

// ---- general acceptance ("Mode F", extension: parity unpinned by the reference) ---------------
// Full-vocabulary temperature + top-p distributions in 64-bit fixed point for target columns
// 0..K and draft columns 0..K-1; accept draft i iff u_accept[i] * q_i(d_i) < p_i(d_i); on the first
// rejection sample the normalized residual max(0, p_i - q_i) with u_residual; after K accepts
// sample column K with u_accept[K].
typedef struct {
    float temperature;
    float top_p;
} orc_general_config;

void orc_general_accept(const uint16_t* target_logits, const uint16_t* draft_logits,
                        int32_t physical_rows, const int32_t* drafts, int32_t K,
                        int32_t token_domain, const orc_general_config* cfg,
                        const float* u_accept, float u_residual, int32_t* length, int32_t* token,
                        int32_t* sampled_out, int32_t* num_sampled, int32_t* accepted,
                        int64_t* stats);

// Fixed-point weights and nucleus of one column, exposed for tests. Returns the nucleus size;
// writes the nucleus mass (sum of fixed-point weights) to *nucleus_mass and the full mass to
// *total_mass. `in_nucleus` (optional) receives 0/1 per token.
int32_t orc_general_column(const uint16_t* column, int32_t token_domain,
                           const orc_general_config* cfg, uint64_t* weights, uint8_t* in_nucleus,
                           uint64_t* nucleus_mass, uint64_t* total_mass);

// ---- commit / rollback / compaction ------------------------------------------------------------
// Quantize-and-commit the prefix [0, commit_count) of T new K/V columns into rows positions[i];
// rejected columns write nothing (restates include/ninfer/ops/kv_cache_append_prefix.h:22-32 for
// an INT8 cache).
void orc_kv_commit_prefix(const uint16_t* k, const uint16_t* v, const int32_t* positions,
                          int32_t T, int32_t commit_count, int32_t Hkv, int32_t D,
                          int32_t padded_context, int8_t* k_codes, int8_t* v_codes,
                          uint16_t* k_scales, uint16_t* v_scales);

// Zero codes and scales of rows positions[i] for i in [keep_count, T).
void orc_kv_rollback(const int32_t* positions, int32_t T, int32_t keep_count, int32_t Hkv,
                     int32_t D, int32_t padded_context, int8_t* k_codes, int8_t* v_codes,
                     uint16_t* k_scales, uint16_t* v_scales);

// Move rows base + path[j] to base + j for j < count (path strictly increasing, path[j] >= j).
void orc_kv_compact_path(int32_t base, const int32_t* path, int32_t count, int32_t Hkv, int32_t D,
                         int32_t padded_context, int8_t* k_codes, int8_t* v_codes,
                         uint16_t* k_scales, uint16_t* v_scales);

// ---- tree verification ---------------------------------------------------------------------------
// Greedy longest accepted root-to-leaf chain. Node u (0 = root, parents[0] = -1) carries draft
// token node_tokens[u] (ignored for the root) and target argmax target_tokens[u]. A child c of an
// accepted node n is accepted iff node_tokens[c] == target_tokens[n]. Among accepted nodes the
// deepest wins; ties go to the lowest node index. Writes the root-to-winner path (node indices)
// to path and returns its length (>= 1). The produced tokens are node_tokens[path[1..]] followed by
// target_tokens[path[last]].
int32_t orc_tree_longest_path(const int32_t* parents, const int32_t* node_tokens,
                              const int32_t* target_tokens, int32_t nodes, int32_t* path);

// ---- test-input generation (synth.cpp; not a restatement) ----------------------------------------
// n seeded N(0, std_dev^2) values as BF16 bits, each replaced by +-outlier_value with probability
// outlier_frac; the result depends on (seed, i) only, not on the thread count.
void orc_fill_normal_bf16(uint64_t seed, size_t n, float std_dev, float outlier_frac,
                          float outlier_value, uint16_t* out, int32_t threads);

#ifdef __cplusplus
}
#endif
