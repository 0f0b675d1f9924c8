/*
 * ninfer_amd — C ABI of the MI355X (gfx950) MTP speculative-decoding verify step.
 *
 * Every entry point validates its arguments on the host before any launch, returns an
 * nmi_status, and launches only hand-written gfx950 kernels on the caller's stream. Nothing
 * allocates device memory, synchronizes, or reads device memory back: state scalars (length,
 * token, commit counts) and sampling parameters are device-resident, so every call can be
 * captured in a HIP graph and replayed. Transient storage is a caller-owned region sized by the
 * matching *_workspace_bytes query (the reference's WorkspaceArena contract).
 *
 * Tensors use the reference's non-owning view (src/core/tensor.h:11-28): a data pointer, a dtype,
 * ne[4] element counts (ne[0] fastest) and nb[4] byte strides. The C++ drop-in layer in
 * include/ninfer_amd/ops.hpp turns statuses back into the reference's exceptions
 * (std::invalid_argument / std::overflow_error).
 *
 * Reference: Neroued/ninfer, include/ninfer/ops/{gqa_attention,argmax,sampling,
 * speculative_round,mtp_round,kv_cache_append_prefix,gated_delta_rule,causal_conv1d_silu,
 * scalar}.h. Entries marked EXTENSION have no reference symbol.
 */
#ifndef NINFER_AMD_H
#define NINFER_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Same object as hipStream_t (0 = the null stream). */
typedef struct ihipStream_t* nmi_stream_t;

typedef enum nmi_status {
    NMI_OK = 0,
    NMI_INVALID_ARGUMENT = 1, /* reference: std::invalid_argument */
    NMI_OVERFLOW = 2,         /* reference: std::overflow_error */
    NMI_HIP_ERROR = 3,        /* launch failure (reference: CUDA_CHECK abort, src/core/device.cu:38-43) */
    NMI_UNSUPPORTED = 4       /* valid request outside the built kernel set */
} nmi_status;

/* src/core/dtype.h:8-16 — same values as ninfer::DType, so a binding converts with a cast. */
typedef enum nmi_dtype {
    NMI_BF16 = 0,
    NMI_FP32 = 1,
    NMI_I32 = 2,
    NMI_U8 = 3,
    NMI_I64 = 4,
    NMI_I8 = 5,
    NMI_FP16 = 6
} nmi_dtype;

/* src/core/tensor.h:11-15 */
typedef struct nmi_tensor {
    void* data;
    int32_t dtype; /* nmi_dtype */
    int32_t ne[4];
    int64_t nb[4];
} nmi_tensor;

/* src/core/kv_cache.h:13-24. INT8-G64: k/v are I8 [D, P, Hkv] (or [D, P, Hkv, B] for a batch of
 * sequences), k_scale/v_scale FP16 [D/64, P, Hkv(, B)], P = padded_context = align_up(max, 128). */
typedef struct nmi_kv_layer_view {
    nmi_tensor k;
    nmi_tensor v;
    nmi_tensor k_scale;
    nmi_tensor v_scale;
    uint32_t max_context;
    uint32_t padded_context;
    int32_t num_kv_heads;
    int32_t head_dim;
    int32_t dtype; /* NMI_I8 (INT8-G64) or NMI_BF16 */
    int32_t quant_group;
} nmi_kv_layer_view;

/* src/core/kv_cache.h:32-43 — cyclic K/V storage: absolute position p lives in row p % capacity.
 * Planes as in nmi_kv_layer_view with P = padded_capacity. */
typedef struct nmi_cyclic_kv_layer_view {
    nmi_tensor k;
    nmi_tensor v;
    nmi_tensor k_scale;
    nmi_tensor v_scale;
    uint32_t capacity;
    uint32_t padded_capacity;
    int32_t num_kv_heads;
    int32_t head_dim;
    int32_t dtype; /* NMI_BF16 (the reference's) or NMI_I8 (INT8-G64) */
    int32_t quant_group;
} nmi_cyclic_kv_layer_view;

/* include/ninfer/ops/gqa_attention.h:13-16 */
typedef struct nmi_gqa_envelope {
    uint32_t min_visible_keys;
    uint32_t max_visible_keys;
} nmi_gqa_envelope;

/* include/ninfer/ops/sampling.h:24-33 — binary-identical device-resident layout (40 bytes). */
typedef struct nmi_sampling_config {
    float temperature;
    int32_t top_k;
    float top_p;
    float min_p;
    float presence_penalty;
    float frequency_penalty;
    unsigned long long seed;
    int32_t* token_counts;
} nmi_sampling_config;

/* include/ninfer/ops/kv_cache_append_prefix.h:18-21 */
typedef struct nmi_commit_envelope {
    uint32_t min_count;
    uint32_t max_count;
} nmi_commit_envelope;

/* EXTENSION: device-resident parameters of the general (Mode F) acceptance. */
typedef struct nmi_general_config {
    float temperature;
    float top_p;
} nmi_general_config;

/* src/core/tensor.h:30-66 — the reference's quantized weight view, field for field. qtype values
 * are ninfer::QType (Q4G64_F16S = 0, Q5G64_F16S = 1, Q6G64_F16S = 2, W8G32_F16S = 3), layout
 * ninfer::QuantLayout (RowSplit = 0). */
typedef struct nmi_weight {
    const void* payload;
    uint64_t payload_bytes;
    uint64_t high_plane_bytes;
    int32_t qtype;
    uint32_t group_size;
    int32_t shape[4];
    int32_t padded_shape[4];
    uint32_t ndim;
    const void* qdata;
    const void* qhigh;
    const void* scales;
    int32_t n;
    int32_t k;
    int32_t group;
    int32_t layout;
    int32_t scale_dtype; /* nmi_dtype */
} nmi_weight;

#define NMI_Q6G64_F16S 2
#define NMI_ROW_SPLIT 0

/* Thread-local text of the last non-OK status. */
const char* nmi_last_error(void);
/* Library build identification (architecture list and kernel set). */
const char* nmi_build_info(void);

/* ---------------------------------------------------------------- verify attention (part a, c) */

/* Replaces gqa_attention_workspace_bytes (include/ninfer/ops/gqa_attention.h:50). The split-K
 * partial count depends on the geometry and on the envelope's max_visible_keys, so both are
 * inputs here. batch = number of sequences (q.ne[3]). */
size_t nmi_gqa_attention_workspace_bytes(int32_t q_heads, int32_t kv_heads, int32_t head_dim,
                                         int32_t tokens, int32_t batch,
                                         uint32_t max_visible_keys);

/* Replaces gqa_attention_workspace_bytes(q_heads, tokens) with its reference signature
 * (include/ninfer/ops/gqa_attention.h:50; src/ops/wrapper/gqa_attention.cpp:229-245), as a status
 * plus the size: the geometry follows from q_heads (24 -> 4 KV heads and 16 -> 2 at head_dim 256,
 * the reference's registered ones; 40 -> 8 at head_dim 128), and the size covers every execution
 * envelope of one sequence (above 32 tokens: the prompt route's launches of 32 and its last one).
 * tokens <= 0 give 0; other q_heads NMI_INVALID_ARGUMENT. */
int nmi_gqa_attention_workspace_bound(int32_t q_heads, int32_t tokens, size_t* bytes);

/* A1, replaces gqa_attention (include/ninfer/ops/gqa_attention.h:71-73): quantize-append the T
 * new K/V columns at rows positions[t] and compute causal GQA over rows [0, positions[t]].
 * q/out BF16 [D, Hq, T(, B)]; k/v BF16 [D, Hkv, T(, B)]; positions I32 [T(, B)] sequential;
 * out may also be FP32 (EXTENSION). T above 32 is the reference's prompt route
 * (src/ops/wrapper/gqa_attention.cpp:202-213): one sequence (B = 1); the rows are appended first,
 * then the tokens attend in launches of 32 through the same workspace. */
int nmi_gqa_attention(const nmi_tensor* q, const nmi_tensor* k, const nmi_tensor* v,
                      const nmi_tensor* positions, float scale, const nmi_kv_layer_view* cache,
                      nmi_gqa_envelope envelope, void* workspace, size_t workspace_bytes,
                      nmi_tensor* out, nmi_stream_t stream);

/* No counterpart in the reference: A1 exactly as nmi_gqa_attention (same validation, kernels and
 * results), for callers that cannot allocate or pass a workspace (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc). The split-K partials go to a static
 * 16 MiB per-device scratch array instead of a workspace, so the call allocates nothing; a plan
 * needing more (NMI_UNSUPPORTED) must use nmi_gqa_attention. Calls that overlap on one GPU (two
 * streams at once) race on that scratch; consecutive calls need no clearing in between. */
int nmi_gqa_attention_noalloc(const nmi_tensor* q, const nmi_tensor* k, const nmi_tensor* v,
                              const nmi_tensor* positions, float scale, const nmi_kv_layer_view* cache,
                              nmi_gqa_envelope envelope, nmi_tensor* out, nmi_stream_t stream);

/* A2, replaces gqa_kv_append (include/ninfer/ops/gqa_attention.h:80-81). */
int nmi_gqa_kv_append(const nmi_tensor* k, const nmi_tensor* v, const nmi_tensor* positions,
                      const nmi_kv_layer_view* cache, nmi_stream_t stream);

/* A3, replaces gqa_attention_cached (include/ninfer/ops/gqa_attention.h:89-91). */
int nmi_gqa_attention_cached(const nmi_tensor* q, const nmi_tensor* positions, float scale,
                             const nmi_kv_layer_view* cache, nmi_gqa_envelope envelope,
                             void* workspace, size_t workspace_bytes, nmi_tensor* out,
                             nmi_stream_t stream);

/* EXTENSION (tree verification): A1/A3 with an ancestor mask. parents I32 [T(, B)], parents[0] =
 * -1, parents[u] < u. Node u occupies row positions[u]; query t sees history rows
 * [0, positions[0]) and the new rows of its ancestors-or-self. A parent outside [0, u) ends the
 * ancestor walk there (nmi_tree_accept_greedy treats it the same way). write_cache = 0 gives A3
 * (k and v may then be NULL). T above 32 returns NMI_UNSUPPORTED (the mask is 32 bits per row). */
int nmi_gqa_attention_tree(const nmi_tensor* q, const nmi_tensor* k, const nmi_tensor* v,
                           const nmi_tensor* positions, const nmi_tensor* parents, float scale,
                           const nmi_kv_layer_view* cache, nmi_gqa_envelope envelope,
                           int32_t write_cache, void* workspace, size_t workspace_bytes,
                           nmi_tensor* out, nmi_stream_t stream);

/* ---------------------------------------------------------------- acceptance (part b) */

/* Replaces argmax (include/ninfer/ops/argmax.h:21): out[t] = min argmax_{v < valid_rows}
 * float(logits[v, t]). logits BF16 [physical_rows, C(, B)], out I32 [C(, B)]. */
int nmi_argmax(const nmi_tensor* logits, nmi_tensor* out, int32_t valid_rows,
               nmi_stream_t stream);

/* Replaces sampling_workspace_bytes (include/ninfer/ops/sampling.h:37). batch = sequences. */
size_t nmi_sampling_workspace_bytes(int32_t token_domain, int32_t columns, int32_t batch);

/* Replaces speculative_prepare_verify_inputs (include/ninfer/ops/speculative_round.h:29-31). */
int nmi_speculative_prepare_verify_inputs(const nmi_tensor* token, const nmi_tensor* drafts,
                                          const nmi_tensor* length, nmi_tensor* verify_ids,
                                          nmi_tensor* positions, nmi_stream_t stream);

/* Replaces speculative_accept_greedy_drafts (include/ninfer/ops/speculative_round.h:68-73):
 * greedy (config->temperature <= 0) or reference stochastic acceptance with the top-20 candidate
 * cap ("Mode R"). `config` is a DEVICE pointer. EXTENSION: a trailing batch dimension
 * (drafts I32 [K, B], logits BF16 [rows, K+1, B], scalars I32 [B], stats I64 [4+K, B]). */
int nmi_speculative_accept_greedy_drafts(const nmi_tensor* target_tokens, const nmi_tensor* logits,
                                         const nmi_tensor* drafts, nmi_tensor* length,
                                         nmi_tensor* token, nmi_tensor* sampled_out,
                                         nmi_tensor* num_sampled, nmi_tensor* accepted,
                                         nmi_tensor* stats, int32_t token_domain,
                                         const nmi_sampling_config* config, void* workspace,
                                         size_t workspace_bytes, nmi_stream_t stream);

/* EXTENSION ("Mode F"): general speculative acceptance with full-vocabulary temperature and
 * top-p for both the target columns (logits BF16 [rows, K+1(, B)]) and the draft columns
 * (draft_logits BF16 [rows, K(, B)]). Accept draft i iff u_accept[i] * q_i(d_i) < p_i(d_i);
 * on the first rejection sample max(0, p_i - q_i) normalized with u_residual; if all K are
 * accepted sample column K with u_accept[K]. uniforms: u_accept FP32 [K+1(, B)],
 * u_residual FP32 [1(, B)]. Probabilities are 64-bit fixed point (bit-exact, order-free).
 * Logits inside the token domain must be finite: a NaN or infinite logit leaves the column's
 * weights, and so the decisions, unspecified. `config` is a DEVICE pointer. */
size_t nmi_general_accept_workspace_bytes(int32_t token_domain, int32_t K, int32_t batch);
int nmi_speculative_accept_general(const nmi_tensor* logits, const nmi_tensor* draft_logits,
                                   const nmi_tensor* drafts, const nmi_tensor* u_accept,
                                   const nmi_tensor* u_residual, nmi_tensor* length,
                                   nmi_tensor* token, nmi_tensor* sampled_out,
                                   nmi_tensor* num_sampled, nmi_tensor* accepted,
                                   nmi_tensor* stats, int32_t token_domain,
                                   const nmi_general_config* config, void* workspace,
                                   size_t workspace_bytes, nmi_stream_t stream);

/* Replaces speculative_select_accepted_hidden (include/ninfer/ops/speculative_round.h:86-87). */
int nmi_speculative_select_accepted_hidden(const nmi_tensor* hidden, const nmi_tensor* accepted,
                                           nmi_tensor* out, nmi_stream_t stream);

/* Replaces mtp_prepare_alignment_ids (include/ninfer/ops/mtp_round.h:19-20): T = K+1 in [2,6];
 * alignment_ids[i] = verify_ids[i+1] for i < K, then alignment_ids[*accepted] = *token (slot K is
 * written only when *accepted == K). A device-side accepted outside [0, K] writes no token. */
int nmi_mtp_prepare_alignment_ids(const nmi_tensor* verify_ids, const nmi_tensor* token,
                                  const nmi_tensor* accepted, nmi_tensor* alignment_ids, nmi_stream_t stream);

/* ---------------------------------------------------------------- commit / rollback (part c) */

/* Replaces kv_cache_append_prefix (include/ninfer/ops/kv_cache_append_prefix.h:34-37) and
 * extends it to INT8-G64 caches and a trailing batch dimension (k/v [D, Hkv, T, B], positions
 * [T, B], commit_count [B]): columns i < commit_count[b] are quantized (INT8) or copied (BF16)
 * into row positions[i]; no byte of a rejected column is written, and a device count outside
 * [envelope.min_count, envelope.max_count] writes nothing. */
int nmi_kv_cache_append_prefix(const nmi_tensor* k, const nmi_tensor* v,
                               const nmi_tensor* positions, const nmi_tensor* commit_count,
                               nmi_commit_envelope envelope, const nmi_kv_layer_view* cache,
                               nmi_stream_t stream);

/* Replaces the cyclic kv_cache_append_prefix overload (include/ninfer/ops/kv_cache_append_prefix.h:
 * 40-51): the same commit into row positions[i] % capacity. The reference fixes capacity at 4096;
 * any power of two from 128 up is accepted, and envelope.max_count must not exceed it. */
int nmi_kv_cache_append_prefix_cyclic(const nmi_tensor* k, const nmi_tensor* v,
                                      const nmi_tensor* positions, const nmi_tensor* commit_count,
                                      nmi_commit_envelope envelope, const nmi_cyclic_kv_layer_view* cache,
                                      nmi_stream_t stream);

/* EXTENSION: explicit rollback — zero codes and scales of rows positions[i] for
 * i in [*keep_count, T). */
int nmi_kv_cache_rollback(const nmi_tensor* positions, const nmi_tensor* keep_count,
                          const nmi_kv_layer_view* cache, nmi_stream_t stream);

/* EXTENSION (tree verification): move rows base + path[j] to base + j for j < *path_len, where
 * base = *base_position (device I32 scalar), path I32 [T] strictly increasing with path[j] >= j.
 * Codes and scales are copied bit-exactly. */
int nmi_kv_cache_compact_path(const nmi_tensor* base_position, const nmi_tensor* path,
                              const nmi_tensor* path_len, const nmi_kv_layer_view* cache,
                              nmi_stream_t stream);

/* EXTENSION (tree verification): greedy longest accepted root-to-leaf chain and commit.
 * parents I32 [N], node_tokens I32 [N] (node 0 = the current token), target_tokens I32 [N]
 * (argmax per node). Writes path I32 [N] (first *path_len entries valid), sampled_out I32 [N]
 * (path tokens then the correction/bonus token, zero padded), num_sampled, accepted, advances
 * length by accepted+1, sets token, and updates stats like the chain case. */
int nmi_tree_accept_greedy(const nmi_tensor* parents, const nmi_tensor* node_tokens,
                           const nmi_tensor* target_tokens, nmi_tensor* path, nmi_tensor* path_len,
                           nmi_tensor* length, nmi_tensor* token, nmi_tensor* sampled_out,
                           nmi_tensor* num_sampled, nmi_tensor* accepted, nmi_tensor* stats,
                           nmi_stream_t stream);

/* ---------------------------------------------------------------- lm_head (logits of the verify columns) */

/* Replaces linear (include/ninfer/ops/linear.h:27) for Q6G64_F16S RowSplit weights:
 * out[n,t] = BF16(sum_k decode(w)[n,k] * x[k,t]), decode = 6-bit code * FP16 group scale. x BF16
 * [K,T], out BF16 [N,T], T >= 1, padded K <= 8192 (the reference registers [248320,5120] and
 * [248320,2048]; other shapes in range are also served). `ws` of the reference is not needed. */
int nmi_linear(const nmi_tensor* x, const nmi_weight* w, nmi_tensor* out, nmi_stream_t stream);

/* EXTENSION: the reference's deferred FUT-F03 linear_argmax
 * (docs/maintainer/qwen3.6-35b-a3b-dflash-op-checklist.md:985-1001): out[t] = lowest v < valid_rows
 * attaining max_v BF16(decode(w)[v,:] . x[:,t]), ties of -0 and +0 equal; the logits are never
 * written. out I32 [T]. Workspace from nmi_linear_argmax_workspace_bytes. */
size_t nmi_linear_argmax_workspace_bytes(int32_t tokens);
int nmi_linear_argmax(const nmi_tensor* x, const nmi_weight* w, int32_t valid_rows, void* workspace,
                      size_t workspace_bytes, nmi_tensor* out, nmi_stream_t stream);

/* EXTENSION: the lm_head and nmi_speculative_accept_greedy_drafts in one call, the logits never
 * written: the top-cap half of the deferred FUT-F03 fusion
 * (docs/maintainer/qwen3.6-35b-a3b-dflash-op-checklist.md:985-1001), replacing the per-tile
 * candidate pass over materialized logits (src/ops/kernel/speculative_round.cuh:169-211).
 * x BF16 [hidden, K+1, B]: the final hidden rows of every verify column; w as for nmi_linear;
 * drafts .. config as for nmi_speculative_accept_greedy_drafts (config a DEVICE pointer). Per column
 * the lm_head keeps the 20 largest keys of the BF16 logits over rows [0, token_domain), penalty
 * adjusted for stochastic sequences and raw for greedy ones (whose target is the largest); the
 * acceptance then runs as in nmi_speculative_accept_greedy_drafts. Decisions equal nmi_linear
 * followed by nmi_argmax and nmi_speculative_accept_greedy_drafts on the same input. */
size_t nmi_speculative_accept_fused_head_workspace_bytes(int32_t K, int32_t batch);
int nmi_speculative_accept_fused_head(const nmi_tensor* x, const nmi_weight* w, const nmi_tensor* drafts,
                                      nmi_tensor* length, nmi_tensor* token, nmi_tensor* sampled_out,
                                      nmi_tensor* num_sampled, nmi_tensor* accepted, nmi_tensor* stats,
                                      int32_t token_domain, const nmi_sampling_config* config, void* workspace,
                                      size_t workspace_bytes, nmi_stream_t stream);

/* ---------------------------------------------------------------- recurrent state (hybrid layers) */

/* Replaces gated_delta_rule_workspace_bytes (include/ninfer/ops/gated_delta_rule.h:18-21), as a
 * status with the size in *bytes. The recurrent kernel needs no transient storage for any T, so
 * a valid geometry gives 0. */
int nmi_gated_delta_rule_workspace_bytes(int32_t head_dim, int32_t qk_heads, int32_t value_heads,
                                         int32_t tokens, int32_t normalize_qk, size_t* bytes);

/* Replaces both gated_delta_rule forms (include/ninfer/ops/gated_delta_rule.h:23-55): for each
 * value head h (q/k head h / (Hv/Hqk)), in token order: alpha = exp(g[h,t]);
 * delta = beta[h,t] * (v[:,h,t] - alpha * S_h * k[:,qh,t]); S_h = alpha * S_h + outer(delta, k);
 * out[:,h,t] = BF16(scale * S_h * q[:,qh,t]). q/k BF16 [S,Hqk,T], v/out BF16 [S,Hv,T], g/beta FP32
 * [Hv,T], states FP32 [S,S,Hv] (row = value index, key index fastest), S in {16,32,64,128},
 * scale = 1/sqrt(S). normalize_qk: q and k rows become x / sqrt(sum(x^2) + 1e-6) first.
 * ssm_state_in and ssm_state_out may be the same storage (the in-place form) or disjoint. */
int nmi_gated_delta_rule(const nmi_tensor* q, const nmi_tensor* k, const nmi_tensor* v,
                         const nmi_tensor* g, const nmi_tensor* beta, float scale,
                         int32_t normalize_qk, const nmi_tensor* ssm_state_in,
                         nmi_tensor* ssm_state_out, nmi_tensor* out, nmi_stream_t stream);

/* Replaces gated_delta_rule_snapshot (include/ninfer/ops/gated_delta_rule.h:57-68): ssm_states FP32
 * [S,S,Hv,Slots], Slots >= T; slot *initial_slot (device I32) supplies the initial state and the
 * state after token t is written to slot t; slots >= T are unchanged. After acceptance the next
 * round starts from slot `accepted` (see nmi_assign_i32_scalar). A device-side initial slot
 * outside [0, Slots) makes the call write nothing. */
int nmi_gated_delta_rule_snapshot(const nmi_tensor* q, const nmi_tensor* k, const nmi_tensor* v,
                                  const nmi_tensor* g, const nmi_tensor* beta, float scale,
                                  int32_t normalize_qk, nmi_tensor* ssm_states,
                                  const nmi_tensor* initial_slot, nmi_tensor* out,
                                  nmi_stream_t stream);

/* Replaces both causal_conv1d_silu forms (include/ninfer/ops/causal_conv1d_silu.h:9-31):
 * out[c,t] = BF16(SiLU(sum_{j<4} weight[c,j] * u[c,t-3+j])) with u = state window (3 values,
 * oldest first) followed by x. x/out BF16 [C,T], weight BF16 [C,4], states BF16 [C,3]; the final
 * window is written to conv_state_out (which may be the same storage as conv_state_in). */
int nmi_causal_conv1d_silu(const nmi_tensor* x, const nmi_tensor* weight,
                           const nmi_tensor* conv_state_in, nmi_tensor* conv_state_out,
                           nmi_tensor* out, nmi_stream_t stream);

/* Replaces causal_conv1d_silu_snapshot (include/ninfer/ops/causal_conv1d_silu.h:33-40):
 * conv_states BF16 [C,3,Slots], Slots >= T; window slot *initial_slot in, window after token t
 * out to slot t. A device-side initial slot outside [0, Slots) makes the call write nothing. */
int nmi_causal_conv1d_silu_snapshot(const nmi_tensor* x, const nmi_tensor* weight,
                                    nmi_tensor* conv_states, const nmi_tensor* initial_slot,
                                    nmi_tensor* out, nmi_stream_t stream);

/* Replace set_i32_scalar / assign_i32_scalar / increment_i32_scalar / increment_i64_scalar
 * (include/ninfer/ops/scalar.h:30-33): one-element device scalars; assign requires distinct
 * storage. assign(accepted -> initial_slot) is the recurrent-state commit of a verify round. */
int nmi_set_i32_scalar(nmi_tensor* destination, int32_t value, nmi_stream_t stream);
int nmi_assign_i32_scalar(const nmi_tensor* source, nmi_tensor* destination, nmi_stream_t stream);
int nmi_increment_i32_scalar(nmi_tensor* scalar, nmi_stream_t stream);
int nmi_increment_i64_scalar(nmi_tensor* scalar, nmi_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* NINFER_AMD_H */
