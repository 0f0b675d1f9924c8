// C++20 drop-in layer over the ninfer_amd C ABI: the reference's ninfer::ops signatures
// (include/ninfer/ops/{gqa_attention,argmax,sampling,speculative_round,mtp_round,
// kv_cache_append_prefix,gated_delta_rule,causal_conv1d_silu,scalar}.h)
// with hipStream_t in place of cudaStream_t. Statuses become the reference's exceptions:
// std::invalid_argument, std::overflow_error, std::runtime_error (launch failure).
//
// Header-only; link against ninfer_amd/libninfer_amd.so.
#pragma once

#include "ninfer_amd.h"

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>
#include <initializer_list>
#include <stdexcept>
#include <string>

namespace ninfer_amd {

enum class DType : int32_t { BF16 = NMI_BF16, FP32 = NMI_FP32, I32 = NMI_I32, U8 = NMI_U8, I64 = NMI_I64, I8 = NMI_I8, FP16 = NMI_FP16 };

inline std::size_t dtype_size(DType d) {
    switch (d) {
    case DType::BF16:
    case DType::FP16: return 2;
    case DType::FP32:
    case DType::I32: return 4;
    case DType::I8:
    case DType::U8: return 1;
    case DType::I64: return 8;
    }
    return 0;
}

// src/core/tensor.h:11-28 — non-owning view, ne[0] fastest, nb in bytes.
struct Tensor {
    void* data = nullptr;
    DType dtype = DType::BF16;
    int32_t ne[4] = {1, 1, 1, 1};
    int64_t nb[4] = {0, 0, 0, 0};

    Tensor() noexcept = default;
    Tensor(void* d, DType t, std::initializer_list<int32_t> shape) : data(d), dtype(t) {
        int i = 0;
        for (int32_t s : shape) { ne[i++] = s; }
        int64_t stride = static_cast<int64_t>(dtype_size(t));
        for (int k = 0; k < 4; ++k) {
            nb[k] = stride;
            stride *= ne[k];
        }
    }
    nmi_tensor c() const {
        nmi_tensor r{};
        r.data = data;
        r.dtype = static_cast<int32_t>(dtype);
        for (int k = 0; k < 4; ++k) {
            r.ne[k] = ne[k];
            r.nb[k] = nb[k];
        }
        return r;
    }
};

// src/core/kv_cache.h:13-24.
struct KVCacheLayerView {
    Tensor k, v, k_scale, v_scale;
    uint32_t max_context = 0;
    uint32_t padded_context = 0;
    int32_t num_kv_heads = 0;
    int32_t head_dim = 0;
    DType dtype = DType::BF16;
    int32_t quant_group = 0;

    nmi_kv_layer_view c() const {
        nmi_kv_layer_view r{};
        r.k = k.c();
        r.v = v.c();
        r.k_scale = k_scale.c();
        r.v_scale = v_scale.c();
        r.max_context = max_context;
        r.padded_context = padded_context;
        r.num_kv_heads = num_kv_heads;
        r.head_dim = head_dim;
        r.dtype = static_cast<int32_t>(dtype);
        r.quant_group = quant_group;
        return r;
    }
};

// src/core/kv_cache.h:32-43 — cyclic storage, absolute position p in row p % capacity.
struct CyclicKVCacheLayerView {
    Tensor k, v, k_scale, v_scale;
    uint32_t capacity = 0;
    uint32_t padded_capacity = 0;
    int32_t num_kv_heads = 0;
    int32_t head_dim = 0;
    DType dtype = DType::BF16;
    int32_t quant_group = 0;

    nmi_cyclic_kv_layer_view c() const {
        nmi_cyclic_kv_layer_view r{};
        r.k = k.c();
        r.v = v.c();
        r.k_scale = k_scale.c();
        r.v_scale = v_scale.c();
        r.capacity = capacity;
        r.padded_capacity = padded_capacity;
        r.num_kv_heads = num_kv_heads;
        r.head_dim = head_dim;
        r.dtype = static_cast<int32_t>(dtype);
        r.quant_group = quant_group;
        return r;
    }
};

using GqaExecutionEnvelope = nmi_gqa_envelope;
using KVCacheAppendPrefixExecutionEnvelope = nmi_commit_envelope;
using SamplingConfig = nmi_sampling_config; // same 40-byte device layout as the reference

// Caller-owned bump arena over device memory (src/core/arena.h WorkspaceArena semantics: ops take
// a scope, sub-allocate 256-byte aligned regions, and release them when the scope ends).
class WorkspaceArena {
  public:
    WorkspaceArena(void* base, std::size_t bytes) : base_(static_cast<char*>(base)), cap_(bytes) {}
    struct Scope {
        WorkspaceArena* a;
        std::size_t mark;
        ~Scope() { a->used_ = mark; }
    };
    Scope scope() { return Scope{this, used_}; }
    void* alloc_bytes(std::size_t n) {
        const std::size_t at = (used_ + 255) & ~static_cast<std::size_t>(255);
        if (at + n > cap_) { throw std::invalid_argument("WorkspaceArena: out of capacity"); }
        used_ = at + n;
        return base_ + at;
    }
    std::size_t remaining() const { return cap_ - ((used_ + 255) & ~static_cast<std::size_t>(255)); }

  private:
    char* base_;
    std::size_t cap_;
    std::size_t used_ = 0;
};

namespace detail {
inline void check(int status) {
    if (status == NMI_OK) { return; }
    const std::string msg = nmi_last_error();
    if (status == NMI_INVALID_ARGUMENT) { throw std::invalid_argument(msg); }
    if (status == NMI_OVERFLOW) { throw std::overflow_error(msg); }
    throw std::runtime_error(msg);
}
inline nmi_stream_t st(hipStream_t s) { return reinterpret_cast<nmi_stream_t>(s); }
} // namespace detail

namespace ops {

// include/ninfer/ops/gqa_attention.h:50, the reference signature: enough for every envelope of one
// sequence at the geometry q_heads implies (24|4 and 16|2 at head_dim 256, 40|8 at 128).
[[nodiscard]] inline std::size_t gqa_attention_workspace_bytes(int32_t q_heads, int32_t tokens) {
    std::size_t n = 0;
    detail::check(nmi_gqa_attention_workspace_bound(q_heads, tokens, &n));
    return n;
}

// The exact size for one geometry, batch and envelope (what the ops below take from the arena).
[[nodiscard]] inline std::size_t gqa_attention_workspace_bytes(int32_t q_heads, int32_t kv_heads,
                                                               int32_t head_dim, int32_t tokens,
                                                               int32_t batch,
                                                               uint32_t max_visible_keys) {
    return nmi_gqa_attention_workspace_bytes(q_heads, kv_heads, head_dim, tokens, batch, max_visible_keys);
}

// A1, include/ninfer/ops/gqa_attention.h:71-73.
inline void gqa_attention(const Tensor& q, const Tensor& k, const Tensor& v, const Tensor& positions,
                          float scale, KVCacheLayerView cache, GqaExecutionEnvelope envelope,
                          WorkspaceArena& workspace, Tensor& out, hipStream_t stream) {
    auto scope = workspace.scope();
    const std::size_t need = gqa_attention_workspace_bytes(q.ne[1], cache.num_kv_heads, q.ne[0], q.ne[2], q.ne[3],
                                                           envelope.max_visible_keys);
    void* ws = need ? workspace.alloc_bytes(need) : nullptr;
    const nmi_tensor cq = q.c(), ck = k.c(), cv = v.c(), cp = positions.c();
    nmi_tensor co = out.c();
    const nmi_kv_layer_view cc = cache.c();
    detail::check(nmi_gqa_attention(&cq, &ck, &cv, &cp, scale, &cc, envelope, ws, need, &co, detail::st(stream)));
}

// No reference counterpart: A1 for callers that cannot allocate or pass a workspace (graph capture,
// serving loops); the split partials use the library's static per-device scratch (16 MiB).
inline void gqa_attention_noalloc(const Tensor& q, const Tensor& k, const Tensor& v, const Tensor& positions,
                                  float scale, KVCacheLayerView cache, GqaExecutionEnvelope envelope, Tensor& out,
                                  hipStream_t stream) {
    const nmi_tensor cq = q.c(), ck = k.c(), cv = v.c(), cp = positions.c();
    nmi_tensor co = out.c();
    const nmi_kv_layer_view cc = cache.c();
    detail::check(nmi_gqa_attention_noalloc(&cq, &ck, &cv, &cp, scale, &cc, envelope, &co, detail::st(stream)));
}

// A2, include/ninfer/ops/gqa_attention.h:80-81.
inline void gqa_kv_append(const Tensor& k, const Tensor& v, const Tensor& positions,
                          KVCacheLayerView cache, hipStream_t stream) {
    const nmi_tensor ck = k.c(), cv = v.c(), cp = positions.c();
    const nmi_kv_layer_view cc = cache.c();
    detail::check(nmi_gqa_kv_append(&ck, &cv, &cp, &cc, detail::st(stream)));
}

// A3, include/ninfer/ops/gqa_attention.h:89-91.
inline void gqa_attention_cached(const Tensor& q, const Tensor& positions, float scale,
                                 const KVCacheLayerView& cache, GqaExecutionEnvelope envelope,
                                 WorkspaceArena& workspace, Tensor& out, hipStream_t stream) {
    auto scope = workspace.scope();
    const std::size_t need = gqa_attention_workspace_bytes(q.ne[1], cache.num_kv_heads, q.ne[0], q.ne[2], q.ne[3],
                                                           envelope.max_visible_keys);
    void* ws = need ? workspace.alloc_bytes(need) : nullptr;
    const nmi_tensor cq = q.c(), cp = positions.c();
    nmi_tensor co = out.c();
    const nmi_kv_layer_view cc = cache.c();
    detail::check(nmi_gqa_attention_cached(&cq, &cp, scale, &cc, envelope, ws, need, &co, detail::st(stream)));
}

// Extension: tree verification (ancestor mask).
inline void gqa_attention_tree(const Tensor& q, const Tensor& k, const Tensor& v, const Tensor& positions,
                               const Tensor& parents, float scale, KVCacheLayerView cache,
                               GqaExecutionEnvelope envelope, bool write_cache, WorkspaceArena& workspace,
                               Tensor& out, hipStream_t stream) {
    auto scope = workspace.scope();
    const std::size_t need = gqa_attention_workspace_bytes(q.ne[1], cache.num_kv_heads, q.ne[0], q.ne[2], q.ne[3],
                                                           envelope.max_visible_keys);
    void* ws = need ? workspace.alloc_bytes(need) : nullptr;
    const nmi_tensor cq = q.c(), ck = k.c(), cv = v.c(), cp = positions.c(), cpar = parents.c();
    nmi_tensor co = out.c();
    const nmi_kv_layer_view cc = cache.c();
    detail::check(nmi_gqa_attention_tree(&cq, &ck, &cv, &cp, &cpar, scale, &cc, envelope, write_cache ? 1 : 0, ws,
                                         need, &co, detail::st(stream)));
}

// include/ninfer/ops/argmax.h:21.
inline void argmax(const Tensor& logits, Tensor& out, int32_t valid_rows, hipStream_t stream) {
    const nmi_tensor cl = logits.c();
    nmi_tensor co = out.c();
    detail::check(nmi_argmax(&cl, &co, valid_rows, detail::st(stream)));
}

// include/ninfer/ops/sampling.h:37.
[[nodiscard]] inline std::size_t sampling_workspace_bytes(int32_t token_domain, int32_t columns) {
    return nmi_sampling_workspace_bytes(token_domain, columns, 1);
}

// include/ninfer/ops/speculative_round.h:29-31.
inline void speculative_prepare_verify_inputs(const Tensor& token, const Tensor& drafts, const Tensor& length,
                                              Tensor& verify_ids, Tensor& positions, hipStream_t stream) {
    const nmi_tensor ct = token.c(), cd = drafts.c(), cl = length.c();
    nmi_tensor cv = verify_ids.c(), cp = positions.c();
    detail::check(nmi_speculative_prepare_verify_inputs(&ct, &cd, &cl, &cv, &cp, detail::st(stream)));
}

// include/ninfer/ops/speculative_round.h:68-73.
inline void speculative_accept_greedy_drafts(const Tensor& target_tokens, const Tensor& logits,
                                             const Tensor& drafts, Tensor& length, Tensor& token,
                                             Tensor& sampled_out, Tensor& num_sampled, Tensor& accepted,
                                             Tensor& stats, int32_t token_domain,
                                             const SamplingConfig* config, WorkspaceArena& workspace,
                                             hipStream_t stream) {
    auto scope = workspace.scope();
    const std::size_t need = nmi_sampling_workspace_bytes(token_domain, drafts.ne[0] + 1, drafts.ne[1]);
    void* ws = need ? workspace.alloc_bytes(need) : nullptr;
    const nmi_tensor ct = target_tokens.c(), cl = logits.c(), cd = drafts.c();
    nmi_tensor clen = length.c(), ctok = token.c(), cso = sampled_out.c(), cns = num_sampled.c(),
               cacc = accepted.c(), cst = stats.c();
    detail::check(nmi_speculative_accept_greedy_drafts(&ct, &cl, &cd, &clen, &ctok, &cso, &cns, &cacc, &cst,
                                                       token_domain, config, ws, need, detail::st(stream)));
}

// Extension: general min(1, p/q) acceptance with residual resampling.
inline void speculative_accept_general(const Tensor& logits, const Tensor& draft_logits, const Tensor& drafts,
                                       const Tensor& u_accept, const Tensor& u_residual, Tensor& length,
                                       Tensor& token, Tensor& sampled_out, Tensor& num_sampled, Tensor& accepted,
                                       Tensor& stats, int32_t token_domain, const nmi_general_config* config,
                                       WorkspaceArena& workspace, hipStream_t stream) {
    auto scope = workspace.scope();
    const std::size_t need = nmi_general_accept_workspace_bytes(token_domain, drafts.ne[0], drafts.ne[1]);
    void* ws = need ? workspace.alloc_bytes(need) : nullptr;
    const nmi_tensor cl = logits.c(), cdl = draft_logits.c(), cd = drafts.c(), cua = u_accept.c(),
                     cur = u_residual.c();
    nmi_tensor clen = length.c(), ctok = token.c(), cso = sampled_out.c(), cns = num_sampled.c(),
               cacc = accepted.c(), cst = stats.c();
    detail::check(nmi_speculative_accept_general(&cl, &cdl, &cd, &cua, &cur, &clen, &ctok, &cso, &cns, &cacc, &cst,
                                                 token_domain, config, ws, need, detail::st(stream)));
}

// include/ninfer/ops/speculative_round.h:86-87.
inline void speculative_select_accepted_hidden(const Tensor& hidden, const Tensor& accepted, Tensor& out,
                                               hipStream_t stream) {
    const nmi_tensor ch = hidden.c(), ca = accepted.c();
    nmi_tensor co = out.c();
    detail::check(nmi_speculative_select_accepted_hidden(&ch, &ca, &co, detail::st(stream)));
}

// include/ninfer/ops/mtp_round.h:19-20.
inline void mtp_prepare_alignment_ids(const Tensor& verify_ids, const Tensor& token, const Tensor& accepted,
                                      Tensor& alignment_ids, hipStream_t stream) {
    const nmi_tensor cv = verify_ids.c(), ct = token.c(), ca = accepted.c();
    nmi_tensor co = alignment_ids.c();
    detail::check(nmi_mtp_prepare_alignment_ids(&cv, &ct, &ca, &co, detail::st(stream)));
}

// include/ninfer/ops/kv_cache_append_prefix.h:34-37 (linear cache; BF16 or INT8-G64).
inline void kv_cache_append_prefix(const Tensor& k, const Tensor& v, const Tensor& positions,
                                   const Tensor& commit_count, KVCacheAppendPrefixExecutionEnvelope envelope,
                                   KVCacheLayerView cache, hipStream_t stream) {
    const nmi_tensor ck = k.c(), cv = v.c(), cp = positions.c(), cc = commit_count.c();
    const nmi_kv_layer_view view = cache.c();
    detail::check(nmi_kv_cache_append_prefix(&ck, &cv, &cp, &cc, envelope, &view, detail::st(stream)));
}

// include/ninfer/ops/kv_cache_append_prefix.h:40-51 (cyclic cache).
inline void kv_cache_append_prefix(const Tensor& k, const Tensor& v, const Tensor& positions,
                                   const Tensor& commit_count, KVCacheAppendPrefixExecutionEnvelope envelope,
                                   CyclicKVCacheLayerView cache, hipStream_t stream) {
    const nmi_tensor ck = k.c(), cv = v.c(), cp = positions.c(), cc = commit_count.c();
    const nmi_cyclic_kv_layer_view view = cache.c();
    detail::check(nmi_kv_cache_append_prefix_cyclic(&ck, &cv, &cp, &cc, envelope, &view, detail::st(stream)));
}

// Extension: explicit rollback of rejected rows.
inline void kv_cache_rollback(const Tensor& positions, const Tensor& keep_count, KVCacheLayerView cache,
                              hipStream_t stream) {
    const nmi_tensor cp = positions.c(), ck = keep_count.c();
    const nmi_kv_layer_view view = cache.c();
    detail::check(nmi_kv_cache_rollback(&cp, &ck, &view, detail::st(stream)));
}

// Extension: compaction of an accepted tree path.
inline void kv_cache_compact_path(const Tensor& base_position, const Tensor& path, const Tensor& path_len,
                                  KVCacheLayerView cache, hipStream_t stream) {
    const nmi_tensor cb = base_position.c(), cp = path.c(), cl = path_len.c();
    const nmi_kv_layer_view view = cache.c();
    detail::check(nmi_kv_cache_compact_path(&cb, &cp, &cl, &view, detail::st(stream)));
}

// Extension: greedy tree acceptance.
inline void tree_accept_greedy(const Tensor& parents, const Tensor& node_tokens, const Tensor& target_tokens,
                               Tensor& path, Tensor& path_len, Tensor& length, Tensor& token, Tensor& sampled_out,
                               Tensor& num_sampled, Tensor& accepted, Tensor& stats, hipStream_t stream) {
    const nmi_tensor cpar = parents.c(), cnt = node_tokens.c(), ctt = target_tokens.c();
    nmi_tensor cpath = path.c(), cpl = path_len.c(), clen = length.c(), ctok = token.c(), cso = sampled_out.c(),
               cns = num_sampled.c(), cacc = accepted.c(), cst = stats.c();
    detail::check(nmi_tree_accept_greedy(&cpar, &cnt, &ctt, &cpath, &cpl, &clen, &ctok, &cso, &cns, &cacc, &cst,
                                         detail::st(stream)));
}

// ---- lm_head ----------------------------------------------------------------------------------------

// include/ninfer/ops/linear.h:27 for Q6G64_F16S RowSplit weights. `w` is the reference's Weight
// (src/core/tensor.h:47-66) copied field for field into nmi_weight by the binding.
inline void linear(const Tensor& x, const nmi_weight& w, Tensor& out, WorkspaceArena& ws, hipStream_t stream) {
    (void)ws;
    const nmi_tensor cx = x.c();
    nmi_tensor co = out.c();
    detail::check(nmi_linear(&cx, &w, &co, detail::st(stream)));
}

// Extension: fused linear -> argmax (the reference's deferred FUT-F03 contract).
[[nodiscard]] inline std::size_t linear_argmax_workspace_bytes(int32_t tokens) {
    return nmi_linear_argmax_workspace_bytes(tokens);
}
inline void linear_argmax(const Tensor& x, const nmi_weight& w, int32_t valid_rows, WorkspaceArena& ws, Tensor& out,
                          hipStream_t stream) {
    const std::size_t need = linear_argmax_workspace_bytes(x.ne[1]);
    auto scope = ws.scope();
    void* p = ws.alloc_bytes(need);
    const nmi_tensor cx = x.c();
    nmi_tensor co = out.c();
    detail::check(nmi_linear_argmax(&cx, &w, valid_rows, p, need, &co, detail::st(stream)));
}

// Extension: the lm_head and speculative_accept_greedy_drafts in one call (the logits never written).
[[nodiscard]] inline std::size_t speculative_accept_fused_head_workspace_bytes(int32_t K, int32_t batch) {
    return nmi_speculative_accept_fused_head_workspace_bytes(K, batch);
}
inline void speculative_accept_fused_head(const Tensor& x, const nmi_weight& w, const Tensor& drafts, Tensor& length,
                                          Tensor& token, Tensor& sampled_out, Tensor& num_sampled, Tensor& accepted,
                                          Tensor& stats, int32_t token_domain, const SamplingConfig* config,
                                          WorkspaceArena& workspace, hipStream_t stream) {
    auto scope = workspace.scope();
    const std::size_t need = speculative_accept_fused_head_workspace_bytes(drafts.ne[0], drafts.ne[1]);
    void* ws = need ? workspace.alloc_bytes(need) : nullptr;
    const nmi_tensor cx = x.c(), cd = drafts.c();
    nmi_tensor clen = length.c(), ctok = token.c(), cso = sampled_out.c(), cns = num_sampled.c(),
               cacc = accepted.c(), cst = stats.c();
    detail::check(nmi_speculative_accept_fused_head(&cx, &w, &cd, &clen, &ctok, &cso, &cns, &cacc, &cst, token_domain,
                                                    config, ws, need, detail::st(stream)));
}

// ---- recurrent state of the hybrid layers -------------------------------------------------------

// include/ninfer/ops/gated_delta_rule.h:18-21
[[nodiscard]] inline std::size_t gated_delta_rule_workspace_bytes(int32_t head_dim, int32_t qk_heads,
                                                                  int32_t value_heads, int32_t tokens,
                                                                  bool normalize_qk) {
    std::size_t n = 0;
    detail::check(nmi_gated_delta_rule_workspace_bytes(head_dim, qk_heads, value_heads, tokens, normalize_qk ? 1 : 0,
                                                       &n));
    return n;
}

// include/ninfer/ops/gated_delta_rule.h:41-43 (in place) and :50-53 (distinct states). The
// recurrent kernel uses no transient storage; `ws` is accepted for signature parity.
inline void gated_delta_rule(const Tensor& q, const Tensor& k, const Tensor& v, const Tensor& g, const Tensor& beta,
                             float scale, bool normalize_qk, const Tensor& ssm_state_in, Tensor& ssm_state_out,
                             Tensor& out, hipStream_t stream) {
    const nmi_tensor cq = q.c(), ck = k.c(), cv = v.c(), cg = g.c(), cb = beta.c(), ci = ssm_state_in.c();
    nmi_tensor co = ssm_state_out.c(), cout = out.c();
    detail::check(nmi_gated_delta_rule(&cq, &ck, &cv, &cg, &cb, scale, normalize_qk ? 1 : 0, &ci, &co, &cout,
                                       detail::st(stream)));
}
inline void gated_delta_rule(const Tensor& q, const Tensor& k, const Tensor& v, const Tensor& g, const Tensor& beta,
                             float scale, bool normalize_qk, WorkspaceArena& ws, Tensor& ssm_state, Tensor& out,
                             hipStream_t stream) {
    (void)ws;
    gated_delta_rule(q, k, v, g, beta, scale, normalize_qk, ssm_state, ssm_state, out, stream);
}
inline void gated_delta_rule(const Tensor& q, const Tensor& k, const Tensor& v, const Tensor& g, const Tensor& beta,
                             float scale, bool normalize_qk, WorkspaceArena& ws, const Tensor& ssm_state_in,
                             Tensor& ssm_state_out, Tensor& out, hipStream_t stream) {
    (void)ws;
    gated_delta_rule(q, k, v, g, beta, scale, normalize_qk, ssm_state_in, ssm_state_out, out, stream);
}

// include/ninfer/ops/gated_delta_rule.h:65-68
inline void gated_delta_rule_snapshot(const Tensor& q, const Tensor& k, const Tensor& v, const Tensor& g,
                                      const Tensor& beta, float scale, bool normalize_qk, WorkspaceArena& ws,
                                      Tensor& ssm_states, const Tensor& initial_slot, Tensor& out,
                                      hipStream_t stream) {
    (void)ws;
    const nmi_tensor cq = q.c(), ck = k.c(), cv = v.c(), cg = g.c(), cb = beta.c(), cs = initial_slot.c();
    nmi_tensor cst = ssm_states.c(), cout = out.c();
    detail::check(nmi_gated_delta_rule_snapshot(&cq, &ck, &cv, &cg, &cb, scale, normalize_qk ? 1 : 0, &cst, &cs,
                                                &cout, detail::st(stream)));
}

// include/ninfer/ops/causal_conv1d_silu.h:24-31
inline void causal_conv1d_silu(const Tensor& x, const Tensor& weight, const Tensor& conv_state_in,
                               Tensor& conv_state_out, Tensor& out, hipStream_t stream) {
    const nmi_tensor cx = x.c(), cw = weight.c(), ci = conv_state_in.c();
    nmi_tensor co = conv_state_out.c(), cout = out.c();
    detail::check(nmi_causal_conv1d_silu(&cx, &cw, &ci, &co, &cout, detail::st(stream)));
}
inline void causal_conv1d_silu(const Tensor& x, const Tensor& weight, Tensor& conv_state, Tensor& out,
                               hipStream_t stream) {
    causal_conv1d_silu(x, weight, conv_state, conv_state, out, stream);
}

// include/ninfer/ops/causal_conv1d_silu.h:39-40
inline void causal_conv1d_silu_snapshot(const Tensor& x, const Tensor& weight, Tensor& conv_states,
                                        const Tensor& initial_slot, Tensor& out, hipStream_t stream) {
    const nmi_tensor cx = x.c(), cw = weight.c(), cs = initial_slot.c();
    nmi_tensor cst = conv_states.c(), cout = out.c();
    detail::check(nmi_causal_conv1d_silu_snapshot(&cx, &cw, &cst, &cs, &cout, detail::st(stream)));
}

// include/ninfer/ops/scalar.h:30-33
inline void set_i32_scalar(Tensor& destination, int32_t value, hipStream_t stream) {
    nmi_tensor cd = destination.c();
    detail::check(nmi_set_i32_scalar(&cd, value, detail::st(stream)));
}
inline void assign_i32_scalar(const Tensor& source, Tensor& destination, hipStream_t stream) {
    const nmi_tensor cs = source.c();
    nmi_tensor cd = destination.c();
    detail::check(nmi_assign_i32_scalar(&cs, &cd, detail::st(stream)));
}
inline void increment_i32_scalar(Tensor& scalar, hipStream_t stream) {
    nmi_tensor cs = scalar.c();
    detail::check(nmi_increment_i32_scalar(&cs, detail::st(stream)));
}
inline void increment_i64_scalar(Tensor& scalar, hipStream_t stream) {
    nmi_tensor cs = scalar.c();
    detail::check(nmi_increment_i64_scalar(&cs, detail::st(stream)));
}

} // namespace ops
} // namespace ninfer_amd
