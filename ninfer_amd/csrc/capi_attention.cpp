// C ABI for the verify attention and the KV cache writes: host validation mirroring the reference
// wrapper (src/ops/wrapper/gqa_attention.cpp:59-136, :278-302) generalized to the BASELINE
// geometry, then dispatch to the gfx950 kernels.
#include "common.h"
#include "ops_internal.h"

#include <algorithm>
#include <cmath>
#include <limits>
#include <string>

namespace nmi {

namespace {

thread_local std::string g_last_error;

void require(bool ok, const std::string& op, const std::string& what) {
    if (!ok) { throw InvalidArgument(op + ": " + what); }
}

void require_tensor(const nmi_tensor* t, const std::string& op, const char* name) {
    require(t != nullptr, op, std::string(name) + " must be non-null");
}

void require_contiguous_nonnull(const nmi_tensor& t, const std::string& op, const char* name) {
    require(is_contiguous(t), op, std::string(name) + " must be contiguous");
    require(t.data != nullptr, op, std::string(name) + " data must be non-null");
}

void require_shape(const nmi_tensor& t, int32_t n0, int32_t n1, int32_t n2, int32_t n3,
                   const std::string& op, const char* name) {
    require(t.ne[0] == n0 && t.ne[1] == n1 && t.ne[2] == n2 && t.ne[3] == n3, op,
            std::string("invalid shape for ") + name);
}

int32_t checked_i32(uint32_t v, const std::string& op, const char* name) {
    if (v > static_cast<uint32_t>(std::numeric_limits<int32_t>::max())) {
        throw Overflow(op + ": " + name + " exceeds int32");
    }
    return static_cast<int32_t>(v);
}

// Cache view checks (reference validate_cache, src/ops/wrapper/gqa_attention.cpp:59-99) with a
// runtime geometry and an optional trailing batch dimension.
// `attention`: the attention kernels also need padded_context to be a multiple of 128 (the
// reference's plan_kv_cache alignment); the commit ops take any padded_context >= max_context, as the
// reference's append validation does (src/ops/wrapper/kv_cache_append_prefix.cpp:62-80).
CacheRef validate_cache(const nmi_kv_layer_view* cache, int32_t kv_heads, int32_t batch,
                        const std::string& op, bool attention = true) {
    require(cache != nullptr, op, "cache must be non-null");
    require(cache->dtype == NMI_I8 || cache->dtype == NMI_BF16, op, "invalid KV cache dtype");
    require(cache->num_kv_heads == kv_heads, op, "invalid KV cache geometry or dtype");
    require(cache->head_dim > 0 && cache->head_dim % kQuantGroup == 0, op, "invalid KV cache head_dim");
    require(cache->max_context != 0 && cache->padded_context >= cache->max_context, op,
            "invalid KV cache capacity");
    require(!attention || cache->padded_context % 128 == 0, op, "padded_context must be a multiple of 128");
    if (cache->dtype == NMI_BF16) {
        require(cache->quant_group == 0, op, "BF16 KV cache must not have quant_group");
    } else {
        require(cache->quant_group == kQuantGroup, op, "I8 KV cache must use quant_group 64");
    }
    const int32_t P = checked_i32(cache->padded_context, op, "padded_context");
    const int32_t D = cache->head_dim;
    // The kernels address one KV head's plane through 32-bit buffer offsets.
    if (static_cast<int64_t>(P) * D * (cache->dtype == NMI_I8 ? 1 : 2) >= (int64_t{1} << 31)) {
        throw Unsupported(op + ": a KV head plane of 2^31 bytes or more (padded_context * head_dim) is not built");
    }
    const int32_t code_dtype = cache->dtype == NMI_I8 ? NMI_I8 : NMI_BF16;
    require(cache->k.dtype == code_dtype && cache->v.dtype == code_dtype, op, "invalid KV cache code dtype");
    require_shape(cache->k, D, P, kv_heads, batch, op, "cache k");
    require_shape(cache->v, D, P, kv_heads, batch, op, "cache v");
    require_contiguous_nonnull(cache->k, op, "cache k");
    require_contiguous_nonnull(cache->v, op, "cache v");
    CacheRef r;
    r.P = P;
    r.Hkv = kv_heads;
    r.D = D;
    r.B = batch;
    r.code_seq = static_cast<int64_t>(D) * P * kv_heads;
    if (cache->dtype == NMI_BF16) {
        require(cache->k_scale.data == nullptr && cache->v_scale.data == nullptr, op,
                "BF16 KV cache must not have scales");
        // Every BF16-cache kernel (the prefix commit, A2, and A1's in-kernel copy of the new rows)
        // stores 16-byte pieces of rows (reference require_vector_aligned on the cache planes,
        // src/ops/wrapper/kv_cache_append_prefix.cpp:77-79,98-100).
        require((reinterpret_cast<uintptr_t>(cache->k.data) & 15u) == 0, op, "cache k must be 16-byte aligned");
        require((reinterpret_cast<uintptr_t>(cache->v.data) & 15u) == 0, op, "cache v must be 16-byte aligned");
        r.kb = static_cast<uint16_t*>(cache->k.data);
        r.vb = static_cast<uint16_t*>(cache->v.data);
        return r;
    }
    const int32_t groups = D / kQuantGroup;
    require(cache->k_scale.dtype == NMI_FP16 && cache->v_scale.dtype == NMI_FP16, op,
            "invalid KV cache scale dtype");
    require_shape(cache->k_scale, groups, P, kv_heads, batch, op, "cache k scale");
    require_shape(cache->v_scale, groups, P, kv_heads, batch, op, "cache v scale");
    require_contiguous_nonnull(cache->k_scale, op, "cache k scale");
    require_contiguous_nonnull(cache->v_scale, op, "cache v scale");
    r.kc = static_cast<int8_t*>(cache->k.data);
    r.vc = static_cast<int8_t*>(cache->v.data);
    r.ks = static_cast<uint16_t*>(cache->k_scale.data);
    r.vs = static_cast<uint16_t*>(cache->v_scale.data);
    r.scale_seq = static_cast<int64_t>(groups) * P * kv_heads;
    return r;
}

void validate_envelope(nmi_gqa_envelope env, const nmi_kv_layer_view* cache, int32_t tokens,
                       const std::string& op) {
    require(env.min_visible_keys != 0 && env.min_visible_keys <= env.max_visible_keys &&
                env.max_visible_keys <= cache->max_context,
            op, "invalid execution envelope");
    require(env.max_visible_keys >= static_cast<uint32_t>(tokens), op,
            "execution envelope is shorter than T");
}

struct AttnShape {
    int32_t D, Hq, Hkv, T, B;
    bool out_f32;
};

// reference validate_attention_tensors (src/ops/wrapper/gqa_attention.cpp:101-136).
AttnShape validate_attention(const nmi_tensor* q, const nmi_tensor* positions,
                             const nmi_tensor* out, const nmi_kv_layer_view* cache,
                             nmi_gqa_envelope env, float scale, const std::string& op) {
    require_tensor(q, op, "q");
    require_tensor(positions, op, "positions");
    require_tensor(out, op, "out");
    require(cache != nullptr, op, "cache must be non-null");
    require(q->dtype == NMI_BF16, op, "q/out must be BF16");
    require(out->dtype == NMI_BF16 || out->dtype == NMI_FP32, op, "q/out must be BF16");
    require(positions->dtype == NMI_I32, op, "positions must be I32");
    AttnShape s{};
    s.D = q->ne[0];
    s.Hq = q->ne[1];
    s.T = q->ne[2];
    s.B = q->ne[3];
    s.Hkv = cache->num_kv_heads;
    s.out_f32 = out->dtype == NMI_FP32;
    require(s.T > 0, op, "T must be positive");
    require(s.B > 0, op, "batch must be positive");
    if (s.T > kAttnMaxTokens && s.B != 1) {
        // the reference's prompt route (T beyond the verify extents) takes one sequence
        throw Unsupported(op + ": T above 32 query tokens (the prompt route) serves one sequence");
    }
    require(s.Hkv > 0 && s.Hq > 0 && s.Hq % s.Hkv == 0, op, "unsupported Q/KV head geometry");
    require(s.Hq / s.Hkv <= kAttnRowsPerTile, op, "unsupported Q/KV head geometry");
    require(s.D == cache->head_dim, op, "q head_dim does not match the cache");
    require(std::isfinite(scale) && std::fabs(scale - 1.0f / std::sqrt(static_cast<float>(s.D))) <= 1.0e-6f, op,
            "scale must be 1/sqrt(head_dim)");
    require_shape(*q, s.D, s.Hq, s.T, s.B, op, "q");
    require_shape(*positions, s.T, s.B, 1, 1, op, "positions");
    require_shape(*out, s.D, s.Hq, s.T, s.B, op, "out");
    require_contiguous_nonnull(*q, op, "q");
    require_contiguous_nonnull(*positions, op, "positions");
    require_contiguous_nonnull(*out, op, "out");
    validate_envelope(env, cache, s.T, op);
    return s;
}

void validate_new_kv(const nmi_tensor* k, const nmi_tensor* v, int32_t D, int32_t Hkv, int32_t T,
                     int32_t B, const std::string& op) {
    require_tensor(k, op, "k");
    require_tensor(v, op, "v");
    require(k->dtype == NMI_BF16 && v->dtype == NMI_BF16, op, "k/v must be BF16");
    require_shape(*k, D, Hkv, T, B, op, "k");
    require_shape(*v, D, Hkv, T, B, op, "v");
    require_contiguous_nonnull(*k, op, "k");
    require_contiguous_nonnull(*v, op, "v");
}

void require_built(const CacheRef& c, const std::string& op) {
    if (c.D != 128 && c.D != 256) { throw Unsupported(op + ": head_dim 128 and 256 kernels are built"); }
}

void require_workspace(void* ws, size_t bytes, size_t need, const std::string& op) {
    require(bytes >= need, op, "workspace is smaller than the size query");
    require(ws != nullptr || need == 0, op, "workspace must be non-null");
    require((reinterpret_cast<uintptr_t>(ws) & 255u) == 0, op, "workspace must be 256-byte aligned");
}

// The prompt route (reference src/ops/wrapper/gqa_attention.cpp:202-213,262-275: T beyond the verify
// extents, one sequence, causal): the new rows are written first (A2), then the query tokens attend
// over the cache in launches of at most kAttnMaxTokens consecutive tokens. Each launch is a verify
// problem of its own: its first position is the history boundary, rows below it (earlier prompt
// tokens included) are visible to all its tokens, and its own rows are masked causally. One
// workspace serves the launches one after another (stream order).
struct PromptChunks {
    int32_t full = 0; // launches of kAttnMaxTokens tokens
    int32_t tail = 0; // tokens of the last, shorter launch (0: none)
};

PromptChunks prompt_chunks(int32_t T) { return PromptChunks{T / kAttnMaxTokens, T % kAttnMaxTokens}; }

// static_ws: the split partials go to the device's static scratch (the allocation-free entry
// point); ws/ws_bytes are then ignored.
int attention_impl(const nmi_tensor* q, const nmi_tensor* k, const nmi_tensor* v,
                   const nmi_tensor* positions, const nmi_tensor* parents, float scale,
                   const nmi_kv_layer_view* cache, nmi_gqa_envelope env, bool write_cache,
                   void* ws, size_t ws_bytes, nmi_tensor* out, hipStream_t stream,
                   const std::string& op, bool static_ws = false) {
    return guarded([&] {
        const AttnShape s = validate_attention(q, positions, out, cache, env, scale, op);
        if (write_cache) { validate_new_kv(k, v, s.D, s.Hkv, s.T, s.B, op); }
        const CacheRef c = validate_cache(cache, s.Hkv, s.B, op);
        if (parents != nullptr) {
            require(parents->dtype == NMI_I32, op, "parents must be I32");
            require_shape(*parents, s.T, s.B, 1, 1, op, "parents");
            require_contiguous_nonnull(*parents, op, "parents");
        }
        require_built(c, op);
        // The 80-row form (INT8, head_dim 128) unless the static scratch of the allocation-free entry
        // cannot hold its partials.
        const auto make_plan = [&](int32_t T) {
            SplitPlan p = plan_attention(s.Hq, s.Hkv, s.D, T, s.B, env.max_visible_keys, c.kb == nullptr);
            if (static_ws && p.bytes > kStaticScratchBytes && p.rows_per_slot != kAttnRowsPerTile) {
                p = plan_attention(s.Hq, s.Hkv, s.D, T, s.B, env.max_visible_keys, false);
            }
            choose_b1_device_plan(p, s.B, env.min_visible_keys, c.kb == nullptr);
            return p;
        };
        if (s.T > kAttnMaxTokens) {
            if (parents != nullptr) { throw Unsupported(op + ": ancestor masks serve at most 32 query tokens"); }
            const PromptChunks pc = prompt_chunks(s.T);
            const SplitPlan full = make_plan(kAttnMaxTokens);
            const SplitPlan last = pc.tail > 0 ? make_plan(pc.tail) : full;
            const size_t need = std::max(full.bytes, last.bytes);
            if (static_ws) {
                ws = static_scratch(need, op);
                ws_bytes = need;
            }
            require_workspace(ws, ws_bytes, need, op);
            if (write_cache) {
                launch_kv_append(static_cast<const uint16_t*>(k->data), static_cast<const uint16_t*>(v->data),
                                 static_cast<const int32_t*>(positions->data), nullptr, CommitBounds{}, s.T, c, stream);
            }
            const size_t out_elem = s.out_f32 ? 4 : 2;
            for (int32_t t0 = 0; t0 < s.T; t0 += kAttnMaxTokens) {
                const int32_t Tc = std::min(kAttnMaxTokens, s.T - t0);
                const size_t off = static_cast<size_t>(t0) * s.Hq * s.D; // [D, Hq, T]: token-major
                launch_verify_attention(static_cast<const uint16_t*>(q->data) + off, nullptr, nullptr,
                                        static_cast<const int32_t*>(positions->data) + t0, nullptr, Tc, s.Hq, c,
                                        scale, env.max_visible_keys, ws, Tc == kAttnMaxTokens ? full : last,
                                        static_cast<char*>(out->data) + off * out_elem, s.out_f32, stream);
            }
            return;
        }
        SplitPlan plan = make_plan(s.T);
        if (static_ws) {
            ws = static_scratch(plan.bytes, op);
            ws_bytes = plan.bytes;
        }
        require_workspace(ws, ws_bytes, plan.bytes, op);
        launch_verify_attention(static_cast<const uint16_t*>(q->data),
                                write_cache ? static_cast<const uint16_t*>(k->data) : nullptr,
                                write_cache ? static_cast<const uint16_t*>(v->data) : nullptr,
                                static_cast<const int32_t*>(positions->data),
                                parents ? static_cast<const int32_t*>(parents->data) : nullptr, s.T,
                                s.Hq, c, scale, env.max_visible_keys, ws, plan, out->data,
                                s.out_f32, stream);
    });
}

// reference kv_cache_append_prefix, both overloads (src/ops/wrapper/kv_cache_append_prefix.cpp:40-123;
// contract include/ninfer/ops/kv_cache_append_prefix.h:22-51), extended to INT8-G64 caches and to a
// trailing batch dimension (k/v [D, Hkv, T, B], positions [T, B], commit_count [B]). A device count
// outside the envelope writes nothing, as in the reference kernel. `slot_mask` selects the cyclic
// form (row = position mod capacity).
void append_prefix_impl(const nmi_tensor* k, const nmi_tensor* v, const nmi_tensor* positions,
                        const nmi_tensor* commit_count, nmi_commit_envelope envelope,
                        const nmi_kv_layer_view* cache, uint32_t capacity, int32_t slot_mask,
                        hipStream_t stream, const std::string& op) {
    require_tensor(k, op, "k");
    require_tensor(v, op, "v");
    require_tensor(positions, op, "positions");
    require_tensor(commit_count, op, "commit_count");
    require(k->dtype == NMI_BF16 && v->dtype == NMI_BF16, op, "k/v must be BF16");
    require(positions->dtype == NMI_I32 && commit_count->dtype == NMI_I32, op,
            "positions/commit_count must be I32");
    const int32_t D = k->ne[0];
    const int32_t Hkv = k->ne[1];
    const int32_t T = k->ne[2];
    const int32_t B = k->ne[3];
    require(T > 0, op, "T must be positive");
    require(Hkv == cache->num_kv_heads && D == cache->head_dim, op, "k/v do not match the cache");
    validate_new_kv(k, v, D, Hkv, T, B, op);
    require((reinterpret_cast<uintptr_t>(k->data) & 15u) == 0 && (reinterpret_cast<uintptr_t>(v->data) & 15u) == 0,
            op, "k/v must be 16-byte aligned");
    require_shape(*positions, T, B, 1, 1, op, "positions");
    require_shape(*commit_count, B, 1, 1, 1, op, "commit_count");
    require_contiguous_nonnull(*positions, op, "positions");
    require_contiguous_nonnull(*commit_count, op, "commit_count");
    require(envelope.min_count <= envelope.max_count && envelope.max_count <= static_cast<uint32_t>(T) &&
                envelope.max_count <= capacity,
            op, "invalid execution envelope");
    const CacheRef c = validate_cache(cache, Hkv, B, op, false);
    if (c.kc != nullptr) { require_built(c, op); }
    require(c.kc != nullptr || D % 8 == 0, op, "BF16 head_dim must be a multiple of 8");
    if (envelope.max_count == 0) { return; }
    CommitBounds bounds;
    bounds.min_count = static_cast<int32_t>(envelope.min_count);
    bounds.max_count = static_cast<int32_t>(envelope.max_count);
    bounds.slot_mask = slot_mask;
    launch_kv_append(static_cast<const uint16_t*>(k->data), static_cast<const uint16_t*>(v->data),
                     static_cast<const int32_t*>(positions->data), static_cast<const int32_t*>(commit_count->data),
                     bounds, T, c, stream);
}

} // namespace

void set_last_error(const std::string& msg) { g_last_error = msg; }

} // namespace nmi

using namespace nmi;

extern "C" {

const char* nmi_last_error(void) { return g_last_error.c_str(); }

const char* nmi_build_info(void) {
    return "ninfer_amd gfx950: verify_attn_partial<{1,2},{128,256}> fp16-MFMA 16x16x32 (INT8-G64 KV), "
           "verify_attn_partial_bf16<{1,2},{128,256}> bf16-MFMA 16x16x32 (BF16 KV), "
           "verify_attn_merge (B = 1) and verify_attn_merge_rows (batches), kv_quant_append, bf16_kv_append, argmax, speculative accept (greedy, top-20 "
           "stochastic, general fixed-point), kv commit/rollback/compaction, gdn_recurrent<{16,32,64,128}> "
           "(snapshot), conv1d_silu (snapshot), device scalars, linear_q6<{4,8,16} cols> f16-MFMA (Q6G64 lm_head, "
           "fused argmax)";
}

size_t nmi_gqa_attention_workspace_bytes(int32_t q_heads, int32_t kv_heads, int32_t head_dim,
                                         int32_t tokens, int32_t batch,
                                         uint32_t max_visible_keys) {
    // 0 for invalid shapes and for batches above 32 tokens (no built route: the op itself reports
    // NMI_UNSUPPORTED)
    if (tokens <= 0 || batch <= 0 || kv_heads <= 0 || q_heads <= 0 || q_heads % kv_heads != 0 || head_dim <= 0 ||
        max_visible_keys == 0 || q_heads / kv_heads > kAttnRowsPerTile || (tokens > kAttnMaxTokens && batch != 1)) {
        return 0;
    }
    // the cache type is not an argument: the larger of the two row forms; the prompt route reuses one
    // workspace for its launches of 32 tokens and its shorter last launch
    const auto bytes = [&](int32_t T) {
        return std::max(plan_attention(q_heads, kv_heads, head_dim, T, batch, max_visible_keys, true).bytes,
                        plan_attention(q_heads, kv_heads, head_dim, T, batch, max_visible_keys, false).bytes);
    };
    if (tokens <= kAttnMaxTokens) { return bytes(tokens); }
    const PromptChunks pc = prompt_chunks(tokens);
    return std::max(bytes(kAttnMaxTokens), pc.tail > 0 ? bytes(pc.tail) : size_t{0});
}

// reference gqa_attention_workspace_bytes(q_heads, tokens) (src/ops/wrapper/gqa_attention.cpp:229-245):
// the registered geometries keyed by query heads (kv_heads_for_q_heads, :24-28) plus the 40/8/128
// verify geometry; the size covers every execution envelope of one sequence.
int nmi_gqa_attention_workspace_bound(int32_t q_heads, int32_t tokens, size_t* bytes) {
    const std::string op = "gqa_attention_workspace_bytes";
    return guarded([&] {
        require(bytes != nullptr, op, "bytes must be non-null");
        *bytes = 0;
        // T <= 0 needs nothing (as in the reference)
        if (tokens <= 0) { return; }
        int32_t kv_heads = 0, head_dim = 0;
        switch (q_heads) {
        case 24: kv_heads = 4; head_dim = 256; break;
        case 16: kv_heads = 2; head_dim = 256; break;
        case 40: kv_heads = 8; head_dim = 128; break;
        default: throw InvalidArgument(op + ": unsupported Q/KV head geometry");
        }
        if (tokens <= kAttnMaxTokens) {
            *bytes = attention_workspace_bound(q_heads, kv_heads, head_dim, tokens);
        } else { // the prompt route's launches of 32 tokens and its shorter last launch
            const PromptChunks pc = prompt_chunks(tokens);
            *bytes = std::max(attention_workspace_bound(q_heads, kv_heads, head_dim, kAttnMaxTokens),
                              pc.tail > 0 ? attention_workspace_bound(q_heads, kv_heads, head_dim, pc.tail) : size_t{0});
        }
    });
}

int nmi_gqa_attention(const nmi_tensor* q, const nmi_tensor* k, const nmi_tensor* v,
                      const nmi_tensor* positions, float scale, const nmi_kv_layer_view* cache,
                      nmi_gqa_envelope envelope, void* workspace, size_t workspace_bytes,
                      nmi_tensor* out, nmi_stream_t stream) {
    return attention_impl(q, k, v, positions, nullptr, scale, cache, envelope, true, workspace,
                          workspace_bytes, out, reinterpret_cast<hipStream_t>(stream),
                          "gqa_attention");
}

int nmi_gqa_attention_noalloc(const nmi_tensor* q, const nmi_tensor* k, const nmi_tensor* v,
                              const nmi_tensor* positions, float scale, const nmi_kv_layer_view* cache,
                              nmi_gqa_envelope envelope, nmi_tensor* out, nmi_stream_t stream) {
    return attention_impl(q, k, v, positions, nullptr, scale, cache, envelope, true, nullptr, 0, out,
                          reinterpret_cast<hipStream_t>(stream), "gqa_attention_noalloc", true);
}

int nmi_gqa_attention_cached(const nmi_tensor* q, const nmi_tensor* positions, float scale,
                             const nmi_kv_layer_view* cache, nmi_gqa_envelope envelope,
                             void* workspace, size_t workspace_bytes, nmi_tensor* out,
                             nmi_stream_t stream) {
    return attention_impl(q, nullptr, nullptr, positions, nullptr, scale, cache, envelope, false,
                          workspace, workspace_bytes, out, reinterpret_cast<hipStream_t>(stream),
                          "gqa_attention_cached");
}

int nmi_gqa_attention_tree(const nmi_tensor* q, const nmi_tensor* k, const nmi_tensor* v,
                           const nmi_tensor* positions, const nmi_tensor* parents, float scale,
                           const nmi_kv_layer_view* cache, nmi_gqa_envelope envelope,
                           int32_t write_cache, void* workspace, size_t workspace_bytes,
                           nmi_tensor* out, nmi_stream_t stream) {
    if (parents == nullptr) {
        set_last_error("gqa_attention_tree: parents must be non-null");
        return NMI_INVALID_ARGUMENT;
    }
    return attention_impl(q, k, v, positions, parents, scale, cache, envelope, write_cache != 0,
                          workspace, workspace_bytes, out, reinterpret_cast<hipStream_t>(stream),
                          "gqa_attention_tree");
}

// reference gqa_kv_append (src/ops/wrapper/gqa_attention.cpp:278-302).
int nmi_gqa_kv_append(const nmi_tensor* k, const nmi_tensor* v, const nmi_tensor* positions,
                      const nmi_kv_layer_view* cache, nmi_stream_t stream) {
    const std::string op = "gqa_kv_append";
    return guarded([&] {
        require_tensor(k, op, "k");
        require_tensor(v, op, "v");
        require_tensor(positions, op, "positions");
        require(k->dtype == NMI_BF16 && v->dtype == NMI_BF16, op, "k/v must be BF16");
        require(positions->dtype == NMI_I32, op, "positions must be I32");
        require(cache != nullptr, op, "cache must be non-null");
        const int32_t D = k->ne[0];
        const int32_t Hkv = k->ne[1];
        const int32_t T = k->ne[2];
        const int32_t B = k->ne[3];
        require(Hkv > 0 && Hkv == cache->num_kv_heads, op, "unsupported KV head geometry");
        require(T > 0, op, "T must be positive");
        require(D == cache->head_dim, op, "k head_dim does not match the cache");
        validate_new_kv(k, v, D, Hkv, T, B, op);
        require_shape(*positions, T, B, 1, 1, op, "positions");
        require_contiguous_nonnull(*positions, op, "positions");
        const CacheRef c = validate_cache(cache, Hkv, B, op, false);
        require(static_cast<uint32_t>(T) <= cache->max_context, op, "T exceeds KV cache capacity");
        require_built(c, op);
        launch_kv_append(static_cast<const uint16_t*>(k->data), static_cast<const uint16_t*>(v->data),
                         static_cast<const int32_t*>(positions->data), nullptr, CommitBounds{}, T, c,
                         reinterpret_cast<hipStream_t>(stream));
    });
}

int nmi_kv_cache_append_prefix(const nmi_tensor* k, const nmi_tensor* v,
                               const nmi_tensor* positions, const nmi_tensor* commit_count,
                               nmi_commit_envelope envelope, const nmi_kv_layer_view* cache,
                               nmi_stream_t stream) {
    const std::string op = "kv_cache_append_prefix";
    return guarded([&] {
        require(cache != nullptr, op, "cache must be non-null");
        append_prefix_impl(k, v, positions, commit_count, envelope, cache, cache->max_context, 0x7FFFFFFF,
                           reinterpret_cast<hipStream_t>(stream), op);
    });
}

int nmi_kv_cache_append_prefix_cyclic(const nmi_tensor* k, const nmi_tensor* v,
                                      const nmi_tensor* positions, const nmi_tensor* commit_count,
                                      nmi_commit_envelope envelope, const nmi_cyclic_kv_layer_view* cache,
                                      nmi_stream_t stream) {
    const std::string op = "kv_cache_append_prefix";
    return guarded([&] {
        require(cache != nullptr, op, "cache must be non-null");
        // reference validate_cyclic_cache (src/ops/wrapper/kv_cache_append_prefix.cpp:82-101) fixes
        // the ring at 4096 slots; any power of two from 128 up is accepted here.
        const uint32_t cap = cache->capacity;
        require(cap >= 128 && cap <= (1u << 30) && (cap & (cap - 1)) == 0, op, "invalid cyclic cache");
        require(cache->padded_capacity >= cap, op, "invalid cyclic cache");
        nmi_kv_layer_view linear{};
        linear.k = cache->k;
        linear.v = cache->v;
        linear.k_scale = cache->k_scale;
        linear.v_scale = cache->v_scale;
        linear.max_context = cap;
        linear.padded_context = cache->padded_capacity;
        linear.num_kv_heads = cache->num_kv_heads;
        linear.head_dim = cache->head_dim;
        linear.dtype = cache->dtype;
        linear.quant_group = cache->quant_group;
        append_prefix_impl(k, v, positions, commit_count, envelope, &linear, cap, static_cast<int32_t>(cap - 1),
                           reinterpret_cast<hipStream_t>(stream), op);
    });
}

// Explicit rollback: positions [T, B], keep_count [B].
int nmi_kv_cache_rollback(const nmi_tensor* positions, const nmi_tensor* keep_count,
                          const nmi_kv_layer_view* cache, nmi_stream_t stream) {
    const std::string op = "kv_cache_rollback";
    return guarded([&] {
        require_tensor(positions, op, "positions");
        require_tensor(keep_count, op, "keep_count");
        require(cache != nullptr, op, "cache must be non-null");
        require(positions->dtype == NMI_I32 && keep_count->dtype == NMI_I32, op, "positions/keep_count must be I32");
        const int32_t T = positions->ne[0];
        const int32_t B = positions->ne[1];
        require(T > 0 && T <= kAttnMaxTokens, op, "T must be in [1, 32]");
        require_shape(*positions, T, B, 1, 1, op, "positions");
        require_shape(*keep_count, B, 1, 1, 1, op, "keep_count");
        require_contiguous_nonnull(*positions, op, "positions");
        require_contiguous_nonnull(*keep_count, op, "keep_count");
        const CacheRef c = validate_cache(cache, cache->num_kv_heads, B, op, false);
        require(c.kc != nullptr, op, "rollback is defined for INT8-G64 caches");
        launch_kv_rollback(static_cast<const int32_t*>(positions->data),
                           static_cast<const int32_t*>(keep_count->data), T, c,
                           reinterpret_cast<hipStream_t>(stream));
    });
}

// Path compaction: base_position [B], path [T, B], path_len [B].
int nmi_kv_cache_compact_path(const nmi_tensor* base_position, const nmi_tensor* path,
                              const nmi_tensor* path_len, const nmi_kv_layer_view* cache,
                              nmi_stream_t stream) {
    const std::string op = "kv_cache_compact_path";
    return guarded([&] {
        require_tensor(base_position, op, "base_position");
        require_tensor(path, op, "path");
        require_tensor(path_len, op, "path_len");
        require(cache != nullptr, op, "cache must be non-null");
        require(base_position->dtype == NMI_I32 && path->dtype == NMI_I32 && path_len->dtype == NMI_I32,
                op, "base_position/path/path_len must be I32");
        const int32_t T = path->ne[0];
        const int32_t B = path->ne[1];
        require(T > 0 && T <= kAttnMaxTokens, op, "path capacity must be in [1, 32]");
        require_shape(*path, T, B, 1, 1, op, "path");
        require_shape(*path_len, B, 1, 1, 1, op, "path_len");
        require_shape(*base_position, B, 1, 1, 1, op, "base_position");
        require_contiguous_nonnull(*path, op, "path");
        require_contiguous_nonnull(*path_len, op, "path_len");
        require_contiguous_nonnull(*base_position, op, "base_position");
        const CacheRef c = validate_cache(cache, cache->num_kv_heads, B, op, false);
        require(c.kc != nullptr, op, "compaction is defined for INT8-G64 caches");
        launch_kv_compact_path(static_cast<const int32_t*>(base_position->data),
                               static_cast<const int32_t*>(path->data),
                               static_cast<const int32_t*>(path_len->data), T, c,
                               reinterpret_cast<hipStream_t>(stream));
    });
}

} // extern "C"
