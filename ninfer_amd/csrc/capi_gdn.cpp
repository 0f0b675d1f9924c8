// C ABI of the recurrent-state ops (Gated DeltaNet recurrence, causal conv1d + SiLU, device scalar
// ops) with host validation restating the reference wrappers:
// src/ops/wrapper/gated_delta_rule.cpp:29-139, src/ops/wrapper/causal_conv1d_silu.cpp:35-200,
// src/ops/wrapper/scalar.cpp:11-41.
#include "common.h"
#include "gdn_internal.h"

#include <cmath>

namespace nmi {
namespace {

void require(bool ok, const std::string& op, const std::string& what) {
    if (!ok) { throw InvalidArgument(op + ": " + what); }
}

void require_tensor(const nmi_tensor* t, int32_t dtype, const std::string& op, const char* name) {
    require(t != nullptr, op, std::string(name) + " must be non-null");
    require(t->dtype == dtype, op, std::string("invalid dtype for ") + name);
}

void require_shape(const nmi_tensor* t, int32_t n0, int32_t n1, int32_t n2, int32_t n3, const std::string& op,
                   const char* name) {
    require(t->ne[0] == n0 && t->ne[1] == n1 && t->ne[2] == n2 && t->ne[3] == n3, op,
            std::string("invalid shape for ") + name);
}

void require_contiguous_nonnull(const nmi_tensor* t, const std::string& op, const char* name) {
    require(is_contiguous(*t), op, std::string(name) + " must be contiguous");
    require(t->data != nullptr, op, std::string(name) + " data must be non-null");
}

size_t byte_size(const nmi_tensor* t) { return static_cast<size_t>(numel(*t)) * dtype_size(t->dtype); }

bool overlap(const nmi_tensor* a, const nmi_tensor* b) {
    const auto* pa = static_cast<const char*>(a->data);
    const auto* pb = static_cast<const char*>(b->data);
    return pa < pb + byte_size(b) && pb < pa + byte_size(a);
}

struct GdnGeometry {
    int32_t S, Hqk, Hv, T;
};

bool supported_head_dim(int32_t s) { return s == 16 || s == 32 || s == 64 || s == 128; }

// src/ops/wrapper/gated_delta_rule.cpp:51-72
GdnGeometry gdn_geometry(const nmi_tensor* q, const nmi_tensor* v, float scale, const std::string& op) {
    require(q != nullptr && v != nullptr, op, "q and v must be non-null");
    const GdnGeometry g{q->ne[0], q->ne[1], v->ne[1], q->ne[2]};
    require(supported_head_dim(g.S), op, "head dimension must be 16, 32, 64, or 128");
    require(g.Hqk >= 1 && g.Hv >= g.Hqk && g.Hv % g.Hqk == 0, op,
            "value heads must be at least q/k heads and divisible by them");
    require(g.T > 0, op, "T must be positive");
    const float expected = 1.0f / std::sqrt(static_cast<float>(g.S));
    require(std::isfinite(scale) && scale > 0.0f && std::abs(scale - expected) <= 1.0e-6f, op,
            "scale must be 1/sqrt(head_dim)");
    return g;
}

GdnArgs gdn_inputs(const nmi_tensor* q, const nmi_tensor* k, const nmi_tensor* v, const nmi_tensor* g,
                   const nmi_tensor* beta, const nmi_tensor* out, float scale, bool normalize_qk,
                   const GdnGeometry& s, const std::string& op) {
    require_tensor(q, NMI_BF16, op, "q");
    require_tensor(k, NMI_BF16, op, "k");
    require_tensor(v, NMI_BF16, op, "v");
    require_tensor(out, NMI_BF16, op, "out");
    require_tensor(g, NMI_FP32, op, "g");
    require_tensor(beta, NMI_FP32, op, "beta");
    require_shape(q, s.S, s.Hqk, s.T, 1, op, "q");
    require_shape(k, s.S, s.Hqk, s.T, 1, op, "k");
    require_shape(v, s.S, s.Hv, s.T, 1, op, "v");
    require_shape(out, s.S, s.Hv, s.T, 1, op, "out");
    require_shape(g, s.Hv, s.T, 1, 1, op, "g");
    require_shape(beta, s.Hv, s.T, 1, 1, op, "beta");
    for (const auto& [t, name] : {std::pair{q, "q"}, {k, "k"}, {v, "v"}, {g, "g"}, {beta, "beta"}, {out, "out"}}) {
        require_contiguous_nonnull(t, op, name);
    }
    for (const auto& [t, name] : {std::pair{q, "q"}, {k, "k"}, {v, "v"}, {g, "g"}, {beta, "beta"}}) {
        require(!overlap(t, out), op, std::string(name) + " must not overlap out");
    }
    GdnArgs a{};
    a.q = static_cast<const uint16_t*>(q->data);
    a.k = static_cast<const uint16_t*>(k->data);
    a.v = static_cast<const uint16_t*>(v->data);
    a.g = static_cast<const float*>(g->data);
    a.beta = static_cast<const float*>(beta->data);
    a.out = static_cast<uint16_t*>(out->data);
    a.scale = scale;
    a.normalize_qk = normalize_qk ? 1 : 0;
    a.T = s.T;
    a.Hqk = s.Hqk;
    a.Hv = s.Hv;
    return a;
}

void require_state_apart(const nmi_tensor* state, const nmi_tensor* const* inputs, int n, const std::string& op,
                         const char* name) {
    for (int i = 0; i < n; ++i) {
        require(!overlap(state, inputs[i]), op, std::string(name) + " must not overlap the inputs or out");
    }
}

// src/ops/wrapper/causal_conv1d_silu.cpp:35-74
ConvArgs conv_inputs(const nmi_tensor* x, const nmi_tensor* weight, const nmi_tensor* out, const std::string& op) {
    require_tensor(x, NMI_BF16, op, "x");
    require_tensor(weight, NMI_BF16, op, "weight");
    require_tensor(out, NMI_BF16, op, "out");
    require(x->ne[2] == 1 && x->ne[3] == 1, op, "x must have shape [C,T]");
    require(x->ne[0] > 0, op, "C must be positive");
    require(x->ne[1] > 0, op, "T must be positive");
    require_shape(weight, x->ne[0], 4, 1, 1, op, "weight ([C,4])");
    require_shape(out, x->ne[0], x->ne[1], 1, 1, op, "out (must match x)");
    require_contiguous_nonnull(x, op, "x");
    require_contiguous_nonnull(weight, op, "weight");
    require_contiguous_nonnull(out, op, "out");
    require(!overlap(x, out) && !overlap(weight, out), op, "x and weight must not overlap out");
    ConvArgs a{};
    a.x = static_cast<const uint16_t*>(x->data);
    a.weight = static_cast<const uint16_t*>(weight->data);
    a.out = static_cast<uint16_t*>(out->data);
    a.C = x->ne[0];
    a.T = x->ne[1];
    return a;
}

void require_slot(const nmi_tensor* initial_slot, const std::string& op) {
    require_tensor(initial_slot, NMI_I32, op, "initial_slot");
    require_shape(initial_slot, 1, 1, 1, 1, op, "initial_slot");
    require_contiguous_nonnull(initial_slot, op, "initial_slot");
}

void require_scalar(const nmi_tensor* t, int32_t dtype, const char* name) {
    const std::string what = std::string(name) + " must be a non-null contiguous scalar";
    if (t == nullptr || t->dtype != dtype || numel(*t) != 1 || !is_contiguous(*t) || t->data == nullptr) {
        throw InvalidArgument(what);
    }
}

} // namespace
} // namespace nmi

using namespace nmi;

extern "C" {

int nmi_gated_delta_rule_workspace_bytes(int32_t head_dim, int32_t qk_heads, int32_t value_heads, int32_t tokens,
                                         int32_t normalize_qk, size_t* bytes) {
    return guarded([&] {
        (void)normalize_qk;
        if (!supported_head_dim(head_dim) || qk_heads < 1 || value_heads < qk_heads || value_heads % qk_heads != 0 ||
            tokens <= 0 || bytes == nullptr) {
            throw InvalidArgument("gated_delta_rule_workspace_bytes: invalid geometry");
        }
        *bytes = 0; // the recurrent kernel keeps every row in registers for any T
    });
}

int nmi_gated_delta_rule(const nmi_tensor* q, const nmi_tensor* k, const nmi_tensor* v, const nmi_tensor* g,
                         const nmi_tensor* beta, float scale, int32_t normalize_qk, const nmi_tensor* ssm_state_in,
                         nmi_tensor* ssm_state_out, nmi_tensor* out, nmi_stream_t stream) {
    const std::string op = "gated_delta_rule";
    return guarded([&] {
        const GdnGeometry s = gdn_geometry(q, v, scale, op);
        GdnArgs a = gdn_inputs(q, k, v, g, beta, out, scale, normalize_qk != 0, s, op);
        require_tensor(ssm_state_in, NMI_FP32, op, "ssm_state_in");
        require_tensor(ssm_state_out, NMI_FP32, op, "ssm_state_out");
        require_shape(ssm_state_in, s.S, s.S, s.Hv, 1, op, "ssm_state_in");
        require_shape(ssm_state_out, s.S, s.S, s.Hv, 1, op, "ssm_state_out");
        require_contiguous_nonnull(ssm_state_in, op, "ssm_state_in");
        require_contiguous_nonnull(ssm_state_out, op, "ssm_state_out");
        require(ssm_state_in->data == ssm_state_out->data || !overlap(ssm_state_in, ssm_state_out), op,
                "ssm_state_in and ssm_state_out must be disjoint or the same storage");
        const nmi_tensor* others[] = {q, k, v, g, beta, out};
        require_state_apart(ssm_state_in, others, 6, op, "ssm_state_in");
        require_state_apart(ssm_state_out, others, 6, op, "ssm_state_out");
        a.state_in = static_cast<const float*>(ssm_state_in->data);
        a.state_out = static_cast<float*>(ssm_state_out->data);
        launch_gdn_recurrent(a, s.S, reinterpret_cast<hipStream_t>(stream));
    });
}

int nmi_gated_delta_rule_snapshot(const nmi_tensor* q, const nmi_tensor* k, const nmi_tensor* v, const nmi_tensor* g,
                                  const nmi_tensor* beta, float scale, int32_t normalize_qk, nmi_tensor* ssm_states,
                                  const nmi_tensor* initial_slot, nmi_tensor* out, nmi_stream_t stream) {
    const std::string op = "gated_delta_rule";
    return guarded([&] {
        const GdnGeometry s = gdn_geometry(q, v, scale, op);
        GdnArgs a = gdn_inputs(q, k, v, g, beta, out, scale, normalize_qk != 0, s, op);
        require_tensor(ssm_states, NMI_FP32, op, "ssm_states");
        require(ssm_states->ne[0] == s.S && ssm_states->ne[1] == s.S && ssm_states->ne[2] == s.Hv &&
                    ssm_states->ne[3] >= s.T,
                op, "invalid shape for ssm_states snapshot");
        require_contiguous_nonnull(ssm_states, op, "ssm_states");
        require_slot(initial_slot, op);
        const nmi_tensor* others[] = {q, k, v, g, beta, out, initial_slot};
        require_state_apart(ssm_states, others, 7, op, "ssm_states");
        a.states = static_cast<float*>(ssm_states->data);
        a.initial_slot = static_cast<const int32_t*>(initial_slot->data);
        a.slots = ssm_states->ne[3];
        launch_gdn_recurrent(a, s.S, reinterpret_cast<hipStream_t>(stream));
    });
}

int nmi_causal_conv1d_silu(const nmi_tensor* x, const nmi_tensor* weight, const nmi_tensor* conv_state_in,
                           nmi_tensor* conv_state_out, nmi_tensor* out, nmi_stream_t stream) {
    const std::string op = "causal_conv1d";
    return guarded([&] {
        ConvArgs a = conv_inputs(x, weight, out, op);
        for (const auto& [t, name] : {std::pair{conv_state_in, "conv_state_in"}, {conv_state_out, "conv_state_out"}}) {
            require_tensor(t, NMI_BF16, op, name);
            require_shape(t, a.C, 3, 1, 1, op, name);
            require_contiguous_nonnull(t, op, name);
        }
        require(conv_state_in->data == conv_state_out->data || !overlap(conv_state_in, conv_state_out), op,
                "conv_state_in and conv_state_out must be disjoint or the same storage");
        const nmi_tensor* others[] = {x, weight, out};
        require_state_apart(conv_state_in, others, 3, op, "conv_state_in");
        require_state_apart(conv_state_out, others, 3, op, "conv_state_out");
        a.state_in = static_cast<const uint16_t*>(conv_state_in->data);
        a.state_out = static_cast<uint16_t*>(conv_state_out->data);
        launch_conv1d_silu(a, reinterpret_cast<hipStream_t>(stream));
    });
}

int nmi_causal_conv1d_silu_snapshot(const nmi_tensor* x, const nmi_tensor* weight, nmi_tensor* conv_states,
                                    const nmi_tensor* initial_slot, nmi_tensor* out, nmi_stream_t stream) {
    const std::string op = "causal_conv1d";
    return guarded([&] {
        ConvArgs a = conv_inputs(x, weight, out, op);
        require_tensor(conv_states, NMI_BF16, op, "conv_states");
        require(conv_states->ne[0] == a.C && conv_states->ne[1] == 3 && conv_states->ne[2] >= a.T &&
                    conv_states->ne[3] == 1,
                op, "conv_states must have shape [C,3,S] with S>=T");
        require_contiguous_nonnull(conv_states, op, "conv_states");
        require_slot(initial_slot, op);
        const nmi_tensor* others[] = {x, weight, out, initial_slot};
        require_state_apart(conv_states, others, 4, op, "conv_states");
        a.states = static_cast<uint16_t*>(conv_states->data);
        a.initial_slot = static_cast<const int32_t*>(initial_slot->data);
        a.slots = conv_states->ne[2];
        launch_conv1d_silu(a, reinterpret_cast<hipStream_t>(stream));
    });
}

int nmi_set_i32_scalar(nmi_tensor* destination, int32_t value, nmi_stream_t stream) {
    return guarded([&] {
        require_scalar(destination, NMI_I32, "set_i32_scalar destination");
        launch_scalar_op(0, nullptr, static_cast<int32_t*>(destination->data), nullptr, value,
                         reinterpret_cast<hipStream_t>(stream));
    });
}

int nmi_assign_i32_scalar(const nmi_tensor* source, nmi_tensor* destination, nmi_stream_t stream) {
    return guarded([&] {
        require_scalar(source, NMI_I32, "assign_i32_scalar source");
        require_scalar(destination, NMI_I32, "assign_i32_scalar destination");
        if (source->data == destination->data) {
            throw InvalidArgument("assign_i32_scalar: source and destination must not alias");
        }
        launch_scalar_op(1, static_cast<const int32_t*>(source->data), static_cast<int32_t*>(destination->data),
                         nullptr, 0, reinterpret_cast<hipStream_t>(stream));
    });
}

int nmi_increment_i32_scalar(nmi_tensor* scalar, nmi_stream_t stream) {
    return guarded([&] {
        require_scalar(scalar, NMI_I32, "increment_i32_scalar scalar");
        launch_scalar_op(2, nullptr, static_cast<int32_t*>(scalar->data), nullptr, 0,
                         reinterpret_cast<hipStream_t>(stream));
    });
}

int nmi_increment_i64_scalar(nmi_tensor* scalar, nmi_stream_t stream) {
    return guarded([&] {
        require_scalar(scalar, NMI_I64, "increment_i64_scalar scalar");
        launch_scalar_op(3, nullptr, nullptr, static_cast<long long*>(scalar->data), 0,
                         reinterpret_cast<hipStream_t>(stream));
    });
}

} // extern "C"
