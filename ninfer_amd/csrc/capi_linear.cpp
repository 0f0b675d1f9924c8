// C ABI of the Q6G64_F16S RowSplit linear and the fused linear -> argmax, with the host checks of
// the reference wrapper (src/ops/linear/linear.cpp:65-152,200-209).
#include "common.h"
#include "linear_internal.h"
#include "sampler_internal.h"

#include <limits>

namespace nmi {
namespace {

void require(bool ok, const std::string& what) {
    if (!ok) { throw InvalidArgument("linear: " + what); }
}

uint64_t checked_mul(uint64_t a, uint64_t b) {
    if (a != 0 && b > std::numeric_limits<uint64_t>::max() / a) { throw Overflow("linear: row-split payload size overflows uint64"); }
    return a * b;
}

uint64_t align_up(uint64_t v, uint64_t a) { return (v + a - 1) / a * a; }

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

struct Checked {
    LinearArgs args;
    int32_t T;
};

// src/ops/linear/linear.cpp:65-152 (shapes, RowSplit metadata, payload size) and :200-209 (Q6
// alignment: 16-byte x/out/code/high, 4-byte scales). out_dtype < 0: no output tensor (the fused
// acceptance form).
Checked check(const nmi_tensor* x, const nmi_weight* w, const nmi_tensor* out, int32_t out_dtype) {
    require(x != nullptr && w != nullptr && (out != nullptr || out_dtype < 0), "x, weight and out must be non-null");
    require(x->dtype == NMI_BF16, "x must be BF16");
    require(x->ne[2] == 1 && x->ne[3] == 1, "x must have shape [K,T]");
    require(w->n > 0 && w->k > 0, "weight n/k must be positive");
    require(x->ne[0] == w->k, "x K dimension must match weight.k");
    const int32_t T = x->ne[1];
    require(T >= 1, "T must be positive");
    if (out_dtype < 0) {
        out = x; // only x is checked below
    } else if (out_dtype == NMI_BF16) {
        require(out->dtype == NMI_BF16 && out->ne[2] == 1 && out->ne[3] == 1 && out->ne[1] == T, "out must have shape [N,T]");
        require(out->ne[0] == w->n, "out N dimension must match weight.n");
    } else {
        require(out->dtype == NMI_I32 && out->ne[0] == T && out->ne[1] == 1 && out->ne[2] == 1 && out->ne[3] == 1,
                "out must be I32 [T]");
    }
    require(is_contiguous(*x) && is_contiguous(*out), "x/out must be contiguous");
    require(x->data != nullptr && out->data != nullptr, "x/out data must be non-null");
    require(w->qtype == NMI_Q6G64_F16S, "only Q6G64_F16S weights are built");
    require(w->layout == NMI_ROW_SPLIT, "weight must be RowSplit");
    require(w->ndim == 2, "weight must be 2-D [N,K]");
    require(w->shape[0] == w->n && w->shape[1] == w->k, "weight shape must match n/k");
    require(w->shape[2] == 1 && w->shape[3] == 1 && w->padded_shape[2] == 1 && w->padded_shape[3] == 1,
            "weight trailing dimensions must be 1");
    require(w->group == 64 && w->group_size == 64u, "weight group is invalid");
    require(w->scale_dtype == NMI_FP16, "weight scale dtype must be FP16");
    const uint64_t Kp = align_up(static_cast<uint64_t>(w->k), 128);
    require(w->padded_shape[0] == w->shape[0] && static_cast<uint64_t>(w->padded_shape[1]) == Kp, "padded shape is invalid");
    const uint64_t kg = Kp / 64;
    const uint64_t groups = checked_mul(static_cast<uint64_t>(w->n), kg);
    const uint64_t nib = checked_mul(groups, 32);
    const uint64_t high = checked_mul(groups, 16);
    const uint64_t sc = checked_mul(groups, 2);
    const uint64_t expected = align_up(nib, 256) + align_up(high, 256) + sc;
    require(w->payload_bytes >= expected, "payload is too small");
    require(w->qdata != nullptr && w->scales != nullptr, "nibble and scale planes must be non-null");
    require(w->qhigh != nullptr && w->high_plane_bytes >= high, "high plane must be non-null");
    require(aligned(x->data, 16) && aligned(out->data, out_dtype == NMI_I32 ? 4 : 16) && aligned(w->qdata, 16) &&
                aligned(w->qhigh, 16) && aligned(w->scales, 4),
            "Q6 RowSplit requires 16-byte x/out/code/high and 4-byte scale alignment");
    if (Kp > static_cast<uint64_t>(kLinearMaxPaddedK) || nib >= (1ull << 31)) {
        throw Unsupported("linear: the Q6 kernel serves padded K <= 8192 and planes below 2 GiB");
    }
    Checked c{};
    LinearArgs& a = c.args;
    a.qdata = static_cast<const uint8_t*>(w->qdata);
    a.qhigh = static_cast<const uint8_t*>(w->qhigh);
    a.scales = static_cast<const uint16_t*>(w->scales);
    a.x = static_cast<const uint16_t*>(x->data);
    a.nib_bytes = static_cast<int64_t>(nib);
    a.high_bytes = static_cast<int64_t>(high);
    a.scale_bytes = static_cast<int64_t>(sc);
    a.N = w->n;
    a.K = w->k;
    a.Kp = static_cast<int32_t>(Kp);
    a.G = static_cast<int32_t>(kg);
    a.T = T;
    a.valid_rows = w->n;
    c.T = T;
    return c;
}

} // namespace
} // namespace nmi

using namespace nmi;

extern "C" {

int nmi_linear(const nmi_tensor* x, const nmi_weight* w, nmi_tensor* out, nmi_stream_t stream) {
    return guarded([&] {
        Checked c = check(x, w, out, NMI_BF16);
        c.args.out = static_cast<uint16_t*>(out->data);
        const LinearPlan p = plan_linear(c.args.N, c.args.Kp, c.T, false, c.args.K);
        launch_linear_q6(c.args, p, reinterpret_cast<hipStream_t>(stream));
    });
}

size_t nmi_linear_argmax_workspace_bytes(int32_t tokens) {
    return tokens >= 1 ? linear_argmax_workspace_bytes(tokens) : 0;
}

int nmi_linear_argmax(const nmi_tensor* x, const nmi_weight* w, int32_t valid_rows, void* workspace,
                      size_t workspace_bytes, nmi_tensor* out, nmi_stream_t stream) {
    return guarded([&] {
        Checked c = check(x, w, out, NMI_I32);
        require(valid_rows >= 1 && valid_rows <= w->n, "valid_rows must be in [1, n]");
        require(workspace != nullptr && workspace_bytes >= linear_argmax_workspace_bytes(c.T) &&
                    aligned(workspace, 256),
                "workspace must be non-null, 256-byte aligned and at least the size query");
        c.args.valid_rows = valid_rows;
        c.args.keys = static_cast<uint64_t*>(workspace);
        const LinearPlan p = plan_linear(c.args.N, c.args.Kp, c.T, false, c.args.K);
        const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
        launch_linear_q6(c.args, p, s);
        launch_linear_argmax_reduce(c.args.keys, c.T, p.grid * p.waves, static_cast<int32_t*>(out->data), s);
    });
}

size_t nmi_speculative_accept_fused_head_workspace_bytes(int32_t K, int32_t batch) {
    if (K < 1 || K + 1 > kMaxColumns || batch < 1) { return 0; }
    return linear_topcap_workspace_bytes((K + 1) * batch);
}

int nmi_speculative_accept_fused_head(const nmi_tensor* x, const nmi_weight* w, const nmi_tensor* drafts,
                                      nmi_tensor* length, nmi_tensor* token, nmi_tensor* sampled_out,
                                      nmi_tensor* num_sampled, nmi_tensor* accepted, nmi_tensor* stats,
                                      int32_t token_domain, const nmi_sampling_config* config, void* workspace,
                                      size_t workspace_bytes, nmi_stream_t stream) {
    const std::string op = "speculative_accept_fused_head";
    return guarded([&] {
        int32_t B = 0;
        SpecArgs s = check_accept_state(drafts, length, token, sampled_out, num_sampled, accepted, stats, config, op, B);
        const int32_t K = s.K;
        require(x != nullptr && x->ne[1] == K + 1 && x->ne[2] == B && x->ne[3] == 1,
                "x must be [hidden, K+1, B] (the verify columns of every sequence)");
        // The kernel reads (K+1) * B packed columns, so x itself must be packed (a view of the first
        // K+1 columns of a wider hidden buffer would hand sequences b >= 1 the wrong rows); x2 below
        // rewrites the batch stride, so it is checked here, before the rewrite.
        require(is_contiguous(*x), "x must be contiguous [hidden, K+1, B]");
        nmi_tensor x2 = *x; // the columns of all sequences as one [hidden, (K+1) * B] operand
        x2.ne[1] = (K + 1) * B;
        x2.ne[2] = 1;
        x2.nb[2] = x2.nb[1] * x2.ne[1];
        Checked c = check(&x2, w, nullptr, -1);
        require(token_domain >= 1 && token_domain <= w->n, "token_domain must be in [1, weight.n]");
        const size_t need = linear_topcap_workspace_bytes(c.T);
        require(workspace != nullptr && workspace_bytes >= need && aligned(workspace, 256),
                "workspace must be non-null, 256-byte aligned and at least the size query");
        const LinearPlan p = plan_linear(c.args.N, c.args.Kp, c.T, true, c.args.K);
        c.args.valid_rows = token_domain;
        c.args.cand = static_cast<uint64_t*>(workspace);
        c.args.config = config;
        c.args.drafts = s.drafts;
        c.args.cols_per_seq = K + 1;
        const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
        launch_linear_q6(c.args, p, st);
        s.target_tokens = nullptr;
        s.partial = c.args.cand;
        s.token_domain = token_domain;
        s.ntiles = p.grid;
        launch_spec_merge_accept_wide(s, B, st);
    });
}

} // extern "C"
