// C ABI of the Q6G64_F16S RowSplit linear and the fused linear -> argmax, with the host checks of
// the reference wrapper (src/ops/linear/linear.cpp:65-152,200-209).
#include "common.h"
#include "linear_internal.h"

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
// alignment: 16-byte x/out/code/high, 4-byte scales).
Checked check(const nmi_tensor* x, const nmi_weight* w, const nmi_tensor* out, int32_t out_dtype) {
    require(x != nullptr && w != nullptr && out != nullptr, "x, weight and out must be non-null");
    require(x->dtype == NMI_BF16, "x must be BF16");
    require(x->ne[2] == 1 && x->ne[3] == 1, "x must have shape [K,T]");
    require(w->n > 0 && w->k > 0, "weight n/k must be positive");
    require(x->ne[0] == w->k, "x K dimension must match weight.k");
    const int32_t T = x->ne[1];
    require(T >= 1, "T must be positive");
    if (out_dtype == NMI_BF16) {
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
    require(aligned(x->data, 16) && aligned(out->data, out_dtype == NMI_BF16 ? 16 : 4) && aligned(w->qdata, 16) &&
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
        const LinearPlan p = plan_linear(c.args.N, c.args.Kp, c.T);
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
        const LinearPlan p = plan_linear(c.args.N, c.args.Kp, c.T);
        const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
        launch_linear_q6(c.args, p, s);
        launch_linear_argmax_reduce(c.args.keys, c.T, p.grid * p.waves, static_cast<int32_t*>(out->data), s);
    });
}

} // extern "C"
