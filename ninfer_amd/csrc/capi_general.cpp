// C ABI of the general speculative acceptance ("Mode F"; no reference counterpart). Validation
// follows the reference accept wrapper's conventions (src/ops/wrapper/speculative_round.cpp:67-102)
// for the shared arguments, then dispatches to general_accept.hip.
#include "common.h"
#include "general_internal.h"
#include "sampler_internal.h"

#include <string>

using namespace nmi;

namespace {

void require(bool ok, const std::string& op, const std::string& what) {
    if (!ok) { throw InvalidArgument(op + ": " + what); }
}

void require_dtype(const nmi_tensor* t, int32_t dtype, const std::string& op, const char* name) {
    require(t != nullptr, op, std::string(name) + " must be non-null");
    require(t->dtype == dtype, op, std::string("invalid dtype for ") + name);
    require(is_contiguous(*t), op, std::string(name) + " must be contiguous");
    require(t->data != nullptr, op, std::string(name) + " data must be non-null");
}

void require_matrix(const nmi_tensor* t, int32_t dtype, int32_t n, int32_t B, const std::string& op,
                    const char* name) {
    require_dtype(t, dtype, op, name);
    require(t->ne[0] == n && t->ne[1] == B && t->ne[2] == 1 && t->ne[3] == 1, op,
            std::string("invalid vector shape for ") + name);
}

bool valid_domain(int32_t token_domain) {
    return token_domain > 0 && token_domain <= kGenTile * kGenMaxTiles;
}

} // namespace

extern "C" {

size_t nmi_general_accept_workspace_bytes(int32_t token_domain, int32_t K, int32_t batch) {
    if (!valid_domain(token_domain) || K <= 0 || batch <= 0) { return 0; }
    return plan_general(token_domain, K, batch).bytes;
}

int nmi_speculative_accept_general(const nmi_tensor* logits, const nmi_tensor* draft_logits,
                                   const nmi_tensor* drafts, const nmi_tensor* u_accept,
                                   const nmi_tensor* u_residual, nmi_tensor* length,
                                   nmi_tensor* token, nmi_tensor* sampled_out,
                                   nmi_tensor* num_sampled, nmi_tensor* accepted,
                                   nmi_tensor* stats, int32_t token_domain,
                                   const nmi_general_config* config, void* workspace,
                                   size_t workspace_bytes, nmi_stream_t stream) {
    const std::string op = "speculative_accept_general";
    return guarded([&] {
        require(drafts != nullptr, op, "drafts must be non-null");
        const int32_t K = drafts->ne[0];
        const int32_t B = drafts->ne[1];
        require(K >= 1, op, "K must be >=1");
        require(K + 1 <= kMaxColumns, op, "K must be <= 15");
        require(B >= 1, op, "batch must be >=1");
        require_matrix(drafts, NMI_I32, K, B, op, "drafts");
        require_dtype(logits, NMI_BF16, op, "logits");
        require(logits->ne[0] > 0 && logits->ne[1] >= K + 1 && logits->ne[2] == B && logits->ne[3] == 1, op,
                "logits must be [physical_rows, >=k+1, batch]");
        require_dtype(draft_logits, NMI_BF16, op, "draft_logits");
        require(draft_logits->ne[0] > 0 && draft_logits->ne[1] >= K && draft_logits->ne[2] == B &&
                    draft_logits->ne[3] == 1,
                op, "draft_logits must be [physical_rows, >=k, batch]");
        require(token_domain > 0 && token_domain <= logits->ne[0] && token_domain <= draft_logits->ne[0], op,
                "token_domain must be in [1, physical rows]");
        require(valid_domain(token_domain), op, "token_domain exceeds 1048576");
        require_matrix(u_accept, NMI_FP32, K + 1, B, op, "u_accept");
        require_matrix(u_residual, NMI_FP32, 1, B, op, "u_residual");
        require_matrix(length, NMI_I32, B, 1, op, "length");
        require_matrix(token, NMI_I32, B, 1, op, "token");
        require_matrix(sampled_out, NMI_I32, K + 1, B, op, "sampled_out");
        require_matrix(num_sampled, NMI_I32, B, 1, op, "num_sampled");
        require_matrix(accepted, NMI_I32, B, 1, op, "accepted");
        require_dtype(stats, NMI_I64, op, "stats");
        require(stats->ne[0] >= 4 + K && stats->ne[1] == B && stats->ne[2] == 1 && stats->ne[3] == 1, op,
                "invalid vector shape for stats");
        require(config != nullptr, op, "config must be non-null");
        const GenPlan plan = plan_general(token_domain, K, B);
        require(workspace_bytes >= plan.bytes, op, "workspace is smaller than the size query");
        require(workspace != nullptr, op, "workspace must be non-null");
        require((reinterpret_cast<uintptr_t>(workspace) & 255u) == 0, op, "workspace must be 256-byte aligned");
        GenLaunch l;
        l.logits = static_cast<const uint16_t*>(logits->data);
        l.draft_logits = static_cast<const uint16_t*>(draft_logits->data);
        l.drafts = static_cast<const int32_t*>(drafts->data);
        l.u_accept = static_cast<const float*>(u_accept->data);
        l.u_residual = static_cast<const float*>(u_residual->data);
        l.length = static_cast<int32_t*>(length->data);
        l.token = static_cast<int32_t*>(token->data);
        l.sampled_out = static_cast<int32_t*>(sampled_out->data);
        l.num_sampled = static_cast<int32_t*>(num_sampled->data);
        l.accepted = static_cast<int32_t*>(accepted->data);
        l.stats = static_cast<int64_t*>(stats->data);
        l.config = config;
        l.logit_col = logits->ne[0];
        l.logit_seq = static_cast<int64_t>(logits->ne[0]) * logits->ne[1];
        l.draft_col = draft_logits->ne[0];
        l.draft_seq = static_cast<int64_t>(draft_logits->ne[0]) * draft_logits->ne[1];
        l.stats_stride = stats->ne[0];
        l.token_domain = token_domain;
        l.K = K;
        l.B = B;
        launch_general_accept(l, plan, workspace, reinterpret_cast<hipStream_t>(stream));
    });
}

} // extern "C"
