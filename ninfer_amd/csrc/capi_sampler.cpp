// C ABI for the acceptance half of the verify step: validation mirroring the reference wrappers
// (src/ops/wrapper/argmax.cpp, src/ops/wrapper/speculative_round.cpp:50-118) plus the batch
// dimension, then dispatch to the gfx950 kernels.
#include "common.h"
#include "sampler_internal.h"

#include <string>

namespace nmi {
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

// [n, B] (B = 1 is the reference's vector [n]).
void require_matrix(const nmi_tensor* t, int32_t dtype, int32_t n, int32_t B, const std::string& op,
                    const char* name) {
    require_dtype(t, dtype, op, name);
    require(n > 0 && t->ne[0] == n && t->ne[1] == B && t->ne[2] == 1 && t->ne[3] == 1, op,
            std::string("invalid vector shape for ") + name);
}

void require_scalars(const nmi_tensor* t, int32_t dtype, int32_t B, const std::string& op,
                     const char* name) {
    require_dtype(t, dtype, op, name);
    require(t->ne[0] == B && t->ne[1] == 1 && t->ne[2] == 1 && t->ne[3] == 1, op,
            std::string("invalid scalar shape for ") + name);
}

void require_workspace(void* ws, size_t bytes, size_t need, const std::string& op) {
    require(bytes >= need, op, "workspace is smaller than the size query");
    require(ws != nullptr || need == 0, op, "workspace must be non-null");
    require((reinterpret_cast<uintptr_t>(ws) & 255u) == 0, op, "workspace must be 256-byte aligned");
}

} // namespace

// Shapes shared by every chain acceptance (src/ops/wrapper/speculative_round.cpp:67-102): drafts
// [K, B], length/token/num_sampled/accepted [B], sampled_out [K+1, B], stats [>=4+K, B], a non-null
// device config; fills the state and output pointers of the kernel arguments.
SpecArgs check_accept_state(const nmi_tensor* drafts, nmi_tensor* length, nmi_tensor* token,
                            nmi_tensor* sampled_out, nmi_tensor* num_sampled, nmi_tensor* accepted,
                            nmi_tensor* stats, const nmi_sampling_config* config, const std::string& op,
                            int32_t& B) {
    require(drafts != nullptr, op, "drafts must be non-null");
    const int32_t K = drafts->ne[0];
    B = drafts->ne[1];
    require(K >= 1, op, "K must be >=1");
    require(K + 1 <= kMaxColumns, op, "K must be <= 15");
    require(B >= 1, op, "batch must be >=1");
    require_matrix(drafts, NMI_I32, K, B, op, "drafts");
    require_scalars(length, NMI_I32, B, op, "length");
    require_scalars(token, NMI_I32, B, op, "token");
    require_matrix(sampled_out, NMI_I32, K + 1, B, op, "sampled_out");
    require_scalars(num_sampled, NMI_I32, B, op, "num_sampled");
    require_scalars(accepted, NMI_I32, B, op, "accepted");
    require_dtype(stats, NMI_I64, op, "stats");
    require(stats->ne[0] >= 4 + K && stats->ne[1] == B && stats->ne[2] == 1 && stats->ne[3] == 1, op,
            "invalid vector shape for stats");
    require(config != nullptr, op, "config must be non-null");
    SpecArgs a{};
    a.drafts = static_cast<const int32_t*>(drafts->data);
    a.length = static_cast<int32_t*>(length->data);
    a.token = static_cast<int32_t*>(token->data);
    a.sampled_out = static_cast<int32_t*>(sampled_out->data);
    a.num_sampled = static_cast<int32_t*>(num_sampled->data);
    a.accepted = static_cast<int32_t*>(accepted->data);
    a.stats = static_cast<int64_t*>(stats->data);
    a.config = config;
    a.K = K;
    a.columns = K + 1;
    a.stats_stride = stats->ne[0];
    return a;
}

} // namespace nmi

using namespace nmi;

extern "C" {

// reference argmax wrapper (src/ops/wrapper/argmax.cpp:35-60); extension: logits [rows, C, B].
int nmi_argmax(const nmi_tensor* logits, nmi_tensor* out, int32_t valid_rows, nmi_stream_t stream) {
    const std::string op = "argmax";
    return guarded([&] {
        require(logits != nullptr && out != nullptr, op, "tensors must be non-null");
        require(logits->dtype == NMI_BF16, op, "logits must be BF16");
        require(out->dtype == NMI_I32, op, "out must be I32");
        require(logits->ne[0] > 0, op, "physical rows must be positive");
        require(logits->ne[3] == 1, op, "logits must be [vocab, T] or [vocab, T, B]");
        require(valid_rows > 0 && valid_rows <= logits->ne[0], op, "valid_rows must be in [1, logits.ne[0]]");
        require(out->ne[0] == logits->ne[1] && out->ne[1] == logits->ne[2] && out->ne[2] == 1 && out->ne[3] == 1,
                op, "out shape must be [logits.ne[1]]");
        require(is_contiguous(*logits) && is_contiguous(*out), op, "tensors must be contiguous");
        require(logits->data != nullptr && out->data != nullptr, op, "data must be non-null");
        launch_argmax(static_cast<const uint16_t*>(logits->data), static_cast<int32_t*>(out->data),
                      logits->ne[0], valid_rows, logits->ne[1] * logits->ne[2],
                      reinterpret_cast<hipStream_t>(stream));
    });
}

size_t nmi_sampling_workspace_bytes(int32_t token_domain, int32_t columns, int32_t batch) {
    if (token_domain <= 0 || columns <= 0 || batch <= 0) { return 0; }
    return plan_spec(token_domain, columns, batch).bytes;
}

int nmi_speculative_prepare_verify_inputs(const nmi_tensor* token, const nmi_tensor* drafts,
                                          const nmi_tensor* length, nmi_tensor* verify_ids,
                                          nmi_tensor* positions, nmi_stream_t stream) {
    const std::string op = "speculative_prepare_verify_inputs";
    return guarded([&] {
        require(drafts != nullptr, op, "drafts must be non-null");
        const int32_t K = drafts->ne[0];
        const int32_t B = drafts->ne[1];
        require(K >= 1, op, "K must be >=1");
        require(B >= 1, op, "batch must be >=1");
        require_scalars(token, NMI_I32, B, op, "token");
        require_matrix(drafts, NMI_I32, K, B, op, "drafts");
        require_scalars(length, NMI_I32, B, op, "length");
        require_matrix(verify_ids, NMI_I32, K + 1, B, op, "verify_ids");
        require_matrix(positions, NMI_I32, K + 1, B, op, "positions");
        launch_prepare_verify_inputs(static_cast<const int32_t*>(token->data),
                                     static_cast<const int32_t*>(drafts->data),
                                     static_cast<const int32_t*>(length->data),
                                     static_cast<int32_t*>(verify_ids->data),
                                     static_cast<int32_t*>(positions->data), K, B,
                                     reinterpret_cast<hipStream_t>(stream));
    });
}

// reference speculative_accept_greedy_drafts wrapper (src/ops/wrapper/speculative_round.cpp:67-102).
int nmi_speculative_accept_greedy_drafts(const nmi_tensor* target_tokens, const nmi_tensor* logits,
                                         const nmi_tensor* drafts, nmi_tensor* length,
                                         nmi_tensor* token, nmi_tensor* sampled_out,
                                         nmi_tensor* num_sampled, nmi_tensor* accepted,
                                         nmi_tensor* stats, int32_t token_domain,
                                         const nmi_sampling_config* config, void* workspace,
                                         size_t workspace_bytes, nmi_stream_t stream) {
    const std::string op = "speculative_accept_greedy_drafts";
    return guarded([&] {
        int32_t B = 0;
        SpecArgs a = check_accept_state(drafts, length, token, sampled_out, num_sampled, accepted, stats, config, op, B);
        const int32_t K = a.K;
        require_matrix(target_tokens, NMI_I32, K + 1, B, op, "target_tokens");
        require_dtype(logits, NMI_BF16, op, "logits");
        require(logits->ne[0] > 0 && logits->ne[1] >= K + 1 && logits->ne[2] == B && logits->ne[3] == 1, op,
                "logits must be [physical_rows, >=k+1]");
        require(token_domain > 0 && token_domain <= logits->ne[0], op, "token_domain must be in [1, logits.ne[0]]");
        const SpecPlan plan = plan_spec(token_domain, K + 1, B);
        require(plan.ntiles <= kMergeMaxTiles, op, "token_domain exceeds the candidate merge capacity (524288)");
        require_workspace(workspace, workspace_bytes, plan.bytes, op);
        char* ws = static_cast<char*>(workspace);
        a.target_tokens = static_cast<const int32_t*>(target_tokens->data);
        a.logits = static_cast<const uint16_t*>(logits->data);
        a.partial = reinterpret_cast<uint64_t*>(ws + plan.partial_offset);
        a.logits_seq_stride = static_cast<int64_t>(logits->ne[0]) * logits->ne[1];
        a.physical_rows = logits->ne[0];
        a.token_domain = token_domain;
        a.ntiles = plan.ntiles;
        launch_spec_accept(a, B, reinterpret_cast<hipStream_t>(stream));
    });
}

// reference speculative_select_accepted_hidden (src/ops/wrapper/speculative_round.cpp:104-118).
int nmi_speculative_select_accepted_hidden(const nmi_tensor* hidden, const nmi_tensor* accepted,
                                           nmi_tensor* out, nmi_stream_t stream) {
    const std::string op = "speculative_select_accepted_hidden";
    return guarded([&] {
        require_dtype(hidden, NMI_BF16, op, "hidden");
        require(hidden->ne[0] > 0 && hidden->ne[1] > 0 && hidden->ne[2] == 1 && hidden->ne[3] == 1, op,
                "invalid hidden shape");
        require_scalars(accepted, NMI_I32, 1, op, "accepted");
        require_dtype(out, NMI_BF16, op, "out");
        require(out->ne[0] == hidden->ne[0] && out->ne[1] == 1 && out->ne[2] == 1 && out->ne[3] == 1, op,
                "invalid output shape");
        launch_select_hidden(static_cast<const uint16_t*>(hidden->data),
                             static_cast<const int32_t*>(accepted->data),
                             static_cast<uint16_t*>(out->data), hidden->ne[0], hidden->ne[1],
                             reinterpret_cast<hipStream_t>(stream));
    });
}

// reference mtp_prepare_alignment_ids (src/ops/wrapper/mtp_round.cpp:36-48).
int nmi_mtp_prepare_alignment_ids(const nmi_tensor* verify_ids, const nmi_tensor* token,
                                  const nmi_tensor* accepted, nmi_tensor* alignment_ids, nmi_stream_t stream) {
    const std::string op = "mtp_prepare_alignment_ids";
    return guarded([&] {
        require(verify_ids != nullptr, op, "verify_ids must be non-null");
        const int32_t T = verify_ids->ne[0];
        require(T >= 2 && T <= 6, op, "T must be in [2,6]");
        require_scalars(verify_ids, NMI_I32, T, op, "verify_ids");
        require_scalars(token, NMI_I32, 1, op, "token");
        require_scalars(accepted, NMI_I32, 1, op, "accepted");
        require_scalars(alignment_ids, NMI_I32, T, op, "alignment_ids");
        require(alignment_ids->data != verify_ids->data, op, "verify_ids and alignment_ids must be distinct");
        launch_mtp_alignment_ids(static_cast<const int32_t*>(verify_ids->data), static_cast<const int32_t*>(token->data),
                                 static_cast<const int32_t*>(accepted->data), static_cast<int32_t*>(alignment_ids->data), T,
                                 reinterpret_cast<hipStream_t>(stream));
    });
}

int nmi_tree_accept_greedy(const nmi_tensor* parents, const nmi_tensor* node_tokens,
                           const nmi_tensor* target_tokens, nmi_tensor* path, nmi_tensor* path_len,
                           nmi_tensor* length, nmi_tensor* token, nmi_tensor* sampled_out,
                           nmi_tensor* num_sampled, nmi_tensor* accepted, nmi_tensor* stats,
                           nmi_stream_t stream) {
    const std::string op = "tree_accept_greedy";
    return guarded([&] {
        require(parents != nullptr, op, "parents must be non-null");
        const int32_t N = parents->ne[0];
        const int32_t B = parents->ne[1];
        require(N >= 1 && N <= kMaxTreeNodes, op, "tree must have 1..32 nodes");
        require(B >= 1, op, "batch must be >=1");
        require_matrix(parents, NMI_I32, N, B, op, "parents");
        require_matrix(node_tokens, NMI_I32, N, B, op, "node_tokens");
        require_matrix(target_tokens, NMI_I32, N, B, op, "target_tokens");
        require_matrix(path, NMI_I32, N, B, op, "path");
        require_scalars(path_len, NMI_I32, B, op, "path_len");
        require_scalars(length, NMI_I32, B, op, "length");
        require_scalars(token, NMI_I32, B, op, "token");
        require_matrix(sampled_out, NMI_I32, N, B, op, "sampled_out");
        require_scalars(num_sampled, NMI_I32, B, op, "num_sampled");
        require_scalars(accepted, NMI_I32, B, op, "accepted");
        require_dtype(stats, NMI_I64, op, "stats");
        require(stats->ne[0] >= 4 && stats->ne[1] == B && stats->ne[2] == 1 && stats->ne[3] == 1, op,
                "invalid vector shape for stats");
        launch_tree_accept(static_cast<const int32_t*>(parents->data),
                           static_cast<const int32_t*>(node_tokens->data),
                           static_cast<const int32_t*>(target_tokens->data), N, B,
                           static_cast<int32_t*>(path->data), static_cast<int32_t*>(path_len->data),
                           static_cast<int32_t*>(length->data), static_cast<int32_t*>(token->data),
                           static_cast<int32_t*>(sampled_out->data),
                           static_cast<int32_t*>(num_sampled->data),
                           static_cast<int32_t*>(accepted->data), static_cast<int64_t*>(stats->data),
                           stats->ne[0], reinterpret_cast<hipStream_t>(stream));
    });
}

} // extern "C"
