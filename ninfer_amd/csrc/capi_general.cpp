// C ABI of the general speculative acceptance ("Mode F"; no reference counterpart).
#include "common.h"

using namespace nmi;

extern "C" {

size_t nmi_general_accept_workspace_bytes(int32_t token_domain, int32_t K, int32_t batch) {
    (void)token_domain;
    (void)K;
    (void)batch;
    return 0;
}

int nmi_speculative_accept_general(const nmi_tensor*, const nmi_tensor*, const nmi_tensor*,
                                   const nmi_tensor*, const nmi_tensor*, nmi_tensor*, nmi_tensor*,
                                   nmi_tensor*, nmi_tensor*, nmi_tensor*, nmi_tensor*, int32_t,
                                   const nmi_general_config*, void*, size_t, nmi_stream_t) {
    set_last_error("speculative_accept_general: not built yet");
    return NMI_UNSUPPORTED;
}

} // extern "C"
