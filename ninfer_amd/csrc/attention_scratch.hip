// Static scratch of the allocation-free verify attention (nmi_gqa_attention_noalloc): the split-K
// partials live in a fixed device array instead of a caller workspace, for callers that cannot
// allocate (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
//
// Each GPU the library runs on holds its own copy of the array until the process ends. Host code
// never passes the array's name to a kernel (on the host it is only a registration handle): the
// device address is resolved once per device with hipGetSymbolAddress, with that device current,
// and kept per device. Every call on one GPU shares that GPU's array and nothing in it needs to
// start at zero (the partial kernel writes every slot the merge reads, and the batch plan's
// sequence table is rewritten by each call), so calls may follow each other freely; calls that
// overlap on one GPU (two streams at once) race on the array.
#include "common.h"
#include "ops_internal.h"

#include <mutex>

static __device__ __align__(256) unsigned char scratch[nmi::kStaticScratchBytes];

namespace nmi {
namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

} // namespace

void* static_scratch(size_t need, const std::string& op) {
    if (need > kStaticScratchBytes) {
        throw Unsupported(op + ": needs " + std::to_string(need) + " bytes of split scratch, more than the " +
                          std::to_string(kStaticScratchBytes) +
                          "-byte static scratch; use the workspace form (nmi_gqa_attention)");
    }
    int dev = 0;
    NMI_HIP_CHECK(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) { throw Unsupported(op + ": device ordinal beyond the static scratch table"); }
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch_ptr[dev] == nullptr) {
        void* p = nullptr;
        NMI_HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        if (p == nullptr || (reinterpret_cast<uintptr_t>(p) & 255u) != 0) {
            throw HipError(op + ": static scratch address is null or misaligned");
        }
        g_scratch_ptr[dev] = p;
    }
    return g_scratch_ptr[dev];
}

} // namespace nmi
