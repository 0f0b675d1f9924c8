// Shared host/device definitions of the ninfer_amd library (gfx950 only).
#pragma once

#include "ninfer_amd.h"

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>

#if defined(__HIP_DEVICE_COMPILE__) && !defined(__gfx950__)
#error "ninfer_amd kernels are written for gfx950 (MI355X) only"
#endif

namespace nmi {

inline constexpr int kQuantGroup = 64;
inline constexpr int kWave = 64;

// ---- host-side errors (converted to nmi_status at the C boundary) ------------------------------
struct InvalidArgument : std::invalid_argument {
    using std::invalid_argument::invalid_argument;
};
struct Overflow : std::overflow_error {
    using std::overflow_error::overflow_error;
};
struct Unsupported : std::runtime_error {
    using std::runtime_error::runtime_error;
};
struct HipError : std::runtime_error {
    using std::runtime_error::runtime_error;
};

void set_last_error(const std::string& msg);

#define NMI_HIP_CHECK(expr)                                                                       \
    do {                                                                                          \
        const hipError_t nmi_err_ = (expr);                                                       \
        if (nmi_err_ != hipSuccess) {                                                             \
            throw ::nmi::HipError(std::string(#expr) + ": " + hipGetErrorString(nmi_err_));      \
        }                                                                                         \
    } while (0)

// Launch check: a kernel launch failure surfaces as the last error.
inline void check_launch(const char* what) {
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) { throw HipError(std::string(what) + ": " + hipGetErrorString(err)); }
}

template <typename F>
int guarded(F&& f) {
    try {
        f();
        return NMI_OK;
    } catch (const InvalidArgument& e) {
        set_last_error(e.what());
        return NMI_INVALID_ARGUMENT;
    } catch (const Overflow& e) {
        set_last_error(e.what());
        return NMI_OVERFLOW;
    } catch (const Unsupported& e) {
        set_last_error(e.what());
        return NMI_UNSUPPORTED;
    } catch (const HipError& e) {
        set_last_error(e.what());
        return NMI_HIP_ERROR;
    } catch (const std::exception& e) {
        set_last_error(e.what());
        return NMI_INVALID_ARGUMENT;
    }
}

// ---- tensor helpers (src/core/tensor.cpp semantics) --------------------------------------------
inline size_t dtype_size(int32_t dt) {
    switch (dt) {
    case NMI_BF16:
    case NMI_FP16: return 2;
    case NMI_FP32:
    case NMI_I32: return 4;
    case NMI_I8:
    case NMI_U8: return 1;
    case NMI_I64: return 8;
    default: throw InvalidArgument("unknown dtype");
    }
}

inline bool is_contiguous(const nmi_tensor& t) {
    int64_t expect = static_cast<int64_t>(dtype_size(t.dtype));
    for (int i = 0; i < 4; ++i) {
        if (t.ne[i] <= 0) { return false; }
        if (t.ne[i] > 1 && t.nb[i] != expect) { return false; }
        expect *= t.ne[i];
    }
    return true;
}

inline int64_t numel(const nmi_tensor& t) {
    return static_cast<int64_t>(t.ne[0]) * t.ne[1] * t.ne[2] * t.ne[3];
}

} // namespace nmi
