// Launch interface of the recurrent-state kernels (gdn_snapshot.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace nmi {

struct GdnArgs {
    const uint16_t* q;     // BF16 [S, Hqk, T]
    const uint16_t* k;     // BF16 [S, Hqk, T]
    const uint16_t* v;     // BF16 [S, Hv, T]
    const float* g;        // FP32 [Hv, T]
    const float* beta;     // FP32 [Hv, T]
    const float* state_in; // FP32 [S, S, Hv] (distinct-state form)
    float* state_out;      // FP32 [S, S, Hv] (may equal state_in)
    float* states;         // FP32 [S, S, Hv, slots] (snapshot form)
    const int32_t* initial_slot; // device I32 scalar; non-null selects the snapshot form
    uint16_t* out;         // BF16 [S, Hv, T]
    float scale;
    int32_t normalize_qk;
    int32_t T;
    int32_t Hqk;
    int32_t Hv;
    int32_t slots;
};

struct ConvArgs {
    const uint16_t* x;      // BF16 [C, T]
    const uint16_t* weight; // BF16 [C, 4]
    const uint16_t* state_in; // BF16 [C, 3]
    uint16_t* state_out;      // BF16 [C, 3] (may equal state_in)
    uint16_t* states;         // BF16 [C, 3, slots] (snapshot form)
    const int32_t* initial_slot;
    uint16_t* out;            // BF16 [C, T]
    int32_t C;
    int32_t T;
    int32_t slots;
};

void launch_gdn_recurrent(const GdnArgs& a, int32_t S, hipStream_t stream);
void launch_conv1d_silu(const ConvArgs& a, hipStream_t stream);
// op: 0 set (dst32 = value), 1 assign (dst32 = *src), 2 increment dst32, 3 increment dst64.
void launch_scalar_op(int32_t op, const int32_t* src, int32_t* dst32, long long* dst64, int32_t value,
                      hipStream_t stream);

} // namespace nmi
