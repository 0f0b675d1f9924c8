// Device helpers shared by the gfx950 kernels: bit conversions, wave reductions, vector types.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace nmi {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef int i4 __attribute__((ext_vector_type(4)));
typedef int i2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
    return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// Round-to-nearest-even FP32 -> BF16 bits (NaN stays NaN).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float x) {
    uint32_t b = __float_as_uint(x);
    if ((b & 0x7fffffffu) > 0x7f800000u) { return static_cast<uint16_t>((b >> 16) | 0x40u); }
    b += 0x7fffu + ((b >> 16) & 1u);
    return static_cast<uint16_t>(b >> 16);
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float x) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(x));
}

// Wave-wide reductions by DPP: shifts by 1, 2, 4, 8 inside each 16-lane row, then lane 15 of rows
// 0 and 2 into rows 1 and 3 (row_bcast:15) and lane 31 into rows 2 and 3 (row_bcast:31), so lane 63
// ends with the whole wave's result, which every lane then reads. A lane whose DPP source is
// outside its row (or masked off) combines with `identity`. No LDS round trip, unlike ds_bpermute
// shuffles.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_from(float v, float identity) {
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(identity), __float_as_int(v), CTRL, ROW_MASK, 0xf, false));
}

__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_from<0x111, 0xf>(v, -INFINITY));
    v = fmaxf(v, dpp_from<0x112, 0xf>(v, -INFINITY));
    v = fmaxf(v, dpp_from<0x114, 0xf>(v, -INFINITY));
    v = fmaxf(v, dpp_from<0x118, 0xf>(v, -INFINITY));
    v = fmaxf(v, dpp_from<0x142, 0xa>(v, -INFINITY));
    v = fmaxf(v, dpp_from<0x143, 0xc>(v, -INFINITY));
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// The lanes' values summed in one fixed order (the same bits on every run).
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_from<0x111, 0xf>(v, 0.0f);
    v += dpp_from<0x112, 0xf>(v, 0.0f);
    v += dpp_from<0x114, 0xf>(v, 0.0f);
    v += dpp_from<0x118, 0xf>(v, 0.0f);
    v += dpp_from<0x142, 0xa>(v, 0.0f);
    v += dpp_from<0x143, 0xc>(v, 0.0f);
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// One step of a wave-wide inclusive scan of an integer: add the value that DPP control CTRL
// brings from another lane (zero where that lane lies outside the row or is masked off), word by
// word with carries.
template <int CTRL, int ROW_MASK, typename T>
__device__ __forceinline__ T dpp_scan_step(T v) {
    constexpr int kWords = sizeof(T) / 4;
    uint32_t w[kWords];
    __builtin_memcpy(w, &v, sizeof(T));
#pragma unroll
    for (int i = 0; i < kWords; ++i) {
        w[i] = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(w[i]), CTRL, ROW_MASK, 0xf, true));
    }
    T o;
    __builtin_memcpy(&o, w, sizeof(T));
    return v + o;
}

// Inclusive scan over the 64 lanes of a wave: shifts by 1, 2, 4, 8 inside each 16-lane row, then
// lane 15 of rows 0 and 2 into rows 1 and 3 (row_bcast:15), then lane 31 into rows 2 and 3
// (row_bcast:31).
template <typename T>
__device__ __forceinline__ T wave_inclusive_scan(T v) {
    v = dpp_scan_step<0x111, 0xf>(v);
    v = dpp_scan_step<0x112, 0xf>(v);
    v = dpp_scan_step<0x114, 0xf>(v);
    v = dpp_scan_step<0x118, 0xf>(v);
    v = dpp_scan_step<0x142, 0xa>(v);
    v = dpp_scan_step<0x143, 0xc>(v);
    return v;
}

// Reduction across the four 16-lane groups that share one MFMA column (lanes c, c+16, c+32, c+48).
// v_permlane32_swap / v_permlane16_swap exchange half-waves and odd/even 16-lane rows in the VALU,
// so each step is a register swap plus one op (no LDS round trip as with ds_bpermute). Both lanes
// of a pair add in the same order, so every lane ends with the same bits.
__device__ __forceinline__ float group4_max(float v) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
    r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ float group4_sum(float v) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Two signed INT8 codes -> one packed FP16 pair, exactly: byte BYTE of `lo` -> low half, byte BYTE
// of `hi` -> high half. One SDWA convert per code reads the byte in place (no shifts, no packing).
template <int BYTE>
__device__ __forceinline__ uint32_t i8x2_to_f16x2(uint32_t lo, uint32_t hi) {
    uint32_t r;
    asm("v_cvt_f16_i16_sdwa %0, sext(%1) dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:BYTE_%2"
        : "=v"(r)
        : "v"(lo), "n"(BYTE));
    asm("v_cvt_f16_i16_sdwa %0, sext(%1) dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_%2"
        : "+v"(r)
        : "v"(hi), "n"(BYTE));
    return r;
}

// Bytes (B0, B1) of one dword -> packed FP16 pair.
template <int B0, int B1>
__device__ __forceinline__ uint32_t i8_bytes_to_f16x2(uint32_t x) {
    uint32_t r;
    asm("v_cvt_f16_i16_sdwa %0, sext(%1) dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:BYTE_%2"
        : "=v"(r)
        : "v"(x), "n"(B0));
    asm("v_cvt_f16_i16_sdwa %0, sext(%1) dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_%2"
        : "+v"(r)
        : "v"(x), "n"(B1));
    return r;
}

} // namespace nmi
