// LDS-DMA helpers shared by the streaming kernels (gfx950): raw buffer resources and the
// buffer_load ... lds forms. Plain (non-template) functions: the host compile pass rejects the DMA
// builtin inside function templates.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#define NMI_AS1 __attribute__((address_space(1)))
#define NMI_AS3 __attribute__((address_space(3)))

namespace nmi {

// Raw byte buffer of `bytes` (< 2^31): loads past the end read zero, offsets are 32-bit.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t raw_buffer(const void* base, int64_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes), 0x00020000);
}

// One LDS-DMA instruction: 16 bytes (or 4) per lane from rsrc + voffset + soffset into
// lds + 16 * lane (4 * lane); the LDS address is M0-based, so only the source is per lane.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t rsrc, NMI_AS3 char* lds, int voff, int soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (NMI_AS3 void*)lds, 16, voff, soff, 0, 0);
}
__device__ __forceinline__ void dma4(__amdgpu_buffer_rsrc_t rsrc, NMI_AS3 char* lds, int voff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (NMI_AS3 void*)lds, 4, voff, 0, 0, 0);
}
__device__ __forceinline__ void dma4s(__amdgpu_buffer_rsrc_t rsrc, NMI_AS3 char* lds, int voff, int soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (NMI_AS3 void*)lds, 4, voff, soff, 0, 0);
}

// Non-temporal forms (cache policy nt, lines evicted first): for streams whose bytes one workgroup
// reads once per call. Measured on MI355X with the attention's K/V code DMAs: C3 120 -> 107 us and
// C2 15.0 -> 14.5 us per layer, the BF16-cache C3 192 -> 171 us, the batch-16 layer 135 -> 130 us;
// the [248320, 5120] lm_head 191 -> 187 us. They cost where other workgroups re-read the lines
// through L2 (row-chunked tree attention: 304 -> 339 us), so attention uses them only with one row
// chunk, and only for the code planes (the small scale DMAs measured faster with the default).
__device__ __forceinline__ void dma16_nt(__amdgpu_buffer_rsrc_t rsrc, NMI_AS3 char* lds, int voff, int soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (NMI_AS3 void*)lds, 16, voff, soff, 0, 2);
}
__device__ __forceinline__ void dma4s_nt(__amdgpu_buffer_rsrc_t rsrc, NMI_AS3 char* lds, int voff, int soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (NMI_AS3 void*)lds, 4, voff, soff, 0, 2);
}

} // namespace nmi
