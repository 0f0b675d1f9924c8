// Bandwidth controls for the benchmark: what one launch that only moves a payload achieves, timed
// beside the ops that move the same bytes.
//  - stream copy: 16-byte loads and stores over a grid of at most 4096 blocks of 256 threads, the
//    reference bench's copy ceiling (bench/ops/gqa_attention_bench.cu:1103-1130, C_copy = 2 x
//    payload / time);
//  - vector read: non-temporal 16-byte loads, eight in flight per thread, folded into a checksum;
//  - LDS-DMA read: the streaming pattern of the attention and linear kernels without their
//    arithmetic: every wave keeps a ring of four 4 KiB stages in flight (buffer_load ... lds).
#include "ninfer_amd_runtime.h"

#include "common.h"
#include "lds_dma.h"

#include <algorithm>

namespace nmi {
namespace {

typedef int i4 __attribute__((ext_vector_type(4)));

constexpr int kCopyThreads = 256;
constexpr int kCopyMaxBlocks = 4096;

__global__ __launch_bounds__(kCopyThreads) void stream_copy_kernel(const i4* __restrict__ src, i4* __restrict__ dst,
                                                                   size_t words) {
    const size_t stride = static_cast<size_t>(gridDim.x) * kCopyThreads;
    for (size_t i = static_cast<size_t>(blockIdx.x) * kCopyThreads + threadIdx.x; i < words; i += stride) {
        dst[i] = src[i];
    }
}

// The checksum is stored only when it equals a value the payload does not produce in practice, so
// the loads stay live without a store per thread.
constexpr uint32_t kSinkMagic = 0x9E3779B9u;

__global__ __launch_bounds__(kCopyThreads) void read_vec_kernel(const i4* __restrict__ src, size_t words,
                                                                uint32_t* sink) {
    constexpr int kUnroll = 8;
    const size_t stride = static_cast<size_t>(gridDim.x) * kCopyThreads;
    size_t i = static_cast<size_t>(blockIdx.x) * kCopyThreads + threadIdx.x;
    i4 acc = {0, 0, 0, 0};
    for (; i + (kUnroll - 1) * stride < words; i += kUnroll * stride) {
        i4 v[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) { v[u] = __builtin_nontemporal_load(src + i + u * stride); }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) { acc ^= v[u]; }
    }
    for (; i < words; i += stride) { acc ^= __builtin_nontemporal_load(src + i); }
    const uint32_t x = static_cast<uint32_t>(acc[0] ^ acc[1] ^ acc[2] ^ acc[3]);
    if (x == kSinkMagic) { sink[0] = x; }
}

constexpr int kDmaWaves = 8;
constexpr int kDmaStages = 4;
constexpr int kDmaChunk = 4096; // bytes of one stage: four 1 KiB DMAs of 64 lanes x 16 B
constexpr int kDmaPerChunk = kDmaChunk / 1024;

// vmcnt(n) with expcnt and lgkmcnt left at their maxima (gfx9 encoding: vmcnt bits 3:0 and 15:14).
constexpr int wait_vm(int n) { return (n & 0xf) | ((n >> 4) << 14) | (0x7 << 4) | (0xf << 8); }
constexpr int kWaitLgkm0 = 0xc07f;

__global__ __launch_bounds__(64 * kDmaWaves) void read_dma_kernel(const char* src, size_t bytes, uint32_t* sink) {
    __shared__ __attribute__((aligned(16))) char smem[kDmaWaves * kDmaStages * kDmaChunk];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    NMI_AS3 char* ring = (NMI_AS3 char*)smem + wave * (kDmaStages * kDmaChunk);
    const size_t chunks = (bytes + kDmaChunk - 1) / kDmaChunk;
    const size_t waves = static_cast<size_t>(gridDim.x) * kDmaWaves;
    const size_t first = static_cast<size_t>(blockIdx.x) * kDmaWaves + wave; // wave-uniform
    const int64_t items = first < chunks ? static_cast<int64_t>((chunks - first + waves - 1) / waves) : 0;
    // Each chunk gets a buffer resource of its own (a 64-bit base, at most 4 KiB of records), so the
    // payload may exceed the 32-bit offsets and the last chunk's loads past the end read zero.
    const auto issue = [&](NMI_AS3 char* stage, int64_t j) {
        const size_t chunk = first + static_cast<size_t>(j) * waves;
        const size_t off = chunk * kDmaChunk;
        const int64_t left = static_cast<int64_t>(bytes - off);
        const __amdgpu_buffer_rsrc_t r = raw_buffer(src + off, left < kDmaChunk ? left : kDmaChunk);
#pragma unroll
        for (int q = 0; q < kDmaPerChunk; ++q) { dma16_nt(r, stage + q * 1024, q * 1024 + 16 * lane, 0); }
    };
#pragma unroll
    for (int s = 0; s < kDmaStages - 1; ++s) {
        if (s < items) { issue(ring + s * kDmaChunk, s); }
    }
    uint32_t acc = 0;
    for (int64_t j = 0; j < items; ++j) {
        if (j + kDmaStages - 1 < items) {
            issue(ring + ((j + kDmaStages - 1) % kDmaStages) * kDmaChunk, j + kDmaStages - 1);
            __builtin_amdgcn_s_waitcnt(wait_vm(kDmaPerChunk * (kDmaStages - 1)));
        } else {
            __builtin_amdgcn_s_waitcnt(wait_vm(0));
        }
        acc ^= *(const NMI_AS3 uint32_t*)(ring + (j % kDmaStages) * kDmaChunk + 4 * lane);
        __builtin_amdgcn_s_waitcnt(kWaitLgkm0); // the stage is read before its next DMA is issued
    }
    if (acc == kSinkMagic) { sink[0] = acc; }
}

void require(bool ok, const char* what) {
    if (!ok) { throw InvalidArgument(std::string("ceiling: ") + what); }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int device_cus() {
    int dev = 0;
    NMI_HIP_CHECK(hipGetDevice(&dev));
    int cus = 0;
    NMI_HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    return cus > 0 ? cus : 1;
}

} // namespace
} // namespace nmi

using nmi::guarded;

extern "C" {

int nmi_rt_stream_copy(void* dst, const void* src, size_t bytes, nmi_stream_t stream) {
    return guarded([&] {
        nmi::require(dst != nullptr && src != nullptr && bytes > 0, "dst, src and bytes must be non-zero");
        nmi::require(bytes % 16 == 0 && nmi::aligned16(dst) && nmi::aligned16(src),
                     "bytes must be a multiple of 16 and both pointers 16-byte aligned");
        const size_t words = bytes / 16;
        const size_t blocks = std::min<size_t>(nmi::kCopyMaxBlocks, (words + nmi::kCopyThreads - 1) / nmi::kCopyThreads);
        hipLaunchKernelGGL(nmi::stream_copy_kernel, dim3(static_cast<unsigned>(blocks)), dim3(nmi::kCopyThreads), 0,
                           reinterpret_cast<hipStream_t>(stream), static_cast<const nmi::i4*>(src),
                           static_cast<nmi::i4*>(dst), words);
        nmi::check_launch("stream_copy_kernel");
    });
}

int nmi_rt_read_ceiling(const void* src, size_t bytes, int32_t form, void* sink, nmi_stream_t stream) {
    return guarded([&] {
        nmi::require(src != nullptr && sink != nullptr && bytes > 0, "src, sink and bytes must be non-zero");
        nmi::require(bytes % 16 == 0 && nmi::aligned16(src), "bytes must be a multiple of 16 and src 16-byte aligned");
        const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
        if (form == NMI_READ_VECTOR) {
            const size_t words = bytes / 16;
            // eight 16-byte loads in flight per thread: 32 KiB per block and pass of the loop
            const size_t blocks = std::min<size_t>(8 * static_cast<size_t>(nmi::device_cus()),
                                                   std::max<size_t>(1, words / (8 * nmi::kCopyThreads)));
            hipLaunchKernelGGL(nmi::read_vec_kernel, dim3(static_cast<unsigned>(blocks)), dim3(nmi::kCopyThreads), 0,
                               s, static_cast<const nmi::i4*>(src), words, static_cast<uint32_t*>(sink));
            nmi::check_launch("read_vec_kernel");
        } else if (form == NMI_READ_LDS_DMA) {
            const size_t chunks = (bytes + nmi::kDmaChunk - 1) / nmi::kDmaChunk;
            const size_t blocks = std::min<size_t>(static_cast<size_t>(nmi::device_cus()),
                                                   (chunks + nmi::kDmaWaves - 1) / nmi::kDmaWaves);
            hipLaunchKernelGGL(nmi::read_dma_kernel, dim3(static_cast<unsigned>(blocks)), dim3(64 * nmi::kDmaWaves), 0,
                               s, static_cast<const char*>(src), bytes, static_cast<uint32_t*>(sink));
            nmi::check_launch("read_dma_kernel");
        } else {
            throw nmi::InvalidArgument("ceiling: form must be NMI_READ_VECTOR or NMI_READ_LDS_DMA");
        }
    });
}

} // extern "C"
