// KV cache commit, rollback and tree-path compaction on gfx950.
//
// The reference never writes a rejected row's bytes when committing a device-selected prefix
// (include/ninfer/ops/kv_cache_append_prefix.h:22-32, BF16 kernel
// src/ops/kernel/kv_cache_append_prefix.cuh) and rolls back implicitly by moving the frontier
// (src/ops/kernel/speculative_round.cuh:150-158). This file adds the explicit forms the verify step
// needs for an INT8-G64 cache: zeroing rejected rows, and moving an accepted tree path's rows to
// contiguous slots. All copies move codes and FP16 scale bits unchanged.
#include "common.h"
#include "device_utils.h"
#include "ops_internal.h"

namespace nmi {
namespace {

// grid (T, B): block zeroes row positions[t, b] of every KV head when t >= keep_count[b].
__global__ __launch_bounds__(256) void kv_rollback_kernel(const int32_t* positions,
                                                          const int32_t* keep_count, int32_t T,
                                                          int32_t Hkv, int32_t D, int32_t P,
                                                          int8_t* kc, int8_t* vc, uint16_t* ks,
                                                          uint16_t* vs, int64_t code_seq,
                                                          int64_t scale_seq) {
    const int t = blockIdx.x;
    const int b = blockIdx.y;
    if (t < keep_count[b]) { return; }
    const int pos = positions[static_cast<int64_t>(b) * T + t];
    if (pos < 0 || pos >= P) { return; }
    const int G = D / 64;
    const int vec_per_row = D / 16;
    for (int i = threadIdx.x; i < Hkv * vec_per_row; i += blockDim.x) {
        const int h = i / vec_per_row;
        const int part = i - h * vec_per_row;
        const int64_t off = static_cast<int64_t>(b) * code_seq + static_cast<int64_t>(D) * (pos + static_cast<int64_t>(P) * h) + 16 * part;
        *reinterpret_cast<i4*>(kc + off) = i4{0, 0, 0, 0};
        *reinterpret_cast<i4*>(vc + off) = i4{0, 0, 0, 0};
    }
    for (int i = threadIdx.x; i < Hkv * G; i += blockDim.x) {
        const int h = i / G;
        const int grp = i - h * G;
        const int64_t off = static_cast<int64_t>(b) * scale_seq + static_cast<int64_t>(G) * (pos + static_cast<int64_t>(P) * h) + grp;
        ks[off] = 0;
        vs[off] = 0;
    }
}

// grid (B, Hkv): one block per (sequence, KV head); the heads are disjoint planes, so they move in
// parallel (one dependent round trip instead of one per head). Every source row of the head is
// staged in LDS before any destination is written, so overlapping moves (path[j] == j' for a later
// j') are safe.
__global__ __launch_bounds__(256) void kv_compact_path_kernel(const int32_t* base_position,
                                                              const int32_t* path,
                                                              const int32_t* path_len, int32_t T,
                                                              int32_t Hkv, int32_t D, int32_t P,
                                                              int8_t* kc, int8_t* vc, uint16_t* ks,
                                                              uint16_t* vs, int64_t code_seq,
                                                              int64_t scale_seq) {
    extern __shared__ int4 smem[];
    const int b = blockIdx.x;
    const int h = blockIdx.y;
    const int G = D / 64;
    const int vec_per_row = D / 16;
    // Codes K|V as 16-byte vectors, then scales as 16-bit words, then the source rows.
    i4* sk = reinterpret_cast<i4*>(smem);
    i4* sv = sk + T * vec_per_row;
    uint16_t* sks = reinterpret_cast<uint16_t*>(sv + T * vec_per_row);
    uint16_t* svs = sks + T * G;
    int32_t* srow = reinterpret_cast<int32_t*>(svs + T * G); // 4-byte aligned: T * (2D + 4G) bytes precede it
    // The path entries load together with the base position and length.
    const int32_t* pth = path + static_cast<int64_t>(b) * T;
    const int pj = static_cast<int>(threadIdx.x) < T ? pth[threadIdx.x] : 0;
    const int base = base_position[b];
    int len = path_len[b];
    len = len < 0 ? 0 : (len > T ? T : len);
    if (static_cast<int>(threadIdx.x) < T) { srow[threadIdx.x] = base + pj; }
    __syncthreads();
    const int64_t head_code = static_cast<int64_t>(b) * code_seq + static_cast<int64_t>(h) * P * D;
    const int64_t head_scale = static_cast<int64_t>(b) * scale_seq + static_cast<int64_t>(h) * P * G;
    for (int i = threadIdx.x; i < len * vec_per_row; i += blockDim.x) {
        const int j = i / vec_per_row;
        const int part = i - j * vec_per_row;
        const int src = srow[j];
        if (src < 0 || src >= P) { continue; }
        sk[i] = *reinterpret_cast<const i4*>(kc + head_code + static_cast<int64_t>(src) * D + 16 * part);
        sv[i] = *reinterpret_cast<const i4*>(vc + head_code + static_cast<int64_t>(src) * D + 16 * part);
    }
    for (int i = threadIdx.x; i < len * G; i += blockDim.x) {
        const int j = i / G;
        const int grp = i - j * G;
        const int src = srow[j];
        if (src < 0 || src >= P) { continue; }
        sks[i] = ks[head_scale + static_cast<int64_t>(src) * G + grp];
        svs[i] = vs[head_scale + static_cast<int64_t>(src) * G + grp];
    }
    __syncthreads();
    for (int i = threadIdx.x; i < len * vec_per_row; i += blockDim.x) {
        const int j = i / vec_per_row;
        const int part = i - j * vec_per_row;
        const int src = srow[j];
        const int dst = base + j;
        if (src == dst || src < 0 || src >= P || dst < 0 || dst >= P) { continue; }
        *reinterpret_cast<i4*>(kc + head_code + static_cast<int64_t>(dst) * D + 16 * part) = sk[i];
        *reinterpret_cast<i4*>(vc + head_code + static_cast<int64_t>(dst) * D + 16 * part) = sv[i];
    }
    for (int i = threadIdx.x; i < len * G; i += blockDim.x) {
        const int j = i / G;
        const int grp = i - j * G;
        const int src = srow[j];
        const int dst = base + j;
        if (src == dst || src < 0 || src >= P || dst < 0 || dst >= P) { continue; }
        ks[head_scale + static_cast<int64_t>(dst) * G + grp] = sks[i];
        vs[head_scale + static_cast<int64_t>(dst) * G + grp] = svs[i];
    }
}

} // namespace

void launch_kv_rollback(const int32_t* positions, const int32_t* keep_count, int32_t T,
                        const CacheRef& c, hipStream_t stream) {
    hipLaunchKernelGGL(kv_rollback_kernel, dim3(T, c.B), dim3(256), 0, stream, positions,
                       keep_count, T, c.Hkv, c.D, c.P, c.kc, c.vc, c.ks, c.vs, c.code_seq,
                       c.scale_seq);
    check_launch("kv_rollback_kernel");
}

void launch_kv_compact_path(const int32_t* base_position, const int32_t* path,
                            const int32_t* path_len, int32_t T, const CacheRef& c,
                            hipStream_t stream) {
    const int G = c.D / 64;
    const size_t lds = static_cast<size_t>(T) * (2 * c.D + 2 * G * 2 + sizeof(int32_t));
    hipLaunchKernelGGL(kv_compact_path_kernel, dim3(c.B, c.Hkv), dim3(256), lds, stream, base_position,
                       path, path_len, T, c.Hkv, c.D, c.P, c.kc, c.vc, c.ks, c.vs, c.code_seq,
                       c.scale_seq);
    check_launch("kv_compact_path_kernel");
}

} // namespace nmi
