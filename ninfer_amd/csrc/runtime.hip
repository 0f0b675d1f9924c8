// Runtime helpers for harnesses (include/ninfer_amd_runtime.h): device memory, streams, events and
// graph capture, so Python tests and the benchmark drive the C ABI without another GPU runtime.
#include "ninfer_amd_runtime.h"

#include "common.h"

#include <cstring>

namespace nmi {
namespace {

__global__ void fill_u8_kernel(uint8_t* dst, uint8_t value, size_t bytes) {
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < bytes; i += stride) {
        dst[i] = value;
    }
}

// Row (*counter mod rows) of a [rows, cols] table into dst, then *counter + 1. Every thread reads
// the counter before thread 0 advances it (the barrier orders the read before the write).
__global__ void next_row_i32_kernel(const int32_t* table, int32_t rows, int32_t cols, int32_t* counter,
                                    int32_t* dst) {
    const int32_t c = *counter;
    const int32_t r = ((c % rows) + rows) % rows;
    for (int i = threadIdx.x; i < cols; i += blockDim.x) { dst[i] = table[static_cast<int64_t>(r) * cols + i]; }
    __syncthreads();
    if (threadIdx.x == 0) { *counter = c + 1; }
}

} // namespace
} // namespace nmi

struct nmi_graph {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
};

using nmi::guarded;

extern "C" {

int nmi_rt_device_count(int32_t* count) {
    return guarded([&] {
        int n = 0;
        NMI_HIP_CHECK(hipGetDeviceCount(&n));
        *count = n;
    });
}

int nmi_rt_device_name(char* buf, size_t len) {
    return guarded([&] {
        hipDeviceProp_t prop;
        NMI_HIP_CHECK(hipGetDeviceProperties(&prop, 0));
        std::snprintf(buf, len, "%s|%s|cu=%d", prop.name, prop.gcnArchName, prop.multiProcessorCount);
    });
}

int nmi_rt_malloc(void** ptr, size_t bytes) {
    return guarded([&] { NMI_HIP_CHECK(hipMalloc(ptr, bytes)); });
}

int nmi_rt_free(void* ptr) {
    return guarded([&] { NMI_HIP_CHECK(hipFree(ptr)); });
}

int nmi_rt_memcpy_htod(void* dst, const void* src, size_t bytes) {
    return guarded([&] { NMI_HIP_CHECK(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice)); });
}

int nmi_rt_memcpy_dtoh(void* dst, const void* src, size_t bytes) {
    return guarded([&] { NMI_HIP_CHECK(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost)); });
}

int nmi_rt_memcpy_dtod(void* dst, const void* src, size_t bytes, nmi_stream_t stream) {
    return guarded([&] {
        NMI_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice,
                                     reinterpret_cast<hipStream_t>(stream)));
    });
}

int nmi_rt_fill_u8(void* dst, uint8_t value, size_t bytes, nmi_stream_t stream) {
    return guarded([&] {
        if (bytes == 0) { return; }
        size_t blocks = (bytes + 255) / 256;
        if (blocks > 4096) { blocks = 4096; }
        hipLaunchKernelGGL(nmi::fill_u8_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                           reinterpret_cast<hipStream_t>(stream), static_cast<uint8_t*>(dst), value, bytes);
        nmi::check_launch("fill_u8_kernel");
    });
}

int nmi_rt_next_row_i32(const int32_t* table, int32_t rows, int32_t cols, int32_t* counter, int32_t* dst,
                        nmi_stream_t stream) {
    return guarded([&] {
        if (table == nullptr || counter == nullptr || dst == nullptr || rows < 1 || cols < 1 || cols > 1024) {
            throw nmi::InvalidArgument("next_row_i32: table, counter and dst must be non-null, rows >= 1, cols in [1, 1024]");
        }
        hipLaunchKernelGGL(nmi::next_row_i32_kernel, dim3(1), dim3(64), 0, reinterpret_cast<hipStream_t>(stream),
                           table, rows, cols, counter, dst);
        nmi::check_launch("next_row_i32_kernel");
    });
}

int nmi_rt_stream_create(nmi_stream_t* stream) {
    return guarded([&] {
        hipStream_t s;
        NMI_HIP_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
        *stream = reinterpret_cast<nmi_stream_t>(s);
    });
}

int nmi_rt_stream_destroy(nmi_stream_t stream) {
    return guarded([&] { NMI_HIP_CHECK(hipStreamDestroy(reinterpret_cast<hipStream_t>(stream))); });
}

int nmi_rt_stream_synchronize(nmi_stream_t stream) {
    return guarded([&] { NMI_HIP_CHECK(hipStreamSynchronize(reinterpret_cast<hipStream_t>(stream))); });
}

int nmi_rt_device_synchronize(void) {
    return guarded([&] { NMI_HIP_CHECK(hipDeviceSynchronize()); });
}

int nmi_rt_event_create(nmi_event_t* event) {
    return guarded([&] {
        hipEvent_t e;
        NMI_HIP_CHECK(hipEventCreate(&e));
        *event = reinterpret_cast<nmi_event_t>(e);
    });
}

int nmi_rt_event_destroy(nmi_event_t event) {
    return guarded([&] { NMI_HIP_CHECK(hipEventDestroy(reinterpret_cast<hipEvent_t>(event))); });
}

int nmi_rt_event_record(nmi_event_t event, nmi_stream_t stream) {
    return guarded([&] {
        NMI_HIP_CHECK(hipEventRecord(reinterpret_cast<hipEvent_t>(event), reinterpret_cast<hipStream_t>(stream)));
    });
}

int nmi_rt_event_elapsed_ms(float* ms, nmi_event_t start, nmi_event_t stop) {
    return guarded([&] {
        NMI_HIP_CHECK(hipEventSynchronize(reinterpret_cast<hipEvent_t>(stop)));
        NMI_HIP_CHECK(hipEventElapsedTime(ms, reinterpret_cast<hipEvent_t>(start), reinterpret_cast<hipEvent_t>(stop)));
    });
}

int nmi_rt_capture_begin(nmi_stream_t stream) {
    return guarded([&] {
        NMI_HIP_CHECK(hipStreamBeginCapture(reinterpret_cast<hipStream_t>(stream), hipStreamCaptureModeThreadLocal));
    });
}

int nmi_rt_capture_end(nmi_stream_t stream, nmi_graph_t* graph) {
    return guarded([&] {
        auto* g = new nmi_graph();
        const hipError_t e1 = hipStreamEndCapture(reinterpret_cast<hipStream_t>(stream), &g->graph);
        if (e1 != hipSuccess) {
            delete g;
            throw nmi::HipError(std::string("hipStreamEndCapture: ") + hipGetErrorString(e1));
        }
        const hipError_t e2 = hipGraphInstantiate(&g->exec, g->graph, nullptr, nullptr, 0);
        if (e2 != hipSuccess) {
            (void)hipGraphDestroy(g->graph);
            delete g;
            throw nmi::HipError(std::string("hipGraphInstantiate: ") + hipGetErrorString(e2));
        }
        *graph = g;
    });
}

int nmi_rt_graph_launch(nmi_graph_t graph, nmi_stream_t stream) {
    return guarded([&] { NMI_HIP_CHECK(hipGraphLaunch(graph->exec, reinterpret_cast<hipStream_t>(stream))); });
}

int nmi_rt_graph_destroy(nmi_graph_t graph) {
    return guarded([&] {
        if (graph == nullptr) { return; }
        if (graph->exec) { NMI_HIP_CHECK(hipGraphExecDestroy(graph->exec)); }
        if (graph->graph) { NMI_HIP_CHECK(hipGraphDestroy(graph->graph)); }
        delete graph;
    });
}

} // extern "C"
