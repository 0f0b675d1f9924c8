/*
 * ninfer_amd runtime helpers — device memory, streams and events for harnesses that drive the
 * C ABI without another GPU framework (the Python tests and bench.py use these through ctypes).
 * They are plumbing, not part of the verify-step op surface, and have no reference counterpart.
 * All return an nmi_status; messages via nmi_last_error().
 */
#ifndef NINFER_AMD_RUNTIME_H
#define NINFER_AMD_RUNTIME_H

#include "ninfer_amd.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipEvent_t* nmi_event_t;

int nmi_rt_device_count(int32_t* count);
int nmi_rt_device_name(char* buf, size_t len);
int nmi_rt_malloc(void** ptr, size_t bytes);
int nmi_rt_free(void* ptr);
int nmi_rt_memcpy_htod(void* dst, const void* src, size_t bytes);
int nmi_rt_memcpy_dtoh(void* dst, const void* src, size_t bytes);
int nmi_rt_memcpy_dtod(void* dst, const void* src, size_t bytes, nmi_stream_t stream);
/* Byte fill with a kernel (graph-safe, no hipMemsetAsync). */
int nmi_rt_fill_u8(void* dst, uint8_t value, size_t bytes, nmi_stream_t stream);
/* Copies row (*counter mod rows) of an int32 [rows, cols] table into dst and adds 1 to *counter
 * (device memory; cols <= 1024): a seeded draft source for a replayed round graph, standing in
 * for the draft model between rounds. */
int nmi_rt_next_row_i32(const int32_t* table, int32_t rows, int32_t cols, int32_t* counter, int32_t* dst,
                        nmi_stream_t stream);
int nmi_rt_stream_create(nmi_stream_t* stream);
int nmi_rt_stream_destroy(nmi_stream_t stream);
int nmi_rt_stream_synchronize(nmi_stream_t stream);
int nmi_rt_device_synchronize(void);
int nmi_rt_event_create(nmi_event_t* event);
int nmi_rt_event_destroy(nmi_event_t event);
int nmi_rt_event_record(nmi_event_t event, nmi_stream_t stream);
int nmi_rt_event_elapsed_ms(float* ms, nmi_event_t start, nmi_event_t stop);
/* Stream capture into a graph and replay (hipStreamBeginCapture / EndCapture / Instantiate). */
typedef struct nmi_graph* nmi_graph_t;
int nmi_rt_capture_begin(nmi_stream_t stream);
int nmi_rt_capture_end(nmi_stream_t stream, nmi_graph_t* graph);
int nmi_rt_graph_launch(nmi_graph_t graph, nmi_stream_t stream);
int nmi_rt_graph_destroy(nmi_graph_t graph);

/* Bandwidth controls for the benchmark (one launch that only moves `bytes`; bytes a multiple of 16,
 * pointers 16-byte aligned). nmi_rt_stream_copy is the reference bench's copy ceiling
 * (bench/ops/gqa_attention_bench.cu:1103-1130); nmi_rt_read_ceiling reads the payload with plain
 * non-temporal vector loads or with the LDS-DMA ring pattern of the attention kernels, storing a
 * checksum to `sink` (4 bytes) only on an improbable value. */
enum { NMI_READ_VECTOR = 0, NMI_READ_LDS_DMA = 1 };
int nmi_rt_stream_copy(void* dst, const void* src, size_t bytes, nmi_stream_t stream);
int nmi_rt_read_ceiling(const void* src, size_t bytes, int32_t form, void* sink, nmi_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* NINFER_AMD_RUNTIME_H */
