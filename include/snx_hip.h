/*
 * snx_hip.h - thin C-ABI over the HIP runtime (allocation, copies, streams,
 * events).  The C host code of libsneppx_quant.so calls only these and the
 * kernel launchers; callers may use them to stage device buffers and to time
 * kernels on the stream they launch on.
 *
 * No reference counterpart: the reference reaches ROCm only through a dlopen
 * shim with host-memory emulation (drivers/rocm/rocm_driver.c:73-133,320-395),
 * which this library does not use.  All functions return 0 on success and -1
 * on failure (message in SNEPPX_qlinear_last_error()).
 */
#ifndef SNX_HIP_H
#define SNX_HIP_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

int snx_hip_device_count(int* count);
int snx_hip_malloc(void** ptr, size_t bytes);
int snx_hip_free(void* ptr);
int snx_hip_malloc_async(void** ptr, size_t bytes, void* stream);
int snx_hip_free_async(void* ptr, void* stream);
int snx_hip_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream);
int snx_hip_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream);
int snx_hip_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream);
int snx_hip_stream_create(void** stream);
int snx_hip_stream_destroy(void* stream);
int snx_hip_stream_sync(void* stream);
int snx_hip_device_sync(void);
int snx_hip_event_create(void** event);
int snx_hip_event_destroy(void* event);
int snx_hip_event_record(void* event, void* stream);
int snx_hip_event_sync(void* event);
int snx_hip_event_elapsed_ms(float* ms, void* start, void* stop);
/* Name of device 0's ISA ("gfx950:sramecc+:xnack-"), CU count and clock. */
int snx_hip_device_info(char* arch, size_t arch_len, int* cu_count, int* clock_khz);

/* HIP graphs for launch-bound loops (a decode step's linears): every call
 * made on `stream` between begin and end is recorded, not run (thread-local
 * capture mode, so other threads' work is unaffected), and end returns an
 * executable graph that graph_launch replays on a stream with one host call.
 * The decode GEMVs take no workspace and record only kernel nodes (no
 * memsets).  Entry points that allocate a workspace the first time they see
 * a shape must have run once on that stream before capture, so that the
 * workspace exists and the capture records kernels only. */
int snx_hip_stream_begin_capture(void* stream);
int snx_hip_stream_end_capture(void* stream, void** graph_exec);
int snx_hip_graph_launch(void* graph_exec, void* stream);
int snx_hip_graph_destroy(void* graph_exec);

#ifdef __cplusplus
}
#endif

#endif /* SNX_HIP_H */
