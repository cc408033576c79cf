/*
 * brasa_hip_rt -- thin device plumbing exported by libbrasa_attn.so for harnesses that drive the
 * attention entry points without another HIP runtime in the process (the Python tests and
 * bench.py use these through ctypes). None of these has a counterpart in the reference's
 * attention interface: they stand in for the reference's `brasa_metal` Buffer / Command / timing
 * (crates/metal/src/runtime.rs:134-425), which the caller of the C ABI owns.
 *
 * All functions return BRASA_OK (0) or BRASA_ERR_LAUNCH with brasa_last_error() set.
 */
#ifndef BRASA_HIP_RT_H
#define BRASA_HIP_RT_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

int brasa_rt_device_count(int* count);
int brasa_rt_set_device(int device);
int brasa_rt_device_name(char* buf, size_t len);
int brasa_rt_malloc(void** ptr, size_t bytes);
int brasa_rt_free(void* ptr);
int brasa_rt_memcpy_htod(void* dst, const void* src, size_t bytes);
int brasa_rt_memcpy_dtoh(void* dst, const void* src, size_t bytes);
int brasa_rt_memcpy_dtod(void* dst, const void* src, size_t bytes, void* stream);
/* Fills `bytes` bytes with `value` using a kernel (not hipMemset). */
int brasa_rt_fill_u8(void* dst, uint8_t value, size_t bytes, void* stream);
int brasa_rt_device_synchronize(void);
int brasa_rt_stream_create(void** stream);
int brasa_rt_stream_destroy(void* stream);
int brasa_rt_stream_synchronize(void* stream);
int brasa_rt_event_create(void** event);
int brasa_rt_event_destroy(void* event);
int brasa_rt_event_record(void* event, void* stream);
int brasa_rt_event_elapsed_ms(float* ms, void* start, void* stop);
int brasa_rt_event_synchronize(void* event);
/*
 * HIP graph capture of the work enqueued on `stream` (hipStreamCaptureModeThreadLocal):
 * begin_capture starts it; end_capture ends it and returns an instantiated, launchable graph
 * (hipGraphExec_t as void*); graph_launch enqueues a replay on `stream`; graph_destroy frees it.
 * The attention entry points allocate nothing and record no memset node, so they can be
 * captured (the conventions in brasa_attn.h say what a captured graph keeps).
 */
int brasa_rt_stream_begin_capture(void* stream);
int brasa_rt_stream_end_capture(void* stream, void** graph_exec);
int brasa_rt_graph_launch(void* graph_exec, void* stream);
int brasa_rt_graph_destroy(void* graph_exec);
/* Free and total device memory of the current device (hipMemGetInfo). */
int brasa_rt_mem_info(size_t* free_bytes, size_t* total_bytes);

/*
 * Synthetic N(0, 1) f32 values for benchmarks: out[i] for i < n is a Box-Muller transform of a
 * counter-based hash of (seed, i). Deterministic per (seed, i) on the device; not bit-identical
 * to any host generator (parity tests generate their inputs on the host instead).
 */
int brasa_rt_fill_normal_f32(float* out, size_t n, uint64_t seed, float scale, void* stream);

#ifdef __cplusplus
}
#endif
#endif
