/*
 * mi_moe_util.h - HIP plumbing exported by libmimoe for callers that have no
 * HIP bindings of their own (the Python ctypes tests and bench.py): device
 * memory, copies, streams and event timing.  No compute; no counterpart in the
 * reference (ggml's backend buffer / tensor_set / tensor_get calls play this
 * role there: moondream.cpp:188-215, moe_decode_driver.hpp:523-545).
 */
#ifndef MI_MOE_UTIL_H
#define MI_MOE_UTIL_H

#include <stddef.h>
#include <stdint.h>

#include "mi_moe.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipEvent_t *mi_event_t;

int mi_device_count(int *count);
int mi_set_device(int device);
/* name (NUL-terminated, up to name_len bytes), CU count, peak engine clock in kHz,
 * gcn arch name (e.g. "gfx950:sramecc+:xnack-") */
int mi_device_info(int device, char *name, int name_len, int *cu_count, int *clock_khz,
                   char *arch, int arch_len);

int mi_dev_malloc(void **ptr, size_t bytes);
int mi_dev_free(void *ptr);
int mi_memcpy_h2d(void *dst, const void *src, size_t bytes);
int mi_memcpy_d2h(void *dst, const void *src, size_t bytes);
int mi_memcpy_d2d(void *dst, const void *src, size_t bytes);
int mi_memset_d(void *dst, int value, size_t bytes);
/* copies ordered on a stream (host memory may be pageable: the call then
 * returns once the host side is staged); wait with mi_stream_synchronize */
int mi_memcpy_h2d_async(void *dst, const void *src, size_t bytes, mi_stream_t s);
int mi_memcpy_d2h_async(void *dst, const void *src, size_t bytes, mi_stream_t s);
int mi_device_synchronize(void);

int mi_stream_create(mi_stream_t *s);
int mi_stream_destroy(mi_stream_t s);
int mi_stream_synchronize(mi_stream_t s);

int mi_event_create(mi_event_t *e);
int mi_event_destroy(mi_event_t e);
int mi_event_record(mi_event_t e, mi_stream_t s);
int mi_event_synchronize(mi_event_t e);
int mi_event_elapsed_ms(float *ms, mi_event_t start, mi_event_t stop);

/* Stream capture into a replayable graph.  mi_moe_forward and
 * mi_moe_expert_ffn may be captured once their context is reserved: after
 * reservation they allocate nothing, set no memory by memset, and wait on
 * nothing on the host (stage profiling, which records events, must be off).
 * Capture mode is relaxed; the stream must not be the null stream.
 * end_capture instantiates the captured work; a graph replays the captured
 * calls with their arguments (pointers, token count) as captured, so the
 * caller rewrites the inputs in place between launches. */
typedef struct mi_graph_s *mi_graph_t;
int mi_stream_begin_capture(mi_stream_t s);
int mi_stream_end_capture(mi_stream_t s, mi_graph_t *graph);
int mi_graph_launch(mi_graph_t graph, mi_stream_t s);
int mi_graph_destroy(mi_graph_t graph);

/* last HIP error string seen by the library (thread-local, static storage) */
const char *mi_last_hip_error(void);

#ifdef __cplusplus
}
#endif
#endif /* MI_MOE_UTIL_H */
