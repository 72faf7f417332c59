/*
 * marian_hip_util.h — device-memory, stream and event helpers exported by the
 * marian-hip library.
 *
 * No counterpart in the reference: the reference never crosses a device
 * boundary on its CPU path.  These exist for callers that have no HIP
 * allocator of their own (the parity tests and the benchmark drive the
 * op-level entry points of marian_hip.h through them) so that no framework is
 * needed to hold device buffers.
 */
#ifndef MARIAN_HIP_UTIL_H
#define MARIAN_HIP_UTIL_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

int marian_hip_device_count(void);
/* "<name> (<gcnArchName>)" of device `device`. */
int marian_hip_device_name(int device, char* buf, size_t cap);
int marian_hip_set_device(int device);

void* marian_hip_device_alloc(size_t bytes); /* NULL on failure */
int marian_hip_device_free(void* ptr);
int marian_hip_memcpy_h2d(void* dst, const void* src, size_t bytes);
int marian_hip_memcpy_d2h(void* dst, const void* src, size_t bytes);
int marian_hip_memcpy_d2d(void* dst, const void* src, size_t bytes);
int marian_hip_memset(void* dst, int value, size_t bytes);

void* marian_hip_stream_create(void); /* default priority */
int marian_hip_stream_destroy(void* stream);
int marian_hip_stream_sync(void* stream); /* NULL = default stream */
int marian_hip_device_sync(void);

void* marian_hip_event_create(void);
int marian_hip_event_destroy(void* event);
int marian_hip_event_record(void* event, void* stream);
int marian_hip_event_sync(void* event);
/* milliseconds between two recorded events */
int marian_hip_event_elapsed(void* start, void* stop, float* ms);

/* Text of the last HIP error seen by the op-level or util entry points. */
const char* marian_hip_last_op_error(void);

/* SHA-256 (hex) of the sources this library was built from: csrc/*.hip,
 * csrc/*.h and include/*.h, in name order, each as name, NUL, contents.
 * Lets a caller check that a prebuilt library matches the checked-out code. */
const char* marian_hip_build_id(void);

#ifdef __cplusplus
}
#endif
#endif
