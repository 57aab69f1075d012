#ifndef KQ_HIP_INTERNAL_H
#define KQ_HIP_INTERNAL_H

#include "kq_hip.h"

/* Synchronous host-to-device copy through the context's two pinned staging
 * buffers (allocated on first use, freed with the context). For sources
 * the copy engines should not read in place, such as mapped file pages.
 * Does not clear the diagnostic. */
kq_status kqi_hip_staged_upload(kq_hip_context *context, void *device_dst,
                                const void *host_src, uint64_t bytes,
                                kq_diagnostic *diagnostic);

/* Context services shared with the sampler's file (kq_hip_sampling.c). */

/* A valid context made current; INVALID_ARGUMENT for a bad context. */
kq_status kqi_context_begin(kq_hip_context *context, kq_diagnostic *diagnostic);
/* The context's stream, as the HIP type (void * in the public header). */
void *kqi_context_stream_ptr(const kq_hip_context *context);
/* Waits for the stream and reports the device status word (then cleared). */
kq_status kqi_context_drain(kq_hip_context *context, kq_diagnostic *diagnostic);
/* DEVICE_FAILURE with the HIP error string. */
kq_status kqi_hip_fail(kq_diagnostic *diagnostic, int hip_error, const char *what);
/* Validates and enqueues logits = W h for one hidden vector (the LM head's
 * product), without waiting. */
kq_status kqi_enqueue_logits(kq_hip_context *context, uint32_t type_id, const void *weights,
                             uint64_t vocabulary, uint64_t columns, const float *hidden,
                             float *logits, kq_diagnostic *diagnostic);

#endif
