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

#endif
