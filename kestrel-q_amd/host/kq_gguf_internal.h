#ifndef KQ_GGUF_INTERNAL_H
#define KQ_GGUF_INTERNAL_H

#include "kq_gguf.h"

/* Maps bytes [byte_offset, byte_offset + byte_count) of a tensor's packed
 * payload (src/kq_gguf.c:1019-1078, kq_gguf_open_tensor_span): the tensor
 * must be one of this GGUF's descriptors (TENSOR_OWNERSHIP_MISMATCH) and
 * the span non-empty and inside its packed bytes. */
/* 1 if tensor is one of gguf's own descriptors */
int kqi_gguf_owns(const kq_gguf *gguf, const kq_gguf_tensor *tensor);

kq_status kqi_gguf_tensor_span(const kq_gguf *gguf, const kq_gguf_tensor *tensor,
                               uint64_t byte_offset, uint64_t byte_count,
                               kq_file_view **out_view, kq_diagnostic *diagnostic);

#endif
