/*
 * kq_hip_gguf.c — packed GGUF tensor bytes into device memory.
 *
 * The reference hands its CPU kernels a pointer into the mapped file
 * (kq_tensor_view_physical_data, src/kq_tensor_view.c; spans from
 * src/kq_gguf.c:1019-1078). Here the same bytes are copied to HBM once:
 * the span is mapped one window at a time and each window goes through the
 * context's pinned staging buffers, so reading the file overlaps the copy.
 * Expert members follow the addressing of kq_tensor_view_open_expert_member
 * (src/kq_tensor_view.c:664-807): experts on the slowest physical axis,
 * each a whole number of quant blocks.
 */
#include "kq_hip.h"

#include "kq_gguf_internal.h"
#include "kq_hip_internal.h"
#include "kq_status_internal.h"

/* mapped window per step: bounds the address space one call holds */
#define KQ_UPLOAD_WINDOW ((uint64_t)1u << 30)

kq_status kq_hip_gguf_expert_member(const kq_gguf_tensor *t, uint32_t expert_id, uint64_t *off,
                                    uint64_t *count, kq_diagnostic *diag) {
    uint64_t experts, member;
    kq_diagnostic_clear(diag);
    if (t == NULL || off == NULL || count == NULL)
        return kq_fail(diag, KQ_STATUS_INVALID_ARGUMENT, "tensor and outputs are required");
    if (t->rank < 2u || t->rank > KQ_GGUF_MAX_DIMS)
        return kq_fail(diag, KQ_STATUS_INVALID_QUANTIZED_GEOMETRY,
                       "an expert stack needs rank 2 or more; the tensor has rank %u", t->rank);
    experts = t->dimensions[t->rank - 1u];
    if ((uint64_t)expert_id >= experts)
        return kq_fail(diag, KQ_STATUS_SPAN_OUT_OF_RANGE, "expert %u is outside a stack of %llu",
                       expert_id, (unsigned long long)experts);
    member = t->element_count / experts;
    if (t->block_elements == 0u || member % t->block_elements != 0u)
        return kq_fail(diag, KQ_STATUS_NONCONTIGUOUS_TENSOR_VIEW,
                       "an expert member of %llu elements is not whole quant blocks",
                       (unsigned long long)member);
    *count = member / t->block_elements * t->bytes_per_block;
    *off = (uint64_t)expert_id * *count;
    return KQ_STATUS_OK;
}

static kq_status upload_span(kq_hip_context *c, const kq_gguf *g, const kq_gguf_tensor *t,
                             uint64_t off, uint64_t bytes, void *dst, uint64_t capacity,
                             kq_diagnostic *diag) {
    uint64_t done = 0u;
    kq_status st = KQ_STATUS_OK;
    if (capacity < bytes)
        return kq_fail(diag, KQ_STATUS_BUFFER_TOO_SMALL,
                       "the device buffer holds %llu bytes; the span needs %llu",
                       (unsigned long long)capacity, (unsigned long long)bytes);
    while (st == KQ_STATUS_OK && done < bytes) {
        const uint64_t n = bytes - done < KQ_UPLOAD_WINDOW ? bytes - done : KQ_UPLOAD_WINDOW;
        kq_file_view *view = NULL;
        st = kqi_gguf_tensor_span(g, t, off + done, n, &view, diag);
        if (st == KQ_STATUS_OK)
            st = kqi_hip_staged_upload(c, (unsigned char *)dst + done, kq_file_view_data(view), n,
                                       diag);
        kq_file_view_close(view);
        done += n;
    }
    return st;
}

static kq_status check_common(const kq_hip_context *c, const kq_gguf *g, const kq_gguf_tensor *t,
                              const void *dst, kq_diagnostic *diag) {
    if (c == NULL || kq_hip_context_stream(c) == NULL || g == NULL || t == NULL || dst == NULL)
        return kq_fail(diag, KQ_STATUS_INVALID_ARGUMENT,
                       "context, GGUF, tensor and device buffer are required");
    if (!kqi_gguf_owns(g, t))
        return kq_fail(diag, KQ_STATUS_TENSOR_OWNERSHIP_MISMATCH,
                       "the tensor descriptor does not belong to this GGUF");
    return KQ_STATUS_OK;
}

kq_status kq_hip_gguf_upload_tensor(kq_hip_context *c, const kq_gguf *g, const kq_gguf_tensor *t,
                                    void *dst, uint64_t capacity, kq_diagnostic *diag) {
    kq_status st;
    kq_diagnostic_clear(diag);
    st = check_common(c, g, t, dst, diag);
    if (st != KQ_STATUS_OK) return st;
    return upload_span(c, g, t, 0u, t->packed_bytes, dst, capacity, diag);
}

kq_status kq_hip_gguf_upload_expert_member(kq_hip_context *c, const kq_gguf *g,
                                           const kq_gguf_tensor *t, uint32_t expert_id, void *dst,
                                           uint64_t capacity, kq_diagnostic *diag) {
    uint64_t off, bytes;
    kq_status st;
    kq_diagnostic_clear(diag);
    st = check_common(c, g, t, dst, diag);
    if (st == KQ_STATUS_OK) st = kq_hip_gguf_expert_member(t, expert_id, &off, &bytes, diag);
    if (st != KQ_STATUS_OK) return st;
    return upload_span(c, g, t, off, bytes, dst, capacity, diag);
}
