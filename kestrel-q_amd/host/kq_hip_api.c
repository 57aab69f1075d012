/*
 * kq_hip_api.c — host side of the kq_hip C ABI (include/kq_hip.h).
 *
 * C17. Validates every call before enqueueing device work, with the
 * reference's status codes and order of checks (src/kq_numeric.c:297-359,
 * :420-503; src/kq_weight_provider.c:378-437; src/kq_moe_qwen38.c:276-330,
 * :604-660), then drives the HIP launchers of the kernel files
 * (kestrel-q_amd/csrc/kq_launch.h) on the context's stream.
 *
 * Device-detected failures are OR-ed by kernels into a device status word;
 * synchronous calls (the default) read it back after the stream drains and
 * report it, asynchronous ones leave it for kq_hip_context_synchronize.
 */
#include "kq_hip.h"

#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "kq_hip_internal.h"
#include "kq_launch.h"
#include "kq_status_internal.h"

#define KQ_MOE_CONFIG_MAGIC 0x4b514d48u /* "KQMH" */
#define KQ_DEV_MALFORMED 1u
#define KQ_DEV_NUMERIC 2u
#define KQ_DEV_INPUT 4u
#define KQ_DEV_RANGE 8u
/* output ranges one call can restore */
#define KQ_SNAP_RANGES 4u

struct kq_hip_context {
    int device;
    int async;
    hipStream_t stream;
    uint32_t *d_status;
    uint32_t *h_status; /* pinned */
    float *part_v;      /* argmax partials */
    uint32_t *part_i;
    uint64_t part_cap;
    void *stage[2];     /* pinned staging for file-backed uploads */
    hipEvent_t stage_done[2];
    void *noalloc;      /* this device's allocation-free LM-head partials */
    void *stage_dev;    /* aligned device copy of a view span that starts off
                           the decoder's alignment, grown on demand */
    uint64_t stage_dev_cap;
    /* commit-on-success of synchronous calls: the outputs' prior contents,
     * copied aside before the call's launches and copied back when it fails */
    int commit;
    void *snap;
    uint64_t snap_cap;
    uint32_t snap_n;
    void *snap_dst[KQ_SNAP_RANGES];
    uint64_t snap_len[KQ_SNAP_RANGES];
};

struct kq_hip_moe_config {
    uint32_t magic;
    kq_hip_moe_dimensions dims;
};

/* ------------------------------------------------------------------ */

static uint64_t align256(uint64_t n) { return (n + 255u) & ~(uint64_t)255u; }

static kq_status hip_fail(kq_diagnostic *diag, hipError_t e, const char *what) {
    return kq_fail(diag, KQ_STATUS_DEVICE_FAILURE, "%s: %s", what, hipGetErrorString(e));
}

static int ctx_ok(const kq_hip_context *c) { return c != NULL && c->stream != NULL; }

static kq_status set_device(kq_hip_context *c, kq_diagnostic *diag) {
    hipError_t e = hipSetDevice(c->device);
    return e == hipSuccess ? KQ_STATUS_OK : hip_fail(diag, e, "hipSetDevice");
}

/* Map the device status word to the reference's codes: a non-finite input
 * is reported first (the reference validates inputs before decoding), then a
 * malformed block scale, then a non-finite result. */
static kq_status device_flags(uint32_t flags, kq_diagnostic *diag) {
    if (flags & KQ_DEV_RANGE)
        return kq_fail(diag, KQ_STATUS_INVALID_ARGUMENT, "an expert id is out of range");
    if (flags & KQ_DEV_INPUT)
        return kq_fail(diag, KQ_STATUS_NUMERIC_DOMAIN, "non-finite input on the device path");
    if (flags & KQ_DEV_MALFORMED)
        return kq_fail(diag, KQ_STATUS_MALFORMED_QUANTIZED_DATA,
                       "quantized block scale is non-finite");
    if (flags & KQ_DEV_NUMERIC)
        return kq_fail(diag, KQ_STATUS_NUMERIC_DOMAIN, "device computation produced a non-finite value");
    return KQ_STATUS_OK;
}

static kq_status drain(kq_hip_context *c, kq_diagnostic *diag) {
    hipError_t e = hipMemcpyAsync(c->h_status, c->d_status, sizeof(uint32_t),
                                  hipMemcpyDeviceToHost, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) return hip_fail(diag, e, "stream synchronize");
    if (*c->h_status != 0u) {
        uint32_t flags = *c->h_status;
        *c->h_status = 0u;
        e = hipMemsetAsync(c->d_status, 0, sizeof(uint32_t), c->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
        if (e != hipSuccess) return hip_fail(diag, e, "status reset");
        return device_flags(flags, diag);
    }
    return KQ_STATUS_OK;
}

/* Copies the outputs of a synchronous call aside before its first launch
 * (commit-on-success, the reference's staged outputs: src/kq_weight_provider.c
 * :420, :480, src/kq_moe_qwen38.c:562-565). n ranges (pointer, bytes); empty
 * or NULL ranges are skipped. Asynchronous calls, and contexts with the
 * commit switched off, take no copy. On an allocation failure nothing has
 * been launched and the outputs are untouched. */
static kq_status snapshot(kq_hip_context *c, uint32_t n, void *const *p, const uint64_t *len,
                          kq_diagnostic *diag) {
    uint64_t total = 0u, off = 0u;
    hipError_t e = hipSuccess;
    /* a call enqueued by another call (the MoE block's stages) runs
     * asynchronously and leaves the outer call's copies in place */
    if (c->async || !c->commit) return KQ_STATUS_OK;
    c->snap_n = 0u;
    for (uint32_t i = 0; i < n; ++i)
        if (p[i] != NULL) total += align256(len[i]);
    if (total == 0u) return KQ_STATUS_OK;
    if (c->snap_cap < total) {
        if (c->snap) {
            (void)hipStreamSynchronize(c->stream);
            (void)hipFree(c->snap);
            c->snap = NULL;
            c->snap_cap = 0u;
        }
        e = hipMalloc(&c->snap, (size_t)total);
        if (e != hipSuccess)
            return kq_fail(diag, KQ_STATUS_OUT_OF_MEMORY,
                           "commit-on-success copy of the outputs (%llu bytes): %s",
                           (unsigned long long)total, hipGetErrorString(e));
        c->snap_cap = total;
    }
    for (uint32_t i = 0; i < n && e == hipSuccess; ++i) {
        if (p[i] == NULL || len[i] == 0u) continue;
        e = hipMemcpyAsync((char *)c->snap + off, p[i], (size_t)len[i], hipMemcpyDeviceToDevice,
                           c->stream);
        c->snap_dst[c->snap_n] = p[i];
        c->snap_len[c->snap_n] = len[i];
        c->snap_n++;
        off += align256(len[i]);
    }
    if (e != hipSuccess) {
        c->snap_n = 0u;
        return hip_fail(diag, e, "commit-on-success copy");
    }
    return KQ_STATUS_OK;
}

static kq_status snapshot1(kq_hip_context *c, void *p, uint64_t len, kq_diagnostic *diag) {
    return snapshot(c, 1u, &p, &len, diag);
}

/* A failed synchronous call: its outputs get their prior contents back
 * (the work it enqueued has drained, or the stream is broken and the copies
 * fail with it). */
static void restore(kq_hip_context *c) {
    uint64_t off = 0u;
    for (uint32_t i = 0; i < c->snap_n; ++i) {
        (void)hipMemcpyAsync(c->snap_dst[i], (char *)c->snap + off, (size_t)c->snap_len[i],
                             hipMemcpyDeviceToDevice, c->stream);
        off += align256(c->snap_len[i]);
    }
    if (c->snap_n != 0u) (void)hipStreamSynchronize(c->stream);
    c->snap_n = 0u;
}

/* The end of a call: asynchronous calls return after enqueueing;
 * synchronous ones drain the stream, report the device status word and, on
 * any failure, restore the outputs copied aside by snapshot(). */
static kq_status finish(kq_hip_context *c, hipError_t launch, const char *what,
                        kq_diagnostic *diag) {
    kq_status st;
    if (c->async && launch == hipSuccess) return KQ_STATUS_OK;
    if (launch != hipSuccess) {
        st = hip_fail(diag, launch, what);
        if (!c->async) {
            (void)hipStreamSynchronize(c->stream);
            restore(c);
        }
        return st;
    }
    st = drain(c, diag);
    if (st != KQ_STATUS_OK)
        restore(c);
    else
        c->snap_n = 0u;
    return st;
}

static int ranges_overlap(const void *a, uint64_t an, const void *b, uint64_t bn) {
    uintptr_t a0 = (uintptr_t)a, b0 = (uintptr_t)b;
    if (a == NULL || b == NULL || an == 0u || bn == 0u) return 0;
    return a0 < b0 + bn && b0 < a0 + an;
}

static int aligned(const void *p, uintptr_t a) { return ((uintptr_t)p % a) == 0u; }


static int u64_mul(uint64_t a, uint64_t b, uint64_t *out) {
    if (a != 0u && b > UINT64_MAX / a) return 0;
    *out = a * b;
    return 1;
}

/* ------------------------------------------------------------------ */
/* context */

kq_status kq_hip_context_create(int device, kq_hip_context **out, kq_diagnostic *diag) {
    kq_hip_context *c;
    hipDeviceProp_t prop;
    hipError_t e;
    int count = 0;
    kq_diagnostic_clear(diag);
    if (out == NULL) return kq_fail(diag, KQ_STATUS_INVALID_ARGUMENT, "context output is required");
    *out = NULL;
    e = hipGetDeviceCount(&count);
    if (e != hipSuccess || count <= 0)
        return kq_fail(diag, KQ_STATUS_DEVICE_FAILURE, "no HIP device is available");
    if (device < 0 || device >= count)
        return kq_fail(diag, KQ_STATUS_INVALID_ARGUMENT, "device %d is out of range", device);
    e = hipGetDeviceProperties(&prop, device);
    if (e != hipSuccess) return hip_fail(diag, e, "hipGetDeviceProperties");
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return kq_fail(diag, KQ_STATUS_DEVICE_FAILURE,
                       "device %d is %s; this library is built for gfx950 only", device,
                       prop.gcnArchName);
    c = (kq_hip_context *)calloc(1, sizeof(*c));
    if (c == NULL) return kq_fail(diag, KQ_STATUS_OUT_OF_MEMORY, "context allocation failed");
    c->device = device;
    c->commit = 1;
    e = hipSetDevice(device);
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipMalloc((void **)&c->d_status, sizeof(uint32_t));
    if (e == hipSuccess) e = hipHostMalloc((void **)&c->h_status, sizeof(uint32_t), hipHostMallocDefault);
    if (e == hipSuccess) e = hipMemsetAsync(c->d_status, 0, sizeof(uint32_t), c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    /* the device address of this device's static partials array, looked up
     * once per device with the device current */
    if (e == hipSuccess) e = kq_launch_noalloc_scratch_init(device, &c->noalloc);
    if (e != hipSuccess) {
        kq_status st = hip_fail(diag, e, "context setup");
        kq_hip_context_destroy(c);
        return st;
    }
    *c->h_status = 0u;
    *out = c;
    return KQ_STATUS_OK;
}

void kq_hip_context_destroy(kq_hip_context *c) {
    if (c == NULL) return;
    (void)hipSetDevice(c->device);
    if (c->stream) (void)hipStreamSynchronize(c->stream);
    if (c->part_v) (void)hipFree(c->part_v);
    if (c->part_i) (void)hipFree(c->part_i);
    if (c->stage_dev) (void)hipFree(c->stage_dev);
    if (c->snap) (void)hipFree(c->snap);
    if (c->d_status) (void)hipFree(c->d_status);
    if (c->h_status) (void)hipHostFree(c->h_status);
    for (int k = 0; k < 2; ++k) {
        if (c->stage[k]) (void)hipHostFree(c->stage[k]);
        if (c->stage_done[k]) (void)hipEventDestroy(c->stage_done[k]);
    }
    if (c->stream) (void)hipStreamDestroy(c->stream);
    free(c);
}

kq_status kq_hip_context_set_async(kq_hip_context *c, int async, kq_diagnostic *diag) {
    kq_diagnostic_clear(diag);
    if (!ctx_ok(c)) return kq_fail(diag, KQ_STATUS_INVALID_ARGUMENT, "valid context is required");
    c->async = async ? 1 : 0;
    return KQ_STATUS_OK;
}

kq_status kq_hip_context_set_commit_on_success(kq_hip_context *c, int commit,
                                               kq_diagnostic *diag) {
    kq_diagnostic_clear(diag);
    if (!ctx_ok(c)) return kq_fail(diag, KQ_STATUS_INVALID_ARGUMENT, "valid context is required");
    c->commit = commit ? 1 : 0;
    return KQ_STATUS_OK;
}

kq_status kq_hip_context_synchronize(kq_hip_context *c, kq_diagnostic *diag) {
    kq_status st;
    kq_diagnostic_clear(diag);
    if (!ctx_ok(c)) return kq_fail(diag, KQ_STATUS_INVALID_ARGUMENT, "valid context is required");
    st = set_device(c, diag);
    if (st != KQ_STATUS_OK) return st;
    return drain(c, diag);
}

kq_status kqi_context_begin(kq_hip_context *c, kq_diagnostic *diag) {
    if (!ctx_ok(c)) return kq_fail(diag, KQ_STATUS_INVALID_ARGUMENT, "valid context is required");
    return set_device(c, diag);
}

void *kqi_context_stream_ptr(const kq_hip_context *c) { return (void *)c->stream; }

kq_status kqi_context_drain(kq_hip_context *c, kq_diagnostic *diag) { return drain(c, diag); }

kq_status kqi_hip_fail(kq_diagnostic *diag, int e, const char *what) {
    return hip_fail(diag, (hipError_t)e, what);
}

void *kq_hip_context_stream(const kq_hip_context *c) {
    return c == NULL ? NULL : (void *)c->stream;
}

kq_status kq_hip_malloc(kq_hip_context *c, uint64_t bytes, void **out, kq_diagnostic *diag) {
    hipError_t e;
    kq_status st;
    kq_diagnostic_clear(diag);
    if (!ctx_ok(c) || out == NULL || bytes == 0u)
        return kq_fail(diag, KQ_STATUS_INVALID_ARGUMENT, "context, size and output are required");
    *out = NULL;
    st = set_device(c, diag);
    if (st != KQ_STATUS_OK) return st;
    e = hipMalloc(out, (size_t)bytes);
    if (e != hipSuccess) {
        *out = NULL;
        return kq_fail(diag, KQ_STATUS_OUT_OF_MEMORY, "hipMalloc of %llu bytes failed: %s",
                       (unsigned long long)bytes, hipGetErrorString(e));
    }
    return KQ_STATUS_OK;
}

void kq_hip_free(kq_hip_context *c, void *p) {
    if (c == NULL || p == NULL) return;
    (void)hipSetDevice(c->device);
    (void)hipStreamSynchronize(c->stream);
    (void)hipFree(p);
}

kq_status kq_hip_upload(kq_hip_context *c, void *dst, const void *src, uint64_t bytes,
                        kq_diagnostic *diag) {
    hipError_t e;
    kq_status st;
    kq_diagnostic_clear(diag);
    if (!ctx_ok(c) || dst == NULL || src == NULL)
        return kq_fail(diag, KQ_STATUS_INVALID_ARGUMENT, "context and buffers are required");
    if (bytes == 0u) return KQ_STATUS_OK;
    st = set_device(c, diag);
    if (st != KQ_STATUS_OK) return st;
    e = hipMemcpyAsync(dst, src, (size_t)bytes, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    return e == hipSuccess ? KQ_STATUS_OK : hip_fail(diag, e, "upload");
}

/* Host memory that the DMA engines may not read directly (a mapped file)
 * is copied through two pinned buffers: while one chunk's copy to the
 * device runs, the CPU fills the other. */
#define KQ_STAGE_BYTES ((uint64_t)16u << 20)

static hipError_t ensure_stage(kq_hip_context *c) {
    hipError_t e = hipSuccess;
    for (int k = 0; k < 2 && e == hipSuccess; ++k) {
        if (c->stage[k] == NULL)
            e = hipHostMalloc(&c->stage[k], (size_t)KQ_STAGE_BYTES, hipHostMallocDefault);
        if (e == hipSuccess && c->stage_done[k] == NULL)
            e = hipEventCreateWithFlags(&c->stage_done[k], hipEventDisableTiming);
    }
    return e;
}

kq_status kqi_hip_staged_upload(kq_hip_context *c, void *dst, const void *src, uint64_t bytes,
                                kq_diagnostic *diag) {
    const unsigned char *from = (const unsigned char *)src;
    int used[2] = {0, 0};
    uint64_t at = 0u;
    hipError_t e, s;
    kq_status st;
    int k = 0;
    if (!ctx_ok(c) || dst == NULL || src == NULL)
        return kq_fail(diag, KQ_STATUS_INVALID_ARGUMENT, "context and buffers are required");
    st = set_device(c, diag);
    if (st != KQ_STATUS_OK) return st;
    e = ensure_stage(c);
    while (e == hipSuccess && at < bytes) {
        const uint64_t n = bytes - at < KQ_STAGE_BYTES ? bytes - at : KQ_STAGE_BYTES;
        if (used[k]) e = hipEventSynchronize(c->stage_done[k]);
        if (e != hipSuccess) break;
        memcpy(c->stage[k], from + at, (size_t)n);
        e = hipMemcpyAsync((unsigned char *)dst + at, c->stage[k], (size_t)n,
                           hipMemcpyHostToDevice, c->stream);
        if (e == hipSuccess) e = hipEventRecord(c->stage_done[k], c->stream);
        used[k] = 1;
        at += n;
        k ^= 1;
    }
    /* the staging buffers must be idle before another call refills them */
    s = hipStreamSynchronize(c->stream);
    if (e == hipSuccess) e = s;
    return e == hipSuccess ? KQ_STATUS_OK : hip_fail(diag, e, "staged upload");
}

kq_status kq_hip_download(kq_hip_context *c, void *dst, const void *src, uint64_t bytes,
                          kq_diagnostic *diag) {
    hipError_t e;
    kq_status st;
    kq_diagnostic_clear(diag);
    if (!ctx_ok(c) || dst == NULL || src == NULL)
        return kq_fail(diag, KQ_STATUS_INVALID_ARGUMENT, "context and buffers are required");
    if (bytes == 0u) return KQ_STATUS_OK;
    st = set_device(c, diag);
    if (st != KQ_STATUS_OK) return st;
    e = hipMemcpyAsync(dst, src, (size_t)bytes, hipMemcpyDeviceToHost, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    return e == hipSuccess ? KQ_STATUS_OK : hip_fail(diag, e, "download");
}

/* ------------------------------------------------------------------ */
/* geometry */

kq_status kq_hip_quant_geometry_for_type(uint32_t type_id, kq_hip_quant_geometry *g,
                                         kq_diagnostic *diag) {
    kq_diagnostic_clear(diag);
    if (g == NULL) return kq_fail(diag, KQ_STATUS_INVALID_ARGUMENT, "output geometry is required");
    memset(g, 0, sizeof(*g));
    switch (type_id) {
    case KQ_HIP_TYPE_F32: g->block_elements = 1u; g->bytes_per_block = 4u; break;
    case KQ_HIP_TYPE_BF16: g->block_elements = 1u; g->bytes_per_block = 2u; break;
    case KQ_HIP_TYPE_Q5_1: g->block_elements = 32u; g->bytes_per_block = 24u; break;
    case KQ_HIP_TYPE_Q8_0: g->block_elements = 32u; g->bytes_per_block = 34u; break;
    case KQ_HIP_TYPE_IQ4_NL: g->block_elements = 32u; g->bytes_per_block = 18u; break;
    case KQ_HIP_TYPE_Q4_K: g->block_elements = 256u; g->bytes_per_block = 144u; break;
    case KQ_HIP_TYPE_Q5_K: g->block_elements = 256u; g->bytes_per_block = 176u; break;
    case KQ_HIP_TYPE_Q6_K: g->block_elements = 256u; g->bytes_per_block = 210u; break;
    default:
        return kq_fail(diag, KQ_STATUS_UNSUPPORTED_TENSOR_TYPE,
                       "GGUF tensor type %u is unsupported", type_id);
    }
    g->type_id = type_id;
    return KQ_STATUS_OK;
}

kq_status kq_hip_quant_packed_size(uint32_t type_id, uint64_t elements, uint64_t *out,
                                   kq_diagnostic *diag) {
    kq_hip_quant_geometry g;
    kq_status st;
    kq_diagnostic_clear(diag);
    if (out == NULL) return kq_fail(diag, KQ_STATUS_INVALID_ARGUMENT, "output byte count is required");
    *out = 0u;
    st = kq_hip_quant_geometry_for_type(type_id, &g, diag);
    if (st != KQ_STATUS_OK) return st;
    if (elements == 0u || elements % g.block_elements != 0u)
        return kq_fail(diag, KQ_STATUS_INVALID_QUANTIZED_GEOMETRY,
                       "element count is not a non-zero whole number of quant blocks");
    if (!u64_mul(elements / g.block_elements, g.bytes_per_block, out))
        return kq_fail(diag, KQ_STATUS_ARITHMETIC_OVERFLOW, "packed byte count overflows uint64");
    return KQ_STATUS_OK;
}

kq_status kq_hip_expert_member_span(uint32_t type_id, uint64_t rows, uint64_t cols,
                                    uint32_t expert_count, uint32_t expert_id,
                                    uint64_t *off, uint64_t *count, kq_diagnostic *diag) {
    uint64_t elements, bytes;
    kq_hip_quant_geometry g;
    kq_status st;
    kq_diagnostic_clear(diag);
    if (off == NULL || count == NULL || rows == 0u || cols == 0u)
        return kq_fail(diag, KQ_STATUS_INVALID_ARGUMENT, "member geometry and outputs are required");
    if (expert_id >= expert_count)
        return kq_fail(diag, KQ_STATUS_SPAN_OUT_OF_RANGE, "expert %u is outside %u experts",
                       expert_id, expert_count);
    if (!u64_mul(rows, cols, &elements))
        return kq_fail(diag, KQ_STATUS_ARITHMETIC_OVERFLOW, "member element count overflows");
    st = kq_hip_quant_packed_size(type_id, elements, &bytes, diag);
    if (st != KQ_STATUS_OK) return st;
    st = kq_hip_quant_geometry_for_type(type_id, &g, diag);
    if (st != KQ_STATUS_OK) return st;
    if (cols % g.block_elements != 0u)
        return kq_fail(diag, KQ_STATUS_INVALID_QUANTIZED_GEOMETRY,
                       "member rows are not whole quant blocks");
    if (!u64_mul(bytes, expert_id, off))
        return kq_fail(diag, KQ_STATUS_ARITHMETIC_OVERFLOW, "member offset overflows");
    *count = bytes;
    return KQ_STATUS_OK;
}

/* every type with a geometry has a device decode; products need a packed
 * quantized type */
static kq_status quant_geometry(uint32_t type_id, uint64_t *be, uint64_t *bb,
                                kq_diagnostic *diag) {
    kq_hip_quant_geometry g;
    kq_status st = kq_hip_quant_geometry_for_type(type_id, &g, diag);
    if (st != KQ_STATUS_OK) return st;
    *be = g.block_elements;
    *bb = g.bytes_per_block;
    return KQ_STATUS_OK;
}

static int packed_quant(uint32_t type_id) {
    return type_id != KQ_HIP_TYPE_F32 && type_id != KQ_HIP_TYPE_BF16;
}

/* base alignment the device decode needs: 16-byte block headers (K-quants
 * whose blocks are multiples of 16 bytes), whole 32-bit words otherwise,
 * 16-bit elements for BF16 */
static uintptr_t packed_alignment(uint32_t type_id) {
    if (type_id == KQ_HIP_TYPE_Q4_K || type_id == KQ_HIP_TYPE_Q5_K) return 16u;
    if (type_id == KQ_HIP_TYPE_BF16) return 2u;
    return 4u;
}

/* ------------------------------------------------------------------ */
/* numeric */

kq_status kq_hip_dequantize_blocks_f32(kq_hip_context *c, uint32_t type_id, const void *packed,
                                       uint64_t packed_bytes, float *output,
                                       uint64_t capacity, uint64_t *count,
                                       kq_diagnostic *diag) {
    uint64_t be, bb, blocks, need, out_bytes;
    kq_status st;
    kq_diagnostic_clear(diag);
    if (!ctx_ok(c) || count == NULL || packed == NULL || packed_bytes == 0u)
        return kq_fail(diag, KQ_STATUS_INVALID_ARGUMENT, "packed input and output count are required");
    *count = 0u;
    st = quant_geometry(type_id, &be, &bb, diag);
    if (st != KQ_STATUS_OK) return st;
    if (packed_bytes % bb != 0u)
        return kq_fail(diag, KQ_STATUS_MALFORMED_QUANTIZED_DATA,
                       "packed bytes are not a bounded whole-block span");
    blocks = packed_bytes / bb;
    if (!u64_mul(blocks, be, &need) || !u64_mul(need, sizeof(float), &out_bytes))
        return kq_fail(diag, KQ_STATUS_ARITHMETIC_OVERFLOW, "decoded output count overflows");
    *count = need;
    if (output == NULL || capacity < need)
        return kq_fail(diag, KQ_STATUS_BUFFER_TOO_SMALL, "decoded output capacity is too small");
    if (ranges_overlap(packed, packed_bytes, output, out_bytes))
        return kq_fail(diag, KQ_STATUS_ALIASING_VIOLATION, "packed input and decoded output overlap");
    if (!aligned(packed, packed_alignment(type_id)) || !aligned(output, 16u))
        return kq_fail(diag, KQ_STATUS_INVALID_ALIGNMENT,
                       "packed input must be 16-byte (Q4_K, Q5_K), 2-byte (BF16) or 4-byte "
                       "aligned, output 16-byte");
    st = set_device(c, diag);
    if (st == KQ_STATUS_OK) st = snapshot1(c, output, out_bytes, diag);
    if (st != KQ_STATUS_OK) return st;
    return finish(c, kq_launch_dequant(type_id, packed, blocks, output, c->d_status, c->stream),
                  "dequant launch", diag);
}

/* ------------------------------------------------------------------ */
/* element ranges, tensor views */

kq_status kq_hip_quant_element_to_block(uint32_t type_id, uint64_t total, uint64_t index,
                                        uint64_t *block, uint64_t *within, kq_diagnostic *diag) {
    kq_hip_quant_geometry g;
    uint64_t ignored;
    kq_status st;
    kq_diagnostic_clear(diag);
    if (block == NULL || within == NULL)
        return kq_fail(diag, KQ_STATUS_INVALID_ARGUMENT,
                       "block index and intra-block outputs are required");
    *block = 0u;
    *within = 0u;
    st = kq_hip_quant_geometry_for_type(type_id, &g, diag);
    if (st == KQ_STATUS_OK) st = kq_hip_quant_packed_size(type_id, total, &ignored, diag);
    if (st != KQ_STATUS_OK) return st;
    if (index >= total)
        return kq_fail(diag, KQ_STATUS_SPAN_OUT_OF_RANGE, "logical element index is outside the tensor");
    *block = index / g.block_elements;
    *within = index % g.block_elements;
    return KQ_STATUS_OK;
}

kq_status kq_hip_quant_range_to_blocks(uint32_t type_id, uint64_t total, uint64_t offset,
                                       uint64_t count, kq_hip_quant_block_span *span,
                                       kq_diagnostic *diag) {
    kq_hip_quant_geometry g;
    uint64_t ignored, end, last, first_el, end_el;
    kq_status st;
    kq_diagnostic_clear(diag);
    if (span == NULL || count == 0u)
        return kq_fail(diag, KQ_STATUS_INVALID_ARGUMENT,
                       "non-zero logical range and output span are required");
    memset(span, 0, sizeof(*span));
    st = kq_hip_quant_geometry_for_type(type_id, &g, diag);
    if (st == KQ_STATUS_OK) st = kq_hip_quant_packed_size(type_id, total, &ignored, diag);
    if (st != KQ_STATUS_OK) return st;
    if (offset > UINT64_MAX - count)
        return kq_fail(diag, KQ_STATUS_ARITHMETIC_OVERFLOW, "logical element range overflows uint64");
    end = offset + count;
    if (offset >= total || end > total)
        return kq_fail(diag, KQ_STATUS_SPAN_OUT_OF_RANGE, "logical element range is outside the tensor");
    span->requested_element_offset = offset;
    span->requested_element_count = count;
    span->first_block = offset / g.block_elements;
    last = (end - 1u) / g.block_elements + 1u;
    span->block_count = last - span->first_block;
    if (!u64_mul(span->first_block, g.bytes_per_block, &span->physical_byte_offset) ||
        !u64_mul(span->block_count, g.bytes_per_block, &span->physical_byte_length) ||
        !u64_mul(span->first_block, g.block_elements, &first_el) ||
        !u64_mul(last, g.block_elements, &end_el))
        return kq_fail(diag, KQ_STATUS_ARITHMETIC_OVERFLOW,
                       "quantized block span arithmetic overflows uint64");
    span->leading_elements = offset - first_el;
    span->trailing_elements = end_el - end;
    return KQ_STATUS_OK;
}

kq_status kq_hip_tensor_view_init(uint32_t type_id, const void *data, uint64_t bytes,
                                  uint32_t layout, kq_hip_tensor_view *view,
                                  kq_diagnostic *diag) {
    kq_hip_quant_geometry g;
    kq_status st;
    kq_diagnostic_clear(diag);
    if (view == NULL || data == NULL || bytes == 0u || layout > KQ_HIP_LAYOUT_FUSED_MEMBER)
        return kq_fail(diag, KQ_STATUS_INVALID_ARGUMENT, "device data, size, layout and view are required");
    memset(view, 0, sizeof(*view));
    st = kq_hip_quant_geometry_for_type(type_id, &g, diag);
    if (st != KQ_STATUS_OK) return st;
    if (bytes % g.bytes_per_block != 0u)
        return kq_fail(diag, KQ_STATUS_MALFORMED_QUANTIZED_DATA, "a view covers whole blocks");
    view->type_id = type_id;
    view->layout = layout;
    view->block_elements = g.block_elements;
    view->bytes_per_block = g.bytes_per_block;
    view->block_count = bytes / g.bytes_per_block;
    view->canonical_contiguous = layout == KQ_HIP_LAYOUT_CANONICAL_CONTIGUOUS ||
                                 layout == KQ_HIP_LAYOUT_FUSED_MEMBER;
    view->device_data = data;
    view->mapped_bytes = bytes;
    return KQ_STATUS_OK;
}

kq_status kq_hip_dequantize_view_blocks_f32(kq_hip_context *c, const kq_hip_tensor_view *v,
                                            uint64_t first, uint64_t count, uint32_t order,
                                            float *out, uint64_t capacity, uint64_t *out_count,
                                            kq_diagnostic *diag) {
    kq_hip_quant_geometry g;
    uint64_t end, off, bytes;
    const char *src;
    kq_status st;
    kq_diagnostic_clear(diag);
    if (v == NULL || out_count == NULL || count == 0u ||
        (order != KQ_HIP_PHYSICAL_ORDER && order != KQ_HIP_REQUIRE_CANONICAL_ORDER))
        return kq_fail(diag, KQ_STATUS_INVALID_ARGUMENT,
                       "valid tensor view, block range and order are required");
    *out_count = 0u;
    if (v->device_data == NULL || v->bytes_per_block == 0u || v->block_elements == 0u ||
        kq_hip_quant_geometry_for_type(v->type_id, &g, NULL) != KQ_STATUS_OK ||
        g.bytes_per_block != v->bytes_per_block || g.block_elements != v->block_elements)
        return kq_fail(diag, KQ_STATUS_TENSOR_OWNERSHIP_MISMATCH,
                       "tensor view is not live or structurally valid");
    if (order == KQ_HIP_REQUIRE_CANONICAL_ORDER &&
        (v->canonical_contiguous == 0u || v->layout == KQ_HIP_LAYOUT_TRANSFORMED_PHYSICAL ||
         v->layout == KQ_HIP_LAYOUT_SPLIT_SEGMENT))
        return kq_fail(diag, KQ_STATUS_TENSOR_LAYOUT_MISMATCH,
                       "view does not provide canonical-contiguous order");
    if (first > UINT64_MAX - count || (end = first + count) > v->block_count ||
        !u64_mul(first, v->bytes_per_block, &off) || !u64_mul(count, v->bytes_per_block, &bytes) ||
        off > v->mapped_bytes || bytes > v->mapped_bytes - off)
        return kq_fail(diag, KQ_STATUS_SPAN_OUT_OF_RANGE, "requested decode blocks are outside the view");
    src = (const char *)v->device_data + off;
    if (!aligned(src, packed_alignment(v->type_id)) && ctx_ok(c)) {
        /* a span that starts off the decoder's alignment (odd blocks of the
         * 34-, 18- and 210-byte formats) is decoded from an aligned copy */
        hipError_t e;
        st = set_device(c, diag);
        if (st != KQ_STATUS_OK) return st;
        if (c->stage_dev_cap < bytes) {
            if (c->stage_dev) {
                (void)hipStreamSynchronize(c->stream);
                (void)hipFree(c->stage_dev);
                c->stage_dev = NULL;
                c->stage_dev_cap = 0u;
            }
            e = hipMalloc(&c->stage_dev, (size_t)bytes);
            if (e != hipSuccess) return kq_fail(diag, KQ_STATUS_OUT_OF_MEMORY, "view staging: %s",
                                                 hipGetErrorString(e));
            c->stage_dev_cap = bytes;
        }
        e = hipMemcpyAsync(c->stage_dev, src, (size_t)bytes, hipMemcpyDeviceToDevice, c->stream);
        if (e != hipSuccess) return hip_fail(diag, e, "view staging copy");
        src = (const char *)c->stage_dev;
    }
    return kq_hip_dequantize_blocks_f32(c, v->type_id, src, bytes, out, capacity, out_count, diag);
}

/* ------------------------------------------------------------------ */
/* GDN layouts */

#define KQ_GDN_QK_ROWS 4096u     /* 2 x 16 key heads x 128 */
#define KQ_GDN_UNITS 48u         /* 16 key heads x 3 value repeats */

/* rows (or columns) the layout maps onto themselves, its identity prefix
 * and unit width; 0 when the layout moves rows (columns) otherwise */
static int gdn_geometry(uint32_t layout, int columns, uint64_t *n, uint64_t *prefix,
                        uint64_t *width) {
    *prefix = 0u;
    switch (layout) {
    case KQ_HIP_GDN_QKV:
    case KQ_HIP_GDN_CONV: *prefix = KQ_GDN_QK_ROWS; *width = 128u; break;
    case KQ_HIP_GDN_GATE: *width = 128u; break;
    case KQ_HIP_GDN_ALPHA:
    case KQ_HIP_GDN_BETA: *width = 1u; break;
    case KQ_HIP_GDN_OUT: *width = 128u; break;
    default: return 0;
    }
    if ((layout == KQ_HIP_GDN_OUT) != (columns != 0)) return 0;
    *n = *prefix + KQ_GDN_UNITS * *width;
    return 1;
}

static uint64_t grouped_to_tiled(uint64_t c, uint64_t w) {
    const uint64_t group = c / (3u * w), within = c % (3u * w);
    return (within / w * 16u + group) * w + within % w;
}

static kq_status gdn_index(uint32_t layout, int columns, uint64_t n, uint64_t index,
                           uint64_t *out, kq_diagnostic *diag) {
    uint64_t want, prefix, width;
    kq_diagnostic_clear(diag);
    if (out == NULL || layout > KQ_HIP_GDN_OUT)
        return kq_fail(diag, KQ_STATUS_INVALID_ARGUMENT, "a GDN layout and an output are required");
    if (index >= n) return kq_fail(diag, KQ_STATUS_SPAN_OUT_OF_RANGE, "index is outside the matrix");
    if (layout == KQ_HIP_GDN_NONE || !gdn_geometry(layout, columns, &want, &prefix, &width)) {
        *out = index; /* rows of GDN_OUT and columns of the row layouts stay */
        return KQ_STATUS_OK;
    }
    if (n != want)
        return kq_fail(diag, KQ_STATUS_TENSOR_LAYOUT_MISMATCH,
                       "this GDN layout maps %llu %s onto themselves, not %llu",
                       (unsigned long long)want, columns ? "columns" : "rows",
                       (unsigned long long)n);
    *out = index < prefix ? index : prefix + grouped_to_tiled(index - prefix, width);
    return KQ_STATUS_OK;
}

kq_status kq_hip_gdn_physical_row(uint32_t layout, uint64_t rows, uint64_t row, uint64_t *out,
                                  kq_diagnostic *diag) {
    return gdn_index(layout, 0, rows, row, out, diag);
}

kq_status kq_hip_gdn_physical_column(uint32_t layout, uint64_t cols, uint64_t col,
                                     uint64_t *out, kq_diagnostic *diag) {
    return gdn_index(layout, 1, cols, col, out, diag);
}

kq_status kq_hip_gdn_canonicalize(kq_hip_context *c, uint32_t layout, uint32_t type_id,
                                  const void *phys, uint64_t rows, uint64_t cols, void *canon,
                                  uint64_t capacity, kq_diagnostic *diag) {
    uint64_t be, bb, row_bytes, bytes, n, prefix, width, units, unit_bytes;
    const int columns = layout == KQ_HIP_GDN_OUT;
    kq_status st;
    kq_diagnostic_clear(diag);
    if (!ctx_ok(c) || phys == NULL || canon == NULL || rows == 0u || cols == 0u ||
        layout > KQ_HIP_GDN_OUT)
        return kq_fail(diag, KQ_STATUS_INVALID_ARGUMENT,
                       "a GDN layout, both matrices and a non-zero shape are required");
    st = quant_geometry(type_id, &be, &bb, diag);
    if (st != KQ_STATUS_OK) return st;
    if (cols % be != 0u)
        return kq_fail(diag, KQ_STATUS_DIMENSION_MISMATCH, "columns are not whole quant blocks");
    row_bytes = cols / be * bb;
    if (!u64_mul(rows, row_bytes, &bytes))
        return kq_fail(diag, KQ_STATUS_ARITHMETIC_OVERFLOW, "matrix byte count overflows");
    if (layout != KQ_HIP_GDN_NONE) {
        gdn_geometry(layout, columns, &n, &prefix, &width);
        if ((columns ? cols : rows) != n)
            return kq_fail(diag, KQ_STATUS_TENSOR_LAYOUT_MISMATCH,
                           "this GDN layout maps %llu %s onto themselves, not %llu",
                           (unsigned long long)n, columns ? "columns" : "rows",
                           (unsigned long long)(columns ? cols : rows));
        if (columns && 128u % be != 0u)
            return kq_fail(diag, KQ_STATUS_UNSUPPORTED_TENSOR_TYPE,
                           "GDN_OUT moves 128-column units: blocks of at most 128 elements");
    }
    if (capacity < bytes)
        return kq_fail(diag, KQ_STATUS_BUFFER_TOO_SMALL, "the canonical copy needs %llu bytes",
                       (unsigned long long)bytes);
    if (ranges_overlap(phys, bytes, canon, bytes))
        return kq_fail(diag, KQ_STATUS_ALIASING_VIOLATION, "the two matrices overlap");
    if (!aligned(phys, 2u) || !aligned(canon, 2u) || bb % 2u != 0u)
        return kq_fail(diag, KQ_STATUS_INVALID_ALIGNMENT, "matrices must be 2-byte aligned");
    units = columns ? rows * KQ_GDN_UNITS : rows;
    unit_bytes = columns ? 128u / be * bb : row_bytes;
    if (layout != KQ_HIP_GDN_NONE && (units > 0x7fffffffu || unit_bytes > 0x7fffffffu))
        return kq_fail(diag, KQ_STATUS_LIMIT_EXCEEDED, "matrix too large for one gather");
    st = set_device(c, diag);
    if (st == KQ_STATUS_OK) st = snapshot1(c, canon, bytes, diag);
    if (st != KQ_STATUS_OK) return st;
    if (layout == KQ_HIP_GDN_NONE)
        return finish(c, hipMemcpyAsync(canon, phys, (size_t)bytes, hipMemcpyDeviceToDevice,
                                        c->stream), "canonical copy", diag);
    return finish(c, kq_launch_gdn_gather(phys, canon, units, (uint32_t)unit_bytes, columns, prefix,
                                          (uint32_t)width, KQ_GDN_UNITS, c->stream),
                  "GDN gather launch", diag);
}

static kq_status ensure_parts(kq_hip_context *c, uint64_t n, kq_diagnostic *diag) {
    hipError_t e;
    if (n <= c->part_cap) return KQ_STATUS_OK;
    if (c->part_v) {
        (void)hipStreamSynchronize(c->stream);
        (void)hipFree(c->part_v);
        (void)hipFree(c->part_i);
        c->part_v = NULL;
        c->part_i = NULL;
        c->part_cap = 0u;
    }
    e = hipMalloc((void **)&c->part_v, (size_t)n * sizeof(float));
    if (e == hipSuccess) e = hipMalloc((void **)&c->part_i, (size_t)n * sizeof(uint32_t));
    if (e != hipSuccess) return kq_fail(diag, KQ_STATUS_OUT_OF_MEMORY, "argmax partials: %s",
                                        hipGetErrorString(e));
    c->part_cap = n;
    return KQ_STATUS_OK;
}

static kq_status validate_matvec(const kq_hip_context *c, uint32_t type_id, const void *w,
                                 uint64_t rows, uint64_t cols, const float *x, uint32_t batch,
                                 const float *y, uint64_t capacity, kq_diagnostic *diag) {
    uint64_t be, bb, w_bytes, need;
    kq_status st;
    if (!ctx_ok(c) || w == NULL || x == NULL || y == NULL || rows == 0u || cols == 0u ||
        batch == 0u)
        return kq_fail(diag, KQ_STATUS_INVALID_ARGUMENT,
                       "weights, input, output and non-zero shape are required");
    st = quant_geometry(type_id, &be, &bb, diag);
    if (st != KQ_STATUS_OK) return st;
    if (!packed_quant(type_id))
        return kq_fail(diag, KQ_STATUS_UNSUPPORTED_TENSOR_TYPE,
                       "device products take Q5_1, Q8_0, IQ4_NL, Q4_K, Q5_K or Q6_K weights");
    if (cols % be != 0u)
        return kq_fail(diag, KQ_STATUS_DIMENSION_MISMATCH, "columns are not whole quant blocks");
    if (rows > UINT32_MAX || batch > 8u)
        return kq_fail(diag, KQ_STATUS_LIMIT_EXCEEDED, "rows must fit 32 bits and batch be <= 8");
    if (cols > UINT32_MAX || !kq_launch_matvec_supported(type_id, (uint32_t)cols, 1u))
        return kq_fail(diag, KQ_STATUS_LIMIT_EXCEEDED,
                       "device matvec takes rows of at most 65536 columns");
    if (!u64_mul(rows, cols / be * bb, &w_bytes) || !u64_mul(rows, batch, &need))
        return kq_fail(diag, KQ_STATUS_ARITHMETIC_OVERFLOW, "matrix byte count overflows");
    /* the kernels address the matrix through one buffer descriptor, whose
     * byte count is 32-bit */
    if (w_bytes > UINT32_MAX)
        return kq_fail(diag, KQ_STATUS_LIMIT_EXCEEDED, "a matrix must be smaller than 4 GiB");
    if (capacity < need)
        return kq_fail(diag, KQ_STATUS_BUFFER_TOO_SMALL, "output capacity is too small");
    if (ranges_overlap(w, w_bytes, y, need * 4u) ||
        ranges_overlap(x, (uint64_t)batch * cols * 4u, y, need * 4u))
        return kq_fail(diag, KQ_STATUS_ALIASING_VIOLATION, "linear output overlaps an input");
    if (!aligned(w, 16u) || !aligned(x, 16u) || !aligned(y, 4u))
        return kq_fail(diag, KQ_STATUS_INVALID_ALIGNMENT,
                       "weights and input must be 16-byte aligned");
    return KQ_STATUS_OK;
}

/* Enqueue y for up to 8 batch columns, in launches of at most 4. */
static hipError_t enqueue_matvec(kq_hip_context *c, uint32_t type_id, const void *w,
                                 uint64_t rows, uint64_t cols, const float *x, uint32_t batch,
                                 float *y, float *pv, uint32_t *pi, uint32_t nparts) {
    uint32_t done = 0u;
    while (done < batch) {
        uint32_t nb = batch - done > 4u ? 4u : batch - done;
        hipError_t e = kq_launch_matvec(type_id, w, (uint32_t)rows, (uint32_t)cols,
                                        x + (size_t)done * cols, nb, y + (size_t)done * rows,
                                        c->d_status, pv ? pv + (size_t)done * nparts : NULL,
                                        pi ? pi + (size_t)done * nparts : NULL, nparts,
                                        c->stream);
        if (e != hipSuccess) return e;
        done += nb;
    }
    return hipSuccess;
}

kq_status kq_hip_quantized_matvec_f32(kq_hip_context *c, uint32_t type_id, const void *w,
                                      uint64_t rows, uint64_t cols, const float *x,
                                      uint32_t batch, float *y, uint64_t capacity,
                                      kq_diagnostic *diag) {
    kq_status st;
    kq_diagnostic_clear(diag);
    st = validate_matvec(c, type_id, w, rows, cols, x, batch, y, capacity, diag);
    if (st != KQ_STATUS_OK) return st;
    st = set_device(c, diag);
    if (st == KQ_STATUS_OK) st = snapshot1(c, y, rows * batch * 4u, diag);
    if (st != KQ_STATUS_OK) return st;
    return finish(c, enqueue_matvec(c, type_id, w, rows, cols, x, batch, y, NULL, NULL, 0u),
                  "matvec launch", diag);
}

kq_status kq_hip_quantized_row_dot_f32(kq_hip_context *c, uint32_t type_id, const void *packed,
                                       uint64_t packed_bytes, const float *x, uint64_t count,
                                       float *out, kq_diagnostic *diag) {
    uint64_t be, bb;
    kq_status st;
    kq_diagnostic_clear(diag);
    if (!ctx_ok(c) || packed == NULL || x == NULL || out == NULL || packed_bytes == 0u ||
        count == 0u)
        return kq_fail(diag, KQ_STATUS_INVALID_ARGUMENT,
                       "row-dot inputs and scalar output are required");
    st = quant_geometry(type_id, &be, &bb, diag);
    if (st != KQ_STATUS_OK) return st;
    if (packed_bytes % bb != 0u)
        return kq_fail(diag, KQ_STATUS_MALFORMED_QUANTIZED_DATA,
                       "row is not a bounded whole-block span");
    if (packed_bytes / bb * be != count)
        return kq_fail(diag, KQ_STATUS_DIMENSION_MISMATCH,
                       "quantized row and activation lengths differ");
    return kq_hip_quantized_matvec_f32(c, type_id, packed, 1u, count, x, 1u, out, 1u, diag);
}

kq_status kq_hip_greedy_argmax_f32(kq_hip_context *c, const float *logits, uint64_t count,
                                   uint32_t batch, uint32_t *ids, kq_diagnostic *diag) {
    uint32_t parts;
    kq_status st;
    kq_diagnostic_clear(diag);
    if (!ctx_ok(c) || logits == NULL || ids == NULL || count == 0u || count > UINT32_MAX ||
        batch == 0u)
        return kq_fail(diag, KQ_STATUS_INVALID_ARGUMENT,
                       "valid finite logits and selection output are required");
    if (ranges_overlap(logits, count * batch * 4u, ids, (uint64_t)batch * 4u))
        return kq_fail(diag, KQ_STATUS_ALIASING_VIOLATION, "logits and ids overlap");
    if (!aligned(logits, 4u) || !aligned(ids, 4u))
        return kq_fail(diag, KQ_STATUS_INVALID_ALIGNMENT, "buffers must be 4-byte aligned");
    st = set_device(c, diag);
    if (st != KQ_STATUS_OK) return st;
    parts = kq_launch_argmax_parts((uint32_t)count);
    st = ensure_parts(c, (uint64_t)parts * batch, diag);
    if (st == KQ_STATUS_OK) st = snapshot1(c, ids, (uint64_t)batch * 4u, diag);
    if (st != KQ_STATUS_OK) return st;
    return finish(c, kq_launch_argmax(logits, (uint32_t)count, batch, c->part_v, c->part_i, ids,
                                      c->d_status, c->stream),
                  "argmax launch", diag);
}

/* The LM head's validation, partial count and launches. noalloc: the
 * partials live in the device's static array (no allocation, at most
 * kq_launch_noalloc_parts() of them per call); otherwise in the context's
 * partials, grown on demand. */
static kq_status lm_head(kq_hip_context *c, uint32_t type_id, const void *w, uint64_t vocab,
                         uint64_t cols, const float *h, uint32_t batch, float *logits,
                         uint32_t *ids, int noalloc, kq_diagnostic *diag) {
    uint32_t nparts;
    float *pv;
    uint32_t *pi;
    hipError_t e;
    kq_status st;
    kq_diagnostic_clear(diag);
    st = validate_matvec(c, type_id, w, vocab, cols, h, batch, logits, vocab * batch, diag);
    if (st != KQ_STATUS_OK) return st;
    if (ids == NULL) return kq_fail(diag, KQ_STATUS_INVALID_ARGUMENT, "token id output is required");
    if (ranges_overlap(ids, (uint64_t)batch * 4u, logits, vocab * batch * 4u))
        return kq_fail(diag, KQ_STATUS_ALIASING_VIOLATION, "logits and ids overlap");
    st = set_device(c, diag);
    if (st != KQ_STATUS_OK) return st;
    /* partials per batch column: the most any launch of the call uses */
    nparts = 0u;
    for (uint32_t done = 0u; done < batch; done += 4u) {
        const uint32_t nb = batch - done > 4u ? 4u : batch - done;
        const uint32_t w_nb = kq_launch_matvec_waves(type_id, (uint32_t)vocab, (uint32_t)cols, nb);
        if (w_nb > nparts) nparts = w_nb;
    }
    if (nparts == 0u)
        return kq_fail(diag, KQ_STATUS_DEVICE_FAILURE, "lm head: no launch configuration");
    if (noalloc) {
        /* The launch shapes keep every call within the array: one row group
         * per wave only below 4 x 4096 groups (at most 16,384 waves in
         * 512-thread workgroups), resident grids above, so 8 columns need
         * at most 131,072 partials. The check stays as the guard should a
         * launch shape change. */
        const uint64_t cap = kq_launch_noalloc_parts();
        if ((uint64_t)nparts * batch > cap)
            return kq_fail(diag, KQ_STATUS_LIMIT_EXCEEDED,
                           "allocation-free lm head: %llu argmax partials needed, the static "
                           "array holds %llu (use kq_hip_lm_head_greedy_f32)",
                           (unsigned long long)nparts * batch, (unsigned long long)cap);
        if (c->noalloc == NULL)
            return kq_fail(diag, KQ_STATUS_DEVICE_FAILURE, "static partials were not set up");
        pv = (float *)c->noalloc;
        pi = (uint32_t *)((char *)c->noalloc + cap * sizeof(float));
    } else {
        void *const outs[2] = {logits, ids};
        const uint64_t lens[2] = {vocab * batch * 4u, (uint64_t)batch * 4u};
        st = ensure_parts(c, (uint64_t)nparts * batch, diag);
        if (st == KQ_STATUS_OK) st = snapshot(c, 2u, outs, lens, diag);
        if (st != KQ_STATUS_OK) return st;
        pv = c->part_v;
        pi = c->part_i;
    }
    e = enqueue_matvec(c, type_id, w, vocab, cols, h, batch, logits, pv, pi, nparts);
    if (e == hipSuccess) e = kq_launch_argmax_from_parts(pv, pi, nparts, batch, ids, c->stream);
    return finish(c, e, "lm head launch", diag);
}

kq_status kqi_enqueue_logits(kq_hip_context *c, uint32_t type_id, const void *w, uint64_t vocab,
                             uint64_t cols, const float *h, float *logits, kq_diagnostic *diag) {
    kq_status st = validate_matvec(c, type_id, w, vocab, cols, h, 1u, logits, vocab, diag);
    if (st != KQ_STATUS_OK) return st;
    st = set_device(c, diag);
    if (st != KQ_STATUS_OK) return st;
    hipError_t e = enqueue_matvec(c, type_id, w, vocab, cols, h, 1u, logits, NULL, NULL, 0u);
    return e == hipSuccess ? KQ_STATUS_OK : hip_fail(diag, e, "lm head launch");
}

kq_status kq_hip_lm_head_greedy_f32(kq_hip_context *c, uint32_t type_id, const void *w,
                                    uint64_t vocab, uint64_t cols, const float *h,
                                    uint32_t batch, float *logits, uint32_t *ids,
                                    kq_diagnostic *diag) {
    return lm_head(c, type_id, w, vocab, cols, h, batch, logits, ids, 0, diag);
}

kq_status kq_hip_lm_head_greedy_f32_noalloc(kq_hip_context *c, uint32_t type_id, const void *w,
                                            uint64_t vocab, uint64_t cols, const float *h,
                                            uint32_t batch, float *logits, uint32_t *ids,
                                            kq_diagnostic *diag) {
    return lm_head(c, type_id, w, vocab, cols, h, batch, logits, ids, 1, diag);
}

kq_status kq_hip_f32_expf(kq_hip_context *c, const float *in, uint64_t n, float *out,
                          kq_diagnostic *diag) {
    kq_status st;
    kq_diagnostic_clear(diag);
    if (!ctx_ok(c) || in == NULL || out == NULL || n == 0u)
        return kq_fail(diag, KQ_STATUS_INVALID_ARGUMENT, "input and output are required");
    if (ranges_overlap(in, n * 4u, out, n * 4u) && in != out)
        return kq_fail(diag, KQ_STATUS_ALIASING_VIOLATION, "input and output overlap");
    st = set_device(c, diag);
    if (st == KQ_STATUS_OK) st = snapshot1(c, out, n * 4u, diag);
    if (st != KQ_STATUS_OK) return st;
    return finish(c, kq_launch_expf(in, n, out, c->stream), "expf launch", diag);
}

/* ------------------------------------------------------------------ */
/* MoE */

static int moe_ok(const kq_hip_moe_config *cfg) {
    return cfg != NULL && cfg->magic == KQ_MOE_CONFIG_MAGIC;
}

static kq_launch_moe_dims launch_dims(const kq_hip_moe_config *cfg) {
    kq_launch_moe_dims d;
    d.hidden = cfg->dims.hidden_size;
    d.experts = cfg->dims.expert_count;
    d.top_k = cfg->dims.top_k;
    d.inter = cfg->dims.routed_intermediate_size;
    d.shared_inter = cfg->dims.shared_intermediate_size;
    return d;
}

kq_status kq_hip_moe_config_create(const kq_hip_moe_dimensions *dims, kq_hip_moe_config **out,
                                   kq_diagnostic *diag) {
    kq_hip_moe_config *cfg;
    kq_launch_moe_dims d;
    kq_diagnostic_clear(diag);
    if (dims == NULL || out == NULL)
        return kq_fail(diag, KQ_STATUS_INVALID_ARGUMENT, "MoE dimensions and output are required");
    *out = NULL;
    if (dims->hidden_size == 0u || dims->expert_count == 0u || dims->top_k == 0u ||
        dims->top_k > dims->expert_count || dims->routed_intermediate_size == 0u ||
        dims->shared_intermediate_size == 0u)
        return kq_fail(diag, KQ_STATUS_INCOMPATIBLE_MOE, "invalid MoE dimensions, top-k, or dtype");
    d.hidden = dims->hidden_size;
    d.experts = dims->expert_count;
    d.top_k = dims->top_k;
    d.inter = dims->routed_intermediate_size;
    d.shared_inter = dims->shared_intermediate_size;
    if (d.experts + 1u > 1024u || d.top_k > 64u)
        return kq_fail(diag, KQ_STATUS_LIMIT_EXCEEDED,
                       "device MoE takes at most 1023 experts and top_k <= 64");
    cfg = (kq_hip_moe_config *)calloc(1, sizeof(*cfg));
    if (cfg == NULL) return kq_fail(diag, KQ_STATUS_OUT_OF_MEMORY, "MoE config allocation failed");
    cfg->magic = KQ_MOE_CONFIG_MAGIC;
    cfg->dims = *dims;
    *out = cfg;
    return KQ_STATUS_OK;
}

void kq_hip_moe_config_close(kq_hip_moe_config *cfg) {
    if (cfg == NULL) return;
    cfg->magic = 0u;
    free(cfg);
}

uint64_t kq_hip_moe_config_scratch_bytes(const kq_hip_moe_config *cfg, uint64_t tokens) {
    kq_launch_moe_dims d;
    if (!moe_ok(cfg) || tokens == 0u || tokens > UINT32_MAX) return 0u;
    d = launch_dims(cfg);
    return kq_launch_moe_ws_bytes(&d, (uint32_t)tokens);
}

#define KQ_MOE_MAX_TOKENS 65536u
/* token count from which the layer runs as grouped expert GEMMs */
#define KQ_GROUPED_MIN_TOKENS 2u

static kq_status moe_common(const kq_hip_context *c, const kq_hip_moe_config *cfg,
                            const float *router, const float *sgw, const float *hidden,
                            uint64_t tokens, void *scratch, uint64_t scratch_bytes,
                            kq_diagnostic *diag) {
    kq_launch_moe_dims d;
    if (!ctx_ok(c) || !moe_ok(cfg) || router == NULL || sgw == NULL || hidden == NULL ||
        scratch == NULL)
        return kq_fail(diag, KQ_STATUS_INVALID_ARGUMENT, "complete MoE arguments are required");
    if (tokens == 0u || tokens > KQ_MOE_MAX_TOKENS)
        return kq_fail(diag, KQ_STATUS_LIMIT_EXCEEDED, "MoE token count is zero or above %u",
                       KQ_MOE_MAX_TOKENS);
    d = launch_dims(cfg);
    if (!kq_launch_moe_supported(&d, NULL))
        return kq_fail(diag, KQ_STATUS_LIMIT_EXCEEDED,
                       "the packed-weight MoE and the route need hidden %% 4 == 0 "
                       "(kq_hip_moe_execute_f32 takes any hidden size)");
    if (scratch_bytes < kq_launch_moe_ws_bytes(&d, (uint32_t)tokens))
        return kq_fail(diag, KQ_STATUS_BUFFER_TOO_SMALL, "MoE device scratch is too small");
    if (!aligned(router, 16u) || !aligned(sgw, 16u) || !aligned(hidden, 16u) ||
        !aligned(scratch, 256u))
        return kq_fail(diag, KQ_STATUS_INVALID_ALIGNMENT,
                       "MoE weights/input need 16-byte and scratch 256-byte alignment");
    if (ranges_overlap(hidden, tokens * d.hidden * 4u, scratch, scratch_bytes))
        return kq_fail(diag, KQ_STATUS_ALIASING_VIOLATION, "MoE input and scratch overlap");
    return KQ_STATUS_OK;
}

kq_status kq_hip_moe_route_f32(kq_hip_context *c, const kq_hip_moe_config *cfg,
                               const float *router, uint64_t router_count, const float *sgw,
                               const float *hidden, uint64_t tokens, float *logits,
                               uint64_t logits_cap, float *probs, uint64_t probs_cap,
                               uint32_t *ids, uint64_t ids_cap, float *weights,
                               uint64_t weights_cap, void *scratch, uint64_t scratch_bytes,
                               kq_diagnostic *diag) {
    kq_launch_moe_dims d;
    kq_launch_moe_ws ws;
    uint64_t need_e, need_k, eb, kb, rb;
    hipError_t e;
    kq_status st;
    kq_diagnostic_clear(diag);
    /* the reference's order of checks (src/kq_moe_qwen38.c:293-349):
     * arguments, shape, output capacities, overlaps */
    if (logits == NULL || probs == NULL || ids == NULL || weights == NULL)
        return kq_fail(diag, KQ_STATUS_INVALID_ARGUMENT, "complete MoE route arguments are required");
    st = moe_common(c, cfg, router, sgw, hidden, tokens, scratch, scratch_bytes, diag);
    if (st != KQ_STATUS_OK) return st;
    d = launch_dims(cfg);
    if (router_count != (uint64_t)d.experts * d.hidden)
        return kq_fail(diag, KQ_STATUS_DIMENSION_MISMATCH,
                       "MoE router weight shape mismatch: %llu values for %u x %u",
                       (unsigned long long)router_count, d.experts, d.hidden);
    need_e = tokens * d.experts;
    need_k = tokens * d.top_k;
    if (logits_cap < need_e || probs_cap < need_e || ids_cap < need_k || weights_cap < need_k)
        return kq_fail(diag, KQ_STATUS_BUFFER_TOO_SMALL,
                       "MoE route output capacity is too small: logits and probabilities need "
                       "%llu values, ids and weights %llu",
                       (unsigned long long)need_e, (unsigned long long)need_k);
    eb = need_e * 4u;
    kb = need_k * 4u;
    rb = router_count * 4u;
    {
        const void *outs[4] = {logits, probs, ids, weights};
        const uint64_t lens[4] = {eb, eb, kb, kb};
        for (int i = 0; i < 4; ++i) {
            int bad = ranges_overlap(router, rb, outs[i], lens[i]) ||
                      ranges_overlap(hidden, tokens * d.hidden * 4u, outs[i], lens[i]) ||
                      ranges_overlap(sgw, (uint64_t)d.hidden * 4u, outs[i], lens[i]) ||
                      ranges_overlap(scratch, scratch_bytes, outs[i], lens[i]);
            for (int j = i + 1; j < 4; ++j) bad |= ranges_overlap(outs[i], lens[i], outs[j], lens[j]);
            if (bad)
                return kq_fail(diag, KQ_STATUS_ALIASING_VIOLATION,
                               "MoE route inputs and outputs must not overlap");
        }
    }
    kq_launch_moe_ws_carve(&d, (uint32_t)tokens, scratch, &ws);
    st = set_device(c, diag);
    if (st != KQ_STATUS_OK) return st;
    /* the results land in scratch; the outputs are written from there, in a
     * synchronous call only once the device reported success (the
     * reference's commit-on-success) */
    e = kq_launch_moe_route(&d, router, sgw, hidden, (uint32_t)tokens, &ws, c->d_status, 0, NULL,
                            NULL, c->stream);
    if (!c->async) {
        st = finish(c, e, "MoE route launch", diag);
        if (st != KQ_STATUS_OK) return st;
    } else if (e != hipSuccess) {
        return hip_fail(diag, e, "MoE route launch");
    }
    e = hipMemcpyAsync(logits, ws.logits, eb, hipMemcpyDeviceToDevice, c->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(probs, ws.probs, eb, hipMemcpyDeviceToDevice, c->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(ids, ws.ids, kb, hipMemcpyDeviceToDevice, c->stream);
    if (e == hipSuccess)
        e = hipMemcpyAsync(weights, ws.weights, kb, hipMemcpyDeviceToDevice, c->stream);
    return finish(c, e, "MoE route copy", diag);
}

/* kq_moe_execute_routed_expert_f32 (src/kq_moe_qwen38.c:461-566): gate,
 * up, activated and the expert's output in scratch, the output copied to
 * the caller's buffer on success */
uint64_t kq_hip_moe_config_one_expert_scratch_bytes(const kq_hip_moe_config *cfg) {
    if (!moe_ok(cfg)) return 0u;
    return 3u * align256((uint64_t)cfg->dims.routed_intermediate_size * 4u) +
           align256((uint64_t)cfg->dims.hidden_size * 4u);
}

kq_status kq_hip_moe_execute_routed_expert_f32(kq_hip_context *c, const kq_hip_moe_config *cfg,
                                               const kq_hip_moe_routed_expert_weights_f32 *w,
                                               uint32_t expert_id, const float *hidden,
                                               float *out, uint64_t capacity, void *scratch,
                                               uint64_t scratch_bytes, kq_diagnostic *diag) {
    uint64_t H, I, member, hb, ib;
    float *gate, *up, *act, *tmp;
    hipError_t e;
    kq_status st;
    kq_diagnostic_clear(diag);
    if (!ctx_ok(c) || !moe_ok(cfg) || w == NULL || hidden == NULL || out == NULL ||
        scratch == NULL)
        return kq_fail(diag, KQ_STATUS_INVALID_ARGUMENT, "complete routed-expert arguments are required");
    H = cfg->dims.hidden_size;
    I = cfg->dims.routed_intermediate_size;
    if (expert_id >= cfg->dims.expert_count)
        return kq_fail(diag, KQ_STATUS_INVALID_ARGUMENT, "routed expert ID is out of range");
    if (capacity < H || scratch_bytes < kq_hip_moe_config_one_expert_scratch_bytes(cfg) ||
        !aligned(scratch, 4u))
        return kq_fail(diag, KQ_STATUS_BUFFER_TOO_SMALL,
                       "routed expert output or scratch is too small (output %llu values, scratch "
                       "%llu bytes)",
                       (unsigned long long)H,
                       (unsigned long long)kq_hip_moe_config_one_expert_scratch_bytes(cfg));
    if (H > UINT32_MAX / 4u || I > UINT32_MAX / 4u || !u64_mul(H, I, &member))
        return kq_fail(diag, KQ_STATUS_ARITHMETIC_OVERFLOW, "routed expert member geometry overflows");
    if (w->gate == NULL || w->up == NULL || w->down == NULL || w->gate_count != member ||
        w->up_count != member || w->down_count != member)
        return kq_fail(diag, KQ_STATUS_DIMENSION_MISMATCH,
                       "MoE routed member gate/up/down shape mismatch: %llu values each",
                       (unsigned long long)member);
    if (!aligned(hidden, 4u) || !aligned(out, 4u) || !aligned(w->gate, 4u) ||
        !aligned(w->up, 4u) || !aligned(w->down, 4u))
        return kq_fail(diag, KQ_STATUS_INVALID_ALIGNMENT, "routed expert buffers need 4-byte alignment");
    hb = H * 4u;
    if (ranges_overlap(hidden, hb, out, hb) || ranges_overlap(hidden, hb, scratch, scratch_bytes) ||
        ranges_overlap(out, hb, scratch, scratch_bytes))
        return kq_fail(diag, KQ_STATUS_ALIASING_VIOLATION, "routed expert buffers must not overlap");
    {
        const void *wp[3] = {w->gate, w->up, w->down};
        for (int i = 0; i < 3; ++i)
            if (ranges_overlap(wp[i], member * 4u, out, hb) ||
                ranges_overlap(wp[i], member * 4u, scratch, scratch_bytes))
                return kq_fail(diag, KQ_STATUS_ALIASING_VIOLATION,
                               "MoE weights must not overlap writable expert buffers");
    }
    ib = align256(I * 4u);
    gate = (float *)scratch;
    up = (float *)((char *)scratch + ib);
    act = (float *)((char *)scratch + 2u * ib);
    tmp = (float *)((char *)scratch + 3u * ib);
    st = set_device(c, diag);
    if (st != KQ_STATUS_OK) return st;
    /* the reference validates gate, up, down, then the input, for finiteness */
    e = kq_launch_f32_scan(w->gate, member, c->d_status, c->stream);
    if (e == hipSuccess) e = kq_launch_f32_scan(w->up, member, c->d_status, c->stream);
    if (e == hipSuccess) e = kq_launch_f32_scan(w->down, member, c->d_status, c->stream);
    if (e == hipSuccess) e = kq_launch_f32_scan(hidden, H, c->d_status, c->stream);
    if (e == hipSuccess)
        e = kq_launch_routed_expert_f32(w->gate, w->up, w->down, hidden, (uint32_t)H,
                                        (uint32_t)I, gate, up, act, tmp, c->d_status, c->stream);
    if (!c->async) {
        st = finish(c, e, "routed expert launch", diag);
        if (st != KQ_STATUS_OK) return st;
    } else if (e != hipSuccess) {
        return hip_fail(diag, e, "routed expert launch");
    }
    return finish(c, hipMemcpyAsync(out, tmp, hb, hipMemcpyDeviceToDevice, c->stream),
                  "routed expert copy", diag);
}

kq_status kq_hip_moe_execute_quantized(kq_hip_context *c, const kq_hip_moe_config *cfg,
                                       const kq_hip_moe_weights *w, const float *hidden,
                                       uint64_t tokens, float *out, uint64_t capacity,
                                       uint32_t *ids, void *scratch, uint64_t scratch_bytes,
                                       kq_diagnostic *diag) {
    kq_launch_moe_dims d;
    kq_launch_moe_weights lw;
    kq_launch_moe_ws ws;
    hipError_t e;
    kq_status st;
    int grouped;
    void *stage;
    kq_diagnostic_clear(diag);
    if (w == NULL || out == NULL)
        return kq_fail(diag, KQ_STATUS_INVALID_ARGUMENT, "complete MoE execution arguments are required");
    st = moe_common(c, cfg, w->router, w->shared_gate_weight, hidden, tokens, scratch,
                    scratch_bytes, diag);
    if (st != KQ_STATUS_OK) return st;
    d = launch_dims(cfg);
    if (w->routed_gate == NULL || w->routed_up == NULL || w->routed_down == NULL ||
        w->shared_gate == NULL || w->shared_up == NULL || w->shared_down == NULL)
        return kq_fail(diag, KQ_STATUS_INVALID_ARGUMENT, "every MoE weight role is required");
    if (capacity < tokens * d.hidden)
        return kq_fail(diag, KQ_STATUS_BUFFER_TOO_SMALL, "MoE output or aligned scratch is too small");
    if (ranges_overlap(hidden, tokens * d.hidden * 4u, out, tokens * d.hidden * 4u) ||
        ranges_overlap(out, tokens * d.hidden * 4u, scratch, scratch_bytes))
        return kq_fail(diag, KQ_STATUS_ALIASING_VIOLATION,
                       "MoE input, output, and scratch must not overlap");
    if (ids != NULL) {
        const uint64_t ib = tokens * d.top_k * 4u;
        if (!aligned(ids, 4u))
            return kq_fail(diag, KQ_STATUS_INVALID_ALIGNMENT, "selected ids need 4-byte alignment");
        if (ranges_overlap(ids, ib, hidden, tokens * d.hidden * 4u) ||
            ranges_overlap(ids, ib, out, tokens * d.hidden * 4u) ||
            ranges_overlap(ids, ib, scratch, scratch_bytes))
            return kq_fail(diag, KQ_STATUS_ALIASING_VIOLATION,
                           "selected ids overlap the MoE input, output or scratch");
    }
    lw.router = w->router;
    lw.gate_type = w->routed_gate_type;
    lw.gate = w->routed_gate;
    lw.up_type = w->routed_up_type;
    lw.up = w->routed_up;
    lw.down_type = w->routed_down_type;
    lw.down = w->routed_down;
    lw.shared_gate_type = w->shared_gate_type;
    lw.shared_gate = w->shared_gate;
    lw.shared_up_type = w->shared_up_type;
    lw.shared_up = w->shared_up;
    lw.shared_down_type = w->shared_down_type;
    lw.shared_down = w->shared_down;
    lw.shared_gate_weight = w->shared_gate_weight;
    if (!kq_launch_moe_supported(&d, &lw))
        return kq_fail(diag, KQ_STATUS_UNSUPPORTED_TENSOR_TYPE,
                       "device MoE needs Q5_1/Q8_0/IQ4_NL/Q4_K/Q5_K/Q6_K roles (gate and up of one "
                       "type, routed and shared each), rows of whole blocks of every type that "
                       "reads them, equal intermediates");
    if (!aligned(w->routed_gate, 16u) || !aligned(w->routed_up, 16u) ||
        !aligned(w->routed_down, 16u) || !aligned(w->shared_gate, 16u) ||
        !aligned(w->shared_up, 16u) || !aligned(w->shared_down, 16u) || !aligned(out, 16u))
        return kq_fail(diag, KQ_STATUS_INVALID_ALIGNMENT,
                       "MoE weights and output must be 16-byte aligned");
    kq_launch_moe_ws_carve(&d, (uint32_t)tokens, scratch, &ws);
    st = set_device(c, diag);
    if (st == KQ_STATUS_OK) {
        void *const outs[2] = {out, ids};
        const uint64_t lens[2] = {tokens * d.hidden * 4u, tokens * d.top_k * 4u};
        st = snapshot(c, 2u, outs, lens, diag);
    }
    if (st != KQ_STATUS_OK) return st;
    /* several tokens: each expert's weights stream once for all of its
     * tokens (grouped MFMA path), whose activation split the route finish
     * forms; one token: the fused decode kernels */
    grouped = tokens >= KQ_GROUPED_MIN_TOKENS && kq_launch_moe_grouped_supported(&d, &lw);
    stage = grouped ? kq_launch_moe_grouped_stage(&d, &lw, &ws) : NULL;
    /* the layer needs the CPU's expert ids exactly and its weights to fp32
     * tolerance: one token may take the certified routing */
    e = kq_launch_moe_route(&d, w->router, w->shared_gate_weight, hidden, (uint32_t)tokens, &ws,
                            c->d_status, 1, tokens == 1u ? ids : NULL, stage, c->stream);
    if (e == hipSuccess && grouped)
        e = kq_launch_moe_grouped(&d, &lw, hidden, (uint32_t)tokens, &ws, stage != NULL, out,
                                  c->d_status, c->stream);
    else if (e == hipSuccess)
        e = kq_launch_moe_experts(&d, &lw, hidden, (uint32_t)tokens, &ws, out, c->d_status,
                                  c->stream);
    /* one token: the route kernel wrote the caller's ids itself */
    if (e == hipSuccess && ids != NULL && tokens > 1u)
        e = hipMemcpyAsync(ids, ws.ids, tokens * d.top_k * 4u, hipMemcpyDeviceToDevice, c->stream);
    return finish(c, e, "MoE execute launch", diag);
}

/* ------------------------------------------------------------------ */
/* MoE on F32 weights (kq_moe_f32.hip) */

#define KQ_F32_MOE_MAX_TOKENS 65535u

static void f32_ws_carve(const kq_launch_moe_dims *d, uint64_t t, void *base,
                         kq_launch_moe_f32_ws *ws, uint64_t *bytes) {
    const uint64_t ip = d->inter > d->shared_inter ? d->inter : d->shared_inter;
    const uint64_t slots = t * (d->top_k + 1u);
    uint8_t *p = (uint8_t *)base;
    uint64_t off = 0u;
#define TAKE(field, type, n)                                  \
    do {                                                      \
        if (ws) ws->field = (type *)(void *)(p + off);        \
        off += align256((uint64_t)(n) * 4u);                  \
    } while (0)
    TAKE(logits, float, t * d->experts);
    TAKE(probs, float, t * d->experts);
    TAKE(ids, uint32_t, t * d->top_k);
    TAKE(order, uint32_t, t * d->top_k);
    TAKE(weights, float, t * d->top_k);
    TAKE(shared_logit, float, t);
    TAKE(shared_scale, float, t);
    TAKE(gate, float, slots * ip);
    TAKE(up, float, slots * ip);
    TAKE(act, float, slots * ip);
    TAKE(out, float, slots * d->hidden);
    TAKE(weighted, float, slots * d->hidden);
    TAKE(routed_sum, float, t * d->hidden);
#undef TAKE
    if (bytes) *bytes = off;
}

uint64_t kq_hip_moe_config_f32_scratch_bytes(const kq_hip_moe_config *cfg, uint64_t tokens) {
    kq_launch_moe_dims d;
    uint64_t n = 0u;
    if (!moe_ok(cfg) || tokens == 0u || tokens > KQ_F32_MOE_MAX_TOKENS) return 0u;
    d = launch_dims(cfg);
    f32_ws_carve(&d, tokens, NULL, NULL, &n);
    return n;
}

/* the reference's count check per role (src/kq_moe_qwen38.c:82-126) */
static kq_status f32_weight_counts(const kq_launch_moe_dims *d, const kq_hip_moe_weights_f32 *w,
                                   kq_diagnostic *diag) {
    const uint64_t routed = (uint64_t)d->inter * d->hidden * d->experts;
    const uint64_t shared = (uint64_t)d->shared_inter * d->hidden;
    const struct {
        const float *p;
        uint64_t have, want;
        const char *what;
    } roles[8] = {
        {w->router, w->router_count, (uint64_t)d->experts * d->hidden, "MoE router shape/data mismatch"},
        {w->routed_gate, w->routed_gate_count, routed, "MoE routed gate shape/data mismatch"},
        {w->routed_up, w->routed_up_count, routed, "MoE routed up shape/data mismatch"},
        {w->routed_down, w->routed_down_count, routed, "MoE routed down shape/data mismatch"},
        {w->shared_gate, w->shared_gate_count, shared, "MoE shared gate shape/data mismatch"},
        {w->shared_up, w->shared_up_count, shared, "MoE shared up shape/data mismatch"},
        {w->shared_down, w->shared_down_count, shared, "MoE shared down shape/data mismatch"},
        {w->shared_gate_weight, w->shared_gate_weight_count, d->hidden,
         "MoE shared scale gate shape/data mismatch"}};
    for (int i = 0; i < 8; ++i) {
        if (roles[i].p == NULL) return kq_fail(diag, KQ_STATUS_INVALID_ARGUMENT, "%s", roles[i].what);
        if (roles[i].have != roles[i].want)
            return kq_fail(diag, KQ_STATUS_DIMENSION_MISMATCH, "%s", roles[i].what);
    }
    return KQ_STATUS_OK;
}

static void emit(kq_hip_moe_checkpoint_observer obs, void *user, kq_hip_moe_checkpoint_kind kind,
                 uint64_t token, uint32_t expert, uint32_t pos, const float *v, uint64_t n) {
    kq_hip_moe_checkpoint c;
    memset(&c, 0, sizeof(c));
    c.kind = kind;
    c.token_index = token;
    c.expert_id = expert;
    c.top_k_position = pos;
    c.rank = 1u;
    c.dimensions[0] = n;
    c.values = v;
    c.value_count = n;
    obs(&c, user);
}

/* The observers, in the reference's order (src/kq_moe_qwen38.c:697-863),
 * over host copies of the device trace. */
static kq_status f32_observe(kq_hip_context *c, const kq_launch_moe_dims *d, uint64_t T,
                             const kq_launch_moe_f32_ws *ws, const float *y,
                             kq_hip_moe_route_observer ro, kq_hip_moe_checkpoint_observer co,
                             void *user, kq_diagnostic *diag) {
    const uint64_t E = d->experts, K = d->top_k, H = d->hidden, ip =
        d->inter > d->shared_inter ? d->inter : d->shared_inter;
    const uint64_t slots = T * (K + 1u);
    /* logits, probs [T][E]; weights, ids, order [T][K]; shared logit and
     * scale [T]; routed sum and output [T][H]; gate, up, act [slots][ip];
     * out, weighted [slots][H] */
    const uint64_t n = T * (2u * E + 3u * K + 2u + 2u * H) + slots * (3u * ip + 2u * H);
    float *h = (float *)malloc(n * 4u);
    kq_status st = KQ_STATUS_OK;
    if (h == NULL) return kq_fail(diag, KQ_STATUS_OUT_OF_MEMORY, "observer copies: out of memory");
    float *logits = h, *probs = logits + T * E, *wts = probs + T * E;
    uint32_t *ids = (uint32_t *)(wts + T * K), *order = ids + T * K;
    float *sl = (float *)(order + T * K), *ss = sl + T, *gate = ss + T, *up = gate + slots * ip;
    float *act = up + slots * ip, *out = act + slots * ip, *wo = out + slots * H;
    float *rsum = wo + slots * H, *yh = rsum + T * H;
    const struct {
        void *dst;
        const void *src;
        uint64_t n;
    } cp[] = {{logits, ws->logits, T * E}, {probs, ws->probs, T * E}, {wts, ws->weights, T * K},
              {ids, ws->ids, T * K},       {order, ws->order, T * K}, {sl, ws->shared_logit, T},
              {ss, ws->shared_scale, T},   {gate, ws->gate, slots * ip}, {up, ws->up, slots * ip},
              {act, ws->act, slots * ip},  {out, ws->out, slots * H}, {wo, ws->weighted, slots * H},
              {rsum, ws->routed_sum, T * H}, {yh, y, T * H}};
    for (size_t i = 0; i < sizeof(cp) / sizeof(cp[0]) && st == KQ_STATUS_OK; ++i)
        st = kq_hip_download(c, cp[i].dst, cp[i].src, cp[i].n * 4u, diag);
    for (uint64_t t = 0; t < T && st == KQ_STATUS_OK; ++t) {
        const float *lt = logits + t * E, *pt = probs + t * E, *wt = wts + t * K;
        const uint32_t *it = ids + t * K;
        if (ro != NULL) {
            kq_hip_moe_route r;
            r.token_index = t;
            r.router_logits = lt;
            r.router_probabilities = pt;
            r.expert_count = E;
            r.selected_expert_ids = it;
            r.selected_weights = wt;
            r.selected_count = (uint32_t)K;
            ro(&r, user);
        }
        if (co == NULL) continue;
        emit(co, user, KQ_HIP_MOE_CHECKPOINT_ROUTER_LOGITS, t, KQ_HIP_MOE_NO_EXPERT, UINT32_MAX, lt, E);
        emit(co, user, KQ_HIP_MOE_CHECKPOINT_ROUTER_PROBABILITIES, t, KQ_HIP_MOE_NO_EXPERT,
             UINT32_MAX, pt, E);
        emit(co, user, KQ_HIP_MOE_CHECKPOINT_SELECTED_WEIGHTS, t, KQ_HIP_MOE_NO_EXPERT, UINT32_MAX,
             wt, K);
        /* experts in ascending id: order[j] is the top-k position of the
         * j-th smallest selected id */
        for (uint64_t j = 0; j < K; ++j) {
            const uint32_t k = order[t * K + j];
            const uint64_t sl_i = t * (K + 1u) + k;
            const uint32_t e = it[k];
            emit(co, user, KQ_HIP_MOE_CHECKPOINT_ROUTED_GATE, t, e, k, gate + sl_i * ip, d->inter);
            emit(co, user, KQ_HIP_MOE_CHECKPOINT_ROUTED_UP, t, e, k, up + sl_i * ip, d->inter);
            emit(co, user, KQ_HIP_MOE_CHECKPOINT_ROUTED_ACTIVATED, t, e, k, act + sl_i * ip,
                 d->inter);
            emit(co, user, KQ_HIP_MOE_CHECKPOINT_ROUTED_EXPERT_OUTPUT, t, e, k, out + sl_i * H, H);
            emit(co, user, KQ_HIP_MOE_CHECKPOINT_ROUTED_WEIGHTED_OUTPUT, t, e, k, wo + sl_i * H, H);
        }
        const uint64_t sh = t * (K + 1u) + K;
        emit(co, user, KQ_HIP_MOE_CHECKPOINT_ROUTED_WEIGHTED_SUM, t, KQ_HIP_MOE_NO_EXPERT,
             UINT32_MAX, rsum + t * H, H);
        emit(co, user, KQ_HIP_MOE_CHECKPOINT_SHARED_GATE_PROJECTION, t, KQ_HIP_MOE_NO_EXPERT,
             UINT32_MAX, gate + sh * ip, d->shared_inter);
        emit(co, user, KQ_HIP_MOE_CHECKPOINT_SHARED_UP_PROJECTION, t, KQ_HIP_MOE_NO_EXPERT,
             UINT32_MAX, up + sh * ip, d->shared_inter);
        emit(co, user, KQ_HIP_MOE_CHECKPOINT_SHARED_ACTIVATED, t, KQ_HIP_MOE_NO_EXPERT, UINT32_MAX,
             act + sh * ip, d->shared_inter);
        emit(co, user, KQ_HIP_MOE_CHECKPOINT_SHARED_OUTPUT, t, KQ_HIP_MOE_NO_EXPERT, UINT32_MAX,
             out + sh * H, H);
        emit(co, user, KQ_HIP_MOE_CHECKPOINT_SHARED_SCALE_LOGIT, t, KQ_HIP_MOE_NO_EXPERT,
             UINT32_MAX, sl + t, 1u);
        emit(co, user, KQ_HIP_MOE_CHECKPOINT_SHARED_SCALE, t, KQ_HIP_MOE_NO_EXPERT, UINT32_MAX,
             ss + t, 1u);
        emit(co, user, KQ_HIP_MOE_CHECKPOINT_GATED_SHARED_OUTPUT, t, KQ_HIP_MOE_NO_EXPERT,
             UINT32_MAX, wo + sh * H, H);
        emit(co, user, KQ_HIP_MOE_CHECKPOINT_OPERATOR_OUTPUT, t, KQ_HIP_MOE_NO_EXPERT, UINT32_MAX,
             yh + t * H, H);
    }
    free(h);
    return st;
}

kq_status kq_hip_moe_execute_f32(kq_hip_context *c, const kq_hip_moe_config *cfg,
                                 const kq_hip_moe_weights_f32 *w, const float *hidden,
                                 uint64_t tokens, float *out, uint64_t capacity, void *scratch,
                                 uint64_t scratch_bytes, kq_hip_moe_route_observer ro,
                                 kq_hip_moe_checkpoint_observer co, void *user,
                                 kq_diagnostic *diag) {
    kq_launch_moe_dims d;
    kq_launch_moe_f32_ws ws;
    kq_launch_moe_f32_weights lw;
    uint64_t need = 0u, vals, vbytes;
    hipError_t e;
    kq_status st;
    kq_diagnostic_clear(diag);
    if (!ctx_ok(c) || !moe_ok(cfg) || w == NULL || hidden == NULL || out == NULL ||
        scratch == NULL)
        return kq_fail(diag, KQ_STATUS_INVALID_ARGUMENT, "complete MoE execution arguments are required");
    d = launch_dims(cfg);
    if (tokens == 0u || tokens > KQ_F32_MOE_MAX_TOKENS || !u64_mul(tokens, d.hidden, &vals) ||
        !u64_mul(vals, 4u, &vbytes))
        return kq_fail(diag, KQ_STATUS_LIMIT_EXCEEDED,
                       "MoE token count is zero, above 65,535 or overflows");
    if (d.experts > 960u)
        return kq_fail(diag, KQ_STATUS_LIMIT_EXCEEDED, "F32 MoE execution takes at most 960 experts");
    f32_ws_carve(&d, tokens, NULL, NULL, &need);
    if (capacity < vals || scratch_bytes < need || !aligned(scratch, 256u))
        return kq_fail(diag, KQ_STATUS_BUFFER_TOO_SMALL, "MoE output or aligned scratch is too small");
    st = f32_weight_counts(&d, w, diag);
    if (st != KQ_STATUS_OK) return st;
    if (!aligned(hidden, 4u) || !aligned(out, 4u))
        return kq_fail(diag, KQ_STATUS_INVALID_ALIGNMENT, "MoE input and output need 4-byte alignment");
    if (ranges_overlap(hidden, vbytes, out, vbytes) ||
        ranges_overlap(hidden, vbytes, scratch, scratch_bytes) ||
        ranges_overlap(out, vbytes, scratch, scratch_bytes))
        return kq_fail(diag, KQ_STATUS_ALIASING_VIOLATION,
                       "MoE input, output, and scratch must not overlap");
    {
        const float *wp[8] = {w->router, w->routed_gate, w->routed_up, w->routed_down,
                              w->shared_gate, w->shared_up, w->shared_down, w->shared_gate_weight};
        const uint64_t wn[8] = {w->router_count, w->routed_gate_count, w->routed_up_count,
                                w->routed_down_count, w->shared_gate_count, w->shared_up_count,
                                w->shared_down_count, w->shared_gate_weight_count};
        for (int i = 0; i < 8; ++i) {
            if (!aligned(wp[i], 4u))
                return kq_fail(diag, KQ_STATUS_INVALID_ALIGNMENT, "MoE weights need 4-byte alignment");
            if (ranges_overlap(wp[i], wn[i] * 4u, out, vbytes) ||
                ranges_overlap(wp[i], wn[i] * 4u, scratch, scratch_bytes))
                return kq_fail(diag, KQ_STATUS_ALIASING_VIOLATION,
                               "MoE weights must not overlap writable execution buffers");
        }
        st = set_device(c, diag);
        if (st == KQ_STATUS_OK) st = snapshot1(c, out, vbytes, diag);
        if (st != KQ_STATUS_OK) return st;
        /* the reference validates the input, then every weight, for finiteness */
        e = kq_launch_f32_scan(hidden, vals, c->d_status, c->stream);
        for (int i = 0; i < 8 && e == hipSuccess; ++i)
            e = kq_launch_f32_scan(wp[i], wn[i], c->d_status, c->stream);
    }
    f32_ws_carve(&d, tokens, scratch, &ws, NULL);
    lw.router = w->router;
    lw.gate = w->routed_gate;
    lw.up = w->routed_up;
    lw.down = w->routed_down;
    lw.shared_gate = w->shared_gate;
    lw.shared_up = w->shared_up;
    lw.shared_down = w->shared_down;
    lw.shared_gate_weight = w->shared_gate_weight;
    if (e == hipSuccess)
        e = kq_launch_moe_f32(&d, &lw, hidden, (uint32_t)tokens, &ws, out, c->d_status, c->stream);
    /* always synchronous: the observers read the results */
    if (!c->async) {
        st = finish(c, e, "F32 MoE launch", diag);
    } else if (e != hipSuccess) {
        st = hip_fail(diag, e, "F32 MoE launch");
    } else {
        st = drain(c, diag);
    }
    if (st != KQ_STATUS_OK) return st;
    if (ro == NULL && co == NULL) return KQ_STATUS_OK;
    return f32_observe(c, &d, tokens, &ws, out, ro, co, user, diag);
}

kq_status kq_hip_moe_token_permutation(kq_hip_context *c, const kq_hip_moe_config *cfg,
                                       const uint32_t *ids, uint64_t tokens, uint32_t *offsets,
                                       uint32_t *pair_token, uint32_t *pair_slot, void *scratch,
                                       uint64_t scratch_bytes, kq_diagnostic *diag) {
    kq_launch_moe_dims d;
    uint64_t pairs;
    kq_status st;
    kq_diagnostic_clear(diag);
    if (!ctx_ok(c) || !moe_ok(cfg) || ids == NULL || offsets == NULL || pair_token == NULL ||
        pair_slot == NULL || scratch == NULL)
        return kq_fail(diag, KQ_STATUS_INVALID_ARGUMENT, "complete permutation arguments are required");
    if (tokens == 0u || tokens > KQ_MOE_MAX_TOKENS)
        return kq_fail(diag, KQ_STATUS_LIMIT_EXCEEDED, "MoE token count is zero or above %u",
                       KQ_MOE_MAX_TOKENS);
    d = launch_dims(cfg);
    if (d.experts > 1023u)
        return kq_fail(diag, KQ_STATUS_LIMIT_EXCEEDED, "the permutation supports up to 1023 experts");
    pairs = tokens * d.top_k;
    if (scratch_bytes < pairs * 4u)
        return kq_fail(diag, KQ_STATUS_BUFFER_TOO_SMALL, "permutation scratch needs %llu bytes",
                       (unsigned long long)(pairs * 4u));
    if (!aligned(ids, 4u) || !aligned(offsets, 4u) || !aligned(pair_token, 4u) ||
        !aligned(pair_slot, 4u) || !aligned(scratch, 4u))
        return kq_fail(diag, KQ_STATUS_INVALID_ALIGNMENT, "permutation buffers need 4-byte alignment");
    if (ranges_overlap(offsets, (d.experts + 1u) * 4u, pair_token, pairs * 4u) ||
        ranges_overlap(offsets, (d.experts + 1u) * 4u, pair_slot, pairs * 4u) ||
        ranges_overlap(pair_token, pairs * 4u, pair_slot, pairs * 4u) ||
        ranges_overlap(ids, pairs * 4u, offsets, (d.experts + 1u) * 4u) ||
        ranges_overlap(ids, pairs * 4u, pair_token, pairs * 4u) ||
        ranges_overlap(ids, pairs * 4u, pair_slot, pairs * 4u) ||
        ranges_overlap(scratch, pairs * 4u, ids, pairs * 4u))
        return kq_fail(diag, KQ_STATUS_ALIASING_VIOLATION, "permutation buffers overlap");
    st = set_device(c, diag);
    if (st == KQ_STATUS_OK) {
        void *const outs[3] = {offsets, pair_token, pair_slot};
        const uint64_t lens[3] = {(d.experts + 1u) * 4u, pairs * 4u, pairs * 4u};
        st = snapshot(c, 3u, outs, lens, diag);
    }
    if (st != KQ_STATUS_OK) return st;
    return finish(c,
                  kq_launch_moe_permute(ids, (uint32_t)tokens, d.top_k, d.experts, offsets,
                                        pair_token, (uint32_t *)scratch, pair_slot, c->d_status,
                                        c->stream),
                  "permutation launch", diag);
}

/* ------------------------------------------------------------------ */
/* gated residual around a layer block */

/* scratch of a gr read: normalized [T][W], rank [T][r], read gates [T][W] */
/* column splits of the dense rank projection (kq_launch_dense_q8) */
#define KQ_GR_SPLITS 8u

/* normalized [T][W], rank [T][r], read_raw [T][W], then the dense
 * projections' room: the rank projection's split partials [S][T][r] (later
 * the split rank rows, hi + lo), and two rows of T scales */
uint64_t kq_hip_gr_scratch_bytes(const kq_hip_gr_dimensions *d, uint64_t tokens) {
    uint64_t w;
    if (d == NULL) return 0u;
    w = (uint64_t)d->branch_count * d->hidden_size;
    return 2u * align256(tokens * w * 4u) + align256(tokens * d->rank * 4u) +
           align256(KQ_GR_SPLITS * tokens * d->rank * 4u) + 2u * align256(tokens * 4u);
}

static kq_status gr_dims_ok(const kq_hip_gr_dimensions *d, uint64_t tokens,
                            kq_diagnostic *diag) {
    if (d == NULL || d->branch_count == 0u || d->hidden_size == 0u || d->rank == 0u ||
        !isfinite(d->rms_epsilon) || !(d->rms_epsilon > 0.0f))
        return kq_fail(diag, KQ_STATUS_INVALID_ARGUMENT,
                       "gated residual needs branches, hidden, rank and a positive epsilon");
    if (d->branch_count > 64u || tokens == 0u || tokens > 65535u ||
        tokens * d->branch_count * (uint64_t)d->hidden_size > (UINT64_C(1) << 30) ||
        (uint64_t)d->rank * d->branch_count * d->hidden_size > (UINT64_C(1) << 31) ||
        tokens * (uint64_t)d->rank > (UINT64_C(1) << 30))
        return kq_fail(diag, KQ_STATUS_LIMIT_EXCEEDED,
                       "gated residual: at most 64 branches, 65,535 tokens, 2^30 state values "
                       "and 2^30 rank values");
    return KQ_STATUS_OK;
}

/* a projection [rows][cols] as F32 or packed rows */
static kq_status gr_proj_ok(uint32_t type, const void *w, uint64_t cols, const char *what,
                            kq_diagnostic *diag) {
    if (w == NULL) return kq_fail(diag, KQ_STATUS_INVALID_ARGUMENT, "gated residual %s is required", what);
    if (!aligned(w, 16u))
        return kq_fail(diag, KQ_STATUS_INVALID_ALIGNMENT, "gated residual %s must be 16-byte aligned", what);
    if (type == KQ_HIP_TYPE_F32) {
        if (cols % 4u != 0u)
            return kq_fail(diag, KQ_STATUS_DIMENSION_MISMATCH,
                           "F32 gated residual %s needs rows of a multiple of 4", what);
        return KQ_STATUS_OK;
    }
    if (!packed_quant(type) || !kq_launch_matvec_supported(type, (uint32_t)cols, 1u))
        return kq_fail(diag, KQ_STATUS_UNSUPPORTED_TENSOR_TYPE,
                       "gated residual %s: F32 or a matvec type with rows of whole blocks", what);
    return KQ_STATUS_OK;
}

/* Tokens from which a Q8_0 projection runs on MFMA: its weights then
 * stream once per 16 tokens instead of once per 4 */
#define KQ_GR_GEMM_MIN_TOKENS 5u

static hipError_t gr_project(kq_hip_context *c, uint32_t type, const void *w, uint64_t rows,
                             uint64_t cols, const float *x, uint32_t tokens, float *y) {
    if (type == KQ_HIP_TYPE_Q8_0 && tokens >= KQ_GR_GEMM_MIN_TOKENS &&
        kq_launch_gemm_q8_0_supported((uint32_t)rows, (uint32_t)cols))
        return kq_launch_gemm_q8_0(w, (uint32_t)rows, (uint32_t)cols, x, tokens, y, c->d_status,
                                   c->stream);
    if (type == KQ_HIP_TYPE_F32)
        return kq_launch_matvec_f32w((const float *)w, (uint32_t)rows, (uint32_t)cols, x, tokens,
                                     y, c->d_status, c->stream);
    if (type == KQ_HIP_TYPE_Q8_0 && cols > 2048u)
        return kq_launch_matvec_q8w(w, (uint32_t)rows, (uint32_t)cols, x, tokens, y,
                                    c->d_status, c->stream);
    return enqueue_matvec(c, type, w, rows, cols, x, tokens, y, NULL, NULL, 0u);
}

kq_status kq_hip_gr_read_f32(kq_hip_context *c, const kq_hip_gr_dimensions *d,
                             const kq_hip_gr_weights *w, const float *x, uint64_t tokens,
                             float *mixed, float *write_gate, void *scratch,
                             uint64_t scratch_bytes, kq_diagnostic *diag) {
    uint64_t W, need;
    float *normalized, *rank, *read_raw, *parts;
    int *sig_dn, *sig_up;
    int dense_dn, dense_up;
    uint32_t slices;
    hipError_t e;
    kq_status st;
    kq_diagnostic_clear(diag);
    if (!ctx_ok(c) || w == NULL || x == NULL || mixed == NULL || write_gate == NULL ||
        scratch == NULL || w->norm == NULL || w->inject == NULL)
        return kq_fail(diag, KQ_STATUS_INVALID_ARGUMENT, "complete gated residual arguments are required");
    st = gr_dims_ok(d, tokens, diag);
    if (st != KQ_STATUS_OK) return st;
    W = (uint64_t)d->branch_count * d->hidden_size;
    st = gr_proj_ok(w->down_type, w->down, W, "down", diag);
    if (st == KQ_STATUS_OK) st = gr_proj_ok(w->up_type, w->up, d->rank, "up", diag);
    if (st != KQ_STATUS_OK) return st;
    need = kq_hip_gr_scratch_bytes(d, tokens);
    if (scratch_bytes < need)
        return kq_fail(diag, KQ_STATUS_BUFFER_TOO_SMALL, "gated residual scratch needs %llu bytes",
                       (unsigned long long)need);
    if (!aligned(x, 16u) || !aligned(scratch, 256u) || !aligned(mixed, 4u) ||
        !aligned(write_gate, 4u) || !aligned(w->norm, 4u) || !aligned(w->inject, 4u))
        return kq_fail(diag, KQ_STATUS_INVALID_ALIGNMENT,
                       "gated residual input 16-byte, scratch 256-byte aligned");
    if (ranges_overlap(x, tokens * W * 4u, scratch, scratch_bytes) ||
        ranges_overlap(mixed, tokens * d->hidden_size * 4u, scratch, scratch_bytes) ||
        ranges_overlap(write_gate, tokens * d->branch_count * 4u, scratch, scratch_bytes) ||
        ranges_overlap(mixed, tokens * d->hidden_size * 4u, write_gate,
                       tokens * d->branch_count * 4u) ||
        ranges_overlap(x, tokens * W * 4u, mixed, tokens * d->hidden_size * 4u) ||
        ranges_overlap(x, tokens * W * 4u, write_gate, tokens * d->branch_count * 4u))
        return kq_fail(diag, KQ_STATUS_ALIASING_VIOLATION,
                       "gated residual input, outputs and scratch must not overlap");
    normalized = (float *)scratch;
    rank = (float *)((char *)scratch + align256(tokens * W * 4u));
    read_raw = (float *)((char *)rank + align256(tokens * d->rank * 4u));
    parts = (float *)((char *)read_raw + align256(tokens * W * 4u));
    sig_dn = (int *)((char *)parts + align256(KQ_GR_SPLITS * tokens * d->rank * 4u));
    sig_up = (int *)((char *)sig_dn + align256(tokens * 4u));
    st = set_device(c, diag);
    if (st == KQ_STATUS_OK) {
        void *const outs[2] = {mixed, write_gate};
        const uint64_t lens[2] = {tokens * d->hidden_size * 4u, tokens * d->branch_count * 4u};
        st = snapshot(c, 2u, outs, lens, diag);
    }
    if (st != KQ_STATUS_OK) return st;
    e = kq_launch_gr_norm(x, w->norm, (uint32_t)tokens, d->branch_count, d->hidden_size,
                          d->rms_epsilon, normalized, c->d_status, c->stream);
    /* Many tokens and Q8_0 projections: the dense MFMA products
     * (kq_launch_dense_q8) on rows split once into fp16 hi + lo. The rank
     * projection's split sits in the read projection's region (free until
     * the up projection writes it), its column splits' partials in `parts`,
     * summed in order by the rank step; the rank rows' split then reuses
     * `parts`. */
    dense_dn = w->down_type == KQ_HIP_TYPE_Q8_0 && tokens >= KQ_GR_GEMM_MIN_TOKENS &&
               kq_launch_dense_q8_supported(d->rank, (uint32_t)W, (uint32_t)tokens);
    dense_up = w->up_type == KQ_HIP_TYPE_Q8_0 && tokens >= KQ_GR_GEMM_MIN_TOKENS &&
               kq_launch_dense_q8_supported((uint32_t)W, d->rank, (uint32_t)tokens);
    slices = dense_dn ? kq_launch_dense_q8_splits((uint32_t)W, KQ_GR_SPLITS) : 1u;
    if (e == hipSuccess && dense_dn) {
        e = kq_launch_dense_split(normalized, (uint32_t)tokens, (uint32_t)W, read_raw,
                                  (char *)read_raw + tokens * W * 2u, sig_dn, 0, c->d_status,
                                  c->stream);
        if (e == hipSuccess)
            e = kq_launch_dense_q8(w->down, NULL, d->rank, (uint32_t)W, read_raw,
                                   (char *)read_raw + tokens * W * 2u, sig_dn, (uint32_t)tokens,
                                   KQ_GR_SPLITS, parts, c->d_status, c->stream);
    } else if (e == hipSuccess) {
        e = gr_project(c, w->down_type, w->down, d->rank, W, normalized, (uint32_t)tokens, rank);
    }
    if (e == hipSuccess)
        e = kq_launch_gr_rank(rank, (uint32_t)(tokens * d->rank), d->branch_count,
                              dense_dn ? parts : NULL, slices, c->d_status, c->stream);
    if (e == hipSuccess && dense_up) {
        e = kq_launch_dense_split(rank, (uint32_t)tokens, d->rank, parts,
                                  (char *)parts + tokens * d->rank * 2u, sig_up, 0, c->d_status,
                                  c->stream);
        if (e == hipSuccess)
            e = kq_launch_dense_q8(w->up, NULL, (uint32_t)W, d->rank, parts,
                                   (char *)parts + tokens * d->rank * 2u, sig_up,
                                   (uint32_t)tokens, 1u, read_raw, c->d_status, c->stream);
    } else if (e == hipSuccess) {
        e = gr_project(c, w->up_type, w->up, W, d->rank, rank, (uint32_t)tokens, read_raw);
    }
    if (e == hipSuccess)
        e = kq_launch_gr_mix(read_raw, normalized, w->inject, (uint32_t)tokens, d->branch_count,
                             d->hidden_size, mixed, write_gate, c->d_status, c->stream);
    return finish(c, e, "gated residual read launch", diag);
}

kq_status kq_hip_gr_write_f32(kq_hip_context *c, const kq_hip_gr_dimensions *d,
                              const float *x, const float *block_output,
                              const float *write_gate, uint64_t tokens, float *out,
                              kq_diagnostic *diag) {
    uint64_t W;
    kq_status st;
    kq_diagnostic_clear(diag);
    if (!ctx_ok(c) || x == NULL || block_output == NULL || write_gate == NULL || out == NULL)
        return kq_fail(diag, KQ_STATUS_INVALID_ARGUMENT, "complete gated residual arguments are required");
    st = gr_dims_ok(d, tokens, diag);
    if (st != KQ_STATUS_OK) return st;
    W = (uint64_t)d->branch_count * d->hidden_size;
    if (!aligned(x, 4u) || !aligned(block_output, 4u) || !aligned(write_gate, 4u) ||
        !aligned(out, 4u))
        return kq_fail(diag, KQ_STATUS_INVALID_ALIGNMENT, "gated residual buffers must be 4-byte aligned");
    if ((out != x && ranges_overlap(x, tokens * W * 4u, out, tokens * W * 4u)) ||
        ranges_overlap(block_output, tokens * d->hidden_size * 4u, out, tokens * W * 4u) ||
        ranges_overlap(write_gate, tokens * d->branch_count * 4u, out, tokens * W * 4u))
        return kq_fail(diag, KQ_STATUS_ALIASING_VIOLATION,
                       "gated residual output may only be the branches themselves");
    st = set_device(c, diag);
    if (st == KQ_STATUS_OK) st = snapshot1(c, out, tokens * W * 4u, diag);
    if (st != KQ_STATUS_OK) return st;
    return finish(c, kq_launch_gr_write(x, block_output, write_gate, (uint32_t)tokens,
                                        d->branch_count, d->hidden_size, out, c->d_status,
                                        c->stream),
                  "gated residual write launch", diag);
}

/* scratch of the MoE block: mixed [T][H], write gates [T][B], MoE output
 * [T][H], then the gated residual's and the MoE's own scratch */
uint64_t kq_hip_moe_block_scratch_bytes(const kq_hip_gr_dimensions *d,
                                        const kq_hip_moe_config *cfg, uint64_t tokens) {
    if (d == NULL || !moe_ok(cfg)) return 0u;
    return 2u * align256(tokens * d->hidden_size * 4u) + align256(tokens * d->branch_count * 4u) +
           kq_hip_gr_scratch_bytes(d, tokens) + align256(kq_hip_moe_config_scratch_bytes(cfg, tokens));
}

kq_status kq_hip_moe_block_f32(kq_hip_context *c, const kq_hip_gr_dimensions *d,
                               const kq_hip_gr_weights *gw, const kq_hip_moe_config *cfg,
                               const kq_hip_moe_weights *mw, const float *x, uint64_t tokens,
                               float *out, uint32_t *ids, void *scratch, uint64_t scratch_bytes,
                               kq_diagnostic *diag) {
    uint64_t W, need, hb, gb;
    char *p;
    float *mixed, *wg, *moe_out;
    int prev;
    kq_status st;
    kq_diagnostic_clear(diag);
    if (!ctx_ok(c) || gw == NULL || mw == NULL || x == NULL || out == NULL || scratch == NULL ||
        !moe_ok(cfg))
        return kq_fail(diag, KQ_STATUS_INVALID_ARGUMENT, "complete MoE block arguments are required");
    st = gr_dims_ok(d, tokens, diag);
    if (st != KQ_STATUS_OK) return st;
    if (cfg->dims.hidden_size != d->hidden_size)
        return kq_fail(diag, KQ_STATUS_DIMENSION_MISMATCH,
                       "the MoE hidden size must be the gated residual's");
    W = (uint64_t)d->branch_count * d->hidden_size;
    need = kq_hip_moe_block_scratch_bytes(d, cfg, tokens);
    if (scratch_bytes < need)
        return kq_fail(diag, KQ_STATUS_BUFFER_TOO_SMALL, "MoE block scratch needs %llu bytes",
                       (unsigned long long)need);
    if (!aligned(scratch, 256u))
        return kq_fail(diag, KQ_STATUS_INVALID_ALIGNMENT, "MoE block scratch must be 256-byte aligned");
    if (ranges_overlap(x, tokens * W * 4u, out, tokens * W * 4u) ||
        ranges_overlap(x, tokens * W * 4u, scratch, scratch_bytes) ||
        ranges_overlap(out, tokens * W * 4u, scratch, scratch_bytes))
        return kq_fail(diag, KQ_STATUS_ALIASING_VIOLATION,
                       "MoE block input, output and scratch must not overlap");
    if (ids != NULL) {
        const uint64_t ib = tokens * cfg->dims.top_k * 4u;
        if (!aligned(ids, 4u))
            return kq_fail(diag, KQ_STATUS_INVALID_ALIGNMENT, "selected ids need 4-byte alignment");
        if (ranges_overlap(ids, ib, x, tokens * W * 4u) ||
            ranges_overlap(ids, ib, out, tokens * W * 4u) ||
            ranges_overlap(ids, ib, scratch, scratch_bytes))
            return kq_fail(diag, KQ_STATUS_ALIASING_VIOLATION,
                           "selected ids overlap the MoE block input, output or scratch");
    }
    hb = align256(tokens * d->hidden_size * 4u);
    gb = kq_hip_gr_scratch_bytes(d, tokens);
    p = (char *)scratch;
    mixed = (float *)p;
    p += hb;
    moe_out = (float *)p;
    p += hb;
    wg = (float *)p;
    p += align256(tokens * d->branch_count * 4u);
    st = set_device(c, diag);
    if (st == KQ_STATUS_OK) {
        void *const outs[2] = {out, ids};
        const uint64_t lens[2] = {tokens * W * 4u, tokens * cfg->dims.top_k * 4u};
        st = snapshot(c, 2u, outs, lens, diag);
    }
    if (st != KQ_STATUS_OK) return st;
    /* one synchronisation for the whole step: the three stages enqueue */
    prev = c->async;
    c->async = 1;
    st = kq_hip_gr_read_f32(c, d, gw, x, tokens, mixed, wg, p, gb, diag);
    if (st == KQ_STATUS_OK)
        st = kq_hip_moe_execute_quantized(c, cfg, mw, mixed, tokens, moe_out,
                                          tokens * d->hidden_size, ids, p + gb,
                                          scratch_bytes - (uint64_t)(p + gb - (char *)scratch),
                                          diag);
    if (st == KQ_STATUS_OK)
        st = kq_hip_gr_write_f32(c, d, x, moe_out, wg, tokens, out, diag);
    c->async = prev;
    if (st != KQ_STATUS_OK) {
        /* stages already enqueued finish before the error is returned */
        if (!prev) {
            kq_diagnostic ignored;
            (void)drain(c, &ignored);
            restore(c);
        }
        return st;
    }
    return finish(c, hipSuccess, "MoE block launch", diag);
}
