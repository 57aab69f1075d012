/*
 * kq_status.c — status strings and diagnostics.
 * Replaces src/kq_status.c:9-159 (kq_status_string, kq_diagnostic_clear,
 * kq_diagnostic_set) for the codes in include/kq_status.h.
 */
#include "kq_status_internal.h"

#include <stdarg.h>
#include <stdio.h>

const char *kq_status_string(kq_status status) {
    switch (status) {
    case KQ_STATUS_OK: return "ok";
    case KQ_STATUS_INVALID_ARGUMENT: return "invalid argument";
    case KQ_STATUS_OUT_OF_MEMORY: return "out of memory";
    case KQ_STATUS_FILE_OPEN_FAILED: return "file open failed";
    case KQ_STATUS_FILE_SIZE_FAILED: return "file size failed";
    case KQ_STATUS_FILE_MAP_FAILED: return "file map failed";
    case KQ_STATUS_TRUNCATED: return "truncated";
    case KQ_STATUS_BAD_MAGIC: return "bad magic";
    case KQ_STATUS_UNSUPPORTED_VERSION: return "unsupported version";
    case KQ_STATUS_MALFORMED_METADATA: return "malformed metadata";
    case KQ_STATUS_UNSUPPORTED_METADATA: return "unsupported metadata";
    case KQ_STATUS_MALFORMED_TENSOR: return "malformed tensor";
    case KQ_STATUS_UNSUPPORTED_TENSOR_TYPE: return "unsupported tensor type";
    case KQ_STATUS_ARITHMETIC_OVERFLOW: return "arithmetic overflow";
    case KQ_STATUS_LIMIT_EXCEEDED: return "limit exceeded";
    case KQ_STATUS_INVALID_ALIGNMENT: return "invalid alignment";
    case KQ_STATUS_SPAN_OUT_OF_RANGE: return "span out of range";
    case KQ_STATUS_DUPLICATE_METADATA: return "duplicate metadata";
    case KQ_STATUS_DUPLICATE_TENSOR: return "duplicate tensor";
    case KQ_STATUS_INCONSISTENT_DATA_SECTION: return "inconsistent data section";
    case KQ_STATUS_INVALID_QUANTIZED_GEOMETRY: return "invalid quantized geometry";
    case KQ_STATUS_NONCONTIGUOUS_TENSOR_VIEW: return "noncontiguous tensor view";
    case KQ_STATUS_TENSOR_LAYOUT_MISMATCH: return "tensor layout mismatch";
    case KQ_STATUS_TENSOR_OWNERSHIP_MISMATCH: return "tensor ownership mismatch";
    case KQ_STATUS_INVALID_TOKEN_ID: return "invalid token id";
    case KQ_STATUS_BUFFER_TOO_SMALL: return "buffer too small";
    case KQ_STATUS_MALFORMED_QUANTIZED_DATA: return "malformed quantized data";
    case KQ_STATUS_NUMERIC_DOMAIN: return "numeric domain error";
    case KQ_STATUS_DIMENSION_MISMATCH: return "dimension mismatch";
    case KQ_STATUS_ALIASING_VIOLATION: return "aliasing violation";
    case KQ_STATUS_INCOMPATIBLE_MOE: return "incompatible MoE";
    case KQ_STATUS_INCOMPATIBLE_SAMPLING: return "incompatible sampling";
    case KQ_STATUS_INVALID_RNG_STATE: return "invalid RNG state";
    case KQ_STATUS_DEVICE_FAILURE: return "device failure";
    default: return "unknown status";
    }
}

void kq_diagnostic_clear(kq_diagnostic *diagnostic) {
    if (diagnostic == NULL) return;
    diagnostic->status = KQ_STATUS_OK;
    diagnostic->message[0] = '\0';
}

kq_status kq_fail(kq_diagnostic *diagnostic, kq_status status, const char *format, ...) {
    va_list args;
    if (diagnostic == NULL) return status;
    diagnostic->status = status;
    diagnostic->message[0] = '\0';
    if (format != NULL) {
        va_start(args, format);
        (void)vsnprintf(diagnostic->message, sizeof(diagnostic->message), format, args);
        va_end(args);
    }
    return status;
}
