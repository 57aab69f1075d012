/*
 * kq_status.h — status codes and the fixed-size diagnostic record used by
 * every kq_hip entry point.
 *
 * Replaces: include/kq_status.h:10-74 (kq_status, kq_diagnostic) and
 * src/kq_status.c:128-159 (kq_diagnostic_clear / kq_diagnostic_set).
 *
 * The numeric values of the codes below are the ones the reference assigns
 * (its enum is positional; the values are restated explicitly here so a
 * caller switching from the reference library keeps the same integers).
 * Only the codes that the quantized-weight path and its GGUF ingestion can
 * return are listed.
 * KQ_STATUS_DEVICE_FAILURE is new: the reference has no device runtime.
 */
#ifndef KQ_STATUS_H
#define KQ_STATUS_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum kq_status {
    KQ_STATUS_OK = 0,
    KQ_STATUS_INVALID_ARGUMENT = 1,
    KQ_STATUS_OUT_OF_MEMORY = 2,
    KQ_STATUS_FILE_OPEN_FAILED = 3,
    KQ_STATUS_FILE_SIZE_FAILED = 4,
    KQ_STATUS_FILE_MAP_FAILED = 5,
    KQ_STATUS_TRUNCATED = 6,
    KQ_STATUS_BAD_MAGIC = 7,
    KQ_STATUS_UNSUPPORTED_VERSION = 8,
    KQ_STATUS_MALFORMED_METADATA = 9,
    KQ_STATUS_UNSUPPORTED_METADATA = 10,
    KQ_STATUS_MALFORMED_TENSOR = 11,
    KQ_STATUS_UNSUPPORTED_TENSOR_TYPE = 12,
    KQ_STATUS_ARITHMETIC_OVERFLOW = 13,
    KQ_STATUS_LIMIT_EXCEEDED = 14,
    KQ_STATUS_INVALID_ALIGNMENT = 15,
    KQ_STATUS_SPAN_OUT_OF_RANGE = 16,
    KQ_STATUS_DUPLICATE_METADATA = 17,
    KQ_STATUS_DUPLICATE_TENSOR = 18,
    KQ_STATUS_INCONSISTENT_DATA_SECTION = 19,
    KQ_STATUS_INVALID_QUANTIZED_GEOMETRY = 25,
    KQ_STATUS_NONCONTIGUOUS_TENSOR_VIEW = 26,
    KQ_STATUS_TENSOR_LAYOUT_MISMATCH = 27,
    KQ_STATUS_TENSOR_OWNERSHIP_MISMATCH = 28,
    KQ_STATUS_INVALID_TOKEN_ID = 31,
    KQ_STATUS_BUFFER_TOO_SMALL = 32,
    KQ_STATUS_MALFORMED_QUANTIZED_DATA = 38,
    KQ_STATUS_NUMERIC_DOMAIN = 39,
    KQ_STATUS_DIMENSION_MISMATCH = 40,
    KQ_STATUS_ALIASING_VIOLATION = 41,
    KQ_STATUS_INCOMPATIBLE_MOE = 46,
    KQ_STATUS_INCOMPATIBLE_SAMPLING = 54,
    KQ_STATUS_INVALID_RNG_STATE = 55,
    /* Extension: a HIP runtime call failed (launch, copy, sync, graph). */
    KQ_STATUS_DEVICE_FAILURE = 1000
} kq_status;

#define KQ_DIAGNOSTIC_CAPACITY 256U

typedef struct kq_diagnostic {
    kq_status status;
    char message[KQ_DIAGNOSTIC_CAPACITY];
} kq_diagnostic;

const char *kq_status_string(kq_status status);
void kq_diagnostic_clear(kq_diagnostic *diagnostic);

#ifdef __cplusplus
}
#endif

#endif
