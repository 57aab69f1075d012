/*
 * kq_gguf.h — GGUF v3 directory parser over a read-only mapped file.
 *
 * Replaces: include/kq_gguf.h:11-117 and src/kq_gguf.c (kq_gguf_open and
 * its accessors). The names, struct layouts, enum values and statuses are
 * the reference's, so a caller switching libraries recompiles unchanged.
 * The contract, in the order the checks run:
 *   - a file shorter than the 24-byte fixed header: TRUNCATED;
 *   - the header and directory are read through one view of at most
 *     512 MiB; reading past it is LIMIT_EXCEEDED when the file is longer
 *     than the view, TRUNCATED otherwise;
 *   - magic "GGUF" (BAD_MAGIC), version 3 (UNSUPPORTED_VERSION), non-zero
 *     tensor and metadata counts (MALFORMED_METADATA), counts whose
 *     descriptor arrays cannot be sized (ARITHMETIC_OVERFLOW), at most 1024
 *     metadata entries and 8192 tensors (LIMIT_EXCEEDED);
 *   - strings at most 128 MiB (LIMIT_EXCEEDED) and well-formed UTF-8
 *     (MALFORMED_METADATA); arrays at most 2,000,000 entries;
 *   - metadata values: UINT16, UINT32, INT32, FLOAT32, BOOL (0 or 1, else
 *     MALFORMED_METADATA), STRING, and ARRAY of INT32, UINT64 or STRING;
 *     anything else UNSUPPORTED_METADATA; repeated keys DUPLICATE_METADATA;
 *   - general.architecture required and a string, general.alignment a
 *     UINT32 (MALFORMED_METADATA); the alignment (default 32) a power of two
 *     up to 4096 (INVALID_ALIGNMENT);
 *   - tensors: unique names (DUPLICATE_TENSOR), rank 1..8 and no zero
 *     dimension (MALFORMED_TENSOR), a dimension product that fits uint64
 *     (ARITHMETIC_OVERFLOW), a supported type (UNSUPPORTED_TENSOR_TYPE), an
 *     aligned relative offset (INVALID_ALIGNMENT), a first dimension of
 *     whole blocks (MALFORMED_TENSOR);
 *   - the data section starts at the directory end rounded up to the
 *     alignment and inside the file (INCONSISTENT_DATA_SECTION); sorted by
 *     offset, the first tensor starts at relative offset 0, none overlaps
 *     the next (INCONSISTENT_DATA_SECTION) and none ends past the file
 *     (SPAN_OUT_OF_RANGE).
 * Parsing reads only the directory: tensor payload bytes are touched later,
 * by the device upload entry points (include/kq_hip.h).
 *
 * One addition: type 14 (Q6_K, 256 elements in 210 bytes) is accepted,
 * because the device path decodes it; the reference's table stops at the
 * seven types below it and fails such a tensor with UNSUPPORTED_TENSOR_TYPE.
 */
#ifndef KQ_GGUF_H
#define KQ_GGUF_H

#include <stdint.h>

#include "kq_file.h"
#include "kq_status.h"

#ifdef __cplusplus
extern "C" {
#endif

#define KQ_GGUF_MAX_DIMS 8U

enum {
    KQ_GGUF_TYPE_F32 = 0,
    KQ_GGUF_TYPE_Q5_1 = 7,
    KQ_GGUF_TYPE_Q8_0 = 8,
    KQ_GGUF_TYPE_Q4_K = 12,
    KQ_GGUF_TYPE_Q5_K = 13,
    KQ_GGUF_TYPE_Q6_K = 14,
    KQ_GGUF_TYPE_IQ4_NL = 20,
    KQ_GGUF_TYPE_BF16 = 30
};

enum {
    KQ_GGUF_VALUE_UINT16 = 2,
    KQ_GGUF_VALUE_UINT32 = 4,
    KQ_GGUF_VALUE_INT32 = 5,
    KQ_GGUF_VALUE_FLOAT32 = 6,
    KQ_GGUF_VALUE_BOOL = 7,
    KQ_GGUF_VALUE_STRING = 8,
    KQ_GGUF_VALUE_ARRAY = 9,
    KQ_GGUF_VALUE_UINT64 = 10
};

/* Bytes inside the mapped directory; not NUL-terminated. */
typedef struct kq_string_view {
    const unsigned char *data;
    uint64_t length;
} kq_string_view;

typedef struct kq_gguf_type_info {
    uint32_t type_id;
    const char *name;
    uint64_t block_elements;
    uint64_t bytes_per_block;
} kq_gguf_type_info;

/* scalar_value holds UINT16/UINT32/INT32/FLOAT32/BOOL bits; arrays keep
 * their element type, length and encoded bytes in array_data. */
typedef struct kq_gguf_metadata {
    kq_string_view key;
    uint32_t value_type;
    uint32_t array_element_type;
    uint64_t array_length;
    uint64_t scalar_value;
    kq_string_view string_value;
    kq_string_view array_data;
} kq_gguf_metadata;

/* dimensions are innermost first (dimensions[0] is the row length);
 * data_offset is absolute in the file. */
typedef struct kq_gguf_tensor {
    kq_string_view name;
    uint32_t rank;
    uint64_t dimensions[KQ_GGUF_MAX_DIMS];
    uint32_t type_id;
    uint64_t block_elements;
    uint64_t bytes_per_block;
    uint64_t element_count;
    uint64_t relative_offset;
    uint64_t data_offset;
    uint64_t packed_bytes;
} kq_gguf_tensor;

typedef struct kq_gguf kq_gguf;

/* The file must stay open until kq_gguf_close. */
kq_status kq_gguf_open(kq_file *file, kq_gguf **out_gguf,
                       kq_diagnostic *diagnostic);
void kq_gguf_close(kq_gguf *gguf);

uint32_t kq_gguf_version(const kq_gguf *gguf);
uint64_t kq_gguf_metadata_count(const kq_gguf *gguf);
uint64_t kq_gguf_tensor_count(const kq_gguf *gguf);
uint64_t kq_gguf_alignment(const kq_gguf *gguf);
uint64_t kq_gguf_directory_end_offset(const kq_gguf *gguf);
uint64_t kq_gguf_data_section_offset(const kq_gguf *gguf);
uint64_t kq_gguf_packed_tensor_bytes(const kq_gguf *gguf);
/* file size minus the packed tensor bytes */
uint64_t kq_gguf_format_overhead_bytes(const kq_gguf *gguf);
/* furthest byte the parser read */
uint64_t kq_gguf_directory_bytes_parsed(const kq_gguf *gguf);
/* payload bytes read while parsing: always 0 */
uint64_t kq_gguf_payload_bytes_accessed(const kq_gguf *gguf);
kq_string_view kq_gguf_architecture(const kq_gguf *gguf);

const kq_gguf_metadata *kq_gguf_metadata_at(const kq_gguf *gguf, uint64_t index);
const kq_gguf_metadata *kq_gguf_find_metadata(const kq_gguf *gguf, const char *key);
const kq_gguf_tensor *kq_gguf_tensor_at(const kq_gguf *gguf, uint64_t index);
const kq_gguf_tensor *kq_gguf_find_tensor(const kq_gguf *gguf, const char *name);

const kq_gguf_type_info *kq_gguf_type_info_for(uint32_t type_id);
int kq_string_view_equal(const kq_string_view *left, const kq_string_view *right);
int kq_string_view_equal_cstr(const kq_string_view *view, const char *text);
/* Typed reads: 1 on success, 0 when the entry is absent or of another type
 * or the index is out of range. */
int kq_gguf_metadata_u16(const kq_gguf_metadata *metadata, uint16_t *value);
int kq_gguf_metadata_u32(const kq_gguf_metadata *metadata, uint32_t *value);
int kq_gguf_metadata_i32(const kq_gguf_metadata *metadata, int32_t *value);
int kq_gguf_metadata_array_i32_at(const kq_gguf_metadata *metadata,
                                  uint64_t index, int32_t *value);
int kq_gguf_metadata_array_u64_at(const kq_gguf_metadata *metadata,
                                  uint64_t index, uint64_t *value);
int kq_gguf_metadata_array_string_at(const kq_gguf_metadata *metadata,
                                     uint64_t index, kq_string_view *value);

#ifdef __cplusplus
}
#endif

#endif
