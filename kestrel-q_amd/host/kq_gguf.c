/*
 * kq_gguf.c — GGUF v3 directory parser (the contract of src/kq_gguf.c:
 * UTF-8 rule at :207-255, metadata values at :349-469, metadata at
 * :471-551, tensors at :553-668, spans at :688-796, open at :798-967,
 * accessors at :979-1237), written over a bounds-checked cursor.
 *
 * Everything is read through one mapped view of the first
 * min(file size, 512 MiB) bytes; descriptors keep string views into it.
 * Duplicate keys and tensor names are found with a hash set instead of
 * pairwise comparison (same result, linear time for 8192 tensors).
 */
#include "kq_gguf.h"

#include <stdlib.h>
#include <string.h>

#include "kq_gguf_internal.h"
#include "kq_status_internal.h"

enum {
    kFixedHeader = 24,
};
#define KQ_GGUF_VIEW_LIMIT (512ull << 20)
#define KQ_GGUF_STRING_LIMIT (128ull << 20)
#define KQ_GGUF_ARRAY_LIMIT 2000000ull
#define KQ_GGUF_METADATA_LIMIT 1024ull
#define KQ_GGUF_TENSOR_LIMIT 8192ull
#define KQ_GGUF_DEFAULT_ALIGNMENT 32ull
#define KQ_GGUF_ALIGNMENT_LIMIT 4096ull

struct kq_gguf {
    kq_file *file;
    kq_file_view *view;
    kq_gguf_metadata *metadata;
    kq_gguf_tensor *tensors;
    uint32_t version;
    uint64_t metadata_count;
    uint64_t tensor_count;
    uint64_t alignment;
    uint64_t directory_end;
    uint64_t data_section;
    uint64_t packed_bytes;
    uint64_t overhead_bytes;
    uint64_t bytes_parsed;
    kq_string_view architecture;
};

/* Block geometry per GGML type id (the GGUF specification's block sizes). */
static const kq_gguf_type_info kTypes[] = {
    {KQ_GGUF_TYPE_F32, "F32", 1u, 4u},
    {KQ_GGUF_TYPE_Q5_1, "Q5_1", 32u, 24u},
    {KQ_GGUF_TYPE_Q8_0, "Q8_0", 32u, 34u},
    {KQ_GGUF_TYPE_Q4_K, "Q4_K", 256u, 144u},
    {KQ_GGUF_TYPE_Q5_K, "Q5_K", 256u, 176u},
    {KQ_GGUF_TYPE_Q6_K, "Q6_K", 256u, 210u},
    {KQ_GGUF_TYPE_IQ4_NL, "IQ4_NL", 32u, 18u},
    {KQ_GGUF_TYPE_BF16, "BF16", 1u, 2u},
};

const kq_gguf_type_info *kq_gguf_type_info_for(uint32_t type_id) {
    size_t i;
    for (i = 0u; i < sizeof(kTypes) / sizeof(kTypes[0]); ++i)
        if (kTypes[i].type_id == type_id) return &kTypes[i];
    return NULL;
}

/* ------------------------------------------------------------------ */
/* cursor over the directory view */

typedef struct cursor {
    const unsigned char *base;
    uint64_t view_bytes;
    uint64_t file_bytes;
    uint64_t at;
    uint64_t furthest;
    kq_diagnostic *diag;
} cursor;

static kq_status cur_take(cursor *c, uint64_t n, const unsigned char **out) {
    uint64_t end;
    if (n > UINT64_MAX - c->at)
        return kq_fail(c->diag, KQ_STATUS_ARITHMETIC_OVERFLOW, "GGUF read position overflows");
    end = c->at + n;
    if (end > c->view_bytes) {
        if (c->view_bytes < c->file_bytes)
            return kq_fail(c->diag, KQ_STATUS_LIMIT_EXCEEDED,
                           "GGUF header and directory pass the %llu-byte limit",
                           (unsigned long long)c->view_bytes);
        return kq_fail(c->diag, KQ_STATUS_TRUNCATED,
                       "GGUF directory needs %llu bytes; the file has %llu",
                       (unsigned long long)end, (unsigned long long)c->view_bytes);
    }
    if (out != NULL) *out = c->base + c->at;
    c->at = end;
    if (end > c->furthest) c->furthest = end;
    return KQ_STATUS_OK;
}

static uint64_t load_le(const unsigned char *p, unsigned n) {
    uint64_t v = 0u;
    while (n-- > 0u) v = (v << 8) | p[n];
    return v;
}

static kq_status cur_uint(cursor *c, unsigned n, uint64_t *v) {
    const unsigned char *p;
    kq_status st = cur_take(c, n, &p);
    if (st == KQ_STATUS_OK) *v = load_le(p, n);
    return st;
}

static kq_status cur_u32(cursor *c, uint32_t *v) {
    uint64_t w = 0u;
    kq_status st = cur_uint(c, 4u, &w);
    *v = (uint32_t)w;
    return st;
}

/* Well-formed UTF-8 (Unicode table 3-7): shortest forms only, no
 * surrogates, nothing above U+10FFFF. */
static int utf8_ok(const unsigned char *s, uint64_t n) {
    uint64_t i = 0u;
    while (i < n) {
        const unsigned b = s[i];
        unsigned len, k;
        uint32_t cp, min;
        if (b < 0x80u) {
            ++i;
            continue;
        }
        if ((b & 0xe0u) == 0xc0u) {
            len = 2u; cp = b & 0x1fu; min = 0x80u;
        } else if ((b & 0xf0u) == 0xe0u) {
            len = 3u; cp = b & 0x0fu; min = 0x800u;
        } else if ((b & 0xf8u) == 0xf0u) {
            len = 4u; cp = b & 0x07u; min = 0x10000u;
        } else {
            return 0;
        }
        if (n - i < len) return 0;
        for (k = 1u; k < len; ++k) {
            if ((s[i + k] & 0xc0u) != 0x80u) return 0;
            cp = (cp << 6) | (s[i + k] & 0x3fu);
        }
        if (cp < min || cp > 0x10ffffu || (cp >= 0xd800u && cp <= 0xdfffu)) return 0;
        i += len;
    }
    return 1;
}

static kq_status cur_string(cursor *c, kq_string_view *out) {
    uint64_t n;
    const unsigned char *p;
    kq_status st = cur_uint(c, 8u, &n);
    if (st != KQ_STATUS_OK) return st;
    if (n > KQ_GGUF_STRING_LIMIT)
        return kq_fail(c->diag, KQ_STATUS_LIMIT_EXCEEDED,
                       "GGUF string of %llu bytes passes the 128 MiB limit", (unsigned long long)n);
    st = cur_take(c, n, &p);
    if (st != KQ_STATUS_OK) return st;
    if (!utf8_ok(p, n))
        return kq_fail(c->diag, KQ_STATUS_MALFORMED_METADATA, "GGUF string is not valid UTF-8");
    out->data = p;
    out->length = n;
    return KQ_STATUS_OK;
}

/* ------------------------------------------------------------------ */
/* string views and a set of them */

int kq_string_view_equal(const kq_string_view *a, const kq_string_view *b) {
    if (a == NULL || b == NULL || a->length != b->length) return 0;
    return a->length == 0u || memcmp(a->data, b->data, (size_t)a->length) == 0;
}

int kq_string_view_equal_cstr(const kq_string_view *v, const char *text) {
    size_t n;
    if (v == NULL || text == NULL) return 0;
    n = strlen(text);
    return (uint64_t)n == v->length && (n == 0u || memcmp(v->data, text, n) == 0);
}

typedef struct name_set {
    const kq_string_view **slot;
    uint64_t mask;
} name_set;

static int set_init(name_set *s, uint64_t count) {
    uint64_t cap = 16u;
    while (cap < 2u * count) cap <<= 1;
    s->slot = (const kq_string_view **)calloc((size_t)cap, sizeof(*s->slot));
    s->mask = cap - 1u;
    return s->slot != NULL;
}

static uint64_t fnv1a(const kq_string_view *v) {
    uint64_t h = 0xcbf29ce484222325ull, i;
    for (i = 0u; i < v->length; ++i) h = (h ^ v->data[i]) * 0x100000001b3ull;
    return h;
}

/* 1 if an equal name is already in the set, else inserts it and returns 0 */
static int set_seen(name_set *s, const kq_string_view *v) {
    uint64_t i = fnv1a(v) & s->mask;
    while (s->slot[i] != NULL) {
        if (kq_string_view_equal(s->slot[i], v)) return 1;
        i = (i + 1u) & s->mask;
    }
    s->slot[i] = v;
    return 0;
}

/* ------------------------------------------------------------------ */
/* metadata */

static kq_status read_scalar(cursor *c, uint32_t type, uint64_t *v) {
    kq_status st;
    switch (type) {
    case KQ_GGUF_VALUE_UINT16:
        return cur_uint(c, 2u, v);
    case KQ_GGUF_VALUE_UINT32:
    case KQ_GGUF_VALUE_INT32:
    case KQ_GGUF_VALUE_FLOAT32:
        return cur_uint(c, 4u, v);
    case KQ_GGUF_VALUE_BOOL:
        st = cur_uint(c, 1u, v);
        if (st == KQ_STATUS_OK && *v > 1u)
            return kq_fail(c->diag, KQ_STATUS_MALFORMED_METADATA,
                           "GGUF bool holds %llu, not 0 or 1", (unsigned long long)*v);
        return st;
    default:
        return kq_fail(c->diag, KQ_STATUS_UNSUPPORTED_METADATA,
                       "GGUF metadata value type %u is not supported", type);
    }
}

static kq_status read_array(cursor *c, kq_gguf_metadata *m) {
    uint64_t n, i, start, width;
    kq_string_view item;
    kq_status st = cur_u32(c, &m->array_element_type);
    if (st == KQ_STATUS_OK) st = cur_uint(c, 8u, &n);
    if (st != KQ_STATUS_OK) return st;
    if (n > KQ_GGUF_ARRAY_LIMIT)
        return kq_fail(c->diag, KQ_STATUS_LIMIT_EXCEEDED,
                       "GGUF array of %llu entries passes the 2,000,000 limit", (unsigned long long)n);
    m->array_length = n;
    start = c->at;
    switch (m->array_element_type) {
    case KQ_GGUF_VALUE_INT32:
    case KQ_GGUF_VALUE_UINT64:
        width = m->array_element_type == KQ_GGUF_VALUE_INT32 ? 4u : 8u;
        st = cur_take(c, n * width, NULL); /* n <= 2e6: no overflow */
        break;
    case KQ_GGUF_VALUE_STRING:
        for (i = 0u; i < n && st == KQ_STATUS_OK; ++i) st = cur_string(c, &item);
        break;
    default:
        return kq_fail(c->diag, KQ_STATUS_UNSUPPORTED_METADATA,
                       "GGUF arrays of value type %u are not supported", m->array_element_type);
    }
    if (st != KQ_STATUS_OK) return st;
    m->array_data.data = c->base + start;
    m->array_data.length = c->at - start;
    return KQ_STATUS_OK;
}

static kq_status read_metadata(cursor *c, kq_gguf *g) {
    name_set seen;
    uint64_t i;
    kq_status st = KQ_STATUS_OK;
    if (!set_init(&seen, g->metadata_count))
        return kq_fail(c->diag, KQ_STATUS_OUT_OF_MEMORY, "metadata key set allocation failed");
    g->alignment = KQ_GGUF_DEFAULT_ALIGNMENT;
    for (i = 0u; i < g->metadata_count && st == KQ_STATUS_OK; ++i) {
        kq_gguf_metadata *m = &g->metadata[i];
        st = cur_string(c, &m->key);
        if (st != KQ_STATUS_OK) break;
        if (set_seen(&seen, &m->key)) {
            st = kq_fail(c->diag, KQ_STATUS_DUPLICATE_METADATA,
                         "GGUF metadata key %llu repeats an earlier key", (unsigned long long)i);
            break;
        }
        st = cur_u32(c, &m->value_type);
        if (st != KQ_STATUS_OK) break;
        if (m->value_type == KQ_GGUF_VALUE_STRING)
            st = cur_string(c, &m->string_value);
        else if (m->value_type == KQ_GGUF_VALUE_ARRAY)
            st = read_array(c, m);
        else
            st = read_scalar(c, m->value_type, &m->scalar_value);
        if (st != KQ_STATUS_OK) break;
        if (kq_string_view_equal_cstr(&m->key, "general.architecture")) {
            if (m->value_type != KQ_GGUF_VALUE_STRING)
                st = kq_fail(c->diag, KQ_STATUS_MALFORMED_METADATA,
                             "general.architecture is not a string");
            else
                g->architecture = m->string_value;
        } else if (kq_string_view_equal_cstr(&m->key, "general.alignment")) {
            if (m->value_type != KQ_GGUF_VALUE_UINT32)
                st = kq_fail(c->diag, KQ_STATUS_MALFORMED_METADATA,
                             "general.alignment is not a uint32");
            else
                g->alignment = m->scalar_value;
        }
    }
    free(seen.slot);
    if (st != KQ_STATUS_OK) return st;
    if (g->architecture.data == NULL)
        return kq_fail(c->diag, KQ_STATUS_MALFORMED_METADATA, "general.architecture is missing");
    if (g->alignment == 0u || g->alignment > KQ_GGUF_ALIGNMENT_LIMIT ||
        (g->alignment & (g->alignment - 1u)) != 0u)
        return kq_fail(c->diag, KQ_STATUS_INVALID_ALIGNMENT,
                       "GGUF alignment %llu is not a power of two up to 4096",
                       (unsigned long long)g->alignment);
    return KQ_STATUS_OK;
}

/* ------------------------------------------------------------------ */
/* tensor directory */

static kq_status read_tensor(cursor *c, kq_gguf *g, uint64_t i) {
    kq_gguf_tensor *t = &g->tensors[i];
    const kq_gguf_type_info *info;
    uint64_t d, elements = 1u, blocks;
    kq_status st = cur_u32(c, &t->rank);
    if (st != KQ_STATUS_OK) return st;
    if (t->rank == 0u || t->rank > KQ_GGUF_MAX_DIMS)
        return kq_fail(c->diag, KQ_STATUS_MALFORMED_TENSOR, "tensor %llu has rank %u",
                       (unsigned long long)i, t->rank);
    for (d = 0u; d < t->rank; ++d) {
        st = cur_uint(c, 8u, &t->dimensions[d]);
        if (st != KQ_STATUS_OK) return st;
        if (t->dimensions[d] == 0u)
            return kq_fail(c->diag, KQ_STATUS_MALFORMED_TENSOR, "tensor %llu has a zero dimension",
                           (unsigned long long)i);
        if (elements > UINT64_MAX / t->dimensions[d])
            return kq_fail(c->diag, KQ_STATUS_ARITHMETIC_OVERFLOW,
                           "tensor %llu element count overflows", (unsigned long long)i);
        elements *= t->dimensions[d];
    }
    st = cur_u32(c, &t->type_id);
    if (st != KQ_STATUS_OK) return st;
    info = kq_gguf_type_info_for(t->type_id);
    if (info == NULL)
        return kq_fail(c->diag, KQ_STATUS_UNSUPPORTED_TENSOR_TYPE,
                       "tensor %llu has GGML type %u, which is not supported",
                       (unsigned long long)i, t->type_id);
    st = cur_uint(c, 8u, &t->relative_offset);
    if (st != KQ_STATUS_OK) return st;
    if (t->relative_offset % g->alignment != 0u)
        return kq_fail(c->diag, KQ_STATUS_INVALID_ALIGNMENT,
                       "tensor %llu offset %llu is not a multiple of %llu", (unsigned long long)i,
                       (unsigned long long)t->relative_offset, (unsigned long long)g->alignment);
    if (t->dimensions[0] % info->block_elements != 0u)
        return kq_fail(c->diag, KQ_STATUS_MALFORMED_TENSOR,
                       "tensor %llu rows of %llu elements are not whole %llu-element blocks",
                       (unsigned long long)i, (unsigned long long)t->dimensions[0],
                       (unsigned long long)info->block_elements);
    blocks = elements / info->block_elements;
    if (blocks > UINT64_MAX / info->bytes_per_block)
        return kq_fail(c->diag, KQ_STATUS_ARITHMETIC_OVERFLOW,
                       "tensor %llu packed size overflows", (unsigned long long)i);
    t->packed_bytes = blocks * info->bytes_per_block;
    t->block_elements = info->block_elements;
    t->bytes_per_block = info->bytes_per_block;
    t->element_count = elements;
    return KQ_STATUS_OK;
}

static kq_status read_tensors(cursor *c, kq_gguf *g) {
    name_set seen;
    uint64_t i;
    kq_status st = KQ_STATUS_OK;
    if (!set_init(&seen, g->tensor_count))
        return kq_fail(c->diag, KQ_STATUS_OUT_OF_MEMORY, "tensor name set allocation failed");
    for (i = 0u; i < g->tensor_count && st == KQ_STATUS_OK; ++i) {
        st = cur_string(c, &g->tensors[i].name);
        if (st != KQ_STATUS_OK) break;
        if (set_seen(&seen, &g->tensors[i].name)) {
            st = kq_fail(c->diag, KQ_STATUS_DUPLICATE_TENSOR,
                         "GGUF tensor %llu repeats an earlier name", (unsigned long long)i);
            break;
        }
        st = read_tensor(c, g, i);
    }
    free(seen.slot);
    return st;
}

typedef struct span_key {
    uint64_t offset;
    uint64_t index;
} span_key;

static int span_cmp(const void *a, const void *b) {
    const span_key *x = (const span_key *)a, *y = (const span_key *)b;
    if (x->offset != y->offset) return x->offset < y->offset ? -1 : 1;
    return x->index < y->index ? -1 : (x->index > y->index);
}

/* Tensors sorted by offset must tile the data section from relative 0
 * without overlap and end inside the file. */
static kq_status check_spans(kq_gguf *g, kq_diagnostic *diag) {
    const uint64_t file_bytes = kq_file_size(g->file);
    uint64_t i, total = 0u;
    span_key *order;
    kq_status st = KQ_STATUS_OK;
    if (g->tensor_count > (uint64_t)(((size_t)-1) / sizeof(span_key)))
        return kq_fail(diag, KQ_STATUS_ARITHMETIC_OVERFLOW, "tensor order does not fit memory");
    order = (span_key *)malloc((size_t)g->tensor_count * sizeof(span_key));
    if (order == NULL) return kq_fail(diag, KQ_STATUS_OUT_OF_MEMORY, "tensor order allocation failed");
    for (i = 0u; i < g->tensor_count; ++i) {
        order[i].offset = g->tensors[i].relative_offset;
        order[i].index = i;
    }
    qsort(order, (size_t)g->tensor_count, sizeof(span_key), span_cmp);
    if (order[0].offset != 0u)
        st = kq_fail(diag, KQ_STATUS_INCONSISTENT_DATA_SECTION,
                     "the first tensor starts at relative offset %llu, not 0",
                     (unsigned long long)order[0].offset);
    for (i = 0u; i < g->tensor_count && st == KQ_STATUS_OK; ++i) {
        const uint64_t k = order[i].index;
        kq_gguf_tensor *t = &g->tensors[k];
        uint64_t rel_end, abs_end;
        if (t->packed_bytes > UINT64_MAX - t->relative_offset ||
            t->relative_offset > UINT64_MAX - g->data_section ||
            t->packed_bytes > UINT64_MAX - (g->data_section + t->relative_offset)) {
            st = kq_fail(diag, KQ_STATUS_ARITHMETIC_OVERFLOW, "tensor %llu span overflows",
                         (unsigned long long)k);
            break;
        }
        rel_end = t->relative_offset + t->packed_bytes;
        t->data_offset = g->data_section + t->relative_offset;
        abs_end = t->data_offset + t->packed_bytes;
        if (abs_end > file_bytes) {
            st = kq_fail(diag, KQ_STATUS_SPAN_OUT_OF_RANGE,
                         "tensor %llu ends at byte %llu of a %llu-byte file", (unsigned long long)k,
                         (unsigned long long)abs_end, (unsigned long long)file_bytes);
            break;
        }
        if (i + 1u < g->tensor_count && rel_end > order[i + 1u].offset) {
            st = kq_fail(diag, KQ_STATUS_INCONSISTENT_DATA_SECTION,
                         "tensor %llu overlaps the tensor after it", (unsigned long long)k);
            break;
        }
        if (t->packed_bytes > UINT64_MAX - total) {
            st = kq_fail(diag, KQ_STATUS_ARITHMETIC_OVERFLOW, "total packed bytes overflow");
            break;
        }
        total += t->packed_bytes;
    }
    free(order);
    if (st != KQ_STATUS_OK) return st;
    if (total > file_bytes)
        return kq_fail(diag, KQ_STATUS_INCONSISTENT_DATA_SECTION,
                       "packed tensor bytes exceed the file size");
    g->packed_bytes = total;
    g->overhead_bytes = file_bytes - total;
    return KQ_STATUS_OK;
}

/* ------------------------------------------------------------------ */
/* open / close */

static kq_status read_directory(kq_gguf *g, uint64_t file_bytes, kq_diagnostic *diag) {
    cursor c;
    uint64_t magic, version, tensors, entries;
    kq_status st;
    c.base = kq_file_view_data(g->view);
    c.view_bytes = kq_file_view_length(g->view);
    c.file_bytes = file_bytes;
    c.at = 0u;
    c.furthest = 0u;
    c.diag = diag;
    st = cur_uint(&c, 4u, &magic);
    if (st != KQ_STATUS_OK) return st;
    if (magic != 0x46554747u) /* "GGUF" little-endian */
        return kq_fail(diag, KQ_STATUS_BAD_MAGIC, "the file does not start with GGUF");
    st = cur_uint(&c, 4u, &version);
    if (st != KQ_STATUS_OK) return st;
    if (version != 3u)
        return kq_fail(diag, KQ_STATUS_UNSUPPORTED_VERSION, "GGUF version %llu; only 3 is read",
                       (unsigned long long)version);
    st = cur_uint(&c, 8u, &tensors);
    if (st == KQ_STATUS_OK) st = cur_uint(&c, 8u, &entries);
    if (st != KQ_STATUS_OK) return st;
    if (tensors == 0u || entries == 0u)
        return kq_fail(diag, KQ_STATUS_MALFORMED_METADATA,
                       "GGUF needs at least one tensor and one metadata entry");
    if (entries > (uint64_t)(((size_t)-1) / sizeof(kq_gguf_metadata)) ||
        tensors > (uint64_t)(((size_t)-1) / sizeof(kq_gguf_tensor)))
        return kq_fail(diag, KQ_STATUS_ARITHMETIC_OVERFLOW,
                       "GGUF directory counts do not fit memory");
    if (entries > KQ_GGUF_METADATA_LIMIT || tensors > KQ_GGUF_TENSOR_LIMIT)
        return kq_fail(diag, KQ_STATUS_LIMIT_EXCEEDED,
                       "GGUF holds %llu metadata entries and %llu tensors (limits 1024 and 8192)",
                       (unsigned long long)entries, (unsigned long long)tensors);
    g->version = (uint32_t)version;
    g->metadata_count = entries;
    g->tensor_count = tensors;
    g->metadata = (kq_gguf_metadata *)calloc((size_t)entries, sizeof(kq_gguf_metadata));
    g->tensors = (kq_gguf_tensor *)calloc((size_t)tensors, sizeof(kq_gguf_tensor));
    if (g->metadata == NULL || g->tensors == NULL)
        return kq_fail(diag, KQ_STATUS_OUT_OF_MEMORY, "GGUF descriptor allocation failed");
    st = read_metadata(&c, g);
    if (st == KQ_STATUS_OK) st = read_tensors(&c, g);
    if (st != KQ_STATUS_OK) return st;
    g->directory_end = c.at;
    g->bytes_parsed = c.furthest;
    /* alignment <= 4096, so only a directory end near 2^64 can overflow */
    if (g->directory_end > UINT64_MAX - (g->alignment - 1u))
        return kq_fail(diag, KQ_STATUS_ARITHMETIC_OVERFLOW, "data section offset overflows");
    g->data_section = (g->directory_end + g->alignment - 1u) & ~(g->alignment - 1u);
    if (g->data_section > file_bytes)
        return kq_fail(diag, KQ_STATUS_INCONSISTENT_DATA_SECTION,
                       "the data section would start past the end of the file");
    return check_spans(g, diag);
}

kq_status kq_gguf_open(kq_file *file, kq_gguf **out, kq_diagnostic *diag) {
    uint64_t file_bytes;
    kq_gguf *g;
    kq_status st;
    kq_diagnostic_clear(diag);
    if (file == NULL || out == NULL)
        return kq_fail(diag, KQ_STATUS_INVALID_ARGUMENT, "file and output GGUF are required");
    *out = NULL;
    file_bytes = kq_file_size(file);
    if (file_bytes < kFixedHeader)
        return kq_fail(diag, KQ_STATUS_TRUNCATED,
                       "a %llu-byte file is shorter than the 24-byte GGUF header",
                       (unsigned long long)file_bytes);
    g = (kq_gguf *)calloc(1u, sizeof(*g));
    if (g == NULL) return kq_fail(diag, KQ_STATUS_OUT_OF_MEMORY, "GGUF allocation failed");
    g->file = file;
    st = kq_file_view_open(file, 0u, file_bytes < KQ_GGUF_VIEW_LIMIT ? file_bytes : KQ_GGUF_VIEW_LIMIT,
                           &g->view, diag);
    if (st == KQ_STATUS_OK) st = read_directory(g, file_bytes, diag);
    if (st != KQ_STATUS_OK) {
        kq_gguf_close(g);
        return st;
    }
    *out = g;
    return KQ_STATUS_OK;
}

void kq_gguf_close(kq_gguf *g) {
    if (g == NULL) return;
    free(g->tensors);
    free(g->metadata);
    kq_file_view_close(g->view);
    free(g);
}

/* ------------------------------------------------------------------ */
/* accessors */

uint32_t kq_gguf_version(const kq_gguf *g) { return g ? g->version : 0u; }
uint64_t kq_gguf_metadata_count(const kq_gguf *g) { return g ? g->metadata_count : 0u; }
uint64_t kq_gguf_tensor_count(const kq_gguf *g) { return g ? g->tensor_count : 0u; }
uint64_t kq_gguf_alignment(const kq_gguf *g) { return g ? g->alignment : 0u; }
uint64_t kq_gguf_directory_end_offset(const kq_gguf *g) { return g ? g->directory_end : 0u; }
uint64_t kq_gguf_data_section_offset(const kq_gguf *g) { return g ? g->data_section : 0u; }
uint64_t kq_gguf_packed_tensor_bytes(const kq_gguf *g) { return g ? g->packed_bytes : 0u; }
uint64_t kq_gguf_format_overhead_bytes(const kq_gguf *g) { return g ? g->overhead_bytes : 0u; }
uint64_t kq_gguf_directory_bytes_parsed(const kq_gguf *g) { return g ? g->bytes_parsed : 0u; }
uint64_t kq_gguf_payload_bytes_accessed(const kq_gguf *g) { (void)g; return 0u; }

kq_string_view kq_gguf_architecture(const kq_gguf *g) {
    kq_string_view none = {NULL, 0u};
    return g ? g->architecture : none;
}

const kq_gguf_metadata *kq_gguf_metadata_at(const kq_gguf *g, uint64_t i) {
    return g != NULL && i < g->metadata_count ? &g->metadata[i] : NULL;
}

const kq_gguf_metadata *kq_gguf_find_metadata(const kq_gguf *g, const char *key) {
    uint64_t i;
    if (g == NULL || key == NULL) return NULL;
    for (i = 0u; i < g->metadata_count; ++i)
        if (kq_string_view_equal_cstr(&g->metadata[i].key, key)) return &g->metadata[i];
    return NULL;
}

const kq_gguf_tensor *kq_gguf_tensor_at(const kq_gguf *g, uint64_t i) {
    return g != NULL && i < g->tensor_count ? &g->tensors[i] : NULL;
}

const kq_gguf_tensor *kq_gguf_find_tensor(const kq_gguf *g, const char *name) {
    uint64_t i;
    if (g == NULL || name == NULL) return NULL;
    for (i = 0u; i < g->tensor_count; ++i)
        if (kq_string_view_equal_cstr(&g->tensors[i].name, name)) return &g->tensors[i];
    return NULL;
}

static int scalar_of(const kq_gguf_metadata *m, uint32_t type, void *out) {
    return m != NULL && out != NULL && m->value_type == type;
}

int kq_gguf_metadata_u16(const kq_gguf_metadata *m, uint16_t *v) {
    if (!scalar_of(m, KQ_GGUF_VALUE_UINT16, v)) return 0;
    *v = (uint16_t)m->scalar_value;
    return 1;
}

int kq_gguf_metadata_u32(const kq_gguf_metadata *m, uint32_t *v) {
    if (!scalar_of(m, KQ_GGUF_VALUE_UINT32, v)) return 0;
    *v = (uint32_t)m->scalar_value;
    return 1;
}

int kq_gguf_metadata_i32(const kq_gguf_metadata *m, int32_t *v) {
    uint32_t bits;
    if (!scalar_of(m, KQ_GGUF_VALUE_INT32, v)) return 0;
    bits = (uint32_t)m->scalar_value;
    memcpy(v, &bits, sizeof(bits));
    return 1;
}

static const unsigned char *array_item(const kq_gguf_metadata *m, uint32_t type,
                                       uint64_t index, const void *out, unsigned width) {
    if (m == NULL || out == NULL || m->value_type != KQ_GGUF_VALUE_ARRAY ||
        m->array_element_type != type || index >= m->array_length || m->array_data.data == NULL)
        return NULL;
    return m->array_data.data + index * width;
}

int kq_gguf_metadata_array_i32_at(const kq_gguf_metadata *m, uint64_t index, int32_t *v) {
    const unsigned char *p = array_item(m, KQ_GGUF_VALUE_INT32, index, v, 4u);
    uint32_t bits;
    if (p == NULL) return 0;
    bits = (uint32_t)load_le(p, 4u);
    memcpy(v, &bits, sizeof(bits));
    return 1;
}

int kq_gguf_metadata_array_u64_at(const kq_gguf_metadata *m, uint64_t index, uint64_t *v) {
    const unsigned char *p = array_item(m, KQ_GGUF_VALUE_UINT64, index, v, 8u);
    if (p == NULL) return 0;
    *v = load_le(p, 8u);
    return 1;
}

/* Walks the length-prefixed strings up to `index` (their bounds were
 * checked while parsing; they are checked again against array_data). */
int kq_gguf_metadata_array_string_at(const kq_gguf_metadata *m, uint64_t index,
                                     kq_string_view *v) {
    uint64_t at = 0u, k, n;
    if (array_item(m, KQ_GGUF_VALUE_STRING, index, v, 0u) == NULL) return 0;
    for (k = 0u;; ++k) {
        if (m->array_data.length - at < 8u) return 0;
        n = load_le(m->array_data.data + at, 8u);
        at += 8u;
        if (n > m->array_data.length - at) return 0;
        if (k == index) {
            v->data = m->array_data.data + at;
            v->length = n;
            return 1;
        }
        at += n;
    }
}

/* ------------------------------------------------------------------ */
/* payload spans (internal) */

int kqi_gguf_owns(const kq_gguf *g, const kq_gguf_tensor *t) {
    uintptr_t at;
    if (g == NULL || t == NULL || (uintptr_t)t < (uintptr_t)g->tensors) return 0;
    at = (uintptr_t)t - (uintptr_t)g->tensors;
    return at < g->tensor_count * sizeof(kq_gguf_tensor) && at % sizeof(kq_gguf_tensor) == 0u;
}

kq_status kqi_gguf_tensor_span(const kq_gguf *g, const kq_gguf_tensor *t, uint64_t byte_offset,
                               uint64_t byte_count, kq_file_view **out, kq_diagnostic *diag) {
    kq_diagnostic_clear(diag);
    if (g == NULL || t == NULL || out == NULL || byte_count == 0u)
        return kq_fail(diag, KQ_STATUS_INVALID_ARGUMENT,
                       "GGUF, tensor, output view and a non-zero span are required");
    *out = NULL;
    if (!kqi_gguf_owns(g, t))
        return kq_fail(diag, KQ_STATUS_TENSOR_OWNERSHIP_MISMATCH,
                       "the tensor descriptor does not belong to this GGUF");
    if (byte_offset > UINT64_MAX - byte_count)
        return kq_fail(diag, KQ_STATUS_ARITHMETIC_OVERFLOW, "tensor span overflows");
    if (byte_offset + byte_count > t->packed_bytes)
        return kq_fail(diag, KQ_STATUS_SPAN_OUT_OF_RANGE,
                       "span [%llu, %llu) passes the tensor's %llu packed bytes",
                       (unsigned long long)byte_offset,
                       (unsigned long long)(byte_offset + byte_count),
                       (unsigned long long)t->packed_bytes);
    return kq_file_view_open(g->file, t->data_offset + byte_offset, byte_count, out, diag);
}
