/*
 * kq_file_posix.c — the reference's read-only file and view layer
 * (include/kq_file.h:16-30, implemented for Windows in src/kq_file_win32.c)
 * on POSIX: a file is an open descriptor and its size; a view maps the
 * pages covering [offset, offset + length) and points at offset.
 */
#define _POSIX_C_SOURCE 200809L
#include "kq_file.h"

#include <errno.h>
#include <fcntl.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include "kq_status_internal.h"

struct kq_file {
    int fd;
    uint64_t size;
};

struct kq_file_view {
    void *base;       /* page-aligned mapping */
    size_t map_bytes; /* bytes mapped from base */
    uint64_t offset;  /* requested file offset */
    uint64_t length;  /* requested length */
    const unsigned char *data;
};

/* UTF-8 bytes of one code point into out (up to 4 bytes); 0 if invalid */
static size_t utf8_encode(uint32_t cp, char *out) {
    if (cp < 0x80u) {
        out[0] = (char)cp;
        return 1u;
    }
    if (cp < 0x800u) {
        out[0] = (char)(0xc0u | (cp >> 6));
        out[1] = (char)(0x80u | (cp & 0x3fu));
        return 2u;
    }
    if (cp >= 0xd800u && cp <= 0xdfffu) return 0u;
    if (cp < 0x10000u) {
        out[0] = (char)(0xe0u | (cp >> 12));
        out[1] = (char)(0x80u | ((cp >> 6) & 0x3fu));
        out[2] = (char)(0x80u | (cp & 0x3fu));
        return 3u;
    }
    if (cp <= 0x10ffffu) {
        out[0] = (char)(0xf0u | (cp >> 18));
        out[1] = (char)(0x80u | ((cp >> 12) & 0x3fu));
        out[2] = (char)(0x80u | ((cp >> 6) & 0x3fu));
        out[3] = (char)(0x80u | (cp & 0x3fu));
        return 4u;
    }
    return 0u;
}

kq_status kq_file_open_readonly(const wchar_t *path, kq_file **out_file,
                                kq_diagnostic *diagnostic) {
    size_t n, i, at = 0u;
    char *utf8;
    kq_status st;
    kq_diagnostic_clear(diagnostic);
    if (path == NULL || out_file == NULL)
        return kq_fail(diagnostic, KQ_STATUS_INVALID_ARGUMENT, "path and output file are required");
    *out_file = NULL;
    n = wcslen(path);
    if (n > ((size_t)-1) / 4u - 1u)
        return kq_fail(diagnostic, KQ_STATUS_ARITHMETIC_OVERFLOW, "path length overflows");
    utf8 = (char *)malloc(n * 4u + 1u);
    if (utf8 == NULL) return kq_fail(diagnostic, KQ_STATUS_OUT_OF_MEMORY, "path conversion failed");
    for (i = 0u; i < n; ++i) {
        const size_t k = utf8_encode((uint32_t)path[i], utf8 + at);
        if (k == 0u) {
            free(utf8);
            return kq_fail(diagnostic, KQ_STATUS_FILE_OPEN_FAILED,
                           "path holds a code point with no UTF-8 form");
        }
        at += k;
    }
    utf8[at] = '\0';
    st = kq_file_open_readonly_utf8(utf8, out_file, diagnostic);
    free(utf8);
    return st;
}

kq_status kq_file_open_readonly_utf8(const char *path, kq_file **out_file,
                                     kq_diagnostic *diagnostic) {
    struct stat sb;
    kq_file *f;
    int fd;
    kq_diagnostic_clear(diagnostic);
    if (path == NULL || out_file == NULL)
        return kq_fail(diagnostic, KQ_STATUS_INVALID_ARGUMENT, "path and output file are required");
    *out_file = NULL;
    fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0)
        return kq_fail(diagnostic, KQ_STATUS_FILE_OPEN_FAILED, "open failed: %s", strerror(errno));
    if (fstat(fd, &sb) != 0 || !S_ISREG(sb.st_mode) || sb.st_size < 0) {
        (void)close(fd);
        return kq_fail(diagnostic, KQ_STATUS_FILE_SIZE_FAILED,
                       "the path is not a regular file of known size");
    }
    f = (kq_file *)calloc(1u, sizeof(*f));
    if (f == NULL) {
        (void)close(fd);
        return kq_fail(diagnostic, KQ_STATUS_OUT_OF_MEMORY, "file allocation failed");
    }
    f->fd = fd;
    f->size = (uint64_t)sb.st_size;
    *out_file = f;
    return KQ_STATUS_OK;
}

uint64_t kq_file_size(const kq_file *file) { return file == NULL ? 0u : file->size; }

void kq_file_close(kq_file *file) {
    if (file == NULL) return;
    (void)close(file->fd);
    free(file);
}

kq_status kq_file_view_open(kq_file *file, uint64_t offset, uint64_t length,
                            kq_file_view **out_view, kq_diagnostic *diagnostic) {
    uint64_t end, page, start, delta;
    kq_file_view *v;
    void *base;
    kq_diagnostic_clear(diagnostic);
    if (file == NULL || out_view == NULL || length == 0u)
        return kq_fail(diagnostic, KQ_STATUS_INVALID_ARGUMENT,
                       "file, output view and a non-zero length are required");
    *out_view = NULL;
    if (offset > UINT64_MAX - length)
        return kq_fail(diagnostic, KQ_STATUS_ARITHMETIC_OVERFLOW, "view offset plus length overflows");
    end = offset + length;
    if (end > file->size)
        return kq_fail(diagnostic, KQ_STATUS_SPAN_OUT_OF_RANGE,
                       "view [%llu, %llu) passes the end of a %llu-byte file",
                       (unsigned long long)offset, (unsigned long long)end,
                       (unsigned long long)file->size);
    page = (uint64_t)sysconf(_SC_PAGESIZE);
    start = offset - offset % page;
    delta = offset - start;
    if (length + delta > (uint64_t)((size_t)-1))
        return kq_fail(diagnostic, KQ_STATUS_ARITHMETIC_OVERFLOW, "view does not fit the address space");
    base = mmap(NULL, (size_t)(length + delta), PROT_READ, MAP_PRIVATE, file->fd, (off_t)start);
    if (base == MAP_FAILED)
        return kq_fail(diagnostic, KQ_STATUS_FILE_MAP_FAILED, "mmap failed: %s", strerror(errno));
    v = (kq_file_view *)calloc(1u, sizeof(*v));
    if (v == NULL) {
        (void)munmap(base, (size_t)(length + delta));
        return kq_fail(diagnostic, KQ_STATUS_OUT_OF_MEMORY, "view allocation failed");
    }
    v->base = base;
    v->map_bytes = (size_t)(length + delta);
    v->offset = offset;
    v->length = length;
    v->data = (const unsigned char *)base + delta;
    *out_view = v;
    return KQ_STATUS_OK;
}

const unsigned char *kq_file_view_data(const kq_file_view *view) {
    return view == NULL ? NULL : view->data;
}

uint64_t kq_file_view_offset(const kq_file_view *view) { return view == NULL ? 0u : view->offset; }

uint64_t kq_file_view_length(const kq_file_view *view) { return view == NULL ? 0u : view->length; }

void kq_file_view_close(kq_file_view *view) {
    if (view == NULL) return;
    (void)munmap(view->base, view->map_bytes);
    free(view);
}
