/*
 * kq_file.h — read-only files and mapped byte views, for POSIX systems.
 *
 * Replaces: include/kq_file.h:16-30 (the reference's file layer), whose only
 * implementation is src/kq_file_win32.c. These are the same entry points
 * with the same statuses, implemented with open/fstat/mmap:
 *   - kq_file_open_readonly: FILE_OPEN_FAILED, FILE_SIZE_FAILED;
 *   - kq_file_view_open: INVALID_ARGUMENT for a zero length,
 *     ARITHMETIC_OVERFLOW when offset + length overflows, SPAN_OUT_OF_RANGE
 *     past the end of the file, FILE_MAP_FAILED when the mapping fails.
 * A view may start at any byte; its data pointer is the requested offset.
 * Paths are wide strings as in the reference (converted to UTF-8), or UTF-8
 * through kq_file_open_readonly_utf8.
 */
#ifndef KQ_FILE_H
#define KQ_FILE_H

#include <stdint.h>
#include <wchar.h>

#include "kq_status.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct kq_file kq_file;
typedef struct kq_file_view kq_file_view;

kq_status kq_file_open_readonly(const wchar_t *path, kq_file **out_file,
                                kq_diagnostic *diagnostic);
/* No counterpart in the reference: the same open for a UTF-8 path. */
kq_status kq_file_open_readonly_utf8(const char *path, kq_file **out_file,
                                     kq_diagnostic *diagnostic);
uint64_t kq_file_size(const kq_file *file);
void kq_file_close(kq_file *file);

kq_status kq_file_view_open(kq_file *file, uint64_t offset, uint64_t length,
                            kq_file_view **out_view, kq_diagnostic *diagnostic);
const unsigned char *kq_file_view_data(const kq_file_view *view);
uint64_t kq_file_view_offset(const kq_file_view *view);
uint64_t kq_file_view_length(const kq_file_view *view);
void kq_file_view_close(kq_file_view *view);

#ifdef __cplusplus
}
#endif

#endif
