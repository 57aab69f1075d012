#ifndef KQ_STATUS_INTERNAL_H
#define KQ_STATUS_INTERNAL_H

#include "kq_status.h"

/* Sets status and a printf-style message; returns status. */
kq_status kq_fail(kq_diagnostic *diagnostic, kq_status status, const char *format, ...)
    __attribute__((format(printf, 3, 4)));

#endif
