// host_err.h -- the library's thread-local error message, shared by its host sources.
//
// Every C-ABI call returns an LFM_* status; on failure the message set here is what
// lfm_last_error() returns on the same thread.
#pragma once

#include <stdarg.h>

// Formats the message, stores it for lfm_last_error() and returns `code`.
__attribute__((visibility("hidden"))) int lfm_vfail(int code, const char *fmt, va_list ap);

__attribute__((format(printf, 2, 3))) static inline int fail(int code, const char *fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    const int rc = lfm_vfail(code, fmt, ap);
    va_end(ap);
    return rc;
}
