// host_err.h -- the library's thread-local error message, shared by its host sources.
//
// Every C-ABI call returns an LFM_* status; on failure the message set here is what
// lfm_last_error() returns on the same thread.
#pragma once

#include <stdarg.h>
#include <stddef.h>
#include <stdint.h>

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

// Checks one tensor's type and shape as lfm_engine_upload_tensor takes
// them (F32 or Q6_K, 1..4 dimensions, none of them zero, Q6_K rows a multiple of
// 256) and sets *want to the bytes the tensor must have.  Host-only: the GGUF
// loaders run it over a whole file before any device work.
__attribute__((visibility("hidden"))) int lfm_check_tensor(const char *name, uint32_t type,
                                                           const uint64_t *ne, uint32_t nd,
                                                           size_t *want);
