/* log.c -- per-thread last error and warnings (RustFox src/log.c:40-105). */
#include "fox_host_internal.h"

#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static _Thread_local char g_err[512];

fox_status fox_fail(fox_status st, const char *fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return st;
}

void fox_warn(const char *fmt, ...)
{
    const char *lv = getenv("FOX_LOG");
    va_list ap;
    if (lv && (strcmp(lv, "error") == 0 || strcmp(lv, "0") == 0)) return;
    fputs("fox warn  ", stderr);
    va_start(ap, fmt);
    vfprintf(stderr, fmt, ap);
    va_end(ap);
    fputc('\n', stderr);
}

fox_status fox_gpu_failed(fox_gpu_status st, const char *what)
{
    const char *m = fox_gpu_last_error();
    return fox_fail((fox_status)st, "%s: %s", what, m && *m ? m : fox_gpu_status_str(st));
}

const char *fox_last_error(void) { return g_err; }

const char *fox_version(void) { return "0.1.0-mi355x"; }

const char *fox_status_str(fox_status s)
{
    switch (s) {
    case FOX_OK: return "ok";
    case FOX_ERR_ARG: return "invalid argument";
    case FOX_ERR_IO: return "i/o error";
    case FOX_ERR_NOMEM: return "out of memory";
    case FOX_ERR_FORMAT: return "bad format";
    case FOX_ERR_UNSUPPORTED: return "unsupported";
    case FOX_ERR_NOTFOUND: return "not found";
    case FOX_ERR_INTERNAL: return "internal error";
    }
    return "unknown status";
}
