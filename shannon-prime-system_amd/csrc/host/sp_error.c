/* sp_error.c -- thread-local error detail (core/io_format/sp_error.c:50-63:
 * one 512-byte buffer per thread, truncating copy, NULL clears). */
#include "sp_l1_abi.h"
#include <string.h>

static _Thread_local char tls_err[512];

const char *sp_last_error(void) { return tls_err; }

void sp_set_error(const char *msg) {
    size_t n = msg ? strlen(msg) : 0;
    if (n > sizeof tls_err - 1) n = sizeof tls_err - 1;
    if (n) memcpy(tls_err, msg, n);
    tls_err[n] = '\0';
}
