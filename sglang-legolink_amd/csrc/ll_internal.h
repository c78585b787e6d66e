// Shared by the library's translation units; not part of the C ABI.
#ifndef LL_INTERNAL_H
#define LL_INTERNAL_H

#include <stdarg.h>

// Records the thread's last error message (ll_last_error) and returns code.
__attribute__((visibility("hidden"))) int ll_record_error(int code, const char *fmt, va_list ap);

#endif  // LL_INTERNAL_H
