// Status codes and the thread-local last-error message shared by the C ABI.
#pragma once

#include <cstdarg>
#include <cstdio>
#include <string>

#include "air_kv.h"

namespace airkv {

std::string &last_error_slot();

// Records `msg` as this thread's last error and returns `code`.
inline int fail(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    last_error_slot() = buf;
    return code;
}

}  // namespace airkv
