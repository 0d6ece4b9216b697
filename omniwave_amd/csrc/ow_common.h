// Shared host-side helpers of libomniwave_amd: thread-local error text and argument checks.
#pragma once

#include <cstdarg>
#include <cstdio>

#include "omniwave_amd.h"

namespace ow {

// Records a printf-style message for ow_last_error() and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

}  // namespace ow

#define OW_CHECK_ARG(cond, ...)                                  \
  do {                                                           \
    if (!(cond)) return ::ow::fail(OW_ERR_INVALID, __VA_ARGS__); \
  } while (0)

#define OW_CHECK_SUPPORTED(cond, ...)                                \
  do {                                                               \
    if (!(cond)) return ::ow::fail(OW_ERR_UNSUPPORTED, __VA_ARGS__); \
  } while (0)
