// tpr_host.h -- host-only internals shared by the planner and the ABI layer.
#pragma once

#include <stdarg.h>
#include <stddef.h>
#include <stdint.h>

namespace tpr {

// Record a printf-style message as this thread's last error; returns `status`.
int fail(int status, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

// Kernel launchers (defined in the .hip translation units). Each returns a
// TprStatus and enqueues on `stream` (hipStream_t passed as void*).
struct FwdArgs;
struct BwdArgs;

}  // namespace tpr
