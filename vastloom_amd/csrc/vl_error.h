// Thread-local last-error message of the C ABI (vl_last_error), shared by the host sources.
#ifndef VL_ERROR_H
#define VL_ERROR_H

namespace vl {

// Records the message for vl_last_error() on this thread and returns code.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

}  // namespace vl

#endif  // VL_ERROR_H
