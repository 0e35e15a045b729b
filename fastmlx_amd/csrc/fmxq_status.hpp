// fmxq_status.hpp -- fmxq::fail, the error recorder behind fmxq_last_error
// (fmxq_status.cpp).  No HIP types, so host-only sources can use it.
#pragma once

namespace fmxq {

// Records a message for fmxq_last_error() and returns code.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

}  // namespace fmxq
