// fmxq_status.cpp -- the library's error messages: fmxq::fail records the text of
// a failing call for fmxq_last_error.  Plain host C++ (no HIP), so the host-side
// parsers can be built and tested on their own.
#include <cstdarg>
#include <cstdio>
#include <mutex>

#include "../../include/fmxq.h"
#include "fmxq_status.hpp"

namespace {

std::mutex g_err_mu;
// The returned pointer must survive until the next failure; keep two buffers
// and alternate so a reader of the previous message is not overwritten mid-read.
char g_err_buf[2][512];
int g_err_slot = 0;

}  // namespace

namespace fmxq {

int fail(int code, const char* fmt, ...) {
  char tmp[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(tmp, sizeof(tmp), fmt, ap);
  va_end(ap);
  std::lock_guard<std::mutex> lk(g_err_mu);
  g_err_slot ^= 1;
  std::snprintf(g_err_buf[g_err_slot], sizeof(g_err_buf[0]), "%s", tmp);
  return code;
}

}  // namespace fmxq

extern "C" const char* fmxq_last_error(void) {
  std::lock_guard<std::mutex> lk(g_err_mu);
  return g_err_buf[g_err_slot];
}
