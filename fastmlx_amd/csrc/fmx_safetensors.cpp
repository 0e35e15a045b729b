// fmx_safetensors.cpp -- the upload of one safetensors tensor into an fmx_array,
// the per-tensor step of compute/loader.go LoadTensors (:61-84).  The header
// parser and the accessors it uses are fmx_st_parse.cpp.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <vector>

#include "../../include/fmx.h"
#include "../../include/fmxq.h"
#include "fmxq_host.hpp"

using fmxq::fail;

extern "C" {

int fmx_safetensors_load(fmx_array* res, const uint8_t* blob, uint64_t len,
                         const fmx_st_header* h, int64_t i) {
  if (!res) return fail(FMXQ_ERR_INVALID_ARGUMENT, "safetensors: null result");
  const char *name = nullptr, *tag = nullptr;
  int ndim = 0;
  const int64_t* shape = nullptr;
  uint64_t b = 0, e = 0, off = 0;
  if (int rc = fmx_safetensors_tensor(h, i, &name, &tag, &ndim, &shape, &b, &e)) return rc;
  fmx_dtype dt;
  if (fmx_safetensors_dtype(tag, &dt) != FMXQ_OK)
    return fail(FMXQ_ERR_UNSUPPORTED, "safetensors: tensor \"%s\" has unsupported dtype \"%s\"",
                name, tag);
  if (int rc = fmx_safetensors_slice(len, fmx_safetensors_data_start(h), b, e, &off)) return rc;
  std::vector<int> sh((size_t)ndim);
  for (int d = 0; d < ndim; ++d) {
    if (shape[d] > INT32_MAX)
      return fail(FMXQ_ERR_SHAPE, "safetensors: tensor \"%s\" axis %d too long", name, d);
    sh[(size_t)d] = (int)shape[d];
  }
  fmx_array a = fmx_array_new_data(blob + off, sh.data(), ndim, dt);
  if (!a.ctx) return FMXQ_ERR_DEVICE;  // fmx_array_new_data set the message
  if (res->ctx) fmx_array_free(*res);
  *res = a;
  return FMXQ_OK;
}

}  // extern "C"
