// fmx_array.cpp -- the array-handle layer of libfmxq.so (include/fmx.h).
//
// The reference reaches the quantized kernels through mlx-c handles
// (mlxgo/binding_cgo.go:71-275 for arrays and streams, :636-682 for the three
// ops).  This file gives those calls the same shapes and ownership rules over the
// raw pointer ABI of fmxq_capi.cpp:
//   * an array is device memory plus shape/dtype; ops allocate their result;
//   * execution is eager: an op has enqueued its kernels on the stream when it
//     returns; eval waits for the producing stream and reports index errors;
//   * result buffers come from a per-(device, stream) cache keyed by rounded
//     size, so a decode loop that frees its intermediates reuses them without
//     hipMalloc.  A buffer returns to the cache of the stream that produced it;
//     reads by other streams are fenced with events before it can be reused;
//   * an input produced on another stream is waited for with an event.
// Validation precedes every HIP call, so a rejected op touches no device state.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/fmx.h"
#include "../../include/fmxq.h"
#include "fmx_shape.hpp"
#include "fmxq_host.hpp"
#include "fmxq_internal.hpp"

using fmxq::check_quant;
using fmxq::fail;
using fmxq::hip_status;
using fmx_shape::dtype_name;
using fmx_shape::dtype_size;
using fmx_shape::is_index_dtype;
using fmx_shape::is_signed_dtype;
using fmx_shape::prod;
using fmx_shape::shape_str;

namespace {

struct Stream {
  hipStream_t s = nullptr;
  bool singleton = false;  // the per-device default stream object; never deleted
};

enum class Storage { kNone, kMalloc, kPooled, kBorrowed };

struct Array {
  std::vector<int64_t> shape;
  fmx_dtype dtype = FMX_FLOAT32;
  void* data = nullptr;
  size_t cap = 0;                 // allocation size (rounded, for the cache)
  Storage storage = Storage::kNone;
  int device = -1;                // -1: borrowed memory of unknown device
  hipStream_t stream = nullptr;   // stream that produces the data (null: already complete)
  bool check_index = false;       // a gather produced it: eval reports index errors
  std::vector<hipStream_t> readers;  // other streams that read it
  std::vector<unsigned char> host;   // host copy behind data_float32 / data_int32
  int64_t numel() const { return prod(shape); }
  size_t nbytes() const { return (size_t)numel() * dtype_size(dtype); }
};

Array* arr(const fmx_array a) { return static_cast<Array*>(a.ctx); }

// ---- device buffer cache ----

fmx_shape::BufferCache g_cache;

int pool_alloc(int dev, hipStream_t s, size_t n, void** out, size_t* cap) {
  const size_t want = fmx_shape::round_bytes(n);
  if (g_cache.take(dev, s, want, out)) {
    *cap = want;
    return FMXQ_OK;
  }
  void* p = nullptr;
  hipError_t e = hipMalloc(&p, want);
  if (e != hipSuccess) {
    // Give cached buffers back to the device and try once more.
    const std::vector<void*> drop = g_cache.drain(dev);
    if (!drop.empty()) {
      (void)hipDeviceSynchronize();
      for (void* b : drop) (void)hipFree(b);
      e = hipMalloc(&p, want);
    }
    if (e != hipSuccess) return hip_status(e, "fmx: hipMalloc");
  }
  *out = p;
  *cap = want;
  return FMXQ_OK;
}

// Fence: work enqueued on `waiter` after this waits for everything enqueued on
// `signaller` so far.
int fence(hipStream_t waiter, hipStream_t signaller) {
  hipEvent_t ev;
  if (int rc = hip_status(hipEventCreateWithFlags(&ev, hipEventDisableTiming), "fmx: event"))
    return rc;
  int rc = hip_status(hipEventRecord(ev, signaller), "fmx: event record");
  if (!rc) rc = hip_status(hipStreamWaitEvent(waiter, ev, 0), "fmx: stream wait");
  (void)hipEventDestroy(ev);
  return rc;
}

void release_storage(Array* a) {
  if (a->storage == Storage::kPooled && a->data) {
    for (hipStream_t r : a->readers) (void)fence(a->stream, r);
    g_cache.put(a->device, a->stream, a->cap, a->data);
  } else if (a->storage == Storage::kMalloc && a->data) {
    (void)hipFree(a->data);
  }
  a->data = nullptr;
  a->cap = 0;
  a->storage = Storage::kNone;
  a->readers.clear();
  a->host.clear();
  a->host.shrink_to_fit();
}

// ---- streams ----

std::mutex g_stream_mu;
std::vector<Stream*> g_default;  // one per device, created on first use

int default_stream(Stream** out) {
  int dev = 0;
  if (int rc = hip_status(hipGetDevice(&dev), "fmx: hipGetDevice")) return rc;
  std::lock_guard<std::mutex> lk(g_stream_mu);
  if ((int)g_default.size() <= dev) g_default.resize(dev + 1, nullptr);
  if (!g_default[dev]) {
    hipStream_t s = nullptr;
    // A blocking stream (default flags) is ordered with the null stream, so work
    // other libraries enqueue there is seen by these ops without extra fences.
    if (int rc = hip_status(hipStreamCreate(&s), "fmx: hipStreamCreate")) return rc;
    g_default[dev] = new Stream{s, true};
  }
  *out = g_default[dev];
  return FMXQ_OK;
}

int resolve_stream(const fmx_stream s, hipStream_t* out) {
  if (s.ctx) {
    *out = static_cast<Stream*>(s.ctx)->s;
    return FMXQ_OK;
  }
  Stream* d = nullptr;
  if (int rc = default_stream(&d)) return rc;
  *out = d->s;
  return FMXQ_OK;
}

// ---- op plumbing ----

int need(const fmx_array h, const char* op, const char* name, Array** out) {
  Array* a = arr(h);
  if (!a) return fail(FMXQ_ERR_INVALID_ARGUMENT, "%s: %s is an empty array", op, name);
  if (a->numel() > 0 && !a->data)
    return fail(FMXQ_ERR_INVALID_ARGUMENT, "%s: %s has no data", op, name);
  *out = a;
  return FMXQ_OK;
}

int need_dtype(const Array* a, int dtype, const char* op, const char* name) {
  if (a->dtype != dtype)
    return fail(FMXQ_ERR_UNSUPPORTED, "%s: %s has dtype %s, need %s", op, name,
                dtype_name(a->dtype), dtype_name(dtype));
  return FMXQ_OK;
}

int need_shape(const Array* a, const std::vector<int64_t>& want, const char* op,
               const char* name) {
  if (a->shape != want)
    return fail(FMXQ_ERR_SHAPE, "%s: %s has shape %s, need %s", op, name,
                shape_str(a->shape).c_str(), shape_str(want).c_str());
  return FMXQ_OK;
}

int unpacked_k(const Array* w, int bits, const char* op, int64_t* K) {
  return fmx_shape::unpacked_k(w->shape, bits, op, K);
}

// Everything an op needs once validation has passed.
struct Launch {
  int dev = 0;
  hipStream_t s = nullptr;
  std::vector<Array*> inputs;
  std::vector<std::pair<void*, size_t>> temps;  // cached index buffers, returned after enqueue
};

int begin(Launch& L, const fmx_stream s, const std::vector<Array*>& inputs) {
  if (int rc = resolve_stream(s, &L.s)) return rc;
  if (int rc = hip_status(hipGetDevice(&L.dev), "fmx: hipGetDevice")) return rc;
  for (Array* a : inputs) {
    if (!a) continue;
    if (a->device >= 0 && a->device != L.dev)
      return fail(FMXQ_ERR_INVALID_ARGUMENT, "fmx: operand lives on device %d, current is %d",
                  a->device, L.dev);
    L.inputs.push_back(a);
  }
  for (Array* a : L.inputs)
    if (a->storage == Storage::kPooled && a->stream != L.s)
      if (int rc = fence(L.s, a->stream)) return rc;
  return FMXQ_OK;
}

int temp(Launch& L, size_t bytes, void** out) {
  size_t cap = 0;
  if (int rc = pool_alloc(L.dev, L.s, bytes, out, &cap)) return rc;
  L.temps.emplace_back(*out, cap);
  return FMXQ_OK;
}

// Called on success and failure alike once kernels may have been enqueued.
void finish(Launch& L) {
  for (Array* a : L.inputs)
    if (a->storage == Storage::kPooled && a->stream != L.s &&
        std::find(a->readers.begin(), a->readers.end(), L.s) == a->readers.end())
      a->readers.push_back(L.s);
  for (auto& t : L.temps) g_cache.put(L.dev, L.s, t.second, t.first);
  L.temps.clear();
}

int new_result(Launch& L, std::vector<int64_t> shape, fmx_dtype dtype, Array** out) {
  Array* r = new Array;
  r->shape = std::move(shape);
  r->dtype = dtype;
  r->device = L.dev;
  r->stream = L.s;
  const size_t n = r->nbytes();
  if (n > 0) {
    if (int rc = pool_alloc(L.dev, L.s, n, &r->data, &r->cap)) {
      delete r;
      return rc;
    }
    r->storage = Storage::kPooled;
  }
  *out = r;
  return FMXQ_OK;
}

// Installs r into *res (replacing what it held) or discards r on failure.
int commit(fmx_array* res, Array* r, int rc) {
  if (rc) {
    release_storage(r);
    delete r;
    return rc;
  }
  if (res->ctx) {
    Array* old = arr(*res);
    release_storage(old);
    *old = std::move(*r);
    delete r;
  } else {
    res->ctx = r;
  }
  return FMXQ_OK;
}

// The flat uint32 index vector a gather kernel reads for `src` (an integer array
// broadcast to `bshape`), or for the arange over `arange_shape` when src is null.
int index_vector(Launch& L, const Array* src, const std::vector<int64_t>& arange_shape,
                 const std::vector<int64_t>& bshape, const uint32_t** out) {
  const int64_t n = prod(bshape);
  const std::vector<int64_t>& sshape = src ? src->shape : arange_shape;
  // Already flat and of the right width: use in place.
  if (src && (src->dtype == FMX_UINT32 || src->dtype == FMX_INT32) &&
      fmx_shape::same_elements(sshape, bshape)) {
    *out = static_cast<const uint32_t*>(src->data);
    return FMXQ_OK;
  }
  fmx_shape::BroadcastMap bm;
  if (int rc = fmx_shape::broadcast_map(sshape, bshape, &bm, "gather_qmm")) return rc;
  static_assert(fmx_shape::kMaxIndexDims == fmxq::kMaxIndexDims, "index axes");
  fmxq::IndexMap m{};
  m.ndim = bm.ndim;
  m.elem_bytes = src ? (int)dtype_size(src->dtype) : 4;
  m.is_signed = src ? is_signed_dtype(src->dtype) : false;
  for (int d = 0; d < bm.ndim; ++d) {
    m.shape[d] = bm.shape[d];
    m.stride[d] = bm.stride[d];
  }
  void* buf = nullptr;
  if (int rc = temp(L, (size_t)n * sizeof(uint32_t), &buf)) return rc;
  if (int rc = hip_status(fmxq::launch_broadcast_index(src ? src->data : nullptr, m,
                                                       static_cast<uint32_t*>(buf), n, L.s),
                          "gather_qmm: index broadcast"))
    return rc;
  *out = static_cast<const uint32_t*>(buf);
  return FMXQ_OK;
}

float half_to_float(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1fu;
  uint32_t m = h & 0x3ffu;
  uint32_t bits;
  if (e == 0x1f) {
    bits = sign | 0x7f800000u | (m << 13);
  } else if (e != 0) {
    bits = sign | ((e + 112u) << 23) | (m << 13);
  } else if (m == 0) {
    bits = sign;
  } else {  // subnormal: normalise
    int shift = 0;
    while (!(m & 0x400u)) {
      m <<= 1;
      ++shift;
    }
    bits = sign | ((uint32_t)(113 - shift) << 23) | ((m & 0x3ffu) << 13);
  }
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

int eval_array(Array* a) {
  if (!a) return fail(FMXQ_ERR_INVALID_ARGUMENT, "eval: empty array");
  if (!a->stream) return FMXQ_OK;
  if (a->check_index) return fmxq_device_error(a->stream);
  return hip_status(hipStreamSynchronize(a->stream), "eval: synchronize");
}

int copy_to_host(Array* a) {
  if (int rc = eval_array(a)) return rc;
  a->host.resize(a->nbytes());
  if (a->host.empty()) return FMXQ_OK;
  return hip_status(hipMemcpy(a->host.data(), a->data, a->host.size(), hipMemcpyDeviceToHost),
                    "fmx: copy to host");
}

fmx_array make_handle(std::vector<int64_t> shape, fmx_dtype dtype) {
  Array* a = new Array;
  a->shape = std::move(shape);
  a->dtype = dtype;
  return fmx_array{a};
}

int read_shape(const int* shape, int dim, std::vector<int64_t>* out, const char* op) {
  return fmx_shape::read_shape(shape, dim, out, op);
}

int qmm_op(fmx_array* res, const fmx_array x, const fmx_array w, const fmx_array scales,
           const fmx_array biases, const fmx_array bias, bool transpose, int group_size,
           int bits, const fmx_stream s, const char* op) {
  if (!res) return fail(FMXQ_ERR_INVALID_ARGUMENT, "%s: null result", op);
  Array *X, *W, *S, *B;
  if (int rc = need(x, op, "x", &X)) return rc;
  if (int rc = need(w, op, "w", &W)) return rc;
  if (int rc = need(scales, op, "scales", &S)) return rc;
  if (int rc = need(biases, op, "biases", &B)) return rc;
  Array* Bias = arr(bias);
  if (int rc = need_dtype(X, FMX_BFLOAT16, op, "x")) return rc;
  if (int rc = need_dtype(W, FMX_UINT32, op, "w")) return rc;
  if (int rc = need_dtype(S, FMX_BFLOAT16, op, "scales")) return rc;
  if (int rc = need_dtype(B, FMX_BFLOAT16, op, "biases")) return rc;
  if (Bias)
    if (int rc = need_dtype(Bias, FMX_BFLOAT16, op, "bias")) return rc;
  fmx_shape::QmmGeom g;
  if (int rc = fmx_shape::qmm_geom(X->shape, W->shape, transpose, group_size, bits, &g, op))
    return rc;
  const int64_t K = g.K, N = g.N, M = g.M;
  if (int rc = need_shape(S, g.sshape, op, "scales")) return rc;
  if (int rc = need_shape(B, g.sshape, op, "biases")) return rc;
  if (Bias)
    if (int rc = need_shape(Bias, {N}, op, "bias")) return rc;
  const std::vector<int64_t>& oshape = g.oshape;

  Launch L;
  if (int rc = begin(L, s, {X, W, S, B, Bias})) return rc;
  Array* r = nullptr;
  if (int rc = new_result(L, oshape, FMX_BFLOAT16, &r)) return rc;
  int rc = fmxq_quantized_matmul_bias(
      static_cast<const uint16_t*>(X->data), static_cast<const uint32_t*>(W->data),
      static_cast<const uint16_t*>(S->data), static_cast<const uint16_t*>(B->data),
      Bias ? static_cast<const uint16_t*>(Bias->data) : nullptr, static_cast<uint16_t*>(r->data),
      M, N, K, transpose, group_size, bits, L.s);
  finish(L);
  return commit(res, r, rc);
}

}  // namespace

extern "C" {

// ---- arrays ----

fmx_array fmx_array_new(void) { return fmx_array{nullptr}; }

fmx_array fmx_array_new_data(const void* data, const int* shape, int dim, fmx_dtype dtype) {
  std::vector<int64_t> sh;
  if (read_shape(shape, dim, &sh, "array_new_data")) return fmx_array{nullptr};
  if (dtype_size(dtype) == 0) {
    fail(FMXQ_ERR_INVALID_ARGUMENT, "array_new_data: invalid dtype %d", (int)dtype);
    return fmx_array{nullptr};
  }
  fmx_array h = make_handle(sh, dtype);
  Array* a = arr(h);
  const size_t n = a->nbytes();
  if (n == 0) return h;
  if (!data) {
    fail(FMXQ_ERR_INVALID_ARGUMENT, "array_new_data: null data for %zu bytes", n);
    delete a;
    return fmx_array{nullptr};
  }
  int dev = 0;
  void* p = nullptr;
  // hipMalloc'd (256-byte aligned) and complete on return, so the array needs no
  // producing stream.
  if (hip_status(hipGetDevice(&dev), "array_new_data: hipGetDevice") ||
      hip_status(hipMalloc(&p, n), "array_new_data: hipMalloc")) {
    delete a;
    return fmx_array{nullptr};
  }
  // A pageable copy may return before its DMA lands; waiting on the null stream
  // makes the data visible to every stream, blocking or not.
  if (hip_status(hipMemcpy(p, data, n, hipMemcpyHostToDevice), "array_new_data: copy") ||
      hip_status(hipStreamSynchronize(nullptr), "array_new_data: synchronize")) {
    (void)hipFree(p);
    delete a;
    return fmx_array{nullptr};
  }
  a->data = p;
  a->cap = n;
  a->storage = Storage::kMalloc;
  a->device = dev;
  return h;
}

fmx_array fmx_array_new_device(void* device_ptr, const int* shape, int dim, fmx_dtype dtype) {
  std::vector<int64_t> sh;
  if (read_shape(shape, dim, &sh, "array_new_device")) return fmx_array{nullptr};
  if (dtype_size(dtype) == 0) {
    fail(FMXQ_ERR_INVALID_ARGUMENT, "array_new_device: invalid dtype %d", (int)dtype);
    return fmx_array{nullptr};
  }
  fmx_array h = make_handle(sh, dtype);
  Array* a = arr(h);
  if (a->numel() > 0 && !device_ptr) {
    fail(FMXQ_ERR_INVALID_ARGUMENT, "array_new_device: null pointer");
    delete a;
    return fmx_array{nullptr};
  }
  a->data = device_ptr;
  a->storage = Storage::kBorrowed;
  return h;
}

int fmx_array_free(fmx_array a) {
  Array* p = arr(a);
  if (!p) return FMXQ_OK;
  release_storage(p);
  delete p;
  return FMXQ_OK;
}

size_t fmx_array_ndim(const fmx_array a) { return arr(a) ? arr(a)->shape.size() : 0; }

int fmx_array_dim(const fmx_array a, int dim) {
  const Array* p = arr(a);
  if (!p || dim < 0 || dim >= (int)p->shape.size()) {
    fail(FMXQ_ERR_INVALID_ARGUMENT, "array_dim: axis %d out of range", dim);
    return 0;
  }
  return (int)p->shape[dim];
}

fmx_dtype fmx_array_dtype(const fmx_array a) { return arr(a) ? arr(a)->dtype : FMX_FLOAT32; }

size_t fmx_array_size(const fmx_array a) { return arr(a) ? (size_t)arr(a)->numel() : 0; }

size_t fmx_array_nbytes(const fmx_array a) { return arr(a) ? arr(a)->nbytes() : 0; }

void* fmx_array_device_ptr(const fmx_array a) { return arr(a) ? arr(a)->data : nullptr; }

int fmx_array_eval(fmx_array a) { return eval_array(arr(a)); }

const float* fmx_array_data_float32(fmx_array a) {
  Array* p = arr(a);
  if (!p) {
    fail(FMXQ_ERR_INVALID_ARGUMENT, "data_float32: empty array");
    return nullptr;
  }
  if (p->dtype != FMX_FLOAT32 && p->dtype != FMX_BFLOAT16 && p->dtype != FMX_FLOAT16) {
    fail(FMXQ_ERR_UNSUPPORTED, "data_float32: dtype %s", dtype_name(p->dtype));
    return nullptr;
  }
  if (copy_to_host(p)) return nullptr;
  if (p->dtype == FMX_FLOAT32) return reinterpret_cast<const float*>(p->host.data());
  const int64_t n = p->numel();
  std::vector<unsigned char> f((size_t)n * 4);
  const uint16_t* src = reinterpret_cast<const uint16_t*>(p->host.data());
  float* dst = reinterpret_cast<float*>(f.data());
  for (int64_t i = 0; i < n; ++i) {
    if (p->dtype == FMX_BFLOAT16) {
      const uint32_t bits = (uint32_t)src[i] << 16;
      std::memcpy(&dst[i], &bits, 4);
    } else {
      dst[i] = half_to_float(src[i]);
    }
  }
  p->host.swap(f);
  return reinterpret_cast<const float*>(p->host.data());
}

const int32_t* fmx_array_data_int32(fmx_array a) {
  Array* p = arr(a);
  if (!p) {
    fail(FMXQ_ERR_INVALID_ARGUMENT, "data_int32: empty array");
    return nullptr;
  }
  if (!is_index_dtype(p->dtype) && p->dtype != FMX_BOOL) {
    fail(FMXQ_ERR_UNSUPPORTED, "data_int32: dtype %s", dtype_name(p->dtype));
    return nullptr;
  }
  if (copy_to_host(p)) return nullptr;
  if (p->dtype == FMX_INT32 || p->dtype == FMX_UINT32)
    return reinterpret_cast<const int32_t*>(p->host.data());
  const int64_t n = p->numel();
  const size_t es = dtype_size(p->dtype);
  const bool sgn = is_signed_dtype(p->dtype);
  std::vector<unsigned char> out((size_t)n * 4);
  int32_t* dst = reinterpret_cast<int32_t*>(out.data());
  for (int64_t i = 0; i < n; ++i) {
    const unsigned char* s = p->host.data() + i * es;
    int64_t v = 0;
    if (es == 1) v = sgn ? (int64_t)(int8_t)s[0] : (int64_t)s[0];
    else if (es == 2) {
      uint16_t u;
      std::memcpy(&u, s, 2);
      v = sgn ? (int64_t)(int16_t)u : (int64_t)u;
    } else {
      uint64_t u;
      std::memcpy(&u, s, 8);
      v = (int64_t)u;
    }
    dst[i] = (int32_t)v;
  }
  p->host.swap(out);
  return reinterpret_cast<const int32_t*>(p->host.data());
}

int fmx_array_to_host(void* dst, size_t nbytes, const fmx_array a) {
  Array* p = arr(a);
  if (!p) return fail(FMXQ_ERR_INVALID_ARGUMENT, "to_host: empty array");
  if (nbytes != p->nbytes())
    return fail(FMXQ_ERR_SHAPE, "to_host: %zu bytes requested, array holds %zu", nbytes,
                p->nbytes());
  if (nbytes == 0) return FMXQ_OK;
  if (!dst) return fail(FMXQ_ERR_INVALID_ARGUMENT, "to_host: null destination");
  if (int rc = eval_array(p)) return rc;
  return hip_status(hipMemcpy(dst, p->data, nbytes, hipMemcpyDeviceToHost), "to_host: copy");
}

// ---- streams ----

fmx_stream fmx_default_gpu_stream_new(void) {
  Stream* s = nullptr;
  if (default_stream(&s)) return fmx_stream{nullptr};
  return fmx_stream{s};
}

fmx_stream fmx_stream_new(void) {
  // Like MLX streams, a stream lives until the process ends: arrays keep the
  // stream that produced them, so destroying it under them is never safe.
  hipStream_t s = nullptr;
  if (hip_status(hipStreamCreate(&s), "stream_new: hipStreamCreate")) return fmx_stream{nullptr};
  return fmx_stream{new Stream{s, false}};
}

fmx_stream fmx_stream_wrap(void* hip_stream) {
  return fmx_stream{new Stream{static_cast<hipStream_t>(hip_stream), false}};
}

int fmx_stream_free(fmx_stream s) {
  Stream* p = static_cast<Stream*>(s.ctx);
  if (p && !p->singleton) delete p;
  return FMXQ_OK;
}

int fmx_synchronize(fmx_stream s) {
  hipStream_t hs = nullptr;
  if (int rc = resolve_stream(s, &hs)) return rc;
  return hip_status(hipStreamSynchronize(hs), "synchronize");
}

// ---- ops ----

int fmx_quantized_matmul(fmx_array* res, const fmx_array x, const fmx_array w,
                         const fmx_array scales, const fmx_array biases, bool transpose,
                         int group_size, int bits, const fmx_stream s) {
  return qmm_op(res, x, w, scales, biases, fmx_array{nullptr}, transpose, group_size, bits, s,
                "quantized_matmul");
}

int fmx_quantized_matmul_bias(fmx_array* res, const fmx_array x, const fmx_array w,
                              const fmx_array scales, const fmx_array biases,
                              const fmx_array bias, bool transpose, int group_size, int bits,
                              const fmx_stream s) {
  return qmm_op(res, x, w, scales, biases, bias, transpose, group_size, bits, s,
                "quantized_matmul_bias");
}

int fmx_moe_combine(fmx_array* res, const fmx_array y, const fmx_array weights,
                    const fmx_array shared, const fmx_array shared_gate, const fmx_stream s) {
  const char* op = "moe_combine";
  if (!res) return fail(FMXQ_ERR_INVALID_ARGUMENT, "%s: null result", op);
  Array *Y, *Wt;
  if (int rc = need(y, op, "y", &Y)) return rc;
  if (int rc = need(weights, op, "weights", &Wt)) return rc;
  Array* Sh = arr(shared);
  Array* Sg = arr(shared_gate);
  if (int rc = need_dtype(Y, FMX_BFLOAT16, op, "y")) return rc;
  if (int rc = need_dtype(Wt, FMX_BFLOAT16, op, "weights")) return rc;
  if (Sh)
    if (int rc = need_dtype(Sh, FMX_BFLOAT16, op, "shared")) return rc;
  if (Sg) {
    if (!Sh) return fail(FMXQ_ERR_INVALID_ARGUMENT, "%s: shared_gate without shared", op);
    if (int rc = need_dtype(Sg, FMX_BFLOAT16, op, "shared_gate")) return rc;
  }
  if (Y->shape.size() < 2) return fail(FMXQ_ERR_SHAPE, "%s: y must be [..., k, D]", op);
  const size_t nd = Y->shape.size();
  const int64_t topk = Y->shape[nd - 2], D = Y->shape[nd - 1];
  std::vector<int64_t> lead(Y->shape.begin(), Y->shape.end() - 2);
  const int64_t T = prod(lead);
  std::vector<int64_t> wshape = lead;
  wshape.push_back(topk);
  // The reference reshapes the scores to [..., k, 1] before the multiply.
  std::vector<int64_t> wshape1 = wshape;
  wshape1.push_back(1);
  if (Wt->shape != wshape && Wt->shape != wshape1)
    return fail(FMXQ_ERR_SHAPE, "%s: weights has shape %s, need %s", op,
                shape_str(Wt->shape).c_str(), shape_str(wshape).c_str());
  std::vector<int64_t> oshape = lead;
  oshape.push_back(D);
  if (Sh)
    if (int rc = need_shape(Sh, oshape, op, "shared")) return rc;
  if (Sg) {
    std::vector<int64_t> g1 = lead;
    g1.push_back(1);
    if (Sg->shape != lead && Sg->shape != g1)
      return fail(FMXQ_ERR_SHAPE, "%s: shared_gate has shape %s, need %s", op,
                  shape_str(Sg->shape).c_str(), shape_str(g1).c_str());
  }
  Launch L;
  if (int rc = begin(L, s, {Y, Wt, Sh, Sg})) return rc;
  Array* r = nullptr;
  if (int rc = new_result(L, oshape, FMX_BFLOAT16, &r)) return rc;
  int rc = fmxq_moe_combine(static_cast<const uint16_t*>(Y->data),
                            static_cast<const uint16_t*>(Wt->data),
                            Sh ? static_cast<const uint16_t*>(Sh->data) : nullptr,
                            Sg ? static_cast<const uint16_t*>(Sg->data) : nullptr,
                            static_cast<uint16_t*>(r->data), T, topk, D, L.s);
  finish(L);
  return commit(res, r, rc);
}

namespace {
int route_handles(fmx_array* inds, fmx_array* weights, const fmx_array logits,
                  const fmx_array bias, int top_k, int n_group, int topk_group, float scale,
                  bool norm, bool group, const fmx_stream s, const char* op) {
  if (!inds || !weights) return fail(FMXQ_ERR_INVALID_ARGUMENT, "%s: null result", op);
  Array* X;
  if (int rc = need(logits, op, "logits", &X)) return rc;
  if (X->dtype != FMX_BFLOAT16 && X->dtype != FMX_FLOAT32)
    return fail(FMXQ_ERR_UNSUPPORTED, "%s: logits must be bfloat16 or float32", op);
  if (X->shape.empty()) return fail(FMXQ_ERR_SHAPE, "%s: logits must be [..., E]", op);
  const int64_t E = X->shape.back();
  Array* Bi = group ? arr(bias) : nullptr;
  if (Bi) {
    if (int rc = need_dtype(Bi, FMX_FLOAT32, op, "bias")) return rc;
    if (int rc = need_shape(Bi, {E}, op, "bias")) return rc;
  }
  std::vector<int64_t> oshape(X->shape.begin(), X->shape.end() - 1);
  const int64_t T = prod(oshape);
  oshape.push_back(top_k);
  Launch L;
  if (int rc = begin(L, s, {X, Bi})) return rc;
  Array *ri = nullptr, *rw = nullptr;
  if (int rc = new_result(L, oshape, FMX_UINT32, &ri)) return rc;
  if (int rc = new_result(L, oshape, X->dtype, &rw)) {
    commit(inds, ri, rc);
    return rc;
  }
  const int bf = X->dtype == FMX_BFLOAT16;
  int rc = group ? fmxq_route_group_topk(X->data, bf, Bi ? static_cast<const float*>(Bi->data)
                                                           : nullptr,
                                         T, E, top_k, n_group, topk_group, scale, norm,
                                         static_cast<uint32_t*>(ri->data), rw->data, bf, L.s)
                 : fmxq_route_softmax_topk(X->data, bf, T, E, top_k, norm,
                                           static_cast<uint32_t*>(ri->data), rw->data, bf, L.s);
  finish(L);
  if (rc) {
    commit(inds, ri, rc);
    return commit(weights, rw, rc);
  }
  commit(inds, ri, 0);
  return commit(weights, rw, 0);
}
}  // namespace

int fmx_route_softmax_topk(fmx_array* inds, fmx_array* weights, const fmx_array logits,
                           int top_k, bool norm_topk_prob, const fmx_stream s) {
  return route_handles(inds, weights, logits, fmx_array{nullptr}, top_k, 1, 1, 1.f,
                       norm_topk_prob, false, s, "route_softmax_topk");
}

int fmx_route_group_topk(fmx_array* inds, fmx_array* weights, const fmx_array gates,
                         const fmx_array bias, int top_k, int n_group, int topk_group,
                         float routed_scaling_factor, bool norm_topk_prob, const fmx_stream s) {
  return route_handles(inds, weights, gates, bias, top_k, n_group, topk_group,
                       routed_scaling_factor, norm_topk_prob, true, s, "route_group_topk");
}

int fmx_gather_qmm(fmx_array* res, const fmx_array x, const fmx_array w,
                   const fmx_array scales, const fmx_array biases, const fmx_array lhs_indices,
                   const fmx_array rhs_indices, bool transpose, int group_size, int bits,
                   bool sorted_indices, const fmx_stream s) {
  const char* op = "gather_qmm";
  if (!res) return fail(FMXQ_ERR_INVALID_ARGUMENT, "%s: null result", op);
  Array *X, *W, *S, *B;
  if (int rc = need(x, op, "x", &X)) return rc;
  if (int rc = need(w, op, "w", &W)) return rc;
  if (int rc = need(scales, op, "scales", &S)) return rc;
  if (int rc = need(biases, op, "biases", &B)) return rc;
  Array* Li = arr(lhs_indices);
  Array* Ri = arr(rhs_indices);
  if (int rc = need_dtype(X, FMX_BFLOAT16, op, "x")) return rc;
  if (int rc = need_dtype(W, FMX_UINT32, op, "w")) return rc;
  if (int rc = need_dtype(S, FMX_BFLOAT16, op, "scales")) return rc;
  if (int rc = need_dtype(B, FMX_BFLOAT16, op, "biases")) return rc;
  if (Li && !is_index_dtype(Li->dtype))
    return fail(FMXQ_ERR_INVALID_ARGUMENT, "%s: lhs_indices must be integral (got %s)", op,
                dtype_name(Li->dtype));
  if (Ri && !is_index_dtype(Ri->dtype))
    return fail(FMXQ_ERR_INVALID_ARGUMENT, "%s: rhs_indices must be integral (got %s)", op,
                dtype_name(Ri->dtype));
  fmx_shape::GatherGeom g;
  if (int rc = fmx_shape::gather_geom(X->shape, W->shape, &S->shape, &B->shape,
                                      Li ? &Li->shape : nullptr, Ri ? &Ri->shape : nullptr,
                                      transpose, group_size, bits, &g))
    return rc;
  const int64_t K = g.K, Mx = g.Mx, N = g.N, batch = g.batch, x_batch = g.x_batch, E = g.E;
  const int64_t lhs_div = g.lhs_div;
  const std::vector<int64_t>& xb = g.xb;
  const std::vector<int64_t>& wb = g.wb;
  const std::vector<int64_t>& bshape = g.bshape;
  const std::vector<int64_t>& oshape = g.oshape;

  Launch L;
  if (int rc = begin(L, s, {X, W, S, B, Li, Ri})) return rc;
  Array* r = nullptr;
  if (int rc = new_result(L, oshape, FMX_BFLOAT16, &r)) return rc;
  r->check_index = true;
  int rc = FMXQ_OK;
  const uint32_t* lp = nullptr;
  const uint32_t* rp = nullptr;
  if (batch > 0 && Mx > 0 && N > 0) {
    if (!Li && lhs_div == 0) rc = index_vector(L, nullptr, xb, bshape, &lp);
    if (Li && !rc) rc = index_vector(L, Li, {}, bshape, &lp);
    if (!rc) rc = index_vector(L, Ri, wb, bshape, &rp);
    if (!rc)
      rc = fmxq_gather_qmm(static_cast<const uint16_t*>(X->data),
                           static_cast<const uint32_t*>(W->data),
                           static_cast<const uint16_t*>(S->data),
                           static_cast<const uint16_t*>(B->data), lp, rp,
                           static_cast<uint16_t*>(r->data), batch, x_batch,
                           lhs_div > 0 ? lhs_div : 1, Mx, N, K, E, transpose, group_size, bits,
                           sorted_indices, L.s);
  }
  finish(L);
  return commit(res, r, rc);
}

int fmx_dequantize(fmx_array* res, const fmx_array w, const fmx_array scales,
                   const fmx_array biases, int group_size, int bits, const fmx_stream s) {
  const char* op = "dequantize";
  if (!res) return fail(FMXQ_ERR_INVALID_ARGUMENT, "%s: null result", op);
  Array *W, *S, *B;
  if (int rc = need(w, op, "w", &W)) return rc;
  if (int rc = need(scales, op, "scales", &S)) return rc;
  if (int rc = need(biases, op, "biases", &B)) return rc;
  if (int rc = need_dtype(W, FMX_UINT32, op, "w")) return rc;
  if (int rc = need_dtype(S, FMX_BFLOAT16, op, "scales")) return rc;
  if (int rc = need_dtype(B, FMX_BFLOAT16, op, "biases")) return rc;
  int64_t K = 0;
  if (int rc = unpacked_k(W, bits, op, &K)) return rc;
  if (int rc = check_quant(group_size, bits, K, true, op)) return rc;
  std::vector<int64_t> sshape(W->shape.begin(), W->shape.end() - 1);
  sshape.push_back(K / group_size);
  if (int rc = need_shape(S, sshape, op, "scales")) return rc;
  if (int rc = need_shape(B, sshape, op, "biases")) return rc;
  std::vector<int64_t> oshape(W->shape.begin(), W->shape.end() - 1);
  oshape.push_back(K);
  if (int rc = fmx_shape::check_elements(oshape, op)) return rc;
  const int64_t rows = prod(W->shape, 0, W->shape.size() - 1);

  Launch L;
  if (int rc = begin(L, s, {W, S, B})) return rc;
  Array* r = nullptr;
  if (int rc = new_result(L, oshape, FMX_BFLOAT16, &r)) return rc;
  int rc = fmxq_dequantize(static_cast<const uint32_t*>(W->data),
                           static_cast<const uint16_t*>(S->data),
                           static_cast<const uint16_t*>(B->data),
                           static_cast<uint16_t*>(r->data), rows, K, group_size, bits, L.s);
  finish(L);
  return commit(res, r, rc);
}

int fmx_dequantize_rows(fmx_array* res, const fmx_array w, const fmx_array scales,
                        const fmx_array biases, const fmx_array idx, int group_size, int bits,
                        const fmx_stream s) {
  const char* op = "dequantize_rows";
  if (!res) return fail(FMXQ_ERR_INVALID_ARGUMENT, "%s: null result", op);
  Array *W, *S, *B, *I;
  if (int rc = need(w, op, "w", &W)) return rc;
  if (int rc = need(scales, op, "scales", &S)) return rc;
  if (int rc = need(biases, op, "biases", &B)) return rc;
  if (int rc = need(idx, op, "idx", &I)) return rc;
  if (int rc = need_dtype(W, FMX_UINT32, op, "w")) return rc;
  if (int rc = need_dtype(S, FMX_BFLOAT16, op, "scales")) return rc;
  if (int rc = need_dtype(B, FMX_BFLOAT16, op, "biases")) return rc;
  if (!is_index_dtype(I->dtype))
    return fail(FMXQ_ERR_INVALID_ARGUMENT, "%s: idx must be integral (got %s)", op,
                dtype_name(I->dtype));
  if (W->shape.size() != 2)
    return fail(FMXQ_ERR_SHAPE, "%s: w must be a [rows, K*bits/32] table (got %s)", op,
                shape_str(W->shape).c_str());
  int64_t K = 0;
  if (int rc = unpacked_k(W, bits, op, &K)) return rc;
  if (int rc = check_quant(group_size, bits, K, true, op)) return rc;
  const std::vector<int64_t> sshape{W->shape[0], K / group_size};
  if (int rc = need_shape(S, sshape, op, "scales")) return rc;
  if (int rc = need_shape(B, sshape, op, "biases")) return rc;
  std::vector<int64_t> oshape = I->shape;
  oshape.push_back(K);
  if (int rc = fmx_shape::check_elements(oshape, op)) return rc;
  const int64_t n = I->numel();

  Launch L;
  if (int rc = begin(L, s, {W, S, B, I})) return rc;
  Array* r = nullptr;
  if (int rc = new_result(L, oshape, FMX_BFLOAT16, &r)) return rc;
  r->check_index = true;
  int rc = FMXQ_OK;
  if (n > 0) {
    const uint32_t* ip = nullptr;
    rc = index_vector(L, I, {}, I->shape, &ip);
    if (!rc)
      rc = fmxq_dequantize_rows(static_cast<const uint32_t*>(W->data),
                                static_cast<const uint16_t*>(S->data),
                                static_cast<const uint16_t*>(B->data), ip,
                                static_cast<uint16_t*>(r->data), n, W->shape[0], K, group_size,
                                bits, L.s);
  }
  finish(L);
  return commit(res, r, rc);
}

int fmx_switch_glu(fmx_array* res, const fmx_array x, const fmx_array inds,
                   const fmx_array w_gate, const fmx_array s_gate, const fmx_array b_gate,
                   const fmx_array w_up, const fmx_array s_up, const fmx_array b_up,
                   const fmx_array w_down, const fmx_array s_down, const fmx_array b_down,
                   int group_size, int bits, const fmx_stream s) {
  const char* op = "switch_glu";
  if (!res) return fail(FMXQ_ERR_INVALID_ARGUMENT, "%s: null result", op);
  Array *X, *Id, *Wg, *Sg, *Bg, *Wu, *Su, *Bu, *Wd, *Sd, *Bd;
  if (int rc = need(x, op, "x", &X)) return rc;
  if (int rc = need(inds, op, "inds", &Id)) return rc;
  // The reference's shape guard (switch_glu.go:13-15, :102-106), same wording.
  if (X->shape.size() != 3 || Id->shape.size() != 3)
    return fail(FMXQ_ERR_SHAPE, "switchGLU: want x [B,L,D] and inds [B,L,top_k], got x %s inds %s",
                shape_str(X->shape).c_str(), shape_str(Id->shape).c_str());
  if (int rc = need(w_gate, op, "w_gate", &Wg)) return rc;
  if (int rc = need(s_gate, op, "s_gate", &Sg)) return rc;
  if (int rc = need(b_gate, op, "b_gate", &Bg)) return rc;
  if (int rc = need(w_up, op, "w_up", &Wu)) return rc;
  if (int rc = need(s_up, op, "s_up", &Su)) return rc;
  if (int rc = need(b_up, op, "b_up", &Bu)) return rc;
  if (int rc = need(w_down, op, "w_down", &Wd)) return rc;
  if (int rc = need(s_down, op, "s_down", &Sd)) return rc;
  if (int rc = need(b_down, op, "b_down", &Bd)) return rc;
  if (int rc = need_dtype(X, FMX_BFLOAT16, op, "x")) return rc;
  if (!is_index_dtype(Id->dtype))
    return fail(FMXQ_ERR_INVALID_ARGUMENT, "%s: inds must be integral (got %s)", op,
                dtype_name(Id->dtype));
  for (Array* q : {Wg, Wu, Wd})
    if (int rc = need_dtype(q, FMX_UINT32, op, "expert weight")) return rc;
  for (Array* q : {Sg, Bg, Su, Bu, Sd, Bd})
    if (int rc = need_dtype(q, FMX_BFLOAT16, op, "expert scales/biases")) return rc;
  const int64_t Bsz = X->shape[0], Lq = X->shape[1], D = X->shape[2], topk = Id->shape[2];
  if (Id->shape[0] != Bsz || Id->shape[1] != Lq)
    return fail(FMXQ_ERR_SHAPE, "switchGLU: want x [B,L,D] and inds [B,L,top_k], got x %s inds %s",
                shape_str(X->shape).c_str(), shape_str(Id->shape).c_str());
  if (bits != 4 && bits != 8)
    return fail(FMXQ_ERR_UNSUPPORTED, "%s: bits=%d not supported (4 or 8)", op, bits);
  if (Wg->shape.size() != 3)
    return fail(FMXQ_ERR_SHAPE, "%s: w_gate must be [E, I, D*bits/32] (got %s)", op,
                shape_str(Wg->shape).c_str());
  const int64_t E = Wg->shape[0], I = Wg->shape[1], pf = 32 / bits;
  if (int rc = check_quant(group_size, bits, D, true, op)) return rc;
  if (int rc = check_quant(group_size, bits, I, true, op)) return rc;
  const std::vector<int64_t> wgu{E, I, D / pf}, sgu{E, I, D / group_size};
  const std::vector<int64_t> wdn{E, D, I / pf}, sdn{E, D, I / group_size};
  if (int rc = need_shape(Wg, wgu, op, "w_gate")) return rc;
  if (int rc = need_shape(Wu, wgu, op, "w_up")) return rc;
  if (int rc = need_shape(Wd, wdn, op, "w_down")) return rc;
  if (int rc = need_shape(Sg, sgu, op, "s_gate")) return rc;
  if (int rc = need_shape(Bg, sgu, op, "b_gate")) return rc;
  if (int rc = need_shape(Su, sgu, op, "s_up")) return rc;
  if (int rc = need_shape(Bu, sgu, op, "b_up")) return rc;
  if (int rc = need_shape(Sd, sdn, op, "s_down")) return rc;
  if (int rc = need_shape(Bd, sdn, op, "b_down")) return rc;

  Launch L;
  if (int rc = begin(L, s, {X, Id, Wg, Sg, Bg, Wu, Su, Bu, Wd, Sd, Bd})) return rc;
  Array* r = nullptr;
  if (int rc = new_result(L, {Bsz, Lq, topk, D}, FMX_BFLOAT16, &r)) return rc;
  r->check_index = true;
  int rc = FMXQ_OK;
  const int64_t T = Bsz * Lq;
  if (T * topk > 0) {
    const uint32_t* ip = nullptr;
    rc = index_vector(L, Id, {}, Id->shape, &ip);
    if (!rc)
      rc = fmxq_switch_glu(
          static_cast<const uint16_t*>(X->data), ip, static_cast<const uint32_t*>(Wg->data),
          static_cast<const uint16_t*>(Sg->data), static_cast<const uint16_t*>(Bg->data),
          static_cast<const uint32_t*>(Wu->data), static_cast<const uint16_t*>(Su->data),
          static_cast<const uint16_t*>(Bu->data), static_cast<const uint32_t*>(Wd->data),
          static_cast<const uint16_t*>(Sd->data), static_cast<const uint16_t*>(Bd->data),
          static_cast<uint16_t*>(r->data), T, topk, E, D, I, group_size, bits, L.s);
  }
  finish(L);
  return commit(res, r, rc);
}

// ---- weight-ingest array ops (mlxgo View / Stack and the int4 bias of
// deepseekv3.go remapInt4) ----

// The bytes of a reinterpreted as dtype: the last axis scales by the ratio of
// the element sizes (mlxgo.View as remapInt4 uses it, deepseekv3.go:513: packed
// u8 [..., K/2] -> u32 [..., K/8]).  The result is a copy on stream s.
int fmx_view(fmx_array* res, const fmx_array a, fmx_dtype dtype, const fmx_stream s) {
  const char* op = "view";
  if (!res) return fail(FMXQ_ERR_INVALID_ARGUMENT, "%s: null result", op);
  Array* A;
  if (int rc = need(a, op, "a", &A)) return rc;
  const size_t from = dtype_size(A->dtype), to = dtype_size(dtype);
  if (!to) return fail(FMXQ_ERR_INVALID_ARGUMENT, "%s: invalid dtype %d", op, (int)dtype);
  std::vector<int64_t> shape = A->shape;
  if (from != to) {
    if (shape.empty())
      return fail(FMXQ_ERR_SHAPE, "%s: a scalar of %s cannot be viewed as %s", op,
                  dtype_name(A->dtype), dtype_name(dtype));
    const int64_t bytes = shape.back() * (int64_t)from;
    if (bytes % (int64_t)to)
      return fail(FMXQ_ERR_SHAPE, "%s: last axis of %s (%lld bytes) is not a multiple of %s", op,
                  shape_str(A->shape).c_str(), (long long)bytes, dtype_name(dtype));
    shape.back() = bytes / (int64_t)to;
  }
  Launch L;
  if (int rc = begin(L, s, {A})) return rc;
  Array* r = nullptr;
  if (int rc = new_result(L, shape, dtype, &r)) return rc;
  int rc = FMXQ_OK;
  if (r->nbytes())
    rc = hip_status(hipMemcpyAsync(r->data, A->data, r->nbytes(), hipMemcpyDeviceToDevice, L.s),
                    "view: copy");
  finish(L);
  return commit(res, r, rc);
}

// n arrays of one shape and dtype joined along a new leading axis (mlxgo.Stack
// with axis 0, as stackExperts calls it, deepseekv3.go:564-592).
int fmx_stack(fmx_array* res, const fmx_array* arrays, size_t n, int axis, const fmx_stream s) {
  const char* op = "stack";
  if (!res) return fail(FMXQ_ERR_INVALID_ARGUMENT, "%s: null result", op);
  if (!arrays || n == 0) return fail(FMXQ_ERR_INVALID_ARGUMENT, "%s: no arrays", op);
  if (axis != 0) return fail(FMXQ_ERR_UNSUPPORTED, "%s: only axis 0 is supported", op);
  std::vector<Array*> parts(n);
  for (size_t i = 0; i < n; ++i) {
    if (int rc = need(arrays[i], op, "part", &parts[i])) return rc;
    if (parts[i]->dtype != parts[0]->dtype || parts[i]->shape != parts[0]->shape)
      return fail(FMXQ_ERR_SHAPE, "%s: part %zu is %s %s, part 0 is %s %s", op, i,
                  dtype_name(parts[i]->dtype), shape_str(parts[i]->shape).c_str(),
                  dtype_name(parts[0]->dtype), shape_str(parts[0]->shape).c_str());
  }
  std::vector<int64_t> shape = parts[0]->shape;
  shape.insert(shape.begin(), (int64_t)n);
  Launch L;
  if (int rc = begin(L, s, parts)) return rc;
  Array* r = nullptr;
  if (int rc = new_result(L, shape, parts[0]->dtype, &r)) return rc;
  const size_t each = parts[0]->nbytes();
  int rc = FMXQ_OK;
  for (size_t i = 0; i < n && !rc && each; ++i)
    rc = hip_status(hipMemcpyAsync(static_cast<char*>(r->data) + i * each, parts[i]->data, each,
                                   hipMemcpyDeviceToDevice, L.s),
                    "stack: copy");
  finish(L);
  return commit(res, r, rc);
}

// -8 * scale in the scale's dtype (bf16, f16 or f32): the affine bias of an int4
// checkpoint whose zero point is 8 (scaleNeg8, deepseekv3.go:539-551).
int fmx_scale_neg8(fmx_array* res, const fmx_array scale, const fmx_stream s) {
  const char* op = "scale_neg8";
  if (!res) return fail(FMXQ_ERR_INVALID_ARGUMENT, "%s: null result", op);
  Array* S;
  if (int rc = need(scale, op, "scale", &S)) return rc;
  const int kind = S->dtype == FMX_BFLOAT16 ? 0 : S->dtype == FMX_FLOAT16 ? 1
                   : S->dtype == FMX_FLOAT32 ? 2 : -1;
  if (kind < 0)
    return fail(FMXQ_ERR_UNSUPPORTED, "%s: scale has dtype %s (bfloat16, float16 or float32)",
                op, dtype_name(S->dtype));
  Launch L;
  if (int rc = begin(L, s, {S})) return rc;
  Array* r = nullptr;
  if (int rc = new_result(L, S->shape, S->dtype, &r)) return rc;
  int rc = hip_status(fmxq::launch_scale_neg8(S->data, r->data, S->numel(), kind, L.s), op);
  finish(L);
  return commit(res, r, rc);
}

// ---- the array ops of the kv_b_proj absorption (deepseekv3.go:609-679) ----
// Arrays here are always row-major and contiguous, so the view-producing MLX
// ops (reshape, split, swapaxes) return contiguous copies and contiguous is a
// copy; the values are the same as MLX's.

namespace {
int copy_op(fmx_array* res, Array* A, std::vector<int64_t> shape, const fmx_stream s,
            const char* op) {
  Launch L;
  if (int rc = begin(L, s, {A})) return rc;
  Array* r = nullptr;
  if (int rc = new_result(L, std::move(shape), A->dtype, &r)) return rc;
  int rc = FMXQ_OK;
  if (r->nbytes())
    rc = hip_status(hipMemcpyAsync(r->data, A->data, r->nbytes(), hipMemcpyDeviceToDevice, L.s),
                    op);
  finish(L);
  return commit(res, r, rc);
}
}  // namespace

// mlx_quantize (mlxgo/binding_cgo.go:684-697): w [..., K] bf16 -> res_0 packed
// [..., K*bits/32] uint32, res_1 scales and res_2 biases [..., K/group] bf16.
int fmx_quantize(fmx_array* res_0, fmx_array* res_1, fmx_array* res_2, const fmx_array w,
                 int group_size, int bits, const fmx_stream s) {
  const char* op = "quantize";
  if (!res_0 || !res_1 || !res_2) return fail(FMXQ_ERR_INVALID_ARGUMENT, "%s: null result", op);
  Array* W;
  if (int rc = need(w, op, "w", &W)) return rc;
  if (W->dtype != FMX_BFLOAT16)
    return fail(FMXQ_ERR_UNSUPPORTED, "%s: w has dtype %s (bfloat16 only)", op,
                dtype_name(W->dtype));
  if (W->shape.size() < 2)
    return fail(FMXQ_ERR_SHAPE, "%s: w must have at least 2 dimensions, got %s", op,
                shape_str(W->shape).c_str());
  const int64_t K = W->shape.back();
  if (int rc = check_quant(group_size, bits, K, true, op)) return rc;
  const int64_t rows = prod(W->shape, 0, W->shape.size() - 1);
  std::vector<int64_t> qshape = W->shape, sshape = W->shape;
  qshape.back() = K * bits / 32;
  sshape.back() = K / group_size;
  Launch L;
  if (int rc = begin(L, s, {W})) return rc;
  Array *rq = nullptr, *rs = nullptr, *rb = nullptr;
  if (int rc = new_result(L, qshape, FMX_UINT32, &rq)) return rc;
  if (int rc = new_result(L, sshape, FMX_BFLOAT16, &rs)) {
    commit(res_0, rq, rc);
    return rc;
  }
  if (int rc = new_result(L, sshape, FMX_BFLOAT16, &rb)) {
    commit(res_0, rq, rc);
    commit(res_1, rs, rc);
    return rc;
  }
  int rc = fmxq_quantize(static_cast<const uint16_t*>(W->data), static_cast<uint32_t*>(rq->data),
                         static_cast<uint16_t*>(rs->data), static_cast<uint16_t*>(rb->data), rows,
                         K, group_size, bits, L.s);
  finish(L);
  if (rc) {
    commit(res_0, rq, rc);
    commit(res_1, rs, rc);
    return commit(res_2, rb, rc);
  }
  commit(res_0, rq, 0);
  commit(res_1, rs, 0);
  return commit(res_2, rb, 0);
}

// mlx_reshape (binding_cgo.go:398-406); one entry may be -1.
int fmx_reshape(fmx_array* res, const fmx_array a, const int* shape, size_t ndim,
                const fmx_stream s) {
  const char* op = "reshape";
  if (!res) return fail(FMXQ_ERR_INVALID_ARGUMENT, "%s: null result", op);
  if (ndim && !shape) return fail(FMXQ_ERR_INVALID_ARGUMENT, "%s: null shape", op);
  Array* A;
  if (int rc = need(a, op, "a", &A)) return rc;
  std::vector<int64_t> out;
  if (int rc = fmx_shape::reshape(A->shape, shape, ndim, &out, op)) return rc;
  return copy_op(res, A, std::move(out), s, op);
}

// mlx_split with explicit indices (binding_cgo.go:463-483): res holds n_res =
// num_indices + 1 handles, part i covering [indices[i-1], indices[i]) of axis
// (indices ascending within [0, dim]).  On failure no handle is touched.
int fmx_split(fmx_array* res, size_t n_res, const fmx_array a, const int* indices,
              size_t num_indices, int axis, const fmx_stream s) {
  const char* op = "split";
  if (!res) return fail(FMXQ_ERR_INVALID_ARGUMENT, "%s: null result", op);
  if (num_indices && !indices) return fail(FMXQ_ERR_INVALID_ARGUMENT, "%s: null indices", op);
  if (n_res != num_indices + 1)
    return fail(FMXQ_ERR_INVALID_ARGUMENT, "%s: %zu result handles for %zu indices (want %zu)",
                op, n_res, num_indices, num_indices + 1);
  Array* A;
  if (int rc = need(a, op, "a", &A)) return rc;
  fmx_shape::SplitPlan sp;
  if (int rc = fmx_shape::split(A->shape, indices, num_indices, axis, &sp, op)) return rc;
  const int ax = sp.axis;
  const int64_t dim = A->shape[ax];
  const std::vector<int64_t>& cut = sp.cut;
  const int64_t outer = sp.outer;
  const size_t inner = (size_t)sp.inner * dtype_size(A->dtype);
  Launch L;
  if (int rc = begin(L, s, {A})) return rc;
  std::vector<Array*> parts(n_res, nullptr);
  int rc = FMXQ_OK;
  for (size_t i = 0; i < n_res && !rc; ++i) {
    std::vector<int64_t> shape = A->shape;
    shape[ax] = cut[i + 1] - cut[i];
    rc = new_result(L, shape, A->dtype, &parts[i]);
    if (!rc && parts[i]->nbytes()) {
      const size_t width = (size_t)shape[ax] * inner;
      rc = hip_status(hipMemcpy2DAsync(parts[i]->data, width,
                                       static_cast<const char*>(A->data) + cut[i] * inner,
                                       (size_t)dim * inner, width, (size_t)outer,
                                       hipMemcpyDeviceToDevice, L.s),
                      "split: copy");
    }
  }
  finish(L);
  for (size_t i = 0; i < n_res; ++i)
    if (parts[i]) commit(&res[i], parts[i], rc);
  return rc;
}

// mlx_swapaxes (binding_cgo.go:715-722).
int fmx_swapaxes(fmx_array* res, const fmx_array a, int axis1, int axis2, const fmx_stream s) {
  const char* op = "swapaxes";
  if (!res) return fail(FMXQ_ERR_INVALID_ARGUMENT, "%s: null result", op);
  Array* A;
  if (int rc = need(a, op, "a", &A)) return rc;
  fmx_shape::SwapPlan sw;
  if (int rc = fmx_shape::swapaxes(A->shape, axis1, axis2, &sw, op)) return rc;
  const int a1 = sw.a1, a2 = sw.a2;
  const std::vector<int64_t>& shape = sw.shape;
  if (a1 == a2) return copy_op(res, A, shape, s, op);
  const size_t es = dtype_size(A->dtype);
  if (es != 1 && es != 2 && es != 4 && es != 8)
    return fail(FMXQ_ERR_UNSUPPORTED, "%s: dtype %s", op, dtype_name(A->dtype));
  Launch L;
  if (int rc = begin(L, s, {A})) return rc;
  Array* r = nullptr;
  if (int rc = new_result(L, shape, A->dtype, &r)) return rc;
  int rc = hip_status(
      fmxq::launch_swap_axes(A->data, r->data, sw.outer, sw.d1, sw.mid, sw.d2, sw.inner,
                             (int)es, L.s),
      op);
  finish(L);
  return commit(res, r, rc);
}

// mlx_contiguous (binding_cgo.go:724-731): a row-major copy.
int fmx_contiguous(fmx_array* res, const fmx_array a, bool allow_col_major, const fmx_stream s) {
  (void)allow_col_major;
  const char* op = "contiguous";
  if (!res) return fail(FMXQ_ERR_INVALID_ARGUMENT, "%s: null result", op);
  Array* A;
  if (int rc = need(a, op, "a", &A)) return rc;
  return copy_op(res, A, A->shape, s, op);
}

}  // extern "C"
