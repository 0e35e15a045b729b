// fmx_shape.cpp -- host-side shape rules of the array-handle layer (fmx_shape.hpp).
//
// The broadcasting and index rules follow mlx_gather_qmm as the reference binds
// it (mlxgo/binding_cgo.go:645-673, called from switch_glu.go:179-186); reshape,
// split and swapaxes follow mlx_reshape / mlx_split / mlx_swapaxes
// (binding_cgo.go:398-406, 463-483, 715-722).  No HIP here.
#include "fmx_shape.hpp"

#include <algorithm>

#include "../../include/fmx.h"
#include "../../include/fmxq.h"
#include "fmxq_status.hpp"

using fmxq::fail;

namespace fmx_shape {

namespace {

// a * b when both are >= 0 and the product stays within kMaxElements.
bool mul_ok(int64_t a, int64_t b, int64_t* out) {
  if (a < 0 || b < 0) return false;
  if (a != 0 && b > kMaxElements / a) return false;
  *out = a * b;
  return true;
}

bool checked_prod(const Shape& s, int64_t* out) {
  int64_t p = 1;
  for (int64_t d : s)
    if (!mul_ok(p, d, &p)) return false;
  *out = p;
  return true;
}

int too_big(const char* op, const Shape& s) {
  return fail(FMXQ_ERR_SHAPE, "%s: shape %s has more than 2^59 elements", op,
              shape_str(s).c_str());
}

int need_shape(const Shape& have, const Shape& want, const char* op, const char* name) {
  if (have != want)
    return fail(FMXQ_ERR_SHAPE, "%s: %s has shape %s, need %s", op, name, shape_str(have).c_str(),
                shape_str(want).c_str());
  return FMXQ_OK;
}

}  // namespace

int check_elements(const Shape& s, const char* op) {
  int64_t n = 0;
  if (!checked_prod(s, &n)) return too_big(op, s);
  return FMXQ_OK;
}

// Packed width -> K (bits is checked first).
int unpacked_k(const Shape& w, int bits, const char* op, int64_t* K) {
  if (bits != 4 && bits != 8)
    return fail(FMXQ_ERR_UNSUPPORTED, "%s: bits=%d not supported (4 or 8)", op, bits);
  if (w.empty()) return fail(FMXQ_ERR_SHAPE, "%s: w must have at least one axis", op);
  if (!mul_ok(w.back(), 32 / bits, K)) return too_big(op, w);
  return FMXQ_OK;
}

size_t dtype_size(int d) {
  switch (d) {
    case FMX_BOOL: case FMX_UINT8: case FMX_INT8: return 1;
    case FMX_UINT16: case FMX_INT16: case FMX_FLOAT16: case FMX_BFLOAT16: return 2;
    case FMX_UINT32: case FMX_INT32: case FMX_FLOAT32: return 4;
    case FMX_UINT64: case FMX_INT64: case FMX_COMPLEX64: case FMX_FLOAT64: return 8;
    default: return 0;
  }
}

bool is_index_dtype(int d) {
  return d == FMX_UINT8 || d == FMX_UINT16 || d == FMX_UINT32 || d == FMX_UINT64 ||
         d == FMX_INT8 || d == FMX_INT16 || d == FMX_INT32 || d == FMX_INT64;
}

bool is_signed_dtype(int d) {
  return d == FMX_INT8 || d == FMX_INT16 || d == FMX_INT32 || d == FMX_INT64;
}

const char* dtype_name(int d) {
  static const char* names[] = {"bool",    "uint8",   "uint16",   "uint32", "uint64",
                                "int8",    "int16",   "int32",    "int64",  "float16",
                                "float32", "bfloat16", "complex64", "float64"};
  return (d >= 0 && d <= FMX_FLOAT64) ? names[d] : "invalid";
}

std::string shape_str(const Shape& s) {
  std::string r = "[";
  for (size_t i = 0; i < s.size(); ++i) {
    if (i) r += " ";
    r += std::to_string(s[i]);
  }
  return r + "]";
}

int64_t prod(const Shape& s, size_t from, size_t to) {
  int64_t p = 1;
  for (size_t i = from; i < std::min(to, s.size()); ++i) p *= s[i];
  return p;
}

int read_shape(const int* shape, int dim, Shape* out, const char* op) {
  if (dim < 0 || (dim > 0 && !shape))
    return fail(FMXQ_ERR_INVALID_ARGUMENT, "%s: bad shape pointer/rank", op);
  out->clear();
  int64_t n = 1;
  for (int i = 0; i < dim; ++i) {
    if (shape[i] < 0) return fail(FMXQ_ERR_SHAPE, "%s: negative dimension %d", op, shape[i]);
    out->push_back(shape[i]);
    if (!mul_ok(n, shape[i], &n)) return too_big(op, *out);
  }
  return FMXQ_OK;
}

int broadcast(const Shape& a, const Shape& b, Shape* out, const char* op) {
  if (int rc = check_elements(a, op)) return rc;
  if (int rc = check_elements(b, op)) return rc;
  const size_t n = std::max(a.size(), b.size());
  Shape r(n, 1);
  for (size_t i = 0; i < n; ++i) {
    const int64_t da = i < n - a.size() ? 1 : a[i - (n - a.size())];
    const int64_t db = i < n - b.size() ? 1 : b[i - (n - b.size())];
    if (da != db && da != 1 && db != 1)
      return fail(FMXQ_ERR_SHAPE, "%s: index shapes %s and %s do not broadcast", op,
                  shape_str(a).c_str(), shape_str(b).c_str());
    r[i] = da == 1 ? db : da;
  }
  int64_t elems = 0;
  if (!checked_prod(r, &elems)) return too_big(op, r);
  *out = std::move(r);
  return FMXQ_OK;
}

int broadcast_map(const Shape& src, const Shape& out, BroadcastMap* m, const char* op) {
  if (int rc = check_elements(src, op)) return rc;
  if (int rc = check_elements(out, op)) return rc;
  const size_t nd = out.size();
  if (nd > (size_t)kMaxIndexDims)
    return fail(FMXQ_ERR_UNSUPPORTED, "%s: index batch has %zu axes (max %d)", op, nd,
                kMaxIndexDims);
  if (src.size() > nd)
    return fail(FMXQ_ERR_SHAPE, "%s: index shape %s has more axes than the batch %s", op,
                shape_str(src).c_str(), shape_str(out).c_str());
  const size_t pad = nd - src.size();
  for (size_t d = 0; d < src.size(); ++d)
    if (src[d] != 1 && src[d] != out[d + pad])
      return fail(FMXQ_ERR_SHAPE, "%s: index shape %s does not broadcast to %s", op,
                  shape_str(src).c_str(), shape_str(out).c_str());
  *m = BroadcastMap{};
  m->ndim = (int)nd;
  int64_t stride = 1;
  for (int d = (int)nd - 1; d >= 0; --d) {
    m->shape[d] = out[d];
    const int64_t sd = d >= (int)pad ? src[d - pad] : 1;
    m->stride[d] = sd == 1 ? 0 : stride;
    stride *= sd;
  }
  return FMXQ_OK;
}

bool same_elements(const Shape& src, const Shape& out) {
  int64_t ns = 0, no = 0;
  if (!checked_prod(src, &ns) || !checked_prod(out, &no)) return false;
  if (src.size() > out.size()) return false;
  const size_t pad = out.size() - src.size();
  for (size_t d = 0; d < src.size(); ++d)
    if (src[d] != 1 && src[d] != out[d + pad]) return false;
  return ns == no;
}

int qmm_geom(const Shape& x, const Shape& w, bool transpose, int group_size, int bits,
             QmmGeom* g, const char* op) {
  if (int rc = check_elements(x, op)) return rc;
  if (int rc = check_elements(w, op)) return rc;
  if (x.empty()) return fail(FMXQ_ERR_SHAPE, "%s: x must have at least one axis", op);
  if (w.size() != 2)
    return fail(FMXQ_ERR_UNSUPPORTED, "%s: w must be [N, K*bits/32] (got %s)", op,
                shape_str(w).c_str());
  int64_t K = 0;
  if (int rc = unpacked_k(w, bits, op, &K)) return rc;
  if (int rc = fmxq::check_quant(group_size, bits, K, transpose, op)) return rc;
  if (x.back() != K)
    return fail(FMXQ_ERR_SHAPE, "%s: x has K=%lld but w packs K=%lld", op, (long long)x.back(),
                (long long)K);
  g->K = K;
  g->N = w[0];
  g->sshape = {g->N, K / group_size};
  g->oshape.assign(x.begin(), x.end() - 1);
  g->oshape.push_back(g->N);
  g->M = prod(x, 0, x.size() - 1);
  int64_t elems = 0;
  if (!checked_prod(g->oshape, &elems)) return too_big(op, g->oshape);
  return FMXQ_OK;
}

int gather_geom(const Shape& x, const Shape& w, const Shape* scales_shape,
                const Shape* biases_shape, const Shape* lhs, const Shape* rhs, bool transpose,
                int group_size, int bits, GatherGeom* g) {
  const char* op = "gather_qmm";
  if (int rc = check_elements(x, op)) return rc;
  if (int rc = check_elements(w, op)) return rc;
  if (x.size() < 2) return fail(FMXQ_ERR_SHAPE, "%s: x must be [..., M, K]", op);
  if (w.size() < 2) return fail(FMXQ_ERR_SHAPE, "%s: w must be [..., N, K*bits/32]", op);
  int64_t K = 0;
  if (int rc = unpacked_k(w, bits, op, &K)) return rc;
  if (int rc = fmxq::check_quant(group_size, bits, K, transpose, op)) return rc;
  if (x.back() != K)
    return fail(FMXQ_ERR_SHAPE, "%s: x has K=%lld but w packs K=%lld", op, (long long)x.back(),
                (long long)K);
  const size_t xnd = x.size(), wnd = w.size();
  g->K = K;
  g->Mx = x[xnd - 2];
  g->N = w[wnd - 2];
  g->xb.assign(x.begin(), x.end() - 2);
  g->wb.assign(w.begin(), w.end() - 2);
  g->sshape = g->wb;
  g->sshape.push_back(g->N);
  g->sshape.push_back(K / group_size);
  if (scales_shape)
    if (int rc = need_shape(*scales_shape, g->sshape, op, "scales")) return rc;
  if (biases_shape)
    if (int rc = need_shape(*biases_shape, g->sshape, op, "biases")) return rc;
  const Shape& lb = lhs ? *lhs : g->xb;
  const Shape& rb = rhs ? *rhs : g->wb;
  if (int rc = broadcast(lb, rb, &g->bshape, op)) return rc;
  g->batch = prod(g->bshape);
  g->x_batch = prod(g->xb);
  g->E = prod(g->wb);
  g->oshape = g->bshape;
  g->oshape.push_back(g->Mx);
  g->oshape.push_back(g->N);
  int64_t elems = 0;
  if (!checked_prod(g->oshape, &elems)) return too_big(op, g->oshape);
  // Implicit lhs: item i reads x item i / lhs_div when x's batch axes are the
  // leading axes of the output batch (the expand_dims choreography of
  // switchGLUCore, switch_glu.go:111-118); any other layout is materialized.
  g->lhs_div = 0;
  if (!lhs) {
    const Shape& xb = g->xb;
    const size_t nd = g->bshape.size();
    if (xb.size() <= nd) {
      const size_t pad = nd - xb.size();
      size_t j = 0;
      while (j < nd && (j >= pad ? xb[j - pad] : 1) == g->bshape[j]) ++j;
      bool flat = true;
      for (size_t d = j; d < nd; ++d)
        if ((d >= pad ? xb[d - pad] : 1) != 1) flat = false;
      if (flat) g->lhs_div = std::max<int64_t>(prod(g->bshape, j), 1);
    }
  }
  return FMXQ_OK;
}

int norm_axis(int axis, size_t ndim, const char* op, int* out) {
  const int n = (int)ndim;
  if (axis < -n || axis >= n)
    return fail(FMXQ_ERR_SHAPE, "%s: axis %d out of range for %d dimensions", op, axis, n);
  *out = axis < 0 ? axis + n : axis;
  return FMXQ_OK;
}

int reshape(const Shape& in, const int* shape, size_t ndim, Shape* out, const char* op) {
  if (ndim && !shape) return fail(FMXQ_ERR_INVALID_ARGUMENT, "%s: null shape", op);
  if (int rc = check_elements(in, op)) return rc;
  Shape r(ndim);
  int infer = -1;
  int64_t known = 1;
  for (size_t i = 0; i < ndim; ++i) {
    if (shape[i] == -1) {
      if (infer >= 0) return fail(FMXQ_ERR_SHAPE, "%s: more than one -1 in the shape", op);
      infer = (int)i;
    } else if (shape[i] < 0) {
      return fail(FMXQ_ERR_SHAPE, "%s: negative size %d", op, shape[i]);
    } else {
      r[i] = shape[i];
      if (!mul_ok(known, shape[i], &known))
        return fail(FMXQ_ERR_SHAPE, "%s: the new shape has more than 2^59 elements", op);
    }
  }
  const int64_t n = prod(in);
  if (infer >= 0) {
    if (known == 0 || n % known)
      return fail(FMXQ_ERR_SHAPE, "%s: cannot infer -1 reshaping %s", op, shape_str(in).c_str());
    r[infer] = n / known;
  } else if (known != n) {
    return fail(FMXQ_ERR_SHAPE, "%s: %s has %lld elements, the new shape %lld", op,
                shape_str(in).c_str(), (long long)n, (long long)known);
  }
  *out = std::move(r);
  return FMXQ_OK;
}

int split(const Shape& in, const int* indices, size_t num_indices, int axis, SplitPlan* p,
          const char* op) {
  if (num_indices && !indices) return fail(FMXQ_ERR_INVALID_ARGUMENT, "%s: null indices", op);
  if (int rc = check_elements(in, op)) return rc;
  int ax = 0;
  if (int rc = norm_axis(axis, in.size(), op, &ax)) return rc;
  const int64_t dim = in[ax];
  std::vector<int64_t> cut{0};
  for (size_t i = 0; i < num_indices; ++i) {
    if (indices[i] < cut.back() || indices[i] > dim)
      return fail(FMXQ_ERR_SHAPE, "%s: index %d out of order or beyond axis size %lld", op,
                  indices[i], (long long)dim);
    cut.push_back(indices[i]);
  }
  cut.push_back(dim);
  p->axis = ax;
  p->cut = std::move(cut);
  p->outer = prod(in, 0, ax);
  p->inner = prod(in, ax + 1);
  return FMXQ_OK;
}

int swapaxes(const Shape& in, int axis1, int axis2, SwapPlan* p, const char* op) {
  if (int rc = check_elements(in, op)) return rc;
  int a1 = 0, a2 = 0;
  if (int rc = norm_axis(axis1, in.size(), op, &a1)) return rc;
  if (int rc = norm_axis(axis2, in.size(), op, &a2)) return rc;
  if (a1 > a2) std::swap(a1, a2);
  p->shape = in;
  std::swap(p->shape[a1], p->shape[a2]);
  p->a1 = a1;
  p->a2 = a2;
  p->outer = prod(in, 0, a1);
  p->d1 = in[a1];
  p->mid = prod(in, a1 + 1, a2);
  p->d2 = in[a2];
  p->inner = prod(in, a2 + 1);
  return FMXQ_OK;
}

size_t round_bytes(size_t n) {
  if (n <= 512) return 512;
  if (n <= ((size_t)1 << 20)) return (n + 511) & ~(size_t)511;
  size_t p = (size_t)1 << 20;
  while (p * 2 <= n) p *= 2;
  const size_t step = p / 8;  // at most 12.5% slack above 1 MiB
  return (n + step - 1) / step * step;
}

bool BufferCache::take(int dev, const void* stream, size_t cap, void** out) {
  std::lock_guard<std::mutex> lk(mu_);
  auto fl = free_.find({dev, stream});
  if (fl == free_.end()) return false;
  auto it = fl->second.find(cap);
  if (it == fl->second.end()) return false;
  *out = it->second;
  fl->second.erase(it);
  return true;
}

void BufferCache::put(int dev, const void* stream, size_t cap, void* p) {
  std::lock_guard<std::mutex> lk(mu_);
  free_[{dev, stream}].emplace(cap, p);
}

std::vector<void*> BufferCache::drain(int dev) {
  std::vector<void*> out;
  std::lock_guard<std::mutex> lk(mu_);
  for (auto& kv : free_)
    if (kv.first.first == dev) {
      for (auto& b : kv.second) out.push_back(b.second);
      kv.second.clear();
    }
  return out;
}

size_t BufferCache::size() const {
  std::lock_guard<std::mutex> lk(mu_);
  size_t n = 0;
  for (auto& kv : free_) n += kv.second.size();
  return n;
}

}  // namespace fmx_shape

namespace fmxq {

int check_quant(int group_size, int bits, int64_t K, bool transpose, const char* op) {
  if (!transpose)
    return fail(FMXQ_ERR_UNSUPPORTED, "%s: transpose=false is not supported (the reference "
                "always passes true)", op);
  if (bits != 4 && bits != 8)
    return fail(FMXQ_ERR_UNSUPPORTED, "%s: bits=%d not supported (4 or 8)", op, bits);
  if (group_size != 32 && group_size != 64 && group_size != 128)
    return fail(FMXQ_ERR_UNSUPPORTED, "%s: group_size=%d not supported (32, 64 or 128)", op,
                group_size);
  if (K <= 0 || K % group_size != 0)
    return fail(FMXQ_ERR_SHAPE, "%s: K=%lld must be a positive multiple of group_size=%d", op,
                (long long)K, group_size);
  return FMXQ_OK;
}

}  // namespace fmxq
