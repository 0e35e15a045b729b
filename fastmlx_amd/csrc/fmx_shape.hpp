// fmx_shape.hpp -- the host-side rules of the array-handle layer (fmx_array.cpp):
// dtypes, shape validation, MLX batch broadcasting for gather_qmm, the geometry of
// reshape / split / swapaxes, and the bookkeeping of the device buffer cache.
//
// Plain host C++ with no HIP types (fmx_shape.cpp), so that the rules can be
// built with g++ under AddressSanitizer and UBSan and fuzzed on their own
// (tests/fuzz/shape_fuzz.cpp).  Every function that can fail returns an
// FMXQ_* status and records its message through fmxq::fail.
#pragma once
#include <stddef.h>
#include <stdint.h>

#include <map>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

namespace fmx_shape {

using Shape = std::vector<int64_t>;

// Arrays hold at most 2^59 elements, so every byte count (at most 8 bytes an
// element) and every product of a shape's axes stays far below 2^63.
constexpr int64_t kMaxElements = int64_t(1) << 59;
// Index broadcasts handle at most this many axes (fmxq::kMaxIndexDims).
constexpr int kMaxIndexDims = 8;

size_t dtype_size(int dtype);  // 0 for an invalid dtype
bool is_index_dtype(int dtype);
bool is_signed_dtype(int dtype);
const char* dtype_name(int dtype);
std::string shape_str(const Shape& s);
// Product of axes [from, to).  Shapes that passed read_shape (or were derived
// from such shapes by the rules below) never overflow it.
int64_t prod(const Shape& s, size_t from = 0, size_t to = SIZE_MAX);

// A caller's int shape of rank `dim`: no negative axis, at most kMaxElements
// elements.
int read_shape(const int* shape, int dim, Shape* out, const char* op);
// FMXQ_ERR_SHAPE unless s has at most kMaxElements elements (and no negative axis).
int check_elements(const Shape& s, const char* op);
// K of a packed weight array w [..., K*bits/32]: bits in {4, 8}, w not a scalar.
int unpacked_k(const Shape& w, int bits, const char* op, int64_t* K);

// MLX broadcasting of two batch shapes (right-aligned; an axis of size 1 takes
// the other's size).
int broadcast(const Shape& a, const Shape& b, Shape* out, const char* op);

// Reading `src` (row-major, right-aligned against `out`) broadcast to `out`:
// element i of `out` (row-major) is element sum_d coord_d(i) * stride[d] of src,
// with stride 0 on the axes src lacks or holds with size 1.
struct BroadcastMap {
  int ndim;
  int64_t shape[kMaxIndexDims];
  int64_t stride[kMaxIndexDims];
};
int broadcast_map(const Shape& src, const Shape& out, BroadcastMap* m, const char* op);
// True when src's elements in row-major order are already out's (src broadcasts
// to out with the same element count), so it can be read in place.
bool same_elements(const Shape& src, const Shape& out);

// quantized_matmul: x [..., K], w [N, K*bits/32]; scales and biases [N, K/group].
struct QmmGeom {
  int64_t K, N, M;
  Shape sshape, oshape;
};
int qmm_geom(const Shape& x, const Shape& w, bool transpose, int group_size, int bits,
             QmmGeom* g, const char* op);

// gather_qmm (mlx_gather_qmm): x [xb..., Mx, K], w [wb..., N, K*bits/32], optional
// index arrays (null: the implicit arange over xb / wb).  scales_shape /
// biases_shape, when given, must equal [wb..., N, K/group].  lhs_div > 0 means item
// i reads x item i / lhs_div (x's batch axes lead the output batch, the
// expand_dims form of switchGLUCore); 0 means the x index is materialized.
struct GatherGeom {
  int64_t K, Mx, N, batch, x_batch, E, lhs_div;
  Shape xb, wb, bshape, oshape, sshape;
};
int gather_geom(const Shape& x, const Shape& w, const Shape* scales_shape,
                const Shape* biases_shape, const Shape* lhs, const Shape* rhs, bool transpose,
                int group_size, int bits, GatherGeom* g);

int norm_axis(int axis, size_t ndim, const char* op, int* out);
// mlx_reshape: `shape` of rank ndim, at most one -1 (inferred).
int reshape(const Shape& in, const int* shape, size_t ndim, Shape* out, const char* op);
// mlx_split with explicit ascending indices: part i covers [cut[i], cut[i+1]) of
// the axis; outer = product of the axes before it, inner = product after it.
struct SplitPlan {
  int axis;
  std::vector<int64_t> cut;  // num_indices + 2 entries, from 0 to the axis size
  int64_t outer, inner;
};
int split(const Shape& in, const int* indices, size_t num_indices, int axis, SplitPlan* p,
          const char* op);
// mlx_swapaxes: the result shape and, when a1 < a2, the five extents of the copy
// [outer, d1, mid, d2, inner] -> [outer, d2, mid, d1, inner] (a1 == a2 is a plain
// copy).
struct SwapPlan {
  Shape shape;
  int a1, a2;
  int64_t outer, d1, mid, d2, inner;
};
int swapaxes(const Shape& in, int axis1, int axis2, SwapPlan* p, const char* op);

// Allocation size of an n-byte buffer in the cache: 512-byte steps up to 1 MiB,
// then steps of an eighth of the power of two below n (at most 12.5% slack).
size_t round_bytes(size_t n);

// Free device buffers of the cache, per (device, stream) and rounded size.  The
// caller allocates on a miss and frees what drain() hands back.
class BufferCache {
 public:
  // A cached buffer of exactly `cap` bytes for (dev, stream), removed from the
  // cache; false if there is none.
  bool take(int dev, const void* stream, size_t cap, void** out);
  void put(int dev, const void* stream, size_t cap, void* p);
  // Every cached buffer of device dev, removed from the cache.
  std::vector<void*> drain(int dev);
  size_t size() const;

 private:
  mutable std::mutex mu_;
  std::map<std::pair<int, const void*>, std::multimap<size_t, void*>> free_;
};

}  // namespace fmx_shape

namespace fmxq {
// The quantization geometry every op supports: transpose, bits in {4, 8},
// group_size in {32, 64, 128}, K a positive multiple of group_size.
int check_quant(int group_size, int bits, int64_t K, bool transpose, const char* op);
}  // namespace fmxq
