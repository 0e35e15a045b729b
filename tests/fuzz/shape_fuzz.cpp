// Fuzz driver for the array-handle layer's host rules (fastmlx_amd/csrc/fmx_shape.cpp),
// built with g++ -fsanitize=address,undefined by tests/test_host_sanitize.py.
//
// Random shapes (small ones, and huge axes that would overflow a naive product) go
// through every rule; whatever a rule accepts is checked against a brute-force
// restatement: MLX broadcasting, the broadcast index map element by element, the
// implicit-lhs shortcut of gather_qmm against the materialized arange, reshape /
// split / swapaxes element counts and the swapaxes copy element by element, the
// cache's size rounding, and the buffer cache's bookkeeping under random take /
// put / drain sequences from several threads.  Any violated invariant aborts.
//
//   shape_fuzz <iterations> [seed]
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <set>
#include <thread>
#include <vector>

#include "../../fastmlx_amd/csrc/fmx_shape.hpp"
#include "fmxq.h"

using fmx_shape::Shape;

namespace {

uint64_t g_state = 0x9E3779B97F4A7C15ull;
uint64_t rnd() {
  uint64_t z = (g_state += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
int64_t pick(int64_t n) { return (int64_t)(rnd() % (uint64_t)n); }

// Accepted cases per rule (the run reports them, so a rule the generator never
// gets past its validation shows up as 0).
long g_ok[10] = {0};
long g_elems = 0;  // elements checked one by one (maps, lhs shortcut, swapaxes)

#define CHECK(c)                                                                 \
  do {                                                                           \
    if (!(c)) {                                                                  \
      std::fprintf(stderr, "check failed at line %d: %s\n", __LINE__, #c);       \
      std::abort();                                                              \
    }                                                                            \
  } while (0)

int64_t small_dim() {
  static const int64_t d[] = {1, 1, 1, 2, 2, 3, 4, 5, 0};
  return d[pick(9)];
}
int64_t any_dim() {
  switch (pick(12)) {
    case 0: return (int64_t)1 << pick(40);
    case 1: return 2147483647;
    case 2: return 65536;
    default: return small_dim();
  }
}
Shape rand_shape(int max_rank, bool huge) {
  Shape s((size_t)pick(max_rank + 1));
  for (auto& d : s) d = huge ? any_dim() : small_dim();
  return s;
}

int64_t prod_checked(const Shape& s, bool* ok) {
  // exact product, flagging anything past 2^59 (no overflow: stop early)
  int64_t p = 1;
  *ok = true;
  for (int64_t d : s) {
    if (d == 0) return 0;
  }
  for (int64_t d : s) {
    if (d < 0 || (p != 0 && d > fmx_shape::kMaxElements / p)) {
      *ok = false;
      return -1;
    }
    p *= d;
  }
  return p;
}

// Row-major coordinates of flat index i in s.
std::vector<int64_t> coords(int64_t i, const Shape& s) {
  std::vector<int64_t> c(s.size());
  for (int d = (int)s.size() - 1; d >= 0; --d) {
    c[d] = s[d] ? i % s[d] : 0;
    i = s[d] ? i / s[d] : 0;
  }
  return c;
}

// Brute-force offset in src of output element i when src is broadcast to out.
int64_t bcast_offset(int64_t i, const Shape& src, const Shape& out) {
  const auto c = coords(i, out);
  const size_t pad = out.size() - src.size();
  int64_t off = 0;
  for (size_t d = 0; d < src.size(); ++d) off = off * src[d] + (src[d] == 1 ? 0 : c[d + pad]);
  return off;
}

void fuzz_read_shape() {
  int dims[10];
  const int rank = (int)pick(10) - 1;  // -1 .. 8
  for (int i = 0; i < 10; ++i) {
    switch (pick(8)) {
      case 0: dims[i] = -(int)pick(5) - 1; break;
      case 1: dims[i] = 2147483647; break;
      case 2: dims[i] = 1 << pick(31); break;
      default: dims[i] = (int)small_dim();
    }
  }
  Shape out;
  const int rc = fmx_shape::read_shape(pick(20) ? dims : nullptr, rank, &out, "fuzz");
  if (rc == FMXQ_OK) {
    CHECK(rank >= 0 && (int)out.size() == rank);
    bool ok = false;
    const int64_t n = prod_checked(out, &ok);
    CHECK(ok && n <= fmx_shape::kMaxElements);
    for (int i = 0; i < rank; ++i) CHECK(out[i] == dims[i] && dims[i] >= 0);
    CHECK(fmx_shape::prod(out) == n);
    ++g_ok[0];
  }
}

void fuzz_broadcast() {
  const bool huge = pick(4) == 0;
  Shape a = rand_shape(5, huge), b = rand_shape(5, huge);
  if (pick(2)) {  // make them compatible more often
    b = a;
    for (auto& d : b)
      if (pick(3) == 0) d = 1;
    if (pick(2) && !b.empty()) b.erase(b.begin(), b.begin() + pick((int64_t)b.size() + 1));
  }
  Shape o1, o2;
  const int r1 = fmx_shape::broadcast(a, b, &o1, "fuzz");
  const int r2 = fmx_shape::broadcast(b, a, &o2, "fuzz");
  CHECK(r1 == r2);
  if (r1 != FMXQ_OK) return;
  CHECK(o1 == o2);
  CHECK(o1.size() == std::max(a.size(), b.size()));
  for (size_t i = 0; i < o1.size(); ++i) {
    const size_t n = o1.size();
    const int64_t da = i < n - a.size() ? 1 : a[i - (n - a.size())];
    const int64_t db = i < n - b.size() ? 1 : b[i - (n - b.size())];
    CHECK(da == db || da == 1 || db == 1);
    CHECK(o1[i] == (da == 1 ? db : da));
  }
  bool ok = false;
  prod_checked(o1, &ok);
  CHECK(ok);
  ++g_ok[1];
}

void fuzz_broadcast_map() {
  Shape out = rand_shape(6, false);
  Shape src = out;
  for (auto& d : src)
    if (pick(3) == 0) d = 1;
  if (pick(2)) src.erase(src.begin(), src.begin() + pick((int64_t)src.size() + 1));
  if (pick(8) == 0 && !src.empty()) src[pick((int64_t)src.size())] += 1;  // sometimes invalid
  fmx_shape::BroadcastMap m;
  const int rc = fmx_shape::broadcast_map(src, out, &m, "fuzz");
  bool valid = src.size() <= out.size() && out.size() <= (size_t)fmx_shape::kMaxIndexDims;
  if (valid)
    for (size_t d = 0; d < src.size(); ++d)
      if (src[d] != 1 && src[d] != out[d + out.size() - src.size()]) valid = false;
  CHECK((rc == FMXQ_OK) == valid);
  if (rc != FMXQ_OK) return;
  CHECK(m.ndim == (int)out.size());
  const int64_t n = fmx_shape::prod(out);
  if (n > 4096) return;
  const bool same = fmx_shape::same_elements(src, out);
  for (int64_t i = 0; i < n; ++i) {
    const auto c = coords(i, out);
    int64_t off = 0;
    for (int d = 0; d < m.ndim; ++d) {
      CHECK(m.shape[d] == out[d]);
      off += c[d] * m.stride[d];
    }
    CHECK(off == bcast_offset(i, src, out));
    CHECK(off >= 0 && (fmx_shape::prod(src) == 0 || off < fmx_shape::prod(src)));
    if (same) CHECK(off == i);
    ++g_elems;
  }
  ++g_ok[2];
}

void fuzz_gather_geom() {
  const bool huge = pick(6) == 0;
  // x [xb..., Mx, K], w [wb..., N, K*bits/32]
  const int bits = pick(5) == 0 ? 3 : (pick(2) ? 4 : 8);
  const int gs = pick(6) == 0 ? 48 : (int)(32 << pick(3));
  const int64_t K = pick(6) == 0 ? 100 : 128 * (1 + pick(3));
  Shape xb = rand_shape(3, huge), wb = rand_shape(3, huge);
  Shape x = xb, w = wb;
  x.push_back(pick(3) + 1);
  x.push_back(pick(8) == 0 ? K + 8 : K);
  w.push_back(pick(3) + 1);
  w.push_back(bits == 3 ? K / 8 : K * bits / 32);
  Shape ss = wb;
  ss.push_back(w[w.size() - 2]);
  ss.push_back(gs > 0 ? K / gs : 0);
  Shape lhs, rhs;
  const bool has_l = pick(2), has_r = pick(2);
  if (has_l) lhs = pick(2) ? xb : rand_shape(3, huge);
  if (has_r) rhs = pick(2) ? wb : rand_shape(3, huge);
  fmx_shape::GatherGeom g;
  const int rc = fmx_shape::gather_geom(x, w, pick(10) ? &ss : nullptr, pick(10) ? &ss : nullptr,
                                        has_l ? &lhs : nullptr, has_r ? &rhs : nullptr,
                                        pick(20) != 0, gs, bits, &g);
  if (rc != FMXQ_OK) return;
  CHECK(bits == 4 || bits == 8);
  CHECK(g.K == K && g.K % gs == 0);
  CHECK(g.oshape.size() == g.bshape.size() + 2);
  CHECK(g.oshape[g.oshape.size() - 2] == g.Mx && g.oshape.back() == g.N);
  CHECK(g.batch == fmx_shape::prod(g.bshape));
  CHECK(g.x_batch == fmx_shape::prod(xb) && g.E == fmx_shape::prod(wb));
  bool ok = false;
  prod_checked(g.oshape, &ok);
  CHECK(ok);
  Shape want_b;
  CHECK(fmx_shape::broadcast(has_l ? lhs : xb, has_r ? rhs : wb, &want_b, "fuzz") == FMXQ_OK);
  CHECK(want_b == g.bshape);
  // The implicit-lhs shortcut reads x item i / lhs_div; it must agree with the
  // arange over xb broadcast to the batch, item by item.
  if (!has_l && g.lhs_div > 0 && g.batch <= 4096) {
    for (int64_t i = 0; i < g.batch; ++i) CHECK(i / g.lhs_div == bcast_offset(i, xb, g.bshape));
    g_elems += g.batch;
    ++g_ok[9];
  }
  ++g_ok[3];
}

void fuzz_qmm_geom() {
  const bool huge = pick(6) == 0;
  const int bits = pick(2) ? 4 : 8;
  const int gs = (int)(32 << pick(3));
  const int64_t K = 128 * (1 + pick(4));
  Shape x = rand_shape(4, huge);
  x.push_back(pick(10) == 0 ? K / 2 : K);
  Shape w{huge ? any_dim() : pick(5) + 1, K * bits / 32};
  if (pick(10) == 0) w.push_back(1);
  fmx_shape::QmmGeom g;
  const int rc = fmx_shape::qmm_geom(x, w, true, gs, bits, &g, "fuzz");
  if (rc != FMXQ_OK) return;
  CHECK(w.size() == 2 && g.K == K && x.back() == K);
  CHECK(g.oshape.size() == x.size() && g.oshape.back() == w[0]);
  CHECK(g.M == fmx_shape::prod(x, 0, x.size() - 1));
  CHECK(g.sshape == Shape({w[0], K / gs}));
  bool ok = false;
  prod_checked(g.oshape, &ok);
  CHECK(ok);
  ++g_ok[4];
}

void fuzz_reshape() {
  Shape in = rand_shape(5, false);
  const int64_t n = fmx_shape::prod(in);
  int req[8];
  const size_t nd = (size_t)pick(7);
  for (size_t i = 0; i < nd; ++i) {
    switch (pick(9)) {
      case 0: req[i] = -1; break;
      case 1: req[i] = -(int)pick(3) - 2; break;
      case 2: req[i] = 2147483647; break;
      case 3: req[i] = (int)n; break;
      default: req[i] = (int)small_dim();
    }
  }
  Shape out;
  const int rc = fmx_shape::reshape(in, req, nd, &out, "fuzz");
  if (rc != FMXQ_OK) return;
  CHECK(out.size() == nd);
  CHECK(fmx_shape::prod(out) == n);
  int minus = 0;
  for (size_t i = 0; i < nd; ++i) {
    if (req[i] == -1) ++minus;
    else CHECK(out[i] == req[i]);
    CHECK(out[i] >= 0);
  }
  CHECK(minus <= 1);
  ++g_ok[5];
}

void fuzz_split() {
  Shape in = rand_shape(4, false);
  if (in.empty()) in.push_back(small_dim());
  const int axis = (int)pick(2 * (int64_t)in.size() + 2) - (int)in.size() - 1;
  int idx[6];
  const size_t ni = (size_t)pick(6);
  int cur = 0;
  for (size_t i = 0; i < ni; ++i) {
    cur += (int)pick(3) - (pick(10) == 0 ? 2 : 0);
    idx[i] = cur;
  }
  fmx_shape::SplitPlan p;
  const int rc = fmx_shape::split(in, ni ? idx : nullptr, ni, axis, &p, "fuzz");
  if (rc != FMXQ_OK) return;
  CHECK(p.axis >= 0 && p.axis < (int)in.size());
  CHECK(p.cut.size() == ni + 2 && p.cut.front() == 0 && p.cut.back() == in[p.axis]);
  for (size_t i = 1; i < p.cut.size(); ++i) CHECK(p.cut[i] >= p.cut[i - 1]);
  CHECK(p.outer * in[p.axis] * p.inner == fmx_shape::prod(in));
  ++g_ok[6];
}

void fuzz_swapaxes() {
  Shape in = rand_shape(5, false);
  const int n = (int)in.size();
  const int a = (int)pick(2 * n + 3) - n - 1, b = (int)pick(2 * n + 3) - n - 1;
  fmx_shape::SwapPlan p;
  const int rc = fmx_shape::swapaxes(in, a, b, &p, "fuzz");
  CHECK((rc == FMXQ_OK) == (a >= -n && a < n && b >= -n && b < n));
  if (rc != FMXQ_OK) return;
  CHECK(p.a1 <= p.a2);
  Shape want = in;
  std::swap(want[(a + n) % n], want[(b + n) % n]);
  CHECK(p.shape == want);
  if (p.a1 == p.a2) return;  // a plain copy: the extents are not used
  CHECK(p.outer * p.d1 * p.mid * p.d2 * p.inner == fmx_shape::prod(in));
  // Element by element: the kernel's copy [outer, d1, mid, d2, inner] ->
  // [outer, d2, mid, d1, inner] against a brute-force transpose.
  const int64_t total = fmx_shape::prod(in);
  if (total > 4096) return;
  for (int64_t i = 0; i < total; ++i) {
    auto c = coords(i, in);
    std::swap(c[p.a1], c[p.a2]);
    int64_t dst = 0;
    for (int d = 0; d < n; ++d) dst = dst * p.shape[d] + c[d];
    const int64_t inner = i % p.inner, r1 = i / p.inner;
    const int64_t e2 = r1 % p.d2, r2 = r1 / p.d2;
    const int64_t m = r2 % p.mid, r3 = r2 / p.mid;
    const int64_t e1 = r3 % p.d1, o = r3 / p.d1;
    const int64_t k = (((o * p.d2 + e2) * p.mid + m) * p.d1 + e1) * p.inner + inner;
    CHECK(k == dst);
    ++g_elems;
  }
  ++g_ok[7];
}

void fuzz_round_bytes() {
  size_t n;
  switch (pick(4)) {
    case 0: n = (size_t)pick(4096); break;
    case 1: n = (size_t)pick((int64_t)1 << 22); break;
    case 2: n = (size_t)1 << pick(45); break;
    default: n = (size_t)(rnd() >> pick(30) >> 24);
  }
  const size_t r = fmx_shape::round_bytes(n);
  CHECK(r >= n && r >= 512 && r % 512 == 0);
  if (n > ((size_t)1 << 20)) CHECK(r - n <= n / 8);
  else CHECK(r - n < 512 || n < 512);
  CHECK(fmx_shape::round_bytes(n + 1) >= r);
  CHECK(fmx_shape::round_bytes(r) == r);
  ++g_ok[8];
}

// Random take / put / drain on one cache from several threads, each with its own
// fake buffers: no buffer is ever handed out while another holder has it, take
// only returns a buffer put under the same key and size, and nothing is lost.
void fuzz_buffer_cache(int steps) {
  fmx_shape::BufferCache cache;
  constexpr int kThreads = 4;
  std::vector<std::thread> th;
  std::vector<int> bad(kThreads, 0);
  for (int t = 0; t < kThreads; ++t) {
    th.emplace_back([&, t] {
      uint64_t st = 0x1234567ull * (t + 1);
      auto r = [&st]() { st ^= st << 13; st ^= st >> 7; st ^= st << 17; return st; };
      const int dev = t % 2;  // two threads per device
      const void* stream = reinterpret_cast<const void*>((uintptr_t)(0x1000 * (t + 1)));
      std::set<uintptr_t> mine, held;  // buffers this thread owns / holds outside the cache
      uintptr_t next = ((uintptr_t)(t + 1) << 40);
      for (int i = 0; i < steps; ++i) {
        const size_t cap = fmx_shape::round_bytes((size_t)(r() % 8192));
        switch (r() % 4) {
          case 0: {  // allocate a new buffer
            held.insert(next);
            mine.insert(next);
            next += 0x10000;
            break;
          }
          case 1: {  // return a held buffer
            if (held.empty()) break;
            const uintptr_t p = *held.begin();
            held.erase(held.begin());
            cache.put(dev, stream, cap, reinterpret_cast<void*>(p));
            break;
          }
          case 2: {  // take one
            void* p = nullptr;
            if (cache.take(dev, stream, cap, &p)) {
              const uintptr_t u = reinterpret_cast<uintptr_t>(p);
              if (!mine.count(u) || held.count(u)) bad[t] = 1;
              held.insert(u);
            }
            break;
          }
          default: {  // the device's drain on a failed hipMalloc: everything cached comes back
            if (r() % 16) break;
            for (void* p : cache.drain(dev)) {
              const uintptr_t u = reinterpret_cast<uintptr_t>(p);
              // another thread of the same device may get this thread's buffers
              held.insert(u);
              if (!mine.count(u)) {
                mine.insert(u);
              }
            }
          }
        }
      }
    });
  }
  for (auto& x : th) x.join();
  for (int t = 0; t < kThreads; ++t) CHECK(!bad[t]);
}

}  // namespace

int main(int argc, char** argv) {
  const long iters = argc > 1 ? std::atol(argv[1]) : 20000;
  if (argc > 2) g_state = std::strtoull(argv[2], nullptr, 10);
  for (long i = 0; i < iters; ++i) {
    fuzz_read_shape();
    fuzz_broadcast();
    fuzz_broadcast_map();
    fuzz_gather_geom();
    fuzz_qmm_geom();
    fuzz_reshape();
    fuzz_split();
    fuzz_swapaxes();
    fuzz_round_bytes();
  }
  fuzz_buffer_cache(20000);
  std::printf("%ld rounds; accepted: read_shape %ld, broadcast %ld, broadcast_map %ld, gather %ld "
              "(implicit-lhs shortcut verified %ld), qmm %ld, reshape %ld, split %ld, swapaxes %ld, "
              "round_bytes %ld; %ld elements checked one by one; buffer cache sequences clean\n",
              iters, g_ok[0], g_ok[1], g_ok[2], g_ok[3], g_ok[9], g_ok[4], g_ok[5], g_ok[6],
              g_ok[7], g_ok[8], g_elems);
  for (int i = 0; i < 10; ++i) CHECK(g_ok[i] > 0);
  return 0;
}
