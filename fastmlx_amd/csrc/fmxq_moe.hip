// fmxq_moe.hip -- the device pieces around gather_qmm in a SwitchGLU MoE layer.
//
// switchGLUCore (compute/models/switch_glu.go:107-153) brackets its three
// gather_qmm calls with argsort / inverse argsort / floor_divide / take (the
// sort branch, :135-150) and silu(gate) * up (:126-127, :146-147).  Here those
// become:
//   - sort_slots_kernel: a counting sort of the flattened routing slots by
//     expert id in one block (replaces argsort + take + floor_divide); the
//     order inside an expert is arbitrary, which cannot change any value
//     because every slot is its own GEMM row.  It also cuts the sorted order
//     into the expert segments the grouped product (fmxq_moe_gemm.hip) runs on;
//   - silu_mul_kernel: h = bf16(bf16(g * bf16(sigmoid(g))) * u), the rounding of
//     the silu (sigmoid then mul, qwen3_forward.go:229-239) then mul op chain;
//   - the unsort is fused into the down projection's store (GatherArgs::yrow).
// moe_combine_kernel is the weighted top-k sum plus optional shared expert of
// qwen3next_forward.go:519-524 and deepseekv3_forward.go:436-440.
#include "fmxq_common.hpp"
#include "fmxq_internal.hpp"

namespace fmxq {

// Exclusive prefix sum of one value per thread over the block; *total gets the
// sum.  wsum: one LDS word per wave.
__device__ __forceinline__ uint32_t block_exclusive_scan(uint32_t v, uint32_t* wsum,
                                                         uint32_t* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  uint32_t inc = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t t = (uint32_t)__shfl_up((int)inc, off, 64);
    if (lane >= off) inc += t;
  }
  if (lane == 63) wsum[wave] = inc;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t run = 0;
    for (int w = 0; w < (int)(blockDim.x >> 6); ++w) {
      const uint32_t t = wsum[w];
      wsum[w] = run;
      run += t;
    }
    *total = run;
  }
  __syncthreads();
  const uint32_t r = wsum[wave] + inc - v;
  __syncthreads();
  return r;
}

// Pieces of a c-slot run cut every `window` slots from its start.
__device__ __forceinline__ uint32_t run_pieces(uint32_t c, uint32_t window) {
  return (c + window - 1) / window;
}

// One block: counts per expert in LDS, exclusive scan, scatter.  Ids >= E go
// to a final bucket (the gather kernels zero those rows and raise the flag).
// Each thread owns a run of consecutive buckets for the scans.  With seg
// non-null, before the scatter: the pieces of every bucket's range
// [off, off + count) cut every `window` slots from off (so a run of c slots has
// ceil(c / window) pieces wherever it starts), as (start, len) pairs in bucket
// order, and their number in *nseg.  With tiles non-null as well, the
// runs of an expert (id < E) with at least long_min slots are not cut into
// window pieces but into tiles of tile_rows slots, written as (start, len) pairs
// to tiles with their number in *ntile (the grouped GEMM's work list).
//
// With sh_T > 0, sh_T shared-expert slots follow the S routed ones: slot S + t
// has id E and x row t, and out-of-range routed ids go to bucket E + 1 and are
// stored as E + 1 in rhs_sorted (so a walk tells the shared expert, id E, from a
// bad id, above E).
//
// STAGED (S + sh_T <= kSortStageSlots): the scatter writes the three sorted
// arrays to LDS and the block then copies them out in order: one block's
// scattered 4-byte stores are one cache line each, the copy is coalesced.
constexpr int64_t kSortStageSlots = 8192;
template <bool STAGED>
__global__ __launch_bounds__(1024) void sort_slots_kernel(const uint32_t* __restrict__ inds,
                                                          int64_t S, int64_t sh_T,
                                                          int64_t lhs_div, int64_t E,
                                                          uint32_t* __restrict__ order,
                                                          uint32_t* __restrict__ rhs_sorted,
                                                          uint32_t* __restrict__ lhs_sorted,
                                                          const uint32_t* __restrict__ lhs,
                                                          uint32_t* __restrict__ seg,
                                                          uint32_t* __restrict__ nseg,
                                                          int window, uint32_t* __restrict__ tiles,
                                                          uint32_t* __restrict__ ntile,
                                                          uint32_t long_min, uint32_t tile_rows) {
  extern __shared__ uint32_t cnt[];  // nb counters, then nb cursors
  __shared__ uint32_t stg[STAGED ? 3 * kSortStageSlots : 1];
  __shared__ uint32_t wsum[16], total;
  const uint32_t bad = (uint32_t)E + (sh_T > 0 ? 1u : 0u);  // bucket of out-of-range ids
  const int64_t nb = (int64_t)bad + 1;
  const int64_t Sa = S + sh_T;
  auto bucket = [&](int64_t s) -> uint32_t {
    if (s >= S) return (uint32_t)E;
    const uint32_t e = inds[s];
    return e < (uint64_t)E ? e : bad;
  };
  uint32_t* cur = cnt + nb;
  for (int64_t i = threadIdx.x; i < nb; i += blockDim.x) cnt[i] = 0;
  __syncthreads();
  for (int64_t s = threadIdx.x; s < Sa; s += blockDim.x) atomicAdd(&cnt[bucket(s)], 1u);
  __syncthreads();
  const int64_t per = (nb + blockDim.x - 1) / blockDim.x;
  const int64_t b0 = threadIdx.x * per < nb ? threadIdx.x * per : nb;
  const int64_t b1 = b0 + per < nb ? b0 + per : nb;
  uint32_t local = 0;
  for (int64_t i = b0; i < b1; ++i) local += cnt[i];
  uint32_t base = block_exclusive_scan(local, wsum, &total);
  for (int64_t i = b0; i < b1; ++i) {
    cur[i] = base;
    base += cnt[i];
  }
  __syncthreads();
  if (seg) {
    auto is_long = [&](int64_t i) { return tiles && i < E && cnt[i] >= long_min; };
    uint32_t lp = 0, lt = 0;
    for (int64_t i = b0; i < b1; ++i) {
      if (is_long(i)) lt += (cnt[i] + tile_rows - 1) / tile_rows;
      else lp += run_pieces(cnt[i], (uint32_t)window);
    }
    uint32_t k = block_exclusive_scan(lp, wsum, &total);
    if (threadIdx.x == 0) *nseg = total;
    uint32_t kt = 0;
    if (tiles) {
      kt = block_exclusive_scan(lt, wsum, &total);
      if (threadIdx.x == 0) *ntile = total;
    }
    for (int64_t i = b0; i < b1; ++i) {
      const uint32_t end = cur[i] + cnt[i];
      if (is_long(i)) {
        for (uint32_t p = cur[i]; p < end; p += tile_rows, ++kt) {
          tiles[2 * kt] = p;
          tiles[2 * kt + 1] = end - p < tile_rows ? end - p : tile_rows;
        }
        continue;
      }
      for (uint32_t p = cur[i]; p < end; p += (uint32_t)window, ++k) {
        seg[2 * k] = p;
        seg[2 * k + 1] = end - p < (uint32_t)window ? end - p : (uint32_t)window;
      }
    }
    __syncthreads();  // the scatter below advances cur
  }
  uint32_t* so = STAGED ? stg : order;
  uint32_t* sr = STAGED ? stg + kSortStageSlots : rhs_sorted;
  uint32_t* sl = STAGED ? stg + 2 * kSortStageSlots : lhs_sorted;
  for (int64_t s = threadIdx.x; s < Sa; s += blockDim.x) {
    const uint32_t b = bucket(s);
    const uint32_t pos = atomicAdd(&cur[b], 1u);
    so[pos] = (uint32_t)s;
    sr[pos] = sh_T > 0 ? b : inds[s];
    sl[pos] = s >= S ? (uint32_t)(s - S) : lhs ? lhs[s] : (uint32_t)(s / lhs_div);
  }
  if constexpr (!STAGED) return;
  __syncthreads();
  for (int64_t i = threadIdx.x; i < Sa; i += blockDim.x) {
    order[i] = so[i];
    rhs_sorted[i] = sr[i];
    lhs_sorted[i] = sl[i];
  }
}

__device__ __forceinline__ float r16(float v) { return bf16_bits_to_f32(f32_to_bf16_rne(v)); }

__global__ __launch_bounds__(256) void fill_u32_kernel(uint32_t* __restrict__ p, uint32_t v,
                                                       int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = v;
}

// 8 elements per thread; n is a multiple of 8.
__global__ __launch_bounds__(256) void silu_mul_kernel(const uint16_t* __restrict__ g,
                                                       const uint16_t* __restrict__ u,
                                                       uint16_t* __restrict__ h, int64_t n8) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n8; i += (int64_t)gridDim.x * 256) {
    const u32x4 gv = reinterpret_cast<const u32x4*>(g)[i];
    const u32x4 uv = reinterpret_cast<const u32x4*>(u)[i];
    u32x4 o;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float g0 = bf16_lo(gv[j]), g1 = bf16_hi(gv[j]);
      const float s0 = r16(1.f / (1.f + __expf(-g0))), s1 = r16(1.f / (1.f + __expf(-g1)));
      const float h0 = r16(r16(g0 * s0) * bf16_lo(uv[j]));
      const float h1 = r16(r16(g1 * s1) * bf16_hi(uv[j]));
      o[j] = f32_to_bf16_rne(h0) | (f32_to_bf16_rne(h1) << 16);
    }
    reinterpret_cast<u32x4*>(h)[i] = o;
  }
}

// out[t] = bf16( bf16(sum_j bf16(y[t,j] * w[t,j])) + shared_term ), shared_term =
// bf16(bf16(sigmoid(sg[t])) * shared[t]) with a gate, shared[t] without, none if
// shared is null.  One thread per (t, d) pair of 2 columns.
__global__ __launch_bounds__(256) void moe_combine_kernel(const uint16_t* __restrict__ y,
                                                          const uint16_t* __restrict__ w,
                                                          const uint16_t* __restrict__ shared,
                                                          const uint16_t* __restrict__ sgate,
                                                          uint16_t* __restrict__ out, int64_t T,
                                                          int64_t topk, int64_t D) {
  const int64_t pairs = D / 2;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < T * pairs;
       i += (int64_t)gridDim.x * 256) {
    const int64_t t = i / pairs, d = (i - t * pairs) * 2;
    float a0 = 0.f, a1 = 0.f;
    // The shared term's loads go first, then up to 16 expert rows are requested
    // before any is summed (the sum still runs in j order).
    uint32_t sv = 0;
    uint16_t sgb = 0;
    if (shared) {
      sv = *reinterpret_cast<const uint32_t*>(shared + t * D + d);
      if (sgate) sgb = sgate[t];
    }
    for (int64_t j0 = 0; j0 < topk; j0 += 16) {
      uint32_t v[16];
      uint16_t wb[16];
#pragma unroll
      for (int jj = 0; jj < 16; ++jj) {
        const int64_t j = j0 + jj < topk ? j0 + jj : topk - 1;
        v[jj] = *reinterpret_cast<const uint32_t*>(y + (t * topk + j) * D + d);
        wb[jj] = w[t * topk + j];
      }
#pragma unroll
      for (int jj = 0; jj < 16; ++jj) {
        if (j0 + jj < topk) {
          const float wj = bf16_bits_to_f32(wb[jj]);
          a0 += r16(bf16_lo(v[jj]) * wj);
          a1 += r16(bf16_hi(v[jj]) * wj);
        }
      }
    }
    a0 = r16(a0);
    a1 = r16(a1);
    if (shared) {
      float s0 = bf16_lo(sv), s1 = bf16_hi(sv);
      if (sgate) {
        const float gt = r16(1.f / (1.f + __expf(-bf16_bits_to_f32(sgb))));
        s0 = r16(gt * s0);
        s1 = r16(gt * s1);
      }
      a0 = r16(a0 + s0);
      a1 = r16(a1 + s1);
    }
    *reinterpret_cast<uint32_t*>(out + t * D + d) = f32_to_bf16_rne(a0) | (f32_to_bf16_rne(a1) << 16);
  }
}

static unsigned grid_for(int64_t items, int64_t per_block) {
  int64_t b = (items + per_block - 1) / per_block;
  if (b > 65536) b = 65536;
  return (unsigned)(b < 1 ? 1 : b);
}

hipError_t launch_sort_slots(const uint32_t* inds, int64_t S, int64_t lhs_div, int64_t E,
                             uint32_t* order, uint32_t* rhs_sorted, uint32_t* lhs_sorted,
                             hipStream_t stream, const uint32_t* lhs, uint32_t* seg,
                             uint32_t* nseg, int window, uint32_t* tiles, uint32_t* ntile,
                             int long_min, int tile_rows, int64_t sh_T) {
  if (seg && (!nseg || window < 1)) return hipErrorInvalidValue;
  if (tiles && (!seg || !ntile || long_min < 1 || tile_rows < 1)) return hipErrorInvalidValue;
  if (sh_T < 0) return hipErrorInvalidValue;
  const size_t lds = (size_t)(E + 1 + (sh_T > 0 ? 1 : 0)) * 2 * sizeof(uint32_t);
  // The staged form holds 96 KiB (and a few words) of static LDS; its counters
  // stay within 56 KiB so the block's total stays below the CU's 160 KiB.
  if (S + sh_T <= kSortStageSlots && lds <= 56 * 1024)
    sort_slots_kernel<true><<<1, 1024, lds, stream>>>(inds, S, sh_T, lhs_div, E, order,
                                                      rhs_sorted, lhs_sorted, lhs, seg, nseg,
                                                      window, tiles, ntile, (uint32_t)long_min,
                                                      (uint32_t)tile_rows);
  else
    sort_slots_kernel<false><<<1, 1024, lds, stream>>>(inds, S, sh_T, lhs_div, E, order,
                                                       rhs_sorted, lhs_sorted, lhs, seg, nseg,
                                                       window, tiles, ntile, (uint32_t)long_min,
                                                       (uint32_t)tile_rows);
  return hipGetLastError();
}

// h rows of the grouped-GEMM tiles: h = silu(g) * u with the op chain's roundings
// (silu_mul_kernel's arithmetic).  Grid (column blocks, tile bound); a block
// covers 256 x 8 values of one tile: rows start .. start + len, n cols.
__global__ __launch_bounds__(256) void silu_mul_tiles_kernel(const uint16_t* __restrict__ g,
                                                             const uint16_t* __restrict__ u,
                                                             uint16_t* __restrict__ h,
                                                             const uint32_t* __restrict__ tiles,
                                                             const uint32_t* __restrict__ ntile,
                                                             int64_t n) {
  const int64_t t = blockIdx.y;
  if (t >= (int64_t)*ntile) return;
  const int64_t start = tiles[2 * t], len = tiles[2 * t + 1];
  const int64_t n8 = n / 8, items = len * n8;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < items;
       i += (int64_t)gridDim.x * 256) {
    const int64_t r = start + i / n8, c = i % n8;
    const u32x4 gv = reinterpret_cast<const u32x4*>(g + r * n)[c];
    const u32x4 uv = reinterpret_cast<const u32x4*>(u + r * n)[c];
    u32x4 o;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float g0 = bf16_lo(gv[j]), g1 = bf16_hi(gv[j]);
      const float s0 = r16(1.f / (1.f + __expf(-g0))), s1 = r16(1.f / (1.f + __expf(-g1)));
      const float h0 = r16(r16(g0 * s0) * bf16_lo(uv[j]));
      const float h1 = r16(r16(g1 * s1) * bf16_hi(uv[j]));
      o[j] = f32_to_bf16_rne(h0) | (f32_to_bf16_rne(h1) << 16);
    }
    reinterpret_cast<u32x4*>(h + r * n)[c] = o;
  }
}

hipError_t launch_silu_mul_tiles(const uint16_t* g, const uint16_t* u, uint16_t* h,
                                 const uint32_t* tiles, const uint32_t* ntile, int64_t max_tiles,
                                 int64_t tile_rows, int64_t n, hipStream_t stream) {
  if (max_tiles <= 0) return hipSuccess;
  if (n % 8 != 0) return hipErrorInvalidValue;
  const int64_t per_tile = tile_rows * (n / 8);
  dim3 grid((unsigned)((per_tile + 255) / 256 < 64 ? (per_tile + 255) / 256 : 64),
            (unsigned)max_tiles);
  silu_mul_tiles_kernel<<<grid, 256, 0, stream>>>(g, u, h, tiles, ntile, n);
  return hipGetLastError();
}

hipError_t launch_silu_mul(const uint16_t* g, const uint16_t* u, uint16_t* h, int64_t n,
                           hipStream_t stream) {
  const int64_t n8 = n / 8;
  silu_mul_kernel<<<grid_for(n8, 256), 256, 0, stream>>>(g, u, h, n8);
  return hipGetLastError();
}

hipError_t launch_moe_combine(const uint16_t* y, const uint16_t* w, const uint16_t* shared,
                              const uint16_t* sgate, uint16_t* out, int64_t T, int64_t topk,
                              int64_t D, hipStream_t stream) {
  moe_combine_kernel<<<grid_for(T * (D / 2), 256), 256, 0, stream>>>(y, w, shared, sgate, out, T,
                                                                     topk, D);
  return hipGetLastError();
}

hipError_t launch_fill_u32(uint32_t* p, uint32_t v, int64_t n, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  fill_u32_kernel<<<(unsigned)((n + 255) / 256), 256, 0, stream>>>(p, v, n);
  return hipGetLastError();
}

}  // namespace fmxq
