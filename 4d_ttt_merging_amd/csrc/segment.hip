// Deterministic segmented reductions of a merge plan: per-destination member
// lists (CSR), mass / log-mass, Q/K/V compaction and the dense restore map.
//
// The reference groups plan members with one stable argsort + bincount per
// corner (vggt_omega/models/token_merging.py:323-333, 40-59) so that every
// reduction runs in a fixed source order; the default sparse-convex mass uses
// atomic scatter_add_ (vggt_omega/models/sparse_convex.py:2448-2450), whose
// float order is unspecified.  Here one stable LSD radix sort (8-bit digits,
// wave-ballot ranking) orders all (destination, corner) pairs at once, and the
// reductions walk those lists sequentially, reproducing the order of
// `deterministic_weighted_normalizer` and of `WeightedBilinearTokenPlan.compact`:
//   mass[k]    = ((1 + S_0) + S_1) + S_2) + S_3,    S_c = sum in source order of w
//   compact[k] = ((x[keep_k] + T_0) + T_1 + T_2 + T_3) / mass[k],  T_c = sum of x*w
// TokenPlan (FastVGGT) compaction is the one-segment case: the members of a
// cluster in ascending token order, divided by their count
// (token_merging.py:176-191).
#include <algorithm>

#include "vgo_common.h"

namespace vgo {
namespace {

constexpr int kSortThreads = 256;
constexpr int kSortRounds = 8;
constexpr int kBlockItems = kSortThreads * kSortRounds;  // 2048 items per block
constexpr int kSortWaves = kSortThreads / 64;

// The first pass reads the caller's keys with `limit` = n_buckets: a key at or
// past it (a negative id too) sorts past the last bucket.  Later passes read
// clamped keys (limit 0: as they are).
__device__ __forceinline__ uint32_t sort_key(const uint32_t* keys, int i, uint32_t limit) {
  const uint32_t k = keys[i];
  return limit != 0u && k > limit ? limit : k;
}

__global__ __launch_bounds__(kSortThreads) void radix_hist_kernel(const uint32_t* __restrict__ keys,
                                                                  int n, int shift,
                                                                  uint32_t* __restrict__ hist,
                                                                  int nblocks, uint32_t limit) {
  __shared__ uint32_t h[256];
  const int tid = threadIdx.x;
  h[tid] = 0;
  __syncthreads();
  const int base = blockIdx.x * kBlockItems;
#pragma unroll
  for (int r = 0; r < kSortRounds; ++r) {
    const int i = base + r * kSortThreads + tid;
    if (i < n) atomicAdd(&h[(sort_key(keys, i, limit) >> shift) & 0xFF], 1u);
  }
  __syncthreads();
  hist[tid * nblocks + blockIdx.x] = h[tid];
}

// In-place exclusive scan of n values by one work-group (contiguous runs).
__global__ __launch_bounds__(1024) void exclusive_scan_kernel(uint32_t* __restrict__ data, int n) {
  __shared__ uint32_t waves[16];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int per = (n + 1023) / 1024;
  const int b = min(n, tid * per), e = min(n, b + per);
  uint32_t sum = 0;
  for (int i = b; i < e; ++i) sum += data[i];
  uint32_t x = sum;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t y = __shfl_up(x, off);
    if (lane >= off) x += y;
  }
  if (lane == 63) waves[wave] = x;
  __syncthreads();
  if (wave == 0) {
    uint32_t w = lane < 16 ? waves[lane] : 0;
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) {
      const uint32_t y = __shfl_up(w, off);
      if (lane >= off) w += y;
    }
    if (lane < 16) waves[lane] = w;
  }
  __syncthreads();
  uint32_t run = (wave > 0 ? waves[wave - 1] : 0) + x - sum;
  for (int i = b; i < e; ++i) {
    const uint32_t v = data[i];
    data[i] = run;
    run += v;
  }
}

// vals_in == nullptr (the first pass): the values are the item indices.
__global__ __launch_bounds__(kSortThreads) void radix_scatter_kernel(
    const uint32_t* __restrict__ keys_in, const uint32_t* __restrict__ vals_in,
    uint32_t* __restrict__ keys_out, uint32_t* __restrict__ vals_out, int n, int shift,
    const uint32_t* __restrict__ hist_scan, int nblocks, uint32_t limit) {
  __shared__ uint32_t base[256];
  __shared__ uint32_t running[256];
  __shared__ uint32_t wcnt[kSortWaves][256];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  base[tid] = hist_scan[tid * nblocks + blockIdx.x];
  running[tid] = 0;
  const uint64_t lt_mask = (uint64_t(1) << lane) - 1;
  for (int r = 0; r < kSortRounds; ++r) {
#pragma unroll
    for (int w = 0; w < kSortWaves; ++w) wcnt[w][tid] = 0;
    __syncthreads();
    const int i = blockIdx.x * kBlockItems + r * kSortThreads + tid;
    const bool valid = i < n;
    uint32_t key = 0, val = 0, d = 0;
    if (valid) {
      key = sort_key(keys_in, i, limit);
      val = vals_in ? vals_in[i] : static_cast<uint32_t>(i);
      d = (key >> shift) & 0xFF;
    }
    uint64_t same = __ballot(valid);
#pragma unroll
    for (int bit = 0; bit < 8; ++bit) {
      const uint64_t ones = __ballot(valid && ((d >> bit) & 1));
      same &= ((d >> bit) & 1) ? ones : ~ones;
    }
    const uint32_t rank = __popcll(same & lt_mask);
    if (valid && rank == 0) wcnt[wave][d] = __popcll(same);
    __syncthreads();
    if (valid) {
      uint32_t pos = base[d] + running[d] + rank;
      for (int w = 0; w < wave; ++w) pos += wcnt[w][d];
      keys_out[pos] = key;
      vals_out[pos] = val;
    }
    __syncthreads();
    uint32_t add = 0;
#pragma unroll
    for (int w = 0; w < kSortWaves; ++w) add += wcnt[w][tid];
    running[tid] += add;
    __syncthreads();
  }
}

// offsets[k] = first position of key k in the sorted keys; offsets[n_buckets] = n_valid.
__global__ __launch_bounds__(256) void bucket_offsets_kernel(const uint32_t* __restrict__ skeys, int n,
                                                             int n_buckets,
                                                             int32_t* __restrict__ offsets) {
  const int e = blockIdx.x * 256 + threadIdx.x;
  if (e >= n) return;
  const int64_t k = min(static_cast<int64_t>(skeys[e]), static_cast<int64_t>(n_buckets));
  const int64_t prev = e > 0 ? min(static_cast<int64_t>(skeys[e - 1]), static_cast<int64_t>(n_buckets)) : -1;
  for (int64_t kk = prev + 1; kk <= k; ++kk) offsets[kk] = e;
  if (e == n - 1)
    for (int64_t kk = k + 1; kk <= n_buckets; ++kk) offsets[kk] = n;
}

__global__ __launch_bounds__(256) void fill_i32_kernel(int32_t* __restrict__ p, int n, int32_t v) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = v;
}

int key_bits(int64_t limit) {
  int bits = 1;
  while ((int64_t(1) << bits) <= limit) ++bits;
  return bits;
}

size_t align_up(size_t x) { return (x + 255) & ~size_t(255); }

// ------------------------------------------------------------- mass ----
__global__ __launch_bounds__(256) void segment_mass_kernel(
    const int32_t* __restrict__ offsets, int segs_per_row, const uint32_t* __restrict__ items,
    const float* __restrict__ weights, int n_weights, int rows, float start,
    float* __restrict__ mass, float* __restrict__ log_mass) {
  const int k = blockIdx.x * 256 + threadIdx.x;
  if (k >= rows) return;
  float m = start;
  for (int c = 0; c < segs_per_row; ++c) {
    const int b = offsets[k * segs_per_row + c], e = offsets[k * segs_per_row + c + 1];
    float s = 0.0f;
    for (int q = b; q < e; ++q) {
      const uint32_t p = items[q];
      s = s + (weights ? (static_cast<int>(p) < n_weights ? weights[p] : 0.0f) : 1.0f);
    }
    m = m + s;
  }
  mass[k] = m;
  if (log_mass) log_mass[k] = logf(m);
}

// ------------------------------------------------------ compaction ----
// out[k] = (base + sum_c sum_{p in seg(k,c)} x[row(p)] * w[p]) / norm[k], in fp32,
// cast to the value type.  Channel c of token t lives at t*ts + (c/64)*hs + c%64
// (hs = 64 for a row-contiguous tensor; a [B,H,N,64] tensor viewed per token
// has ts = 64, hs = N*64), so head-major attention operands are read and written
// without a transpose copy.
template <typename T, int U>
__global__ __launch_bounds__(256) void compact_kernel(
    const T* __restrict__ x, int64_t xts, int64_t xhs, int64_t x_rows,
    const int64_t* __restrict__ base_rows, const int32_t* __restrict__ offsets, int segs_per_row,
    const uint32_t* __restrict__ items, int item_shift, const int64_t* __restrict__ item_rows,
    const float* __restrict__ weights, int n_weights, const float* __restrict__ norm, int rows,
    int dim, T* __restrict__ out, int64_t ots, int64_t ohs) {
  const int lane = threadIdx.x & 63;
  const int k = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (k >= rows) return;
  for (int c0 = 0; c0 < dim; c0 += 64 * U) {
    float acc[U];
    const int64_t b = base_rows ? base_rows[k] : -1;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = c0 + u * 64 + lane;
      acc[u] = (b >= 0 && b < x_rows && c < dim)
                   ? to_f32(x[b * xts + (c >> 6) * xhs + (c & 63)])
                   : 0.0f;
    }
    for (int sgi = 0; sgi < segs_per_row; ++sgi) {
      const int sb = offsets[k * segs_per_row + sgi], se = offsets[k * segs_per_row + sgi + 1];
      if (sb >= se) continue;
      float seg[U];
#pragma unroll
      for (int u = 0; u < U; ++u) seg[u] = 0.0f;
      for (int q = sb; q < se; ++q) {
        const uint32_t p = items[q];
        const int64_t i = static_cast<int64_t>(p >> item_shift);
        const int64_t row = item_rows ? item_rows[i] : i;
        const float w = weights ? (static_cast<int>(p) < n_weights ? weights[p] : 0.0f) : 1.0f;
        if (row < 0 || row >= x_rows) continue;
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int c = c0 + u * 64 + lane;
          if (c < dim) seg[u] = seg[u] + to_f32(x[row * xts + (c >> 6) * xhs + (c & 63)]) * w;
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) acc[u] = acc[u] + seg[u];
    }
    const float nk = norm ? norm[k] : 1.0f;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = c0 + u * 64 + lane;
      if (c < dim) out[static_cast<int64_t>(k) * ots + (c >> 6) * ohs + (c & 63)] = from_f32<T>(acc[u] / nk);
    }
  }
}

// Vectorised compaction: lane l owns 16 contiguous channels [16 l, 16 l + 16)
// of every 1024-channel slab (a head is four lanes), loaded and stored as
// 16-byte vectors.  With ln_w != NULL every gathered row is first normalised
// per 64-channel head (LayerNorm, eps, shared affine) in fp32 -- the q_norm /
// k_norm of vggt_omega/models/layers/attention.py:337-339 fused into the pooling
// -- and the output may be a narrower dtype than the input, so q/k go from the
// bf16 projection to bf16 attention operands with one rounding.
template <typename T>
struct V16;
template <>
struct V16<bf16_t> {
  typedef bf16x8 half;
  static constexpr int kLoads = 2;
};
template <>
struct V16<f16_t> {
  typedef f16x8 half;
  static constexpr int kLoads = 2;
};
template <>
struct V16<float> {
  typedef f32x4 half;
  static constexpr int kLoads = 4;
};

template <typename T>
__device__ __forceinline__ void v16_load(const T* p, float* v) {
  typedef typename V16<T>::half V;
  constexpr int kPer = 16 / V16<T>::kLoads;
#pragma unroll
  for (int i = 0; i < V16<T>::kLoads; ++i) {
    const V x = *reinterpret_cast<const V*>(p + i * kPer);
#pragma unroll
    for (int j = 0; j < kPer; ++j) v[i * kPer + j] = to_f32(x[j]);
  }
}

// 16 values of T as loaded (not yet widened), so the next member's row can be
// in flight while the current one is normalised.
template <typename T>
struct V16Raw {
  typename V16<T>::half h[V16<T>::kLoads];
};

template <typename T>
__device__ __forceinline__ void v16_load_raw(const T* p, V16Raw<T>& r) {
  typedef typename V16<T>::half V;
  constexpr int kPer = 16 / V16<T>::kLoads;
#pragma unroll
  for (int i = 0; i < V16<T>::kLoads; ++i) r.h[i] = *reinterpret_cast<const V*>(p + i * kPer);
}

template <typename T>
__device__ __forceinline__ void v16_widen(const V16Raw<T>& r, float* v) {
  constexpr int kPer = 16 / V16<T>::kLoads;
#pragma unroll
  for (int i = 0; i < V16<T>::kLoads; ++i)
#pragma unroll
    for (int j = 0; j < kPer; ++j) v[i * kPer + j] = to_f32(r.h[i][j]);
}

template <typename T>
__device__ __forceinline__ void v16_store(T* p, const float* v) {
  typedef typename V16<T>::half V;
  constexpr int kPer = 16 / V16<T>::kLoads;
#pragma unroll
  for (int i = 0; i < V16<T>::kLoads; ++i) {
    V x;
#pragma unroll
    for (int j = 0; j < kPer; ++j) x[j] = from_f32<T>(v[i * kPer + j]);
    *reinterpret_cast<V*>(p + i * kPer) = x;
  }
}

// Outputs of one compaction launch that share its segments: output g reads
// the channels at element offset x_off[g] of every member row, optionally
// LayerNorms them per head, and writes out[g] with its own strides.
template <typename TO, int G>
struct CompactOuts {
  int64_t x_off[G];
  const float* ln_w[G];
  const float* ln_b[G];
  TO* out[G];
  int64_t ots[G], ohs[G];
};

// One output of a launch, as a wave sees it.
template <typename TO>
struct CompactOut {
  int64_t x_off;
  const float* ln_w;
  const float* ln_b;
  TO* out;
  int64_t ots, ohs;
};

// acc[j] = acc[j] / n, correctly rounded as the division (n is the row's
// normalizer, the same in every lane).  n == 1 leaves acc as it is.
// Otherwise, when 1 <= n <= 2^16 (cluster counts and masses) and every value of
// the wave lies in [2^-100, FLT_MAX], each takes three operations instead of a
// division: with r = RN(1/n), q = RN(a*r) and the exact residual
// e = fma(-q, n, a), fma(e, r, q) is the correctly rounded a/n (Markstein's
// theorem: r within half an ulp of 1/n, q within one ulp of a/n, e exact).
// These ranges keep q finite and q and e clear of the subnormals, where the
// residual can round; anything else (zeros, subnormals, infinities, NaNs, other
// normalizers) takes the division.
__device__ __forceinline__ void divide_by_normalizer(float (&acc)[16], float n) {
  if (n == 1.0f) return;
  float lo = __builtin_inff(), hi = 0.0f;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    lo = fminf(lo, fabsf(acc[j]));
    hi = __builtin_elementwise_maximum(hi, fabsf(acc[j]));  // a NaN propagates
  }
  const bool in_range = lo >= 0x1p-100f && hi <= 3.40282347e+38f && n >= 1.0f && n <= 65536.0f;
  if (__ballot(!in_range) == 0) {
    const float r = 1.0f / n;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const float a = acc[j];
      const float q = a * r;
      acc[j] = fmaf(fmaf(-q, n, a), r, q);
    }
  } else {
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[j] = acc[j] / n;
  }
}

// Compact row k of one output: (f(x[base_rows[k]]) + sum over the row's segments
// of the segment's sum of weights[p] * f(x[row of p])) / norm[k], f = the
// output's per-head LayerNorm (parameters staged in LDS: ln_w / ln_b) or the
// identity.  kFold (one segment per row, no base row): the segment's sum is the
// row's sum, so members add into acc directly -- acc starts at +0 as a segment
// sum does, and a sum that starts at +0 is never -0, so 0 + seg would equal seg.
template <typename TI, typename TO, bool kFold>
__device__ __forceinline__ void compact16_row(
    const TI* __restrict__ x, int64_t xts, int64_t xhs, int64_t x_rows,
    const int64_t* __restrict__ base_rows, const int32_t* __restrict__ offsets, int segs_per_row,
    const uint32_t* __restrict__ items, int item_shift, const int64_t* __restrict__ item_rows,
    const float* __restrict__ weights, int n_weights, const float* __restrict__ norm, int k,
    int dim, float ln_eps, const CompactOut<TO>& o, const float* ln_w, const float* ln_b) {
  const int lane = threadIdx.x & 63;
  const int d0 = (lane * 16) & 63;  // the same in every 1024-channel chunk
  const int64_t b = base_rows ? base_rows[k] : -1;
  const float nk = norm ? norm[k] : 1.0f;
  auto layer_norm = [&](float* v) {
    if (o.ln_w) head_layer_norm(v, ln_w + d0, ln_b + d0, ln_eps);
  };
  for (int c0 = 0; c0 < dim; c0 += 1024) {
    const int c = c0 + lane * 16;
    // Whole 4-lane head groups are active together (dim % 64 == 0).  Lanes past
    // the row read its first channels instead and store nothing, so every load
    // below is under a wave-uniform condition only.
    const bool active = c < dim;
    const int cl = active ? c : 0;
    const int64_t xoff = static_cast<int64_t>(cl >> 6) * xhs + (cl & 63) + o.x_off;
    float acc[16], v[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[j] = 0.0f;
    if (b >= 0 && b < x_rows) {
      v16_load(x + b * xts + xoff, acc);
      layer_norm(acc);
    }
    // The row's members over all its segments (segment t holds items[ob[t]] ..
    // items[ob[t + 1] - 1]) as one stream, software-pipelined: while member q
    // is normalised and pooled, member q + 1's row is in flight, member q + 2's
    // row id and member q + 3's item are being fetched, so a row costs a couple
    // of round trips rather than one chain per member.  The sums keep the
    // reference's order: seg over a segment's members, then acc += seg for
    // every non-empty segment.
    const int32_t* ob = offsets + static_cast<int64_t>(k) * segs_per_row;
    // Segment ends ob[1..4] up front (plans have one or four segments per row);
    // further ones are read when reached.
    const int o1 = ob[1];
    const int o2 = segs_per_row >= 2 ? ob[2] : 0;
    const int o3 = segs_per_row >= 3 ? ob[3] : 0;
    const int o4 = segs_per_row >= 4 ? ob[4] : 0;
    auto seg_end = [&](int t1) -> int {  // ob[t1], 1 <= t1 <= segs_per_row
      return t1 == 1 ? o1 : t1 == 2 ? o2 : t1 == 3 ? o3 : t1 == 4 ? o4 : ob[t1];
    };
    int q = ob[0];
    const int q_end = seg_end(segs_per_row);
    if (q < q_end) {
      int t = 0;
      int t_end = o1;
      while (t_end <= q && t + 1 < segs_per_row) t_end = seg_end(++t + 1);
      auto row_of = [&](uint32_t p) -> int64_t {
        const int64_t i = static_cast<int64_t>(p >> item_shift);
        return item_rows ? item_rows[i] : i;
      };
      auto weight_of = [&](uint32_t p) -> float {
        return weights ? (static_cast<int>(p) < n_weights ? weights[p] : 0.0f) : 1.0f;
      };
      auto usable = [&](int64_t row) { return row >= 0 && row < x_rows; };
      const uint32_t p0 = items[q];
      uint32_t p1 = q + 1 < q_end ? items[q + 1] : 0u;
      uint32_t p2 = q + 2 < q_end ? items[q + 2] : 0u;
      const int64_t row0 = row_of(p0);
      int64_t row1 = q + 1 < q_end ? row_of(p1) : -1;
      // Two row buffers used in turn (an unrolled pair of steps), so no
      // register copy has to wait for a row still in flight.
      V16Raw<TI> ra, rb;
      bool ok_a = usable(row0), ok_b = false;
      float w_a = weight_of(p0), w_b = 0.0f;
      if (ok_a) v16_load_raw(x + row0 * xts + xoff, ra);
      float seg_own[kFold ? 1 : 16];
      float* seg = kFold ? acc : seg_own;
      if constexpr (!kFold) {
#pragma unroll
        for (int j = 0; j < 16; ++j) seg[j] = 0.0f;
      }
      // One member: request member q + 1's row into `nxt` (and member q + 2's
      // row id, member q + 3's item), then pool member q from `cur`.
      auto step = [&](V16Raw<TI>& cur, bool ok_c, float w_c, V16Raw<TI>& nxt, bool& ok_n, float& w_n) {
        ok_n = q + 1 < q_end && usable(row1);
        w_n = q + 1 < q_end ? weight_of(p1) : 0.0f;
        if (ok_n) v16_load_raw(x + row1 * xts + xoff, nxt);
        const int64_t row2 = q + 2 < q_end ? row_of(p2) : -1;
        const uint32_t p3 = q + 3 < q_end ? items[q + 3] : 0u;
        if (ok_c) {
          v16_widen(cur, v);
          layer_norm(v);
          if (weights) {
#pragma unroll
            for (int j = 0; j < 16; ++j) seg[j] = seg[j] + v[j] * w_c;
          } else {  // w_c == 1
#pragma unroll
            for (int j = 0; j < 16; ++j) seg[j] = seg[j] + v[j];
          }
        }
        if (!kFold && q + 1 == t_end) {
#pragma unroll
          for (int j = 0; j < 16; ++j) {
            acc[j] = acc[j] + seg[j];
            seg[j] = 0.0f;
          }
          // Empty segments that follow add nothing.
          while (t + 1 < segs_per_row && t_end <= q + 1) t_end = seg_end(++t + 1);
        }
        p1 = p2;
        p2 = p3;
        row1 = row2;
        ++q;
      };
      while (true) {
        step(ra, ok_a, w_a, rb, ok_b, w_b);
        if (q >= q_end) break;
        step(rb, ok_b, w_b, ra, ok_a, w_a);
        if (q >= q_end) break;
      }
    }
    if (active) {
      divide_by_normalizer(acc, nk);
      v16_store(o.out + static_cast<int64_t>(k) * o.ots + static_cast<int64_t>(c >> 6) * o.ohs + (c & 63), acc);
    }
  }
}

// G outputs that share one segment structure, one output per wave: wave w
// pools output w % G of compact row w / G.  A wave holds one output's sums and
// row buffers (89-105 VGPRs: five or four waves per SIMD to cover each row's
// index round trips, where three outputs in one wave took 238, two per SIMD);
// the index loads repeat per output through the scalar cache.  The outputs'
// LayerNorm parameters are staged in LDS once per work-group.
template <typename TI, typename TO, int G, bool kFold>
__global__ __launch_bounds__(256) void compact16_kernel(
    const TI* __restrict__ x, int64_t xts, int64_t xhs, int64_t x_rows,
    const int64_t* __restrict__ base_rows, const int32_t* __restrict__ offsets, int segs_per_row,
    const uint32_t* __restrict__ items, int item_shift, const int64_t* __restrict__ item_rows,
    const float* __restrict__ weights, int n_weights, const float* __restrict__ norm, int rows,
    int dim, float ln_eps, CompactOuts<TO, G> o) {
  __shared__ float ln_lds[G][2][64];
  for (int e = threadIdx.x; e < G * 128; e += blockDim.x) {
    const int g = e >> 7, h = (e >> 6) & 1, j = e & 63;
    const float* src = h ? o.ln_b[g] : o.ln_w[g];
    ln_lds[g][h][j] = src ? src[j] : 0.0f;
  }
  __syncthreads();
  // Persistent waves: wave w pools units w, w + W, ... (unit u = output u % G of
  // compact row u / G), so the LayerNorm parameters are staged once per resident
  // work-group.  The unit is wave-uniform: its index loads (offsets, items, row ids)
  // go through the scalar cache, apart from the member rows' vector loads.
  const int units = rows * G;
  const int stride = gridDim.x * 4;
  for (int w = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6)); w < units;
       w += stride) {
    const int k = w / G;
    const int gs = w - k * G;
    // Output gs's fields, selected with compile-time indices (indexing the
    // kernel-argument arrays at run time would copy them to scratch).
    CompactOut<TO> o1{o.x_off[0], o.ln_w[0], o.ln_b[0], o.out[0], o.ots[0], o.ohs[0]};
#pragma unroll
    for (int g = 1; g < G; ++g)
      if (gs == g) o1 = CompactOut<TO>{o.x_off[g], o.ln_w[g], o.ln_b[g], o.out[g], o.ots[g], o.ohs[g]};
    compact16_row<TI, TO, kFold>(x, xts, xhs, x_rows, base_rows, offsets, segs_per_row, items, item_shift,
                                 item_rows, weights, n_weights, norm, k, dim, ln_eps, o1, ln_lds[gs][0],
                                 ln_lds[gs][1]);
  }
}

// Launch of compact16_kernel for `rows` compact rows of G outputs.
template <typename TI, typename TO, int G>
int launch_compact16(const TI* x, int64_t xts, int64_t xhs, int64_t x_rows, const int64_t* base_rows,
                     const int32_t* offsets, int sp, const uint32_t* items, int item_shift,
                     const int64_t* item_rows, const float* weights, int nw, const float* normalizer,
                     int rows, int dim, float ln_eps, const CompactOuts<TO, G>& o, hipStream_t s,
                     const char* what) {
  // Resident work-groups only (the kernel loops over its units).
  int per_cu = 0, dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    cus = 256;
  const bool fold = sp == 1 && !base_rows;
  if ((fold ? hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, compact16_kernel<TI, TO, G, true>, 256, 0)
            : hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, compact16_kernel<TI, TO, G, false>, 256, 0)) !=
          hipSuccess ||
      per_cu <= 0)
    per_cu = 1;
  const int64_t need = (static_cast<int64_t>(rows) * G + 3) / 4;
  const dim3 grid(static_cast<unsigned>(std::min<int64_t>(need, static_cast<int64_t>(cus) * per_cu)));
  if (sp == 1 && !base_rows)
    hipLaunchKernelGGL((compact16_kernel<TI, TO, G, true>), grid, dim3(256), 0, s, x, xts, xhs, x_rows,
                       base_rows, offsets, sp, items, item_shift, item_rows, weights, nw, normalizer, rows,
                       dim, ln_eps, o);
  else
    hipLaunchKernelGGL((compact16_kernel<TI, TO, G, false>), grid, dim3(256), 0, s, x, xts, xhs, x_rows,
                       base_rows, offsets, sp, items, item_shift, item_rows, weights, nw, normalizer, rows,
                       dim, ln_eps, o);
  return check_launch(what);
}

// ---------------------------------------------------- restore map ----
// Dense [N,4] (index, weight) rows for the top-4 projection:
//   kept token keep[k]              -> (k,k,k,k), (1,0,0,0)
//   source token source[i]          -> parent[i,:], w[i,:]
//   token with inverse[t] = k (TokenPlan)     -> (k,k,k,k), (1,0,0,0)
__global__ __launch_bounds__(256) void restore_map_kernel(
    const int64_t* __restrict__ keep, int n_keep, const int64_t* __restrict__ source,
    const int64_t* __restrict__ parent, const float* __restrict__ w, int n_source,
    const int64_t* __restrict__ inverse, int total, int32_t* __restrict__ index,
    float* __restrict__ weight) {
  const int e = blockIdx.x * 256 + threadIdx.x;
  if (inverse) {
    if (e >= total) return;
    const int64_t k = inverse[e];
    const int32_t kk = static_cast<int32_t>(k);
    index[4 * e + 0] = kk;
    index[4 * e + 1] = kk;
    index[4 * e + 2] = kk;
    index[4 * e + 3] = kk;
    weight[4 * e + 0] = k >= 0 ? 1.0f : 0.0f;
    weight[4 * e + 1] = 0.0f;
    weight[4 * e + 2] = 0.0f;
    weight[4 * e + 3] = 0.0f;
    return;
  }
  if (e < n_keep) {
    const int64_t t = keep[e];
    if (t < 0 || t >= total) return;
    for (int c = 0; c < 4; ++c) {
      index[4 * t + c] = e;
      weight[4 * t + c] = c == 0 ? 1.0f : 0.0f;
    }
  } else if (e < n_keep + n_source) {
    const int i = e - n_keep;
    const int64_t t = source[i];
    if (t < 0 || t >= total) return;
    for (int c = 0; c < 4; ++c) {
      index[4 * t + c] = static_cast<int32_t>(parent[4 * i + c]);
      weight[4 * t + c] = w[4 * i + c];
    }
  }
}

}  // namespace
}  // namespace vgo

using namespace vgo;

extern "C" int vgo_csr_workspace(int64_t n_items, int64_t n_buckets, size_t* bytes) {
  VGO_REQUIRE(n_items >= 0 && n_buckets >= 1, "csr_build: bad size");
  VGO_REQUIRE(n_items < (1LL << 31) && n_buckets < (1LL << 31) - 1, "csr_build: size too large");
  const int64_t nblocks = (n_items + kBlockItems - 1) / kBlockItems;
  size_t b = 0;
  b += 3 * align_up(static_cast<size_t>(n_items) * 4);  // keys x2, vals ping
  b += align_up(static_cast<size_t>(256) * (nblocks > 0 ? nblocks : 1) * 4);
  *bytes = b;
  return VGO_OK;
}

extern "C" int vgo_csr_build(const uint32_t* keys, int64_t n_items, int64_t n_buckets,
                             void* workspace, size_t workspace_bytes, uint32_t* order,
                             int32_t* offsets, void* stream) {
  size_t need = 0;
  int st = vgo_csr_workspace(n_items, n_buckets, &need);
  if (st != VGO_OK) return st;
  VGO_REQUIRE(offsets, "csr_build: null offsets");
  hipStream_t s = as_stream(stream);
  const int n = static_cast<int>(n_items);
  const int nb = static_cast<int>(n_buckets);
  if (n == 0) {
    hipLaunchKernelGGL(fill_i32_kernel, dim3((nb + 1 + 255) / 256), dim3(256), 0, s, offsets, nb + 1, 0);
    return check_launch("csr_build");
  }
  VGO_REQUIRE(keys && order && workspace, "csr_build: null pointer");
  VGO_REQUIRE(workspace_bytes >= need && aligned(workspace, 256), "csr_build: workspace too small or misaligned");
  char* ws = static_cast<char*>(workspace);
  uint32_t* ka = reinterpret_cast<uint32_t*>(ws);
  uint32_t* kb = reinterpret_cast<uint32_t*>(ws + align_up(size_t(n) * 4));
  uint32_t* va = reinterpret_cast<uint32_t*>(ws + 2 * align_up(size_t(n) * 4));
  uint32_t* hist = reinterpret_cast<uint32_t*>(ws + 3 * align_up(size_t(n) * 4));
  const int nblocks = (n + kBlockItems - 1) / kBlockItems;
  const int passes = (key_bits(n_buckets) + 7) / 8;
  // Value buffers ping-pong between va and `order` so the last pass lands in `order`.
  uint32_t* vbuf[2] = {va, order};
  uint32_t* kbuf[2] = {ka, kb};
  int cur = passes % 2 == 0 ? 1 : 0;  // pass p writes buffer (cur + p + 1) % 2
  // Pass 0 reads the caller's keys (clamped as it reads them) and the item
  // indices; after `passes` flips the values end in vbuf[(cur + passes) % 2] == order.
  for (int p = 0; p < passes; ++p) {
    const int shift = 8 * p;
    const uint32_t* kin = p == 0 ? keys : kbuf[cur];
    const uint32_t* vin = p == 0 ? nullptr : vbuf[cur];
    const uint32_t limit = p == 0 ? static_cast<uint32_t>(nb) : 0u;
    hipLaunchKernelGGL(radix_hist_kernel, dim3(nblocks), dim3(kSortThreads), 0, s, kin, n, shift, hist,
                       nblocks, limit);
    hipLaunchKernelGGL(exclusive_scan_kernel, dim3(1), dim3(1024), 0, s, hist, 256 * nblocks);
    hipLaunchKernelGGL(radix_scatter_kernel, dim3(nblocks), dim3(kSortThreads), 0, s, kin, vin,
                       kbuf[1 - cur], vbuf[1 - cur], n, shift, hist, nblocks, limit);
    cur = 1 - cur;
  }
  hipLaunchKernelGGL(bucket_offsets_kernel, dim3((n + 255) / 256), dim3(256), 0, s, kbuf[cur], n,
                     nb, offsets);
  return check_launch("csr_build");
}

extern "C" int vgo_segment_mass(const int32_t* offsets, int64_t segs_per_row, const uint32_t* items,
                                const float* weights, int64_t n_weights, int64_t rows, float start,
                                float* mass, float* log_mass, void* stream) {
  VGO_REQUIRE(rows >= 0 && segs_per_row >= 1, "segment_mass: bad size");
  if (rows == 0) return VGO_OK;
  // items may be NULL when every segment is empty (a plan with no merged sources).
  VGO_REQUIRE(offsets && mass, "segment_mass: null pointer");
  hipLaunchKernelGGL(segment_mass_kernel, dim3(static_cast<unsigned>((rows + 255) / 256)), dim3(256), 0,
                     as_stream(stream), offsets, static_cast<int>(segs_per_row), items, weights,
                     static_cast<int>(n_weights), static_cast<int>(rows), start, mass, log_mass);
  return check_launch("segment_mass");
}

extern "C" int vgo_compact(const void* x, int64_t x_token_stride, int64_t x_head_stride, int64_t x_rows,
                           const int64_t* base_rows, const int32_t* offsets, int64_t segs_per_row,
                           const uint32_t* items, int item_shift, const int64_t* item_rows,
                           const float* weights, int64_t n_weights, const float* normalizer,
                           int64_t rows, int64_t dim, const float* ln_weight, const float* ln_bias,
                           float ln_eps, void* out, int64_t out_token_stride, int64_t out_head_stride,
                           int in_dtype, int out_dtype, void* stream) {
  VGO_REQUIRE(rows >= 0 && dim >= 0 && segs_per_row >= 1, "compact: bad size");
  if (rows == 0 || dim == 0) return VGO_OK;
  VGO_REQUIRE(x && offsets && out, "compact: null pointer");
  VGO_REQUIRE(item_shift >= 0 && item_shift < 8, "compact: bad item shift");
  VGO_REQUIRE(rows < (1LL << 31) && dim < (1 << 20), "compact: size too large");
  VGO_REQUIRE((ln_weight == nullptr) == (ln_bias == nullptr), "compact: LayerNorm weight and bias go together");
  hipStream_t s = as_stream(stream);
  const dim3 grid(static_cast<unsigned>((rows + 3) / 4));
  const int r = static_cast<int>(rows), d = static_cast<int>(dim), sp = static_cast<int>(segs_per_row);
  const int nw = static_cast<int>(n_weights);
  const int64_t in_vec = in_dtype == VGO_F32 ? 4 : 8;
  const int64_t out_vec = out_dtype == VGO_F32 ? 4 : 8;
  const bool vec = dim % 64 == 0 && x_token_stride % in_vec == 0 && x_head_stride % in_vec == 0 &&
                   out_token_stride % out_vec == 0 && out_head_stride % out_vec == 0 &&
                   aligned(x, 16) && aligned(out, 16);
  if (vec) {
#define VGO_C16(TI, TO)                                                                            \
  {                                                                                                \
    const CompactOuts<TO, 1> o{{0}, {ln_weight}, {ln_bias}, {static_cast<TO*>(out)},               \
                               {out_token_stride}, {out_head_stride}};                            \
    return launch_compact16<TI, TO, 1>(static_cast<const TI*>(x), x_token_stride, x_head_stride,   \
                                       x_rows, base_rows, offsets, sp, items, item_shift,          \
                                       item_rows, weights, nw, normalizer, r, d, ln_eps, o, s,     \
                                       "compact");                                                 \
  }
    if (in_dtype == VGO_F32 && out_dtype == VGO_F32) { VGO_C16(float, float); }
    if (in_dtype == VGO_BF16 && out_dtype == VGO_BF16) { VGO_C16(bf16_t, bf16_t); }
    if (in_dtype == VGO_F16 && out_dtype == VGO_F16) { VGO_C16(f16_t, f16_t); }
    if (in_dtype == VGO_BF16 && out_dtype == VGO_F32) { VGO_C16(bf16_t, float); }
    if (in_dtype == VGO_F32 && out_dtype == VGO_BF16) { VGO_C16(float, bf16_t); }
#undef VGO_C16
    return fail(VGO_EINVAL, "compact: unsupported dtype pair");
  }
  VGO_REQUIRE(in_dtype == out_dtype && ln_weight == nullptr,
              "compact: LayerNorm and dtype conversion need 64-aligned channels and 16-byte rows");
  switch (in_dtype) {
    case VGO_F32:
      hipLaunchKernelGGL((compact_kernel<float, 16>), grid, dim3(256), 0, s, static_cast<const float*>(x),
                         x_token_stride, x_head_stride, x_rows, base_rows, offsets, sp, items, item_shift,
                         item_rows, weights, nw, normalizer, r, d, static_cast<float*>(out),
                         out_token_stride, out_head_stride);
      break;
    case VGO_BF16:
      hipLaunchKernelGGL((compact_kernel<bf16_t, 16>), grid, dim3(256), 0, s,
                         static_cast<const bf16_t*>(x), x_token_stride, x_head_stride, x_rows, base_rows,
                         offsets, sp, items, item_shift, item_rows, weights, nw, normalizer, r, d,
                         static_cast<bf16_t*>(out), out_token_stride, out_head_stride);
      break;
    case VGO_F16:
      hipLaunchKernelGGL((compact_kernel<f16_t, 16>), grid, dim3(256), 0, s, static_cast<const f16_t*>(x),
                         x_token_stride, x_head_stride, x_rows, base_rows, offsets, sp, items, item_shift,
                         item_rows, weights, nw, normalizer, r, d, static_cast<f16_t*>(out),
                         out_token_stride, out_head_stride);
      break;
    default:
      return fail(VGO_EINVAL, "compact: unknown dtype");
  }
  return check_launch("compact");
}

extern "C" int vgo_restore_map(const int64_t* keep, int64_t n_keep, const int64_t* source,
                               const int64_t* parent, const float* weight, int64_t n_source,
                               const int64_t* inverse, int64_t total, int32_t* index_out,
                               float* weight_out, void* stream) {
  VGO_REQUIRE(total >= 0 && n_keep >= 0 && n_source >= 0, "restore_map: bad size");
  VGO_REQUIRE(total < (1LL << 31), "restore_map: size too large");
  if (total == 0) return VGO_OK;
  VGO_REQUIRE(index_out && weight_out, "restore_map: null pointer");
  hipStream_t s = as_stream(stream);
  const int64_t work = inverse ? total : n_keep + n_source;
  if (!inverse) VGO_REQUIRE(keep && (n_source == 0 || (source && parent && weight)), "restore_map: null pointer");
  if (work == 0) return VGO_OK;
  hipLaunchKernelGGL(restore_map_kernel, dim3(static_cast<unsigned>((work + 255) / 256)), dim3(256), 0, s,
                     keep, static_cast<int>(n_keep), source, parent, weight, static_cast<int>(n_source),
                     inverse, static_cast<int>(total), index_out, weight_out);
  return check_launch("restore_map");
}

namespace vgo {
namespace {

template <typename TI, typename TO, int G>
int launch_compact_multi(const void* x, int64_t xts, int64_t xhs, int64_t x_rows, const int64_t* base_rows,
                         const int32_t* offsets, int sp, const uint32_t* items, int item_shift,
                         const int64_t* item_rows, const float* weights, int nw, const float* normalizer,
                         int rows, int dim, const int64_t* x_offsets, const float* const* ln_weights,
                         const float* const* ln_biases, float ln_eps, void* const* outs,
                         const int64_t* ots, const int64_t* ohs, hipStream_t s) {
  CompactOuts<TO, G> o;
  for (int g = 0; g < G; ++g) {
    o.x_off[g] = x_offsets[g];
    o.ln_w[g] = ln_weights ? ln_weights[g] : nullptr;
    o.ln_b[g] = ln_biases ? ln_biases[g] : nullptr;
    o.out[g] = static_cast<TO*>(outs[g]);
    o.ots[g] = ots[g];
    o.ohs[g] = ohs[g];
  }
  return launch_compact16<TI, TO, G>(static_cast<const TI*>(x), xts, xhs, x_rows, base_rows, offsets, sp,
                                     items, item_shift, item_rows, weights, nw, normalizer, rows, dim, ln_eps,
                                     o, s, "compact_multi");
}

template <typename T>
int dispatch_compact_multi(int n, const void* x, int64_t xts, int64_t xhs, int64_t x_rows,
                           const int64_t* base_rows, const int32_t* offsets, int sp, const uint32_t* items,
                           int item_shift, const int64_t* item_rows, const float* weights, int nw,
                           const float* normalizer, int rows, int dim, const int64_t* x_offsets,
                           const float* const* lw, const float* const* lb, float eps, void* const* outs,
                           const int64_t* ots, const int64_t* ohs, hipStream_t s) {
#define VGO_CM(G)                                                                                      \
  return launch_compact_multi<T, T, G>(x, xts, xhs, x_rows, base_rows, offsets, sp, items, item_shift,  \
                                       item_rows, weights, nw, normalizer, rows, dim, x_offsets, lw, lb, \
                                       eps, outs, ots, ohs, s)
  switch (n) {
    case 1: VGO_CM(1);
    case 2: VGO_CM(2);
    default: VGO_CM(3);
  }
#undef VGO_CM
}

}  // namespace
}  // namespace vgo

extern "C" int vgo_compact_multi(const void* x, int64_t x_token_stride, int64_t x_head_stride, int64_t x_rows,
                                 const int64_t* base_rows, const int32_t* offsets, int64_t segs_per_row,
                                 const uint32_t* items, int item_shift, const int64_t* item_rows,
                                 const float* weights, int64_t n_weights, const float* normalizer,
                                 int64_t rows, int64_t dim, int n_outputs, const int64_t* x_offsets,
                                 const float* const* ln_weights, const float* const* ln_biases,
                                 float ln_eps, void* const* outs, const int64_t* out_token_strides,
                                 const int64_t* out_head_strides, int dtype, void* stream) {
  VGO_REQUIRE(rows >= 0 && dim >= 0 && segs_per_row >= 1, "compact_multi: bad size");
  VGO_REQUIRE(n_outputs >= 1 && n_outputs <= 3, "compact_multi: 1 to 3 outputs");
  if (rows == 0 || dim == 0) return VGO_OK;
  VGO_REQUIRE(x && offsets && x_offsets && outs && out_token_strides && out_head_strides,
              "compact_multi: null pointer");
  VGO_REQUIRE(item_shift >= 0 && item_shift < 8, "compact_multi: bad item shift");
  VGO_REQUIRE(rows < (1LL << 31) && dim < (1 << 20), "compact_multi: size too large");
  const int64_t vec = dtype == VGO_F32 ? 4 : 8;
  bool ok = dim % 64 == 0 && x_token_stride % vec == 0 && x_head_stride % vec == 0 && aligned(x, 16);
  for (int g = 0; g < n_outputs; ++g) {
    VGO_REQUIRE(outs[g], "compact_multi: null output");
    VGO_REQUIRE((ln_weights == nullptr || ln_weights[g] == nullptr) ==
                    (ln_biases == nullptr || ln_biases[g] == nullptr),
                "compact_multi: LayerNorm weight and bias go together");
    ok = ok && x_offsets[g] >= 0 && x_offsets[g] % vec == 0 && out_token_strides[g] % vec == 0 &&
         out_head_strides[g] % vec == 0 && aligned(outs[g], 16);
  }
  VGO_REQUIRE(ok, "compact_multi: needs 64-aligned channels, 16-byte rows and vector-aligned offsets");
  hipStream_t s = as_stream(stream);
  const int r = static_cast<int>(rows), d = static_cast<int>(dim), sp = static_cast<int>(segs_per_row);
  const int nw = static_cast<int>(n_weights);
  switch (dtype) {
    case VGO_BF16:
      return dispatch_compact_multi<bf16_t>(n_outputs, x, x_token_stride, x_head_stride, x_rows, base_rows, offsets,
                                            sp, items, item_shift, item_rows, weights, nw, normalizer, r, d,
                                            x_offsets, ln_weights, ln_biases, ln_eps, outs, out_token_strides,
                                            out_head_strides, s);
    case VGO_F16:
      return dispatch_compact_multi<f16_t>(n_outputs, x, x_token_stride, x_head_stride, x_rows, base_rows, offsets,
                                           sp, items, item_shift, item_rows, weights, nw, normalizer, r, d,
                                           x_offsets, ln_weights, ln_biases, ln_eps, outs, out_token_strides,
                                           out_head_strides, s);
    case VGO_F32:
      return dispatch_compact_multi<float>(n_outputs, x, x_token_stride, x_head_stride, x_rows, base_rows, offsets,
                                           sp, items, item_shift, item_rows, weights, nw, normalizer, r, d,
                                           x_offsets, ln_weights, ln_biases, ln_eps, outs, out_token_strides,
                                           out_head_strides, s);
    default:
      return fail(VGO_EINVAL, "compact_multi: unsupported dtype");
  }
}
