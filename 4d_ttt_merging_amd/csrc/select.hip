// Rank-and-select that turns FastVGGT match scores into a merge plan.
//
// Work of vggt_omega/models/token_merging.py:1112-1121:
//   ranked  = best.argsort(descending=True, stable=True)
//   removed = sources[ranked[:r]];  target = destinations[targets[ranked[:r]]]
//   keep    = ascending non-removed ids;  inverse: kept -> compact id,
//             removed -> compact id of its target.
// Only the *set* of the r best sources matters (keep is re-sorted, inverse is
// per token), so instead of a full sort one work-group per batch element runs
// a four-pass radix select on the order-preserving 32-bit image of `best`
// (coalesced histogram passes, parallel digit search), then breaks ties at the
// threshold by source position (the stable sort's rule) and builds keep /
// inverse, both with ballot-based ordered ranks (one block scan per 64 chunks
// of 1024 elements).  Integer work, bit-exact, deterministic.
#include "vgo_common.h"

namespace vgo {
namespace {

constexpr int kThreads = 1024;
constexpr int kWavesS = kThreads / 64;

// Order-preserving map float -> uint32 (NaN above +inf, -0 folded onto +0),
// matching the comparison order of torch's descending stable sort.
__device__ __forceinline__ uint32_t ord32(float x) {
  if (x != x) return 0xFFFFFFFFu;
  uint32_t b = __float_as_uint(x);
  if (b == 0x80000000u) b = 0;
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// Exclusive prefix sum over the work-group (kThreads threads); returns the
// thread's exclusive prefix and writes the total to *total.
__device__ int block_exclusive_scan(int v, int* lds_waves, int* total) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  int x = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(x, off);
    if (lane >= off) x += y;
  }
  if (lane == 63) lds_waves[wave] = x;
  __syncthreads();
  if (wave == 0) {
    int w = lane < kWavesS ? lds_waves[lane] : 0;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int y = __shfl_up(w, off);
      if (lane >= off) w += y;
    }
    if (lane < kWavesS) lds_waves[lane] = w;  // inclusive scan of wave totals
  }
  __syncthreads();
  const int wave_base = wave > 0 ? lds_waves[wave - 1] : 0;
  const int t = lds_waves[kWavesS - 1];
  __syncthreads();
  *total = t;
  return wave_base + x - v;
}

// Ranks, in index order, of the elements whose flag is set: element i = c*kThreads
// + tid of chunk c.  Chunks are processed 64 at a time: per (chunk, wave) counts
// from ballots go to LDS, one block scan over those 1024 counts gives every
// (chunk, wave) its offset, and a lane adds the set flags of lower lanes.
// `flag(c)` is evaluated twice per chunk; `emit(c, rank)` is called for every
// set flag.  Returns the number of set flags.
template <typename Flag, typename Emit>
__device__ int ordered_ranks(int n_chunks, Flag flag, Emit emit, int* cnt_lds, int* scan_lds) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  int running = 0;
  for (int c0 = 0; c0 < n_chunks; c0 += 64) {
    const int nc = min(64, n_chunks - c0);
    for (int c = 0; c < 64; ++c) {
      const uint64_t m = c < nc ? __ballot(flag(c0 + c)) : 0ull;
      if (lane == 0) cnt_lds[c * kWavesS + wave] = __popcll(m);
    }
    __syncthreads();
    const int mine = cnt_lds[threadIdx.x];  // kThreads == 64 * kWavesS entries
    int sum = 0;
    const int pre = block_exclusive_scan(mine, scan_lds, &sum);
    cnt_lds[threadIdx.x] = pre;
    __syncthreads();
    const uint64_t below = (1ull << lane) - 1ull;
    for (int c = 0; c < nc; ++c) {
      const bool f = flag(c0 + c);
      const uint64_t m = __ballot(f);
      if (f) emit(c0 + c, running + cnt_lds[c * kWavesS + wave] + __popcll(m & below));
    }
    running += sum;
    __syncthreads();
  }
  return running;
}

// hist[digit] += 1 for every lane with `valid`.  Keys here cluster in a few
// digits (bf16-rounded scores), and same-address LDS atomics serialise, so a
// wave first adds whole groups of equal digits through a leader lane; after a
// few groups the remaining lanes fall back to one atomic each.
__device__ __forceinline__ void hist_add(int* hist, bool valid, uint32_t digit) {
  const int lane = threadIdx.x & 63;
  uint64_t active = __ballot(valid);
#pragma unroll
  for (int round = 0; round < 4; ++round) {
    if (active == 0) return;
    const int leader = __ffsll(static_cast<long long>(active)) - 1;
    const uint32_t d = __shfl(digit, leader);
    const uint64_t same = __ballot(valid && digit == d) & active;
    if (lane == leader) atomicAdd(&hist[d], __popcll(same));
    active &= ~same;
  }
  if ((active >> lane) & 1ull) atomicAdd(&hist[digit], 1);
}

// Keys per thread held in registers (sources beyond kThreads * kKeyRegs are
// re-read from global memory in batches of the same size).
constexpr int kKeyRegs = 32;

__global__ __launch_bounds__(kThreads) void fastvggt_assemble_kernel(
    const float* __restrict__ best, const int32_t* __restrict__ target,
    const int64_t* __restrict__ source_ids, const int64_t* __restrict__ dest_ids, int ns, int nd,
    int total, int removed, int64_t* __restrict__ keep, int64_t* __restrict__ inverse,
    uint8_t* __restrict__ removed_flag) {
  __shared__ int hist[256];
  __shared__ int scan_lds[kWavesS];
  __shared__ int cnt_lds[kThreads];
  __shared__ uint32_t sel_prefix;
  __shared__ int sel_above;

  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const float* bb = best + static_cast<int64_t>(b) * ns;
  const int32_t* tb = target + static_cast<int64_t>(b) * ns;
  int64_t* inv = inverse + static_cast<int64_t>(b) * total;
  int64_t* kp = keep + static_cast<int64_t>(b) * (total - removed);
  uint8_t* flag = removed_flag + static_cast<int64_t>(b) * ns;
  const int s_chunks = (ns + kThreads - 1) / kThreads;
  const int t_chunks = (total + kThreads - 1) / kThreads;

  // Keys of chunks [0, kKeyRegs) in registers; key(c) reads further chunks from global.
  uint32_t kreg[kKeyRegs];
#pragma unroll
  for (int c = 0; c < kKeyRegs; ++c) {
    const int i = c * kThreads + tid;
    kreg[c] = i < ns ? ord32(bb[i]) : 0u;
  }
  auto key = [&](int c) -> uint32_t {  // chunks >= kKeyRegs
    const int i = c * kThreads + tid;
    return i < ns ? ord32(bb[i]) : 0u;
  };

  // ---- radix select (8-bit digits, most significant first) of the r-th largest key.
  if (tid == 0) {
    sel_prefix = 0;
    sel_above = 0;
  }
  for (int pass = 0; pass < 4; ++pass) {
    const int shift = 24 - 8 * pass;
    if (tid < 256) hist[tid] = 0;
    __syncthreads();
    const uint32_t prefix = sel_prefix;
    const uint32_t pmask = pass == 0 ? 0u : (0xFFFFFFFFu << (32 - 8 * pass));
#pragma unroll
    for (int c = 0; c < kKeyRegs; ++c) {
      if (c < s_chunks)  // wave-uniform
        hist_add(hist, c * kThreads + tid < ns && (kreg[c] & pmask) == prefix, (kreg[c] >> shift) & 0xFF);
    }
    for (int c = kKeyRegs; c < s_chunks; ++c) {
      const int i = c * kThreads + tid;
      const uint32_t o = i < ns ? ord32(bb[i]) : 0u;
      hist_add(hist, i < ns && (o & pmask) == prefix, (o >> shift) & 0xFF);
    }
    __syncthreads();
    if (tid < 64) {
      // Lane l owns digits 4l..4l+3; c(d) = keys with digit >= d.  The digit
      // sought is the largest d with c(d) >= need.
      const int need = removed - sel_above;
      int h[4], local = 0;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        h[q] = hist[4 * lane + q];
        local += h[q];
      }
      int suffix = local;  // inclusive suffix sum over lanes >= lane
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const int y = __shfl_down(suffix, off);
        if (lane + off < 64) suffix += y;
      }
      int c = suffix - local;  // keys in digits above this lane's range
      int found = -1, above = 0;
#pragma unroll
      for (int q = 3; q >= 0; --q) {
        if (found < 0 && c + h[q] >= need) {
          found = 4 * lane + q;
          above = c;
        }
        c += h[q];
      }
      const uint64_t hit = __ballot(found >= 0);
      const int top = 63 - __clzll(hit);  // highest lane holding the digit
      if (lane == top) {
        sel_above += above;
        sel_prefix = prefix | (static_cast<uint32_t>(found) << shift);
      }
    }
    __syncthreads();
  }
  const uint32_t thresh = sel_prefix;
  const int need_ties = removed - sel_above;  // ties at the threshold to remove, lowest position first

  // ---- removed sources: keys above the threshold, and the first need_ties ties.
  // inv[t] holds 0 for kept tokens and -1 for removed ones until compaction.
  for (int t0 = 0; t0 < total; t0 += kThreads * 8) {
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int t = t0 + q * kThreads + tid;
      if (t < total) inv[t] = 0;
    }
  }
  __syncthreads();
#pragma unroll
  for (int c = 0; c < kKeyRegs; ++c) {
    const int i = c * kThreads + tid;
    if (i < ns) flag[i] = kreg[c] > thresh ? 1 : 0;
  }
#pragma unroll
  for (int c = 0; c < kKeyRegs; ++c) {
    const int i = c * kThreads + tid;
    const int64_t sid = (i < ns && kreg[c] > thresh) ? source_ids[i] : -1;
    if (sid >= 0 && sid < total) inv[sid] = -1;
  }
  for (int c = kKeyRegs; c < s_chunks; ++c) {
    const int i = c * kThreads + tid;
    if (i < ns) {
      const bool rm = key(c) > thresh;
      flag[i] = rm ? 1 : 0;
      if (rm) {
        const int64_t sid = source_ids[i];
        if (sid >= 0 && sid < total) inv[sid] = -1;
      }
    }
  }
  __syncthreads();
  uint32_t tie_bits = 0;  // chunks < kKeyRegs
#pragma unroll
  for (int c = 0; c < kKeyRegs; ++c)
    tie_bits |= (c * kThreads + tid < ns && kreg[c] == thresh ? 1u : 0u) << c;
  ordered_ranks(
      s_chunks,
      [&](int c) {
        if (c < kKeyRegs) return ((tie_bits >> c) & 1u) != 0u;
        return c * kThreads + tid < ns && key(c) == thresh;
      },
      [&](int c, int rank) {
        if (rank < need_ties) {
          const int i = c * kThreads + tid;
          flag[i] = 1;
          const int64_t sid = source_ids[i];
          if (sid >= 0 && sid < total) inv[sid] = -1;
        }
      },
      cnt_lds, scan_lds);

  // ---- compact ids of kept tokens (ascending), keep list.  Kept flags of the
  // first 64 token chunks are read once into a bit mask.
  uint64_t kept_bits = 0;
  {
    const int nc = min(t_chunks, 64);
    for (int c0 = 0; c0 < nc; c0 += 8) {
      int64_t v[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const int t = (c0 + q) * kThreads + tid;
        v[q] = (c0 + q < nc && t < total) ? inv[t] : -1;
      }
#pragma unroll
      for (int q = 0; q < 8; ++q) kept_bits |= (v[q] == 0 ? 1ull : 0ull) << (c0 + q);
    }
  }
  const int n_keep = total - removed;
  ordered_ranks(
      t_chunks,
      [&](int c) {
        if (c < 64) return ((kept_bits >> c) & 1ull) != 0ull;
        const int t = c * kThreads + tid;
        return t < total && inv[t] == 0;
      },
      [&](int c, int rank) {
        const int t = c * kThreads + tid;
        inv[t] = rank;
        if (rank < n_keep) kp[rank] = t;  // always true for a valid (disjoint) source list
      },
      cnt_lds, scan_lds);

  // ---- removed sources point at their target's compact id (eight independent
  // load chains per thread in flight).
  for (int c0 = 0; c0 < s_chunks; c0 += 8) {
    int64_t sid[8], dst[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int i = (c0 + q) * kThreads + tid;
      sid[q] = -1;
      dst[q] = -1;
      if (i < ns && flag[i]) {
        sid[q] = source_ids[i];
        const int32_t d = tb[i];
        dst[q] = (d >= 0 && d < nd) ? dest_ids[d] : -1;
      }
    }
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      if (sid[q] >= 0 && sid[q] < total) inv[sid[q]] = (dst[q] >= 0 && dst[q] < total) ? inv[dst[q]] : -1;
    }
  }
}


// Sparse-convex plan assembly (vggt_omega/models/sparse_convex.py:2435-2455):
//   selected = fit >= threshold; sources = candidates[selected] (ascending);
//   keep = ascending non-sources; o2c = compact id or -1;
//   parent_compact = o2c[support[selected]]; weights = alpha[selected].
// Buffers are sized for the worst case (n sources, total kept); stats[0] = M
// (sources), stats[1] = hard candidates, stats[2] = fallback candidates (copied
// from the device counter), stats[3] = sum of the selected fits.
__global__ __launch_bounds__(kThreads) void sparse_convex_assemble_kernel(
    const float* __restrict__ fit, const float* __restrict__ alpha,
    const int64_t* __restrict__ support, const int64_t* __restrict__ candidate,
    const float* __restrict__ top1, float easy_threshold, const int* __restrict__ failed_count,
    int n, int total, float threshold, int64_t* __restrict__ keep, int64_t* __restrict__ o2c,
    int64_t* __restrict__ source, int64_t* __restrict__ parent, float* __restrict__ weight,
    float* __restrict__ stats) {
  __shared__ int scan_lds[kWavesS];
  __shared__ float red[kWavesS];
  const int tid = threadIdx.x;
  const int es = (n + kThreads - 1) / kThreads;
  const int s_begin = min(n, tid * es), s_end = min(n, s_begin + es);
  const int et = (total + kThreads - 1) / kThreads;
  const int t_begin = min(total, tid * et), t_end = min(total, t_begin + et);

  int mine = 0, hard = 0;
  float fsum = 0.0f;
  for (int r = s_begin; r < s_end; ++r) {
    const bool sel = fit[r] >= threshold;
    mine += sel;
    if (sel) fsum += fit[r];
    hard += !(top1 && top1[r] >= easy_threshold);
  }
  int n_sel = 0;
  int pos = block_exclusive_scan(mine, scan_lds, &n_sel);
  int n_hard = 0;
  block_exclusive_scan(hard, scan_lds, &n_hard);
  for (int t = t_begin; t < t_end; ++t) o2c[t] = 0;
  __syncthreads();
  for (int r = s_begin; r < s_end; ++r) {
    if (fit[r] >= threshold) {
      const int64_t c = candidate[r];
      source[pos] = c;
#pragma unroll
      for (int k = 0; k < 4; ++k) weight[4 * pos + k] = alpha[4 * r + k];
      if (c >= 0 && c < total) o2c[c] = -1;
      ++pos;
    }
  }
  __syncthreads();
  int kept = 0;
  for (int t = t_begin; t < t_end; ++t) kept += o2c[t] == 0;
  int kept_total = 0;
  int base = block_exclusive_scan(kept, scan_lds, &kept_total);
  for (int t = t_begin; t < t_end; ++t) {
    if (o2c[t] == 0) {
      o2c[t] = base;
      keep[base] = t;
      ++base;
    }
  }
  __syncthreads();
  // Second walk over the selected rows in the same order to fill parent ids.
  int pos2 = 0;
  {
    int dummy = 0;
    pos2 = block_exclusive_scan(mine, scan_lds, &dummy);
  }
  for (int r = s_begin; r < s_end; ++r) {
    if (fit[r] >= threshold) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int64_t sup = support[4 * r + k];
        parent[4 * pos2 + k] = (sup >= 0 && sup < total) ? o2c[sup] : -1;
      }
      ++pos2;
    }
  }
  // Deterministic fit sum (fixed thread/wave order).
  float v = fsum;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
  if ((tid & 63) == 0) red[tid >> 6] = v;
  __syncthreads();
  if (tid == 0) {
    float s = 0.0f;
    for (int w = 0; w < kWavesS; ++w) s += red[w];
    stats[0] = static_cast<float>(n_sel);
    stats[1] = static_cast<float>(n_hard);
    stats[2] = failed_count ? static_cast<float>(*failed_count) : 0.0f;
    stats[3] = s;
  }
}

// ---------------------------------------------------------------------------
// Multi-work-group FastVGGT assembly (the workspace entry).  The same rule as
// fastvggt_assemble_kernel, spread over the chip as a chain of short kernels:
//   init     inverse = 0, workspace histograms cleared
//   hist p   (p = 0..3) histogram of digit p of the keys matching the prefix
//            chosen from digits 0..p-1 (each work-group re-derives that
//            prefix from the previous histogram; work-group 0 records it)
//   mark     threshold; keys above it are removed; ties counted per group
//   ties     the first need_ties ties in source order are removed
//   kcount   kept tokens per 512-token group
//   compact  compact ids (ascending) and the keep list
//   inverse  removed sources take their target's compact id
// Every step is integer work; the result is bit-identical to the one-group
// kernel.
constexpr int kAThreads = 256;
// Two elements per thread: 512-element groups spread each step over 4x the
// work-groups of 2048-element ones (47 / 65 at C4 instead of 12 / 17), which took
// the C4 plan build from 500 to 480 us.
constexpr int kAPer = 2;                     // elements per thread, contiguous
constexpr int kAChunk = kAThreads * kAPer;  // elements per work-group
constexpr int kASel = 4 * 256;               // sel[5][4] follows hist[4][256]
constexpr int kAGroupsAt = kASel + 20;       // per-group counts follow

__host__ __device__ inline int64_t fv_ws_ints(int s_groups, int t_groups) {
  return kAGroupsAt + s_groups + t_groups;
}

// Exclusive prefix over the 256 threads; *total receives the sum.
__device__ int scan256(int v, int* lds4, int* total) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  int x = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(x, off);
    if (lane >= off) x += y;
  }
  if (lane == 63) lds4[wave] = x;
  __syncthreads();
  int base = 0;
  for (int w = 0; w < wave; ++w) base += lds4[w];
  const int t = lds4[0] + lds4[1] + lds4[2] + lds4[3];
  __syncthreads();
  *total = t;
  return base + x - v;
}

// Wave 0: from a 256-bin digit histogram of the keys matching `prefix`, with
// `above` keys known to lie above them, the digit of the `removed`-th largest
// key; writes the extended prefix and count above it to *out_prefix/*out_above.
__device__ void fv_select(const int* hist, uint32_t prefix, int above, int removed, int shift,
                          uint32_t* out_prefix, int* out_above) {
  const int lane = threadIdx.x & 63;
  const int need = removed - above;
  int h[4], local = 0;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    h[q] = hist[4 * lane + q];
    local += h[q];
  }
  int suffix = local;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_down(suffix, off);
    if (lane + off < 64) suffix += y;
  }
  int c = suffix - local;
  int found = -1, more = 0;
#pragma unroll
  for (int q = 3; q >= 0; --q) {
    if (found < 0 && c + h[q] >= need) {
      found = 4 * lane + q;
      more = c;
    }
    c += h[q];
  }
  const uint64_t hit = __ballot(found >= 0);
  const int top = 63 - __clzll(hit);
  if (lane == top) {
    *out_above = above + more;
    *out_prefix = prefix | (static_cast<uint32_t>(found) << shift);
  }
}

__global__ __launch_bounds__(kAThreads) void fva_init_kernel(int total, int64_t* __restrict__ inverse,
                                                            int* __restrict__ ws, int64_t ws_ints) {
  const int b = blockIdx.y;
  int64_t* inv = inverse + static_cast<int64_t>(b) * total;
  const int t0 = blockIdx.x * kAChunk + threadIdx.x * kAPer;
#pragma unroll
  for (int k = 0; k < kAPer; ++k)
    if (t0 + k < total) inv[t0 + k] = 0;
  if (blockIdx.x == 0) {
    int* w = ws + b * ws_ints;
    for (int i = threadIdx.x; i < kAGroupsAt; i += kAThreads) w[i] = 0;
  }
}

__global__ __launch_bounds__(kAThreads) void fva_hist_kernel(const float* __restrict__ best, int ns,
                                                            int removed, int pass, int* __restrict__ ws,
                                                            int64_t ws_ints) {
  __shared__ int lh[256];
  __shared__ uint32_t s_prefix;
  __shared__ int s_above;
  const int b = blockIdx.y;
  int* w = ws + b * ws_ints;
  const int tid = threadIdx.x;
  if (pass == 0) {
    if (tid == 0) {
      s_prefix = 0;
      s_above = 0;
    }
  } else if (tid < 64) {
    fv_select(w + (pass - 1) * 256, static_cast<uint32_t>(w[kASel + 4 * (pass - 1)]),
              w[kASel + 4 * (pass - 1) + 1], removed, 32 - 8 * pass, &s_prefix, &s_above);
  }
  lh[tid] = 0;
  __syncthreads();
  if (blockIdx.x == 0 && tid == 0) {
    w[kASel + 4 * pass] = static_cast<int>(s_prefix);
    w[kASel + 4 * pass + 1] = s_above;
  }
  const uint32_t prefix = s_prefix;
  const uint32_t pmask = pass == 0 ? 0u : (0xFFFFFFFFu << (32 - 8 * pass));
  const int shift = 24 - 8 * pass;
  const float* bb = best + static_cast<int64_t>(b) * ns;
  const int i0 = blockIdx.x * kAChunk + tid * kAPer;
#pragma unroll
  for (int k = 0; k < kAPer; ++k) {
    const int i = i0 + k;
    const uint32_t key = i < ns ? ord32(bb[i]) : 0u;
    hist_add(lh, i < ns && (key & pmask) == prefix, (key >> shift) & 0xFF);
  }
  __syncthreads();
  if (lh[tid]) atomicAdd(&w[pass * 256 + tid], lh[tid]);
}

__global__ __launch_bounds__(kAThreads) void fva_mark_kernel(const float* __restrict__ best,
                                                            const int64_t* __restrict__ source_ids,
                                                            int ns, int total, int removed,
                                                            int64_t* __restrict__ inverse,
                                                            uint8_t* __restrict__ removed_flag,
                                                            int* __restrict__ ws, int64_t ws_ints) {
  __shared__ uint32_t s_prefix;
  __shared__ int s_above;
  __shared__ int lds4[4];
  const int b = blockIdx.y;
  int* w = ws + b * ws_ints;
  const int tid = threadIdx.x;
  if (tid < 64)
    fv_select(w + 3 * 256, static_cast<uint32_t>(w[kASel + 12]), w[kASel + 13], removed, 0, &s_prefix,
              &s_above);
  __syncthreads();
  const uint32_t thresh = s_prefix;
  if (blockIdx.x == 0 && tid == 0) {
    w[kASel + 16] = static_cast<int>(thresh);
    w[kASel + 17] = removed - s_above;  // ties to remove, lowest position first
  }
  const float* bb = best + static_cast<int64_t>(b) * ns;
  int64_t* inv = inverse + static_cast<int64_t>(b) * total;
  uint8_t* flag = removed_flag + static_cast<int64_t>(b) * ns;
  const int i0 = blockIdx.x * kAChunk + tid * kAPer;
  int ties = 0;
#pragma unroll
  for (int k = 0; k < kAPer; ++k) {
    const int i = i0 + k;
    if (i < ns) {
      const uint32_t key = ord32(bb[i]);
      const bool rm = key > thresh;
      flag[i] = rm ? 1 : 0;
      ties += key == thresh;
      if (rm) {
        const int64_t sid = source_ids[i];
        if (sid >= 0 && sid < total) inv[sid] = -1;
      }
    }
  }
  int n = 0;
  scan256(ties, lds4, &n);
  if (tid == 0) w[kAGroupsAt + blockIdx.x] = n;
}

__global__ __launch_bounds__(kAThreads) void fva_ties_kernel(const float* __restrict__ best,
                                                            const int64_t* __restrict__ source_ids,
                                                            int ns, int total,
                                                            int64_t* __restrict__ inverse,
                                                            uint8_t* __restrict__ removed_flag,
                                                            const int* __restrict__ ws, int64_t ws_ints) {
  __shared__ int lds4[4];
  const int b = blockIdx.y;
  const int* w = ws + b * ws_ints;
  const int tid = threadIdx.x;
  const uint32_t thresh = static_cast<uint32_t>(w[kASel + 16]);
  const int need = w[kASel + 17];
  int before = 0;  // ties in earlier groups
  for (int g = tid; g < static_cast<int>(blockIdx.x); g += kAThreads) before += w[kAGroupsAt + g];
  int sum = 0;
  scan256(before, lds4, &sum);
  before = sum;
  if (before >= need) return;  // uniform
  const float* bb = best + static_cast<int64_t>(b) * ns;
  int64_t* inv = inverse + static_cast<int64_t>(b) * total;
  uint8_t* flag = removed_flag + static_cast<int64_t>(b) * ns;
  const int i0 = blockIdx.x * kAChunk + tid * kAPer;
  uint32_t tie_bits = 0;
#pragma unroll
  for (int k = 0; k < kAPer; ++k) {
    const int i = i0 + k;
    tie_bits |= (i < ns && ord32(bb[i]) == thresh ? 1u : 0u) << k;
  }
  int n = 0;
  int rank = before + scan256(__popc(tie_bits), lds4, &n);
#pragma unroll
  for (int k = 0; k < kAPer; ++k) {
    if ((tie_bits >> k) & 1u) {
      if (rank < need) {
        const int i = i0 + k;
        flag[i] = 1;
        const int64_t sid = source_ids[i];
        if (sid >= 0 && sid < total) inv[sid] = -1;
      }
      ++rank;
    }
  }
}

__global__ __launch_bounds__(kAThreads) void fva_kcount_kernel(int total, const int64_t* __restrict__ inverse,
                                                              int* __restrict__ ws, int64_t ws_ints,
                                                              int s_groups) {
  __shared__ int lds4[4];
  const int b = blockIdx.y;
  const int64_t* inv = inverse + static_cast<int64_t>(b) * total;
  const int t0 = blockIdx.x * kAChunk + threadIdx.x * kAPer;
  int kept = 0;
#pragma unroll
  for (int k = 0; k < kAPer; ++k) kept += (t0 + k < total && inv[t0 + k] == 0) ? 1 : 0;
  int n = 0;
  scan256(kept, lds4, &n);
  if (threadIdx.x == 0) ws[b * ws_ints + kAGroupsAt + s_groups + blockIdx.x] = n;
}

__global__ __launch_bounds__(kAThreads) void fva_compact_kernel(int total, int removed,
                                                               int64_t* __restrict__ inverse,
                                                               int64_t* __restrict__ keep,
                                                               const int* __restrict__ ws, int64_t ws_ints,
                                                               int s_groups) {
  __shared__ int lds4[4];
  const int b = blockIdx.y;
  const int* w = ws + b * ws_ints + kAGroupsAt + s_groups;
  const int tid = threadIdx.x;
  int before = 0;
  for (int g = tid; g < static_cast<int>(blockIdx.x); g += kAThreads) before += w[g];
  int sum = 0;
  scan256(before, lds4, &sum);
  int64_t* inv = inverse + static_cast<int64_t>(b) * total;
  int64_t* kp = keep + static_cast<int64_t>(b) * (total - removed);
  const int t0 = blockIdx.x * kAChunk + tid * kAPer;
  uint32_t kept_bits = 0;
#pragma unroll
  for (int k = 0; k < kAPer; ++k) kept_bits |= (t0 + k < total && inv[t0 + k] == 0 ? 1u : 0u) << k;
  int n = 0;
  int rank = sum + scan256(__popc(kept_bits), lds4, &n);
  const int n_keep = total - removed;
#pragma unroll
  for (int k = 0; k < kAPer; ++k) {
    if ((kept_bits >> k) & 1u) {
      inv[t0 + k] = rank;
      if (rank < n_keep) kp[rank] = t0 + k;  // always true for a valid (disjoint) source list
      ++rank;
    }
  }
}

__global__ __launch_bounds__(kAThreads) void fva_inverse_kernel(const int32_t* __restrict__ target,
                                                               const int64_t* __restrict__ source_ids,
                                                               const int64_t* __restrict__ dest_ids,
                                                               int ns, int nd, int total,
                                                               int64_t* __restrict__ inverse,
                                                               const uint8_t* __restrict__ removed_flag) {
  const int b = blockIdx.y;
  const int32_t* tb = target + static_cast<int64_t>(b) * ns;
  int64_t* inv = inverse + static_cast<int64_t>(b) * total;
  const uint8_t* flag = removed_flag + static_cast<int64_t>(b) * ns;
  const int i0 = blockIdx.x * kAChunk + threadIdx.x * kAPer;
  int64_t sid[kAPer], dst[kAPer];
#pragma unroll
  for (int k = 0; k < kAPer; ++k) {
    const int i = i0 + k;
    sid[k] = -1;
    dst[k] = -1;
    if (i < ns && flag[i]) {
      sid[k] = source_ids[i];
      const int32_t d = tb[i];
      dst[k] = (d >= 0 && d < nd) ? dest_ids[d] : -1;
    }
  }
#pragma unroll
  for (int k = 0; k < kAPer; ++k)
    if (sid[k] >= 0 && sid[k] < total) inv[sid[k]] = (dst[k] >= 0 && dst[k] < total) ? inv[dst[k]] : -1;
}

}  // namespace
}  // namespace vgo

extern "C" int vgo_fastvggt_assemble(const float* best, const int32_t* target,
                                     const int64_t* source_ids, const int64_t* dest_ids,
                                     int64_t batch, int64_t n_sources, int64_t n_dest,
                                     int64_t total_tokens, int64_t removed, int64_t* keep,
                                     int64_t* inverse, uint8_t* removed_flag, void* stream) {
  using namespace vgo;
  VGO_REQUIRE(batch >= 0 && n_sources >= 0 && n_dest >= 0 && total_tokens >= 0,
              "fastvggt_assemble: negative size");
  VGO_REQUIRE(removed >= 1 && removed <= n_sources, "fastvggt_assemble: removed must lie in [1, sources]");
  VGO_REQUIRE(n_sources + n_dest <= total_tokens && total_tokens < (1LL << 30),
              "fastvggt_assemble: inconsistent token counts");
  if (batch == 0) return VGO_OK;
  VGO_REQUIRE(best && target && source_ids && dest_ids && keep && inverse && removed_flag,
              "fastvggt_assemble: null pointer");
  hipLaunchKernelGGL(fastvggt_assemble_kernel, dim3(static_cast<unsigned>(batch)), dim3(kThreads),
                     0, as_stream(stream), best, target, source_ids, dest_ids,
                     static_cast<int>(n_sources), static_cast<int>(n_dest),
                     static_cast<int>(total_tokens), static_cast<int>(removed), keep, inverse,
                     removed_flag);
  return check_launch("fastvggt_assemble");
}

extern "C" int vgo_sparse_convex_assemble(const float* fit, const float* alpha, const int64_t* support,
                                          const int64_t* candidate, const float* top1,
                                          float easy_threshold, const int* failed_count,
                                          int64_t n_candidates, int64_t total_tokens, float threshold,
                                          int64_t* keep, int64_t* original_to_compact, int64_t* source,
                                          int64_t* parent, float* weight, float* stats, void* stream) {
  using namespace vgo;
  VGO_REQUIRE(n_candidates >= 0 && total_tokens >= n_candidates && total_tokens < (1LL << 30),
              "sparse_convex_assemble: bad size");
  VGO_REQUIRE(keep && original_to_compact && stats, "sparse_convex_assemble: null pointer");
  VGO_REQUIRE(n_candidates == 0 || (fit && alpha && support && candidate && source && parent && weight),
              "sparse_convex_assemble: null pointer");
  hipLaunchKernelGGL(sparse_convex_assemble_kernel, dim3(1), dim3(kThreads), 0, as_stream(stream), fit,
                     alpha, support, candidate, top1, easy_threshold, failed_count,
                     static_cast<int>(n_candidates), static_cast<int>(total_tokens), threshold, keep,
                     original_to_compact, source, parent, weight, stats);
  return check_launch("sparse_convex_assemble");
}

extern "C" int vgo_fastvggt_assemble_workspace(int64_t batch, int64_t n_sources, int64_t total_tokens,
                                               size_t* bytes) {
  using namespace vgo;
  VGO_REQUIRE(bytes, "fastvggt_assemble: null size pointer");
  VGO_REQUIRE(batch >= 0 && n_sources >= 0 && total_tokens >= 0 && total_tokens < (1LL << 30),
              "fastvggt_assemble: bad size");
  const int s_groups = static_cast<int>((n_sources + kAChunk - 1) / kAChunk);
  const int t_groups = static_cast<int>((total_tokens + kAChunk - 1) / kAChunk);
  *bytes = static_cast<size_t>(batch) * fv_ws_ints(s_groups, t_groups) * sizeof(int);
  return VGO_OK;
}

extern "C" int vgo_fastvggt_assemble_ws(const float* best, const int32_t* target,
                                        const int64_t* source_ids, const int64_t* dest_ids,
                                        int64_t batch, int64_t n_sources, int64_t n_dest,
                                        int64_t total_tokens, int64_t removed, int64_t* keep,
                                        int64_t* inverse, uint8_t* removed_flag, void* workspace,
                                        size_t workspace_bytes, void* stream) {
  using namespace vgo;
  VGO_REQUIRE(batch >= 0 && n_sources >= 0 && n_dest >= 0 && total_tokens >= 0,
              "fastvggt_assemble: negative size");
  VGO_REQUIRE(removed >= 1 && removed <= n_sources, "fastvggt_assemble: removed must lie in [1, sources]");
  VGO_REQUIRE(n_sources + n_dest <= total_tokens && total_tokens < (1LL << 30),
              "fastvggt_assemble: inconsistent token counts");
  VGO_REQUIRE(batch <= 0xffff, "fastvggt_assemble: batch too large");
  if (batch == 0) return VGO_OK;
  VGO_REQUIRE(best && target && source_ids && dest_ids && keep && inverse && removed_flag,
              "fastvggt_assemble: null pointer");
  const int ns = static_cast<int>(n_sources), total = static_cast<int>(total_tokens);
  const int s_groups = (ns + kAChunk - 1) / kAChunk;
  const int t_groups = (total + kAChunk - 1) / kAChunk;
  const int64_t ws_ints = fv_ws_ints(s_groups, t_groups);
  if (workspace == nullptr ||
      workspace_bytes < static_cast<size_t>(batch) * ws_ints * sizeof(int))
    return fail(VGO_EWORKSPACE, "fastvggt_assemble: workspace too small");
  VGO_REQUIRE(aligned(workspace, 4), "fastvggt_assemble: workspace must be 4-byte aligned");
  int* ws = static_cast<int*>(workspace);
  hipStream_t s = as_stream(stream);
  const unsigned nb = static_cast<unsigned>(batch);
  hipLaunchKernelGGL(fva_init_kernel, dim3(t_groups, nb), dim3(kAThreads), 0, s, total, inverse, ws, ws_ints);
  for (int pass = 0; pass < 4; ++pass)
    hipLaunchKernelGGL(fva_hist_kernel, dim3(s_groups, nb), dim3(kAThreads), 0, s, best, ns,
                       static_cast<int>(removed), pass, ws, ws_ints);
  hipLaunchKernelGGL(fva_mark_kernel, dim3(s_groups, nb), dim3(kAThreads), 0, s, best, source_ids, ns, total,
                     static_cast<int>(removed), inverse, removed_flag, ws, ws_ints);
  hipLaunchKernelGGL(fva_ties_kernel, dim3(s_groups, nb), dim3(kAThreads), 0, s, best, source_ids, ns, total,
                     inverse, removed_flag, ws, ws_ints);
  hipLaunchKernelGGL(fva_kcount_kernel, dim3(t_groups, nb), dim3(kAThreads), 0, s, total, inverse, ws,
                     ws_ints, s_groups);
  hipLaunchKernelGGL(fva_compact_kernel, dim3(t_groups, nb), dim3(kAThreads), 0, s, total,
                     static_cast<int>(removed), inverse, keep, ws, ws_ints, s_groups);
  hipLaunchKernelGGL(fva_inverse_kernel, dim3(s_groups, nb), dim3(kAThreads), 0, s, target, source_ids,
                     dest_ids, ns, static_cast<int>(n_dest), total, inverse, removed_flag);
  return check_launch("fastvggt_assemble");
}
