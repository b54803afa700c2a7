// Rank-and-select that turns FastVGGT match scores into a merge plan.
//
// Work of vggt_omega/models/token_merging.py:1112-1121:
//   ranked  = best.argsort(descending=True, stable=True)
//   removed = sources[ranked[:r]];  target = destinations[targets[ranked[:r]]]
//   keep    = ascending non-removed ids;  inverse: kept -> compact id,
//             removed -> compact id of its target.
// Only the *set* of the r best sources matters (keep is re-sorted, inverse is
// per token), so instead of a full sort one work-group per batch element runs
// a four-pass radix select on the order-preserving 32-bit image of `best`,
// then breaks ties at the threshold by source position (the stable sort's
// rule) with a block-wide prefix count, and finally builds keep/inverse with
// one block scan over the tokens.  Integer work, bit-exact, deterministic.
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

__global__ __launch_bounds__(kThreads) void fastvggt_assemble_kernel(
    const float* __restrict__ best, const int32_t* __restrict__ target,
    const int64_t* __restrict__ source_ids, const int64_t* __restrict__ dest_ids, int ns, int nd,
    int total, int removed, int64_t* __restrict__ keep, int64_t* __restrict__ inverse,
    uint8_t* __restrict__ removed_flag) {
  __shared__ int hist[256];
  __shared__ int scan_lds[kWavesS];
  __shared__ uint32_t sel_prefix;
  __shared__ int sel_above;

  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  const float* bb = best + static_cast<int64_t>(b) * ns;
  const int32_t* tb = target + static_cast<int64_t>(b) * ns;
  int64_t* inv = inverse + static_cast<int64_t>(b) * total;
  int64_t* kp = keep + static_cast<int64_t>(b) * (total - removed);
  uint8_t* flag = removed_flag + static_cast<int64_t>(b) * ns;

  const int es = (ns + kThreads - 1) / kThreads;  // sources per thread (contiguous run)
  const int s_begin = min(ns, tid * es), s_end = min(ns, s_begin + es);
  const int et = (total + kThreads - 1) / kThreads;  // tokens per thread
  const int t_begin = min(total, tid * et), t_end = min(total, t_begin + et);

  // ---- radix select: find the r-th largest key T and how many keys exceed it.
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
    for (int i = s_begin; i < s_end; ++i) {
      const uint32_t o = ord32(bb[i]);
      if ((o & pmask) == prefix) atomicAdd(&hist[(o >> shift) & 0xFF], 1);
    }
    __syncthreads();
    if (tid == 0) {
      const int need = removed - sel_above;  // >= 1 while we are still inside the run
      int above = 0;
      int digit = 255;
      for (; digit > 0; --digit) {
        if (above + hist[digit] >= need) break;
        above += hist[digit];
      }
      sel_above += above;
      sel_prefix = prefix | (static_cast<uint32_t>(digit) << shift);
    }
    __syncthreads();
  }
  const uint32_t thresh = sel_prefix;
  const int need_ties = removed - sel_above;  // ties at the threshold to remove, lowest position first

  // ---- tie ranks in source order, then mark removed sources.
  int my_ties = 0;
  for (int i = s_begin; i < s_end; ++i) my_ties += ord32(bb[i]) == thresh;
  int ties_total = 0;
  int tie_rank = block_exclusive_scan(my_ties, scan_lds, &ties_total);
  for (int t = t_begin; t < t_end; ++t) inv[t] = 0;  // 0 = kept
  __syncthreads();
  for (int i = s_begin; i < s_end; ++i) {
    const uint32_t o = ord32(bb[i]);
    bool rm = o > thresh;
    if (o == thresh) rm = (tie_rank++) < need_ties;
    flag[i] = rm ? 1 : 0;
    const int64_t sid = source_ids[i];
    if (rm && sid >= 0 && sid < total) inv[sid] = -1;
  }
  __syncthreads();

  // ---- compact ids of kept tokens, keep list.
  int my_kept = 0;
  for (int t = t_begin; t < t_end; ++t) my_kept += inv[t] == 0;
  int kept_total = 0;
  int base = block_exclusive_scan(my_kept, scan_lds, &kept_total);
  const int n_keep = total - removed;
  for (int t = t_begin; t < t_end; ++t) {
    if (inv[t] == 0) {
      inv[t] = base;
      if (base < n_keep) kp[base] = t;  // always true for a valid (disjoint) source list
      ++base;
    }
  }
  __syncthreads();

  // ---- removed sources point at their target's compact id.
  for (int i = s_begin; i < s_end; ++i) {
    const int64_t sid = source_ids[i];
    if (flag[i] && sid >= 0 && sid < total) {
      const int32_t d = tb[i];
      const int64_t dst = (d >= 0 && d < nd) ? dest_ids[d] : -1;
      inv[sid] = (dst >= 0 && dst < total) ? inv[dst] : -1;
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
