// Exact four-support simplex fit of the sparse-convex planner.
//
// Work of `_convex_fit` (vggt_omega/models/sparse_convex.py:2260-2304) as used
// at :2415-2434: for a source x and four parent features s_0..s_3 (each
// L2-normalised twice with eps 1e-6, as :2384 and :2421-2422 do),
//   min_a ||S a - x||^2  over the probability simplex,
// solved by enumerating the 15 active sets.  Each set's KKT system is the 5x5
// matrix the reference builds (2 G on the active block plus a 2e-4 ridge,
// identity rows for pinned variables, the sum-to-one row) and is solved here
// by Gaussian elimination with partial pivoting, the algorithm of the LAPACK
// getrf/getrs pair behind `torch.linalg.solve_ex`.  Candidates with negative
// weights beyond 1e-5 or a singular system are infeasible; the feasible
// candidate with the lowest objective wins (first index on ties), its cosine
// fit is compared with the single best parent (rhs[0]) and the one-hot
// solution is taken when that is better.  Rows whose local top-1 score clears
// the early-accept threshold keep the one-hot fit without solving (:2415-2418).
//
// One wave per row: the five rows are normalised in registers, the 10 Gram
// and 4 right-hand-side dot products are wave reductions, lanes 0..14 each
// solve one active set, and a lane reduction picks the winner.  Results for
// valid inputs are within fp32 rounding of the reference; threshold decisions
// can differ only for fits within that rounding of the threshold.
#include "vgo_common.h"

namespace vgo {
namespace {

constexpr int kMaxPerLane = 16;  // dim <= 1024

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

template <typename T>
__device__ __forceinline__ void load_normalised(const T* row, int dim, float eps, float* v) {
  const int lane = threadIdx.x & 63;
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < kMaxPerLane; ++i) {
    const int e = i * 64 + lane;
    v[i] = e < dim ? to_f32(row[e]) : 0.0f;
    ss = fmaf(v[i], v[i], ss);
  }
  // F.normalize twice: x / max(||x||, eps), then the same on the result.
  const float d1 = fmaxf(sqrtf(wave_sum(ss)), eps);
  float ss2 = 0.0f;
#pragma unroll
  for (int i = 0; i < kMaxPerLane; ++i) {
    v[i] = v[i] / d1;
    ss2 = fmaf(v[i], v[i], ss2);
  }
  const float d2 = fmaxf(sqrtf(wave_sum(ss2)), eps);
#pragma unroll
  for (int i = 0; i < kMaxPerLane; ++i) v[i] = v[i] / d2;
}

// Active set `set` (0..14) in the reference's order (sparse_convex.py:22-28).
__device__ __forceinline__ bool is_active(int set, int var) {
  constexpr unsigned char kMask[15] = {0xF, 0x7, 0xB, 0xD, 0xE, 0x3, 0x5, 0x9,
                                       0x6, 0xA, 0xC, 0x1, 0x2, 0x4, 0x8};
  return (kMask[set] >> var) & 1;
}

// Solve the 5x5 KKT system of one active set; returns false when singular.
__device__ bool solve_set(int set, const float g[4][4], const float rhs[4], float ridge, float sol[5]) {
  float m[5][6];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const bool ai = is_active(set, i);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bool aj = is_active(set, j);
      float val = 2.0f * g[i][j] * ((ai && aj) ? 1.0f : 0.0f);
      if (i == j) val = ai ? val + 2.0f * ridge : 1.0f;
      m[i][j] = val;
    }
    m[i][4] = ai ? 1.0f : 0.0f;
    m[i][5] = ai ? 2.0f * rhs[i] : 0.0f;
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) m[4][j] = 1.0f;
  m[4][4] = 0.0f;
  m[4][5] = 1.0f;
  // Gaussian elimination with partial pivoting (first maximal |pivot|).
#pragma unroll
  for (int col = 0; col < 5; ++col) {
    int piv = col;
    float best = fabsf(m[col][col]);
#pragma unroll
    for (int r = col + 1; r < 5; ++r) {
      const float a = fabsf(m[r][col]);
      if (a > best) {
        best = a;
        piv = r;
      }
    }
    if (best == 0.0f) return false;
    if (piv != col) {
#pragma unroll
      for (int c = 0; c < 6; ++c) {
        const float t = m[col][c];
        m[col][c] = m[piv][c];
        m[piv][c] = t;
      }
    }
    const float inv = 1.0f / m[col][col];
#pragma unroll
    for (int r = col + 1; r < 5; ++r) {
      const float f = m[r][col] * inv;
#pragma unroll
      for (int c = col; c < 6; ++c) m[r][c] = m[r][c] - f * m[col][c];
    }
  }
#pragma unroll
  for (int r = 4; r >= 0; --r) {
    float acc = m[r][5];
#pragma unroll
    for (int c = r + 1; c < 5; ++c) acc = acc - m[r][c] * sol[c];
    sol[r] = acc / m[r][r];
  }
  return true;
}

template <typename T>
__global__ __launch_bounds__(256) void convex_fit_kernel(
    const T* __restrict__ tokens, int64_t token_stride, int64_t n_tokens,
    const int64_t* __restrict__ rows, int64_t* __restrict__ supports,
    const int64_t* __restrict__ list_supports, const float* __restrict__ top1,
    float easy_threshold, const int32_t* __restrict__ row_list,
    const int* __restrict__ n_list_dev, int n, int dim, float eps, float ridge,
    float* __restrict__ fit, float* __restrict__ alpha) {
  const int lane = threadIdx.x & 63;
  const int w = blockIdx.x * 4 + (threadIdx.x >> 6);
  int count = n;
  if (row_list && n_list_dev) count = min(count, *n_list_dev);
  if (w >= count) return;
  const int r = row_list ? row_list[w] : w;
  if (r < 0 || r >= n) return;

  if (top1 && top1[r] >= easy_threshold) {
    if (lane < 4) alpha[4 * r + lane] = lane == 0 ? 1.0f : 0.0f;
    if (lane == 0) fit[r] = top1[r];
    return;
  }
  int64_t ids[5];
  ids[0] = rows[r];
#pragma unroll
  for (int c = 0; c < 4; ++c)
    ids[c + 1] = list_supports ? list_supports[4 * w + c] : supports[4 * r + c];
  // New supports of a listed row replace its old ones (reference :2431).
  if (list_supports && lane < 4) supports[4 * r + lane] = ids[lane + 1];
  bool ok = true;
#pragma unroll
  for (int c = 0; c < 5; ++c) ok = ok && ids[c] >= 0 && ids[c] < n_tokens;
  if (!ok) {  // invalid ids: no fit (never accepted), no out-of-bounds read
    if (lane < 4) alpha[4 * r + lane] = lane == 0 ? 1.0f : 0.0f;
    if (lane == 0) fit[r] = -__builtin_inff();
    return;
  }

  float x[kMaxPerLane], s[kMaxPerLane];
  load_normalised(tokens + ids[0] * token_stride, dim, eps, x);
  float g[4][4], rhs[4];
  // Parents one at a time; keep their normalised rows for the Gram entries.
  float sp[4][kMaxPerLane];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    load_normalised(tokens + ids[c + 1] * token_stride, dim, eps, s);
#pragma unroll
    for (int i = 0; i < kMaxPerLane; ++i) sp[c][i] = s[i];
  }
#pragma unroll
  for (int a = 0; a < 4; ++a) {
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < kMaxPerLane; ++i) acc = fmaf(sp[a][i], x[i], acc);
    rhs[a] = wave_sum(acc);
#pragma unroll
    for (int b = a; b < 4; ++b) {
      float gg = 0.0f;
#pragma unroll
      for (int i = 0; i < kMaxPerLane; ++i) gg = fmaf(sp[a][i], sp[b][i], gg);
      g[a][b] = wave_sum(gg);
      g[b][a] = g[a][b];
    }
  }

  // Lane `set` (< 15) evaluates one active set.
  float cand[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  float objective = __builtin_inff();
  if (lane < 15) {
    float sol[5];
    const bool solved = solve_set(lane, g, rhs, ridge, sol);
    if (solved) {
      bool feasible = true;
      float sum = 0.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        feasible = feasible && sol[i] >= -1e-5f;
        cand[i] = fmaxf(sol[i], 0.0f);
        sum = sum + cand[i];
      }
      sum = fmaxf(sum, 1e-12f);
#pragma unroll
      for (int i = 0; i < 4; ++i) cand[i] = cand[i] / sum;
      float quad = 0.0f, lin = 0.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float q = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j) q = q + g[i][j] * cand[j];
        quad = quad + cand[i] * q;
        lin = lin + cand[i] * rhs[i];
      }
      if (feasible) objective = quad - 2.0f * lin;
    }
  }
  // argmin over lanes 0..14, first index on ties (torch.argmin).
  float best_obj = objective;
  int best_set = lane < 15 ? lane : 15;
#pragma unroll
  for (int off = 8; off >= 1; off >>= 1) {
    const float o = __shfl_xor(best_obj, off);
    const int ss = __shfl_xor(best_set, off);
    if (o < best_obj || (o == best_obj && ss < best_set)) {
      best_obj = o;
      best_set = ss;
    }
  }
  if (best_set > 14) best_set = 0;  // all candidates infeasible: argmin of all-inf is index 0
  float a[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) a[i] = __shfl(cand[i], best_set);

  if (lane == 0) {
    float num = 0.0f, sq = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) num = num + a[i] * rhs[i];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float q = 0.0f;
#pragma unroll
      for (int j = 0; j < 4; ++j) q = q + g[i][j] * a[j];
      sq = sq + a[i] * q;
    }
    const float cosine = num / sqrtf(fmaxf(sq, 1e-12f));
    const float single = rhs[0];
    if (single > cosine) {
      a[0] = 1.0f;
      a[1] = a[2] = a[3] = 0.0f;
    }
    fit[r] = fmaxf(cosine, single);
#pragma unroll
    for (int i = 0; i < 4; ++i) alpha[4 * r + i] = a[i];
  }
}

// Stable list of rows with fit < threshold among rows whose top1 is below the
// early-accept threshold (the reference's `failed`, :2424), plus its length.
__global__ __launch_bounds__(1024) void failed_rows_kernel(const float* __restrict__ fit,
                                                           const float* __restrict__ top1,
                                                           float easy_threshold, int n,
                                                           float threshold,
                                                           int32_t* __restrict__ list,
                                                           int* __restrict__ count) {
  __shared__ int waves[16];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int per = (n + 1023) / 1024;
  const int b = min(n, tid * per), e = min(n, b + per);
  auto failed = [&](int r) {
    const bool hard = !(top1 && top1[r] >= easy_threshold);
    return hard && fit[r] < threshold;
  };
  int mine = 0;
  for (int r = b; r < e; ++r) mine += failed(r);
  int x = mine;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(x, off);
    if (lane >= off) x += y;
  }
  if (lane == 63) waves[wave] = x;
  __syncthreads();
  if (wave == 0) {
    int v = lane < 16 ? waves[lane] : 0;
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) {
      const int y = __shfl_up(v, off);
      if (lane >= off) v += y;
    }
    if (lane < 16) waves[lane] = v;
  }
  __syncthreads();
  int pos = (wave > 0 ? waves[wave - 1] : 0) + x - mine;
  for (int r = b; r < e; ++r)
    if (failed(r)) list[pos++] = r;
  if (tid == 0) *count = waves[15];
}

}  // namespace
}  // namespace vgo

using namespace vgo;

extern "C" int vgo_convex_fit(const void* tokens, int64_t token_row_stride, int64_t n_tokens, int dtype,
                              const int64_t* rows, int64_t* supports, const int64_t* list_supports,
                              const float* top1,
                              float easy_threshold, const int32_t* row_list, const int* n_list_device,
                              int64_t n, int64_t dim, float eps, float ridge, float* fit, float* alpha,
                              void* stream) {
  VGO_REQUIRE(n >= 0 && dim > 0 && n_tokens >= 0, "convex_fit: bad size");
  if (n == 0) return VGO_OK;
  VGO_REQUIRE(dim <= 64 * kMaxPerLane, "convex_fit: dim > 1024 is not supported");
  VGO_REQUIRE(tokens && rows && supports && fit && alpha, "convex_fit: null pointer");
  VGO_REQUIRE(n < (1LL << 31), "convex_fit: too many rows");
  VGO_REQUIRE((row_list == nullptr) == (n_list_device == nullptr),
              "convex_fit: row_list and its device count go together");
  VGO_REQUIRE(list_supports == nullptr || row_list != nullptr,
              "convex_fit: list_supports needs a row_list");
  hipStream_t s = as_stream(stream);
  const dim3 grid(static_cast<unsigned>((n + 3) / 4));
  const int ni = static_cast<int>(n), d = static_cast<int>(dim);
  switch (dtype) {
    case VGO_F32:
      hipLaunchKernelGGL((convex_fit_kernel<float>), grid, dim3(256), 0, s, static_cast<const float*>(tokens),
                         token_row_stride, n_tokens, rows, supports, list_supports, top1, easy_threshold,
                         row_list, n_list_device, ni, d, eps, ridge, fit, alpha);
      break;
    case VGO_BF16:
      hipLaunchKernelGGL((convex_fit_kernel<bf16_t>), grid, dim3(256), 0, s, static_cast<const bf16_t*>(tokens),
                         token_row_stride, n_tokens, rows, supports, list_supports, top1, easy_threshold,
                         row_list, n_list_device, ni, d, eps, ridge, fit, alpha);
      break;
    default:
      return fail(VGO_EINVAL, "convex_fit: unsupported dtype");
  }
  return check_launch("convex_fit");
}

extern "C" int vgo_failed_rows(const float* fit, const float* top1, float easy_threshold, int64_t n,
                               float threshold, int32_t* list, int* count, void* stream) {
  VGO_REQUIRE(n >= 0 && n < (1LL << 31), "failed_rows: bad size");
  VGO_REQUIRE(fit && list && count, "failed_rows: null pointer");
  hipLaunchKernelGGL(failed_rows_kernel, dim3(1), dim3(1024), 0, as_stream(stream), fit, top1,
                     easy_threshold, static_cast<int>(n), threshold, list, count);
  return check_launch("failed_rows");
}
