// Four-variable simplex least-squares solvers on given Gram / right-hand-side
// inputs: min_a a^T G a - 2 r^T a over the probability simplex, one problem
// per row (G [N,4,4], r [N,4], fp32).
//
// * four_support_active_set (vggt_omega/models/sparse_convex_kernels.py:
//   102-212, 332-353): the 15 active sets of the reference's table (:316-323),
//   each solved in closed form on the reduced simplex -- the last active
//   variable p is eliminated (a_p = 1 - sum of the others), the 1x1 / 2x2 /
//   3x3 system in the remaining active variables is solved by Cramer's rule on
//   G + ridge I, singular systems (|det| <= 1e-12) and candidates with a weight
//   below -1e-5 are infeasible -- then the feasible candidate with the lowest
//   objective (on G without the ridge; first set on ties), renormalised, and
//   the one-hot weights (1,0,0,0) when r_0 exceeds the cosine of the fit.
// * four_support_projected_gradient (:214-296): `steps` projected-gradient
//   steps from (1,0,0,0) with step 0.95 / max(max_i sum_j |G_ij|, 1e-4); the
//   projection onto the simplex takes its threshold from a four-value sorting
//   network, the weights keep the support order.
//
// One lane per row: a problem is 80 bytes in and 16 out with a few hundred
// flops, so the kernels are bound by HBM (96 B per row) and launch latency;
// every lane reads its 64-byte Gram block as four 16-byte loads (one wave
// reads 4 KB of consecutive rows).
#include "vgo_common.h"

namespace vgo {
namespace {

__device__ __forceinline__ void load_row(const float* __restrict__ gram, const float* __restrict__ rhs,
                                         int64_t row, float g[16], float r[4]) {
  const f32x4* gp = reinterpret_cast<const f32x4*>(gram + row * 16);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const f32x4 v = gp[q];
#pragma unroll
    for (int e = 0; e < 4; ++e) g[4 * q + e] = v[e];
  }
  const f32x4 rv = *reinterpret_cast<const f32x4*>(rhs + row * 4);
#pragma unroll
  for (int e = 0; e < 4; ++e) r[e] = rv[e];
}

// Active set s (0..14): size and variables in the reference's table order
// (singletons, pairs, triples, the full set); the last listed variable is the
// one eliminated through the sum-to-one constraint.
struct ActiveSet {
  int count, i0, i1, i2, p;
};
__device__ __forceinline__ ActiveSet active_set(int s) {
  constexpr signed char kIds[15][4] = {
      {0, 0, 0, 0}, {1, 1, 1, 1}, {2, 2, 2, 2}, {3, 3, 3, 3}, {0, 1, 1, 1},
      {0, 2, 2, 2}, {0, 3, 3, 3}, {1, 2, 2, 2}, {1, 3, 3, 3}, {2, 3, 3, 3},
      {0, 1, 2, 2}, {0, 1, 3, 3}, {0, 2, 3, 3}, {1, 2, 3, 3}, {0, 1, 2, 3}};
  constexpr signed char kCount[15] = {1, 1, 1, 1, 2, 2, 2, 2, 2, 2, 3, 3, 3, 3, 4};
  ActiveSet a;
  a.count = kCount[s];
  a.i0 = kIds[s][0];
  a.i1 = kIds[s][1];
  a.i2 = kIds[s][2];
  a.p = kIds[s][kCount[s] - 1];
  return a;
}

__global__ __launch_bounds__(256) void active_set_kernel(const float* __restrict__ gram,
                                                         const float* __restrict__ rhs, int64_t rows,
                                                         float ridge, float* __restrict__ out) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (row >= rows) return;
  float g[16], r[4];
  load_row(gram, rhs, row, g, r);
  auto ge = [&](int a, int b) { return g[4 * a + b] + (a == b ? ridge : 0.0f); };

  float best_obj = 0.0f, best[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int s = 0; s < 15; ++s) {
    const ActiveSet as = active_set(s);
    const int i0 = as.i0, i1 = as.i1, i2 = as.i2, p = as.p;
    const float hp = ge(p, p);
    const float rp = r[p];
    // Reduced Hessian and right-hand side in the variables i0, i1, i2.
    const float h00 = ge(i0, i0) - 2.0f * ge(i0, p) + hp;
    const float h01 = ge(i0, i1) - ge(i0, p) - ge(p, i1) + hp;
    const float h02 = ge(i0, i2) - ge(i0, p) - ge(p, i2) + hp;
    const float h10 = ge(i1, i0) - ge(i1, p) - ge(p, i0) + hp;
    const float h11 = ge(i1, i1) - 2.0f * ge(i1, p) + hp;
    const float h12 = ge(i1, i2) - ge(i1, p) - ge(p, i2) + hp;
    const float h20 = ge(i2, i0) - ge(i2, p) - ge(p, i0) + hp;
    const float h21 = ge(i2, i1) - ge(i2, p) - ge(p, i1) + hp;
    const float h22 = ge(i2, i2) - 2.0f * ge(i2, p) + hp;
    const float c0 = r[i0] - rp - ge(i0, p) + hp;
    const float c1 = r[i1] - rp - ge(i1, p) + hp;
    const float c2 = r[i2] - rp - ge(i2, p) + hp;
    const int dimension = as.count - 1;
    float b0 = 0.0f, b1 = 0.0f, b2 = 0.0f;
    bool stable = as.count == 1;
    // One reciprocal of the determinant per system (the reference divides by it).
    if (dimension == 1) {
      stable = fabsf(h00) > 1.0e-12f;
      b0 = c0 / (stable ? h00 : 1.0f);
    } else if (dimension == 2) {
      const float det2 = h00 * h11 - h01 * h10;
      stable = fabsf(det2) > 1.0e-12f;
      const float inv = 1.0f / (stable ? det2 : 1.0f);
      b0 = (c0 * h11 - h01 * c1) * inv;
      b1 = (h00 * c1 - h10 * c0) * inv;
    } else if (dimension == 3) {
      const float det3 = h00 * (h11 * h22 - h12 * h21) - h01 * (h10 * h22 - h12 * h20) +
                         h02 * (h10 * h21 - h11 * h20);
      stable = fabsf(det3) > 1.0e-12f;
      const float inv = 1.0f / (stable ? det3 : 1.0f);
      b0 = (c0 * (h11 * h22 - h12 * h21) - h01 * (c1 * h22 - h12 * c2) + h02 * (c1 * h21 - h11 * c2)) * inv;
      b1 = (h00 * (c1 * h22 - h12 * c2) - c0 * (h10 * h22 - h12 * h20) + h02 * (h10 * c2 - c1 * h20)) * inv;
      b2 = (h00 * (h11 * c2 - c1 * h21) - h01 * (h10 * c2 - c1 * h20) + c0 * (h10 * h21 - h11 * h20)) * inv;
    }
    const float ap = 1.0f - b0 - b1 - b2;
    // Scatter onto the four weights (for a singleton p == i0 and b0 == 0).
    float a[4];
#pragma unroll
    for (int v = 0; v < 4; ++v)
      a[v] = (i0 == v ? b0 : 0.0f) + (i1 == v ? b1 : 0.0f) + (i2 == v ? b2 : 0.0f) + (p == v ? ap : 0.0f);
    bool feasible = stable;
#pragma unroll
    for (int v = 0; v < 4; ++v) feasible = feasible & (a[v] >= -1.0e-5f);
#pragma unroll
    for (int v = 0; v < 4; ++v) a[v] = fmaxf(a[v], 0.0f);
    const float inv_total = 1.0f / fmaxf(a[0] + a[1] + a[2] + a[3], 1.0e-12f);
#pragma unroll
    for (int v = 0; v < 4; ++v) a[v] = a[v] * inv_total;
    // Objective a^T G a - 2 r^T a on the Gram without the ridge.
    float quad = 0.0f, lin = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float q = fmaf(g[4 * i + 3], a[3], fmaf(g[4 * i + 2], a[2], fmaf(g[4 * i + 1], a[1], g[4 * i] * a[0])));
      quad = fmaf(a[i], q, quad);
      lin = fmaf(a[i], r[i], lin);
    }
    const float obj = feasible ? quad - 2.0f * lin : __builtin_inff();
    // argmin, first index on ties: set 0 seeds the choice even when infeasible.
    if (s == 0 || obj < best_obj) {
      best_obj = obj;
#pragma unroll
      for (int v = 0; v < 4; ++v) best[v] = a[v];
    }
  }

  float alpha[4];
  const float inv_total = 1.0f / fmaxf(best[0] + best[1] + best[2] + best[3], 1.0e-12f);
#pragma unroll
  for (int v = 0; v < 4; ++v) alpha[v] = best[v] * inv_total;
  float numerator = 0.0f, squared_norm = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float q = g[4 * i] * alpha[0] + g[4 * i + 1] * alpha[1] + g[4 * i + 2] * alpha[2] +
                    g[4 * i + 3] * alpha[3];
    numerator += alpha[i] * r[i];
    squared_norm += alpha[i] * q;
  }
  const float cosine = numerator / sqrtf(fmaxf(squared_norm, 1.0e-12f));
  if (r[0] > cosine) {
    alpha[0] = 1.0f;
    alpha[1] = alpha[2] = alpha[3] = 0.0f;
  }
  const f32x4 o = {alpha[0], alpha[1], alpha[2], alpha[3]};
  *reinterpret_cast<f32x4*>(out + row * 4) = o;
}

__global__ __launch_bounds__(256) void projected_gradient_kernel(const float* __restrict__ gram,
                                                                 const float* __restrict__ rhs,
                                                                 int64_t rows, int steps,
                                                                 float* __restrict__ out) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (row >= rows) return;
  float g[16], r[4];
  load_row(gram, rhs, row, g, r);
  float lipschitz = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float norm = fabsf(g[4 * i]) + fabsf(g[4 * i + 1]) + fabsf(g[4 * i + 2]) + fabsf(g[4 * i + 3]);
    lipschitz = i == 0 ? norm : fmaxf(lipschitz, norm);
  }
  const float step = 0.95f / fmaxf(lipschitz, 1.0e-4f);
  float a[4] = {1.0f, 0.0f, 0.0f, 0.0f};
  for (int it = 0; it < steps; ++it) {
    float p[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      // Fused multiply-adds, as the reference's compiler forms them.
      const float dot = fmaf(g[4 * i + 3], a[3], fmaf(g[4 * i + 2], a[2], fmaf(g[4 * i + 1], a[1], g[4 * i] * a[0])));
      p[i] = fmaf(-step, dot - r[i], a[i]);
    }
    // Descending sorting network; only the threshold comes from the sorted values.
    float s0 = fmaxf(p[0], p[1]), s1 = fminf(p[0], p[1]);
    float s2 = fmaxf(p[2], p[3]), s3 = fminf(p[2], p[3]);
    float t = fmaxf(s0, s2);
    s2 = fminf(s0, s2);
    s0 = t;
    t = fmaxf(s1, s3);
    s3 = fminf(s1, s3);
    s1 = t;
    t = fmaxf(s1, s2);
    s2 = fminf(s1, s2);
    s1 = t;
    float theta = s0 - 1.0f;
    const float theta2 = (s0 + s1 - 1.0f) * 0.5f;
    theta = s1 > theta2 ? theta2 : theta;
    const float theta3 = (s0 + s1 + s2 - 1.0f) * (1.0f / 3.0f);  // a multiply, not a divide
    theta = s2 > theta3 ? theta3 : theta;
    const float theta4 = (s0 + s1 + s2 + s3 - 1.0f) * 0.25f;
    theta = s3 > theta4 ? theta4 : theta;
#pragma unroll
    for (int i = 0; i < 4; ++i) a[i] = fmaxf(p[i] - theta, 0.0f);
  }
  const f32x4 o = {a[0], a[1], a[2], a[3]};
  *reinterpret_cast<f32x4*>(out + row * 4) = o;
}

int check_inputs(const float* gram, const float* rhs, int64_t rows, const float* out, const char* what) {
  VGO_REQUIRE(rows >= 0, what);
  VGO_REQUIRE(rows < (int64_t(1) << 40), what);
  if (rows == 0) return VGO_OK;
  VGO_REQUIRE(gram && rhs && out, what);
  VGO_REQUIRE(aligned(gram, 16) && aligned(rhs, 16) && aligned(out, 16), what);
  return VGO_OK;
}

}  // namespace
}  // namespace vgo

extern "C" int vgo_four_support_active_set(const float* gram, const float* rhs, int64_t rows,
                                           float ridge, float* out, void* stream) {
  using namespace vgo;
  const int st = check_inputs(gram, rhs, rows, out,
                              "four_support_active_set: bad arguments (rows >= 0, 16-byte aligned "
                              "contiguous [N,4,4] / [N,4] fp32)");
  if (st != VGO_OK || rows == 0) return st;
  const int64_t blocks = (rows + 255) / 256;
  VGO_REQUIRE(blocks < (int64_t(1) << 31), "four_support_active_set: too many rows");
  hipLaunchKernelGGL(active_set_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     as_stream(stream), gram, rhs, rows, ridge, out);
  return check_launch("four_support_active_set");
}

extern "C" int vgo_four_support_projected_gradient(const float* gram, const float* rhs, int64_t rows,
                                                   int steps, float* out, void* stream) {
  using namespace vgo;
  VGO_REQUIRE(steps >= 0, "four_support_projected_gradient: steps must be >= 0");
  const int st = check_inputs(gram, rhs, rows, out,
                              "four_support_projected_gradient: bad arguments (rows >= 0, 16-byte "
                              "aligned contiguous [N,4,4] / [N,4] fp32)");
  if (st != VGO_OK || rows == 0) return st;
  const int64_t blocks = (rows + 255) / 256;
  VGO_REQUIRE(blocks < (int64_t(1) << 31), "four_support_projected_gradient: too many rows");
  hipLaunchKernelGGL(projected_gradient_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     as_stream(stream), gram, rhs, rows, steps, out);
  return check_launch("four_support_projected_gradient");
}
