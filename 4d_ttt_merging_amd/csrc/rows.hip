// Residual-stream rows of a transformer block in one pass per row:
//   s[r,:]  = x[r,:] + gamma * branch[r,:]          (LayerScale + residual add)
//   n[r,:]  = (s[r,:] - mean) * rsqrt(var + eps) * w + b   (LayerNorm over dim)
// The block is vggt_omega/models/layers/block.py:126-127 and :219-226,
//   x_attn = x + ls1(attn(norm1(x)));  x_ffn = x_attn + ls2(mlp(norm2(x_attn))),
// with LayerScale = `x * gamma` (layer_scale.py:38) and torch LayerNorm.  Under
// bf16 autocast the reference runs each of these as its own pass over the fp32
// stream (multiply, add, layer_norm, then the cast autocast puts in front of the
// next Linear); here one wave reads a row once and writes the new stream row
// and its normalised, already-cast copy.
//
// Optionally also u = n / max(||n||_2, unit_eps), the F.normalize(...).to(bf16)
// front end of the merge planners (token_merging.py:1102-1103), from the fp32
// n in registers, bit-identical to normalize_rows applied to the fp32 n.
//
// s is bit-identical to the reference's: the branch element is widened to fp32,
// multiplied by gamma and added to x with separate IEEE roundings (no fused
// multiply-add; the library is built with -ffp-contract=off), exactly the two
// fp32 ops torch performs.  The LayerNorm uses two passes over the row held in
// registers (mean, then the mean of squared deviations) and differs from torch's
// Welford pass only by fp32 rounding.
//
// One wave per row, four rows per work-group; lane l owns elements 4(l + 64i) ..
// 4(l + 64i) + 3, so each load or store instruction of a wave covers one
// contiguous 1 KB (fp32) or 512 B (16-bit) span.  HBM-bound: per row it reads
// 4*dim (x) + s_b*dim (branch) and writes 4*dim (s) + s_n*dim (n).
//
// Restore variant (vgo_restore_residual_layer_norm): the branch row is the
// merge plan's restore of the attention output, branch[r,:] =
// sum_c w[r,c] * table[index[r,c],:] rounded as the projection kernel rounds it
// (token_merging.py:387-414, 193-196: weight and each product in the value type,
// fp32 sum, result in the value type), so the restored rows never go to memory:
// the row's (index, weight) is loaded first, the table rows of its non-zero
// weights next, under the loads of x and the parameter vectors.  A token plan
// restores by a one-hot map, branch[r,:] = table[index[r],:] (its `inverse`,
// token_merging.py:193-196); with weight == NULL, index is that [rows] array
// and the pass reads 4 bytes of map per row instead of 32.
#include <algorithm>

#include "vgo_common.h"

namespace vgo {
namespace {

// 4-element chunks per lane: dim <= 4 * 64 * kChunks.  Two instantiations,
// kChunks = 4 (dim <= 1024) and 8 (dim <= 2048), keep the register budget of the
// common case small.
constexpr int kRowChunks = 8;

// Butterfly sum: every lane ends with the same value (each exchange adds the
// same two operands in either order).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

struct RowArgs {
  const float* x;
  int64_t x_stride;
  const void* branch;
  int64_t branch_stride;
  const float* gamma;
  const float* ln_w;
  const float* ln_b;
  float eps;
  int64_t rows;
  int dim;
  float* x_out;
  int64_t x_out_stride;
  void* norm;
  int64_t norm_stride;
  float* norm_f32;
  int64_t norm_f32_stride;
  void* unit;
  int64_t unit_stride;
  float unit_eps;
  // Restore variant: branch is the [table_rows, dim] table, branch_stride its row stride.
  const int32_t* r_index;  // [rows, 4]
  const float* r_weight;   // [rows, 4]
  int64_t table_rows;
};

// kGather: 0 no restore; 1 restore by a [rows, 4] (index, weight) map; 2 restore
// by a one-hot [rows] index (a token plan's inverse): the map row (k, 1, 0, 0, 0)
// for k >= 0, a zero row for k < 0, with the same rounding.
template <int kChunks, bool kBranch, int kGather, typename TB, typename TN>
__device__ __forceinline__ void residual_ln_row(const RowArgs& a, int64_t r, int lane, const int (&off)[kChunks],
                                                const bool (&live)[kChunks], const f32x4 (&g)[kChunks],
                                                const f32x4 (&w)[kChunks], const f32x4 (&bias)[kChunks],
                                                int32_t one_hot_id) {
  // The restore map of the row goes out before everything else: only the
  // table loads wait for it.
  constexpr int kCorners = kGather == 2 ? 1 : 4;
  i32x4 id4 = {0, 0, 0, 0};
  f32x4 w4 = {0.0f, 0.0f, 0.0f, 0.0f};
  if constexpr (kGather == 1) {
    id4 = *reinterpret_cast<const i32x4*>(a.r_index + 4 * r);
    w4 = *reinterpret_cast<const f32x4*>(a.r_weight + 4 * r);
  } else if constexpr (kGather == 2) {
    id4[0] = one_hot_id;
    w4[0] = id4[0] >= 0 ? 1.0f : 0.0f;
  }
  const int chunks = a.dim >> 2;
  const float* xr = a.x + r * a.x_stride;
  f32x4 v[kChunks];
#pragma unroll
  for (int i = 0; i < kChunks; ++i) v[i] = *reinterpret_cast<const f32x4*>(xr + off[i]);
  if constexpr (kBranch) {
    f32x4 b[kChunks];
    if constexpr (!kGather) {
      const TB* br = static_cast<const TB*>(a.branch) + r * a.branch_stride;
#pragma unroll
      for (int i = 0; i < kChunks; ++i) b[i] = load4(br + off[i]);
    }
    if constexpr (kGather) {
      // Table rows of the non-zero weights, raw, all requested before any is
      // used; an out-of-range id with a non-zero weight makes the row NaN, as
      // in the projection kernel (the table is never read out of range).
      typedef typename Vec4<TB>::type Raw;
      Raw y[4][kChunks];
      bool use[4];
      bool bad = false;
#pragma unroll
      for (int c = 0; c < kCorners; ++c) {
        use[c] = w4[c] != 0.0f;
        if (use[c] && static_cast<uint32_t>(id4[c]) >= static_cast<uint64_t>(a.table_rows)) {
          bad = true;
          use[c] = false;
        }
        if (use[c]) {
          const TB* tr = static_cast<const TB*>(a.branch) + static_cast<int64_t>(id4[c]) * a.branch_stride;
#pragma unroll
          for (int i = 0; i < kChunks; ++i) y[c][i] = *reinterpret_cast<const Raw*>(tr + off[i]);
        }
      }
      f32x4 acc[kChunks];
#pragma unroll
      for (int i = 0; i < kChunks; ++i) acc[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int c = 0; c < kCorners; ++c) {
        if (!use[c]) continue;
        const float wq = weight_as_value<TB>(w4[c]);
#pragma unroll
        for (int i = 0; i < kChunks; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[i][j] = acc[i][j] + rounded_product<TB>(to_f32(y[c][i][j]), wq);
      }
      // The restored element in the value type, widened again as the branch.
#pragma unroll
      for (int i = 0; i < kChunks; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) b[i][j] = to_f32(from_f32<TB>(bad ? __builtin_nanf("") : acc[i][j]));
    }
    // Empty asm reading the loaded registers: the loads that are only used
    // under a NULL test cannot sink into that branch behind a wait of their own.
#pragma unroll
    for (int i = 0; i < kChunks; ++i) asm volatile("" : "+v"(b[i]));
#pragma unroll
    for (int i = 0; i < kChunks; ++i) {
      if (a.gamma) b[i] = b[i] * g[i];
      v[i] = v[i] + b[i];
    }
  }
  if (a.x_out) {
    float* xo = a.x_out + r * a.x_out_stride;
#pragma unroll
    for (int i = 0; i < kChunks; ++i)
      if (live[i]) *reinterpret_cast<f32x4*>(xo + off[i]) = v[i];
  }
  if (!a.norm && !a.norm_f32 && !a.unit) return;

  const float inv_dim = 1.0f / static_cast<float>(a.dim);
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < kChunks; ++i)
    s += live[i] ? (v[i][0] + v[i][1]) + (v[i][2] + v[i][3]) : 0.0f;
  const float mean = wave_sum(s) * inv_dim;
  float q = 0.0f;
#pragma unroll
  for (int i = 0; i < kChunks; ++i) {
    const f32x4 d = v[i] - mean;
    v[i] = d;
    q += live[i] ? (d[0] * d[0] + d[1] * d[1]) + (d[2] * d[2] + d[3] * d[3]) : 0.0f;
  }
  const float rstd = 1.0f / sqrtf(wave_sum(q) * inv_dim + a.eps);
  TN* no = a.norm ? static_cast<TN*>(a.norm) + r * a.norm_stride : nullptr;
  float* nf = a.norm_f32 ? a.norm_f32 + r * a.norm_f32_stride : nullptr;
#pragma unroll
  for (int i = 0; i < kChunks; ++i) {
    f32x4 n = v[i] * rstd;
    if (a.ln_w) n = n * w[i];
    if (a.ln_b) n = n + bias[i];
    v[i] = n;
    if (!live[i]) continue;
    if (no) store4(no + off[i], n);
    if (nf) *reinterpret_cast<f32x4*>(nf + off[i]) = n;
  }
  if (!a.unit) return;
  // F.normalize of the normalised row, from the same fp32 values and in the
  // same order as normalize_rows over norm_f32, so the two agree bit for bit.
  float vv[kChunks][4];
#pragma unroll
  for (int i = 0; i < kChunks; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) vv[i][j] = v[i][j];
  const float denom = row_l2_denominator<kChunks>(vv, lane, chunks, a.unit_eps);
  TN* uo = static_cast<TN*>(a.unit) + r * a.unit_stride;
#pragma unroll
  for (int i = 0; i < kChunks; ++i)
    if (live[i]) store4(uo + off[i], v[i] / denom);
}

// The plain pass runs one row per wave.  The restore variants run persistent
// waves (as many work-groups as are resident): wave w takes rows w, w + W, ...
// with the parameter vectors (gamma, LayerNorm weight and bias) loaded once and
// the one-hot map's next id fetched a row ahead, so the table row's load waits
// on no index load (C4 restore in the aggregator: 66.7 -> 64.7 us; the plain
// pass gained nothing from it and ran fewer waves per SIMD).  Every load is
// unconditional, so one wait covers them all: a lane's chunk offset is clamped
// into the row and chunks past its end are zeroed after loading; a NULL
// parameter vector reads x's first row in its place and the value is then
// replaced by the identity.
template <int kChunks, bool kBranch, int kGather, typename TB, typename TN>
__global__ __launch_bounds__(256) void residual_ln_kernel(RowArgs a) {
  const int lane = lane_id();
  const int chunks = a.dim >> 2;
  int off[kChunks];
  bool live[kChunks];
#pragma unroll
  for (int i = 0; i < kChunks; ++i) {
    const int c = i * 64 + lane;
    live[i] = c < chunks;
    off[i] = 4 * (live[i] ? c : chunks - 1);
  }
  const float* gp = a.gamma ? a.gamma : a.x;
  const float* wp = a.ln_w ? a.ln_w : a.x;
  const float* bp = a.ln_b ? a.ln_b : a.x;
  f32x4 g[kChunks], w[kChunks], bias[kChunks];
#pragma unroll
  for (int i = 0; i < kChunks; ++i) {
    g[i] = kBranch ? *reinterpret_cast<const f32x4*>(gp + off[i]) : f32x4{1.0f, 1.0f, 1.0f, 1.0f};
    w[i] = *reinterpret_cast<const f32x4*>(wp + off[i]);
    bias[i] = *reinterpret_cast<const f32x4*>(bp + off[i]);
  }
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * 4 +
                    __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  if constexpr (kGather == 0) {  // one row per wave
    if (r0 < a.rows) residual_ln_row<kChunks, kBranch, kGather, TB, TN>(a, r0, lane, off, live, g, w, bias, 0);
    return;
  }
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 4;
  int32_t next_id = kGather == 2 && r0 < a.rows ? a.r_index[r0] : 0;
  for (int64_t r = r0; r < a.rows; r += stride) {
    const int32_t id = next_id;
    if (kGather == 2 && r + stride < a.rows) next_id = a.r_index[r + stride];
    residual_ln_row<kChunks, kBranch, kGather, TB, TN>(a, r, lane, off, live, g, w, bias, id);
  }
}

// Resident work-groups of one kernel (its occupancy on every CU).
template <typename K>
int64_t resident_groups(K kernel) {
  int dev = 0, cus = 0, per_cu = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    cus = 256;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, 256, 0) != hipSuccess || per_cu <= 0)
    per_cu = 1;
  return static_cast<int64_t>(cus) * per_cu;
}

template <bool kBranch, typename TB, typename TN, int kGather = 0>
int launch_rows(const RowArgs& a, hipStream_t s) {
  const int64_t need = (a.rows + 3) / 4;
  if (a.dim <= 4 * 64 * 4) {
    auto k = residual_ln_kernel<4, kBranch, kGather, TB, TN>;
    const dim3 grid(static_cast<unsigned>(kGather ? std::min<int64_t>(need, resident_groups(k)) : need));
    hipLaunchKernelGGL(k, grid, dim3(256), 0, s, a);
  } else {
    auto k = residual_ln_kernel<kRowChunks, kBranch, kGather, TB, TN>;
    const dim3 grid(static_cast<unsigned>(kGather ? std::min<int64_t>(need, resident_groups(k)) : need));
    hipLaunchKernelGGL(k, grid, dim3(256), 0, s, a);
  }
  return check_launch(kGather ? "restore_residual_layer_norm" : "residual_layer_norm");
}

template <typename TN>
int dispatch_branch(const RowArgs& a, int branch_dtype, hipStream_t s) {
  if (!a.branch) return launch_rows<false, float, TN>(a, s);
  switch (branch_dtype) {
    case VGO_BF16: return launch_rows<true, bf16_t, TN>(a, s);
    case VGO_F16: return launch_rows<true, f16_t, TN>(a, s);
    case VGO_F32: return launch_rows<true, float, TN>(a, s);
    default: return fail(VGO_EINVAL, "residual_layer_norm: unsupported branch dtype");
  }
}

template <typename TN, int kGather>
int dispatch_restore(const RowArgs& a, int table_dtype, hipStream_t s) {
  switch (table_dtype) {
    case VGO_BF16: return launch_rows<true, bf16_t, TN, kGather>(a, s);
    case VGO_F16: return launch_rows<true, f16_t, TN, kGather>(a, s);
    case VGO_F32: return launch_rows<true, float, TN, kGather>(a, s);
    default: return fail(VGO_EINVAL, "restore_residual_layer_norm: unsupported table dtype");
  }
}
template <typename TN>
int dispatch_restore(const RowArgs& a, int table_dtype, hipStream_t s) {
  return a.r_weight ? dispatch_restore<TN, 1>(a, table_dtype, s) : dispatch_restore<TN, 2>(a, table_dtype, s);
}

size_t dtype_bytes(int dtype) { return dtype == VGO_F32 ? 4 : 2; }

}  // namespace
}  // namespace vgo

extern "C" int vgo_residual_layer_norm(const float* x, int64_t x_row_stride, const void* branch,
                                       int64_t branch_row_stride, int branch_dtype,
                                       const float* gamma, const float* ln_weight,
                                       const float* ln_bias, float eps, int64_t rows, int64_t dim,
                                       float* x_out, int64_t x_out_row_stride, void* norm_out,
                                       int64_t norm_row_stride, int norm_dtype, float* norm_f32,
                                       int64_t norm_f32_row_stride, void* unit_out,
                                       int64_t unit_row_stride, float unit_eps, void* stream) {
  using namespace vgo;
  VGO_REQUIRE(rows >= 0 && dim >= 0, "residual_layer_norm: negative size");
  if (rows == 0 || dim == 0) return VGO_OK;
  VGO_REQUIRE(x, "residual_layer_norm: null x");
  VGO_REQUIRE(x_out || norm_out || norm_f32 || unit_out, "residual_layer_norm: no output");
  VGO_REQUIRE(!unit_out || norm_out, "residual_layer_norm: unit_out needs norm_out (same dtype)");
  VGO_REQUIRE(branch || !x_out || x_out == x,
              "residual_layer_norm: x_out without a branch must be NULL or x itself");
  VGO_REQUIRE(dim % 4 == 0 && dim <= 4 * 64 * kRowChunks,
              "residual_layer_norm: dim must be a multiple of 4 and at most 2048");
  VGO_REQUIRE(rows < (int64_t(1) << 33), "residual_layer_norm: too many rows");
  VGO_REQUIRE(norm_dtype == VGO_BF16 || norm_dtype == VGO_F16 || !norm_out,
              "residual_layer_norm: norm_out must be bf16 or f16");
  VGO_REQUIRE(branch_dtype == VGO_BF16 || branch_dtype == VGO_F16 || branch_dtype == VGO_F32 || !branch,
              "residual_layer_norm: unsupported branch dtype");
  // Four-element vector accesses: every row start must be 4-element aligned.
  auto vec_ok = [](const void* p, int64_t stride, size_t elem) {
    return !p || (aligned(p, 4 * elem) && stride % 4 == 0);
  };
  VGO_REQUIRE(vec_ok(x, x_row_stride, 4) && vec_ok(x_out, x_out_row_stride, 4) &&
                  vec_ok(norm_f32, norm_f32_row_stride, 4) &&
                  vec_ok(branch, branch_row_stride, dtype_bytes(branch_dtype)) &&
                  vec_ok(norm_out, norm_row_stride, 2) && vec_ok(unit_out, unit_row_stride, 2) &&
                  vec_ok(gamma, 0, 4) &&
                  vec_ok(ln_weight, 0, 4) && vec_ok(ln_bias, 0, 4),
              "residual_layer_norm: pointers must be 4-element aligned and row strides multiples of 4");
  VGO_REQUIRE(!x_out || x_out == x || x_out_row_stride != 0,
              "residual_layer_norm: zero x_out row stride");
  RowArgs a{x, x_row_stride, branch, branch_row_stride, gamma, ln_weight, ln_bias, eps, rows,
            static_cast<int>(dim), x_out, x_out_row_stride, norm_out, norm_row_stride, norm_f32,
            norm_f32_row_stride, unit_out, unit_row_stride, unit_eps, nullptr, nullptr, 0};
  hipStream_t s = as_stream(stream);
  if (norm_out && norm_dtype == VGO_F16) return dispatch_branch<f16_t>(a, branch_dtype, s);
  return dispatch_branch<bf16_t>(a, branch_dtype, s);
}

extern "C" int vgo_restore_residual_layer_norm(
    const float* x, int64_t x_row_stride, const void* table, int64_t table_row_stride,
    int64_t table_rows, int table_dtype, const int32_t* index, const float* weight,
    const float* gamma, const float* ln_weight, const float* ln_bias, float eps, int64_t rows,
    int64_t dim, float* x_out, int64_t x_out_row_stride, void* norm_out, int64_t norm_row_stride,
    int norm_dtype, void* stream) {
  using namespace vgo;
  VGO_REQUIRE(rows >= 0 && dim >= 0 && table_rows >= 0, "restore_residual_layer_norm: negative size");
  if (rows == 0 || dim == 0) return VGO_OK;
  VGO_REQUIRE(x && table && index, "restore_residual_layer_norm: null input");
  VGO_REQUIRE(x_out || norm_out, "restore_residual_layer_norm: no output");
  VGO_REQUIRE(dim % 4 == 0 && dim <= 4 * 64 * kRowChunks,
              "restore_residual_layer_norm: dim must be a multiple of 4 and at most 2048");
  VGO_REQUIRE(rows < (int64_t(1) << 33) && table_rows < (int64_t(1) << 31),
              "restore_residual_layer_norm: too many rows");
  VGO_REQUIRE(norm_dtype == VGO_BF16 || norm_dtype == VGO_F16 || !norm_out,
              "restore_residual_layer_norm: norm_out must be bf16 or f16");
  VGO_REQUIRE(table_dtype == VGO_BF16 || table_dtype == VGO_F16 || table_dtype == VGO_F32,
              "restore_residual_layer_norm: unsupported table dtype");
  auto vec_ok = [](const void* p, int64_t stride, size_t elem) {
    return !p || (aligned(p, 4 * elem) && stride % 4 == 0);
  };
  VGO_REQUIRE(vec_ok(x, x_row_stride, 4) && vec_ok(x_out, x_out_row_stride, 4) &&
                  vec_ok(table, table_row_stride, dtype_bytes(table_dtype)) &&
                  vec_ok(norm_out, norm_row_stride, 2) && vec_ok(gamma, 0, 4) &&
                  vec_ok(ln_weight, 0, 4) && vec_ok(ln_bias, 0, 4) &&
                  (weight ? vec_ok(index, 0, 4) : aligned(index, 4)) && vec_ok(weight, 0, 4),
              "restore_residual_layer_norm: pointers must be 4-element aligned and row strides multiples of 4");
  VGO_REQUIRE(!x_out || x_out == x || x_out_row_stride != 0,
              "restore_residual_layer_norm: zero x_out row stride");
  RowArgs a{x, x_row_stride, table, table_row_stride, gamma, ln_weight, ln_bias, eps, rows,
            static_cast<int>(dim), x_out, x_out_row_stride, norm_out, norm_row_stride, nullptr, 0,
            nullptr, 0, 0.0f, index, weight, table_rows};
  hipStream_t s = as_stream(stream);
  if (norm_out && norm_dtype == VGO_F16) return dispatch_restore<f16_t>(a, table_dtype, s);
  return dispatch_restore<bf16_t>(a, table_dtype, s);
}
