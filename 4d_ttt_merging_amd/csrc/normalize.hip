// Row gather + L2 normalisation, the matching front end of the merge planners:
//   out[r,:] = x[rows[r],:] / max(||x[rows[r],:]||_2, eps)
// Work of `F.normalize(tokens[:, ids].float(), dim=-1)` followed by `.to(bf16)`
// in vggt_omega/models/token_merging.py:1102-1103 (eps 1e-12) and
// vggt_omega/models/sparse_convex.py:2384, 2403 (eps 1e-6).  The norm is
// accumulated in fp32; the quotient is rounded once to the output dtype.
// One wave per row; HBM-bound (reads dim*s_in, writes dim*s_out per row).
#include "vgo_common.h"

namespace vgo {
namespace {

template <typename TI, typename TO, bool kVec>
__global__ __launch_bounds__(256) void normalize_rows_kernel(
    const TI* __restrict__ x, int64_t row_stride, int64_t x_rows, const int64_t* __restrict__ rows,
    int64_t n_rows, int dim, float eps, TO* __restrict__ out, int64_t out_stride) {
  const int lane = lane_id();
  const int64_t r = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (r >= n_rows) return;
  const int64_t src = rows ? rows[r] : r;
  TO* orow = out + r * out_stride;
  if (src < 0 || src >= x_rows) {  // bad row id: NaN row, no out-of-bounds read
    for (int e = lane; e < dim; e += 64) orow[e] = from_f32<TO>(__builtin_nanf(""));
    return;
  }
  const TI* xr = x + src * row_stride;
  // Lane l holds elements 4(l + 64i) + j (i < kNormChunks, j < 4); the sum of
  // squares runs over i, then j, then the butterfly -- the order
  // row_l2_denominator fixes, shared with the fused LayerNorm row pass.
  float v[kNormChunks][4];
  const int chunks = dim >> 2;
#pragma unroll
  for (int i = 0; i < kNormChunks; ++i) {
    const int c = i * 64 + lane;
    if (kVec && c < chunks) {
      const f32x4 x4 = load4(xr + 4 * c);
#pragma unroll
      for (int j = 0; j < 4; ++j) v[i][j] = x4[j];
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) v[i][j] = c < chunks ? to_f32(xr[4 * c + j]) : 0.0f;
    }
  }
  const float denom = row_l2_denominator<kNormChunks>(v, lane, chunks, eps);
#pragma unroll
  for (int i = 0; i < kNormChunks; ++i) {
    const int c = i * 64 + lane;
    if (c < chunks) {
#pragma unroll
      for (int j = 0; j < 4; ++j) orow[4 * c + j] = from_f32<TO>(v[i][j] / denom);
    }
  }
}

template <typename TI, typename TO>
int launch_norm(const void* x, int64_t row_stride, int64_t x_rows, const int64_t* rows,
                int64_t n_rows, int dim, float eps, void* out, int64_t out_stride, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>((n_rows + 3) / 4));
  if (aligned(x, 4 * sizeof(TI)) && row_stride % 4 == 0)
    hipLaunchKernelGGL((normalize_rows_kernel<TI, TO, true>), grid, dim3(256), 0, s,
                       static_cast<const TI*>(x), row_stride, x_rows, rows, n_rows, dim, eps,
                       static_cast<TO*>(out), out_stride);
  else
    hipLaunchKernelGGL((normalize_rows_kernel<TI, TO, false>), grid, dim3(256), 0, s,
                       static_cast<const TI*>(x), row_stride, x_rows, rows, n_rows, dim, eps,
                       static_cast<TO*>(out), out_stride);
  return check_launch("normalize_rows");
}

}  // namespace
}  // namespace vgo

extern "C" int vgo_normalize_rows(const void* x, int64_t x_row_stride, int64_t x_rows,
                                  int x_dtype, const int64_t* rows, int64_t n_rows, int64_t dim, float eps,
                                  void* out, int64_t out_row_stride, int out_dtype, void* stream) {
  using namespace vgo;
  VGO_REQUIRE(n_rows >= 0 && dim >= 0, "normalize_rows: negative size");
  if (n_rows == 0 || dim == 0) return VGO_OK;
  VGO_REQUIRE(x && out, "normalize_rows: null pointer");
  VGO_REQUIRE(dim <= 4 * 64 * kNormChunks && dim % 4 == 0,
              "normalize_rows: dim must be a multiple of 4 and at most 2048");
  VGO_REQUIRE(n_rows < (int64_t(1) << 33), "normalize_rows: too many rows");
  hipStream_t s = as_stream(stream);
  const int d = static_cast<int>(dim);
  if (x_dtype == VGO_F32 && out_dtype == VGO_BF16)
    return launch_norm<float, bf16_t>(x, x_row_stride, x_rows, rows, n_rows, d, eps, out, out_row_stride, s);
  if (x_dtype == VGO_F32 && out_dtype == VGO_F32)
    return launch_norm<float, float>(x, x_row_stride, x_rows, rows, n_rows, d, eps, out, out_row_stride, s);
  if (x_dtype == VGO_BF16 && out_dtype == VGO_BF16)
    return launch_norm<bf16_t, bf16_t>(x, x_row_stride, x_rows, rows, n_rows, d, eps, out, out_row_stride, s);
  if (x_dtype == VGO_BF16 && out_dtype == VGO_F32)
    return launch_norm<bf16_t, float>(x, x_row_stride, x_rows, rows, n_rows, d, eps, out, out_row_stride, s);
  if (x_dtype == VGO_F16 && out_dtype == VGO_BF16)
    return launch_norm<f16_t, bf16_t>(x, x_row_stride, x_rows, rows, n_rows, d, eps, out, out_row_stride, s);
  if (x_dtype == VGO_F16 && out_dtype == VGO_F32)
    return launch_norm<f16_t, float>(x, x_row_stride, x_rows, rows, n_rows, d, eps, out, out_row_stride, s);
  return fail(VGO_EINVAL, "normalize_rows: unsupported dtype pair");
}
