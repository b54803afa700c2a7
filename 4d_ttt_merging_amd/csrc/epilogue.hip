// Fused QKV epilogue: per-head LayerNorm(64) of q and k, optional axial RoPE,
// and the split of the packed projection into head-major q/k/v operands.
//
// Work of vggt_omega/models/layers/attention.py:334-341: reshape of the packed
// qkv projection to [B, N, 3, H, 64], `q_norm` / `k_norm` (LayerNorm over the
// 64 channels of every head, eps 1e-5, shared affine), RoPE on the patch
// tokens (`apply_rope`, :243-262, with the prefix of special tokens left
// unrotated), and the transposes to [B, H, N, 64] -- one pass over the
// projection instead of a LayerNorm kernel per tensor, a concat for the RoPE
// prefix, elementwise RoPE kernels and dtype casts.
//
// Layout: lane l of a wave owns channels [16 l, 16 l + 16) of a 1024-channel
// row, so a head is four lanes and its LayerNorm statistics are two xor
// shuffles; RoPE's rotate_half partner (channel +-32) is lane l ^ 2.
// Arithmetic follows the reference's dtypes: LayerNorm and RoPE in fp32, one
// rounding to the output dtype.  HBM-bound: reads 3*C*s_in and writes up to
// 3*C*s_out bytes per token.
#include <algorithm>

#include "vgo_common.h"

namespace vgo {
namespace {

template <typename T>
struct Pack16;  // 16 values of T
template <>
struct Pack16<bf16_t> {
  typedef bf16x8 half;
  static constexpr int kLoads = 2;
};
template <>
struct Pack16<f16_t> {
  typedef f16x8 half;
  static constexpr int kLoads = 2;
};
template <>
struct Pack16<float> {
  typedef f32x4 half;
  static constexpr int kLoads = 4;
};

template <typename T>
__device__ __forceinline__ void load16(const T* p, float* v) {
  typedef typename Pack16<T>::half V;
  constexpr int kPer = 16 / Pack16<T>::kLoads;
#pragma unroll
  for (int i = 0; i < Pack16<T>::kLoads; ++i) {
    const V x = *reinterpret_cast<const V*>(p + i * kPer);
#pragma unroll
    for (int j = 0; j < kPer; ++j) v[i * kPer + j] = to_f32(x[j]);
  }
}

template <typename T>
__device__ __forceinline__ void store16(T* p, const float* v) {
  typedef typename Pack16<T>::half V;
  constexpr int kPer = 16 / Pack16<T>::kLoads;
#pragma unroll
  for (int i = 0; i < Pack16<T>::kLoads; ++i) {
    V x;
#pragma unroll
    for (int j = 0; j < kPer; ++j) x[j] = from_f32<T>(v[i * kPer + j]);
    *reinterpret_cast<V*>(p + i * kPer) = x;
  }
}

// x*cos + rotate_half(x)*sin over a 64-channel head; the partner half lives in lane ^ 2.
__device__ __forceinline__ void rope16(float* v, const float* sin_row, const float* cos_row, int d0) {
  const bool first_half = d0 < 32;
  float rot[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const float partner = quad_xor<2>(v[j]);
    rot[j] = first_half ? -partner : partner;
  }
#pragma unroll
  for (int j = 0; j < 16; ++j) v[j] = v[j] * cos_row[d0 + j] + rot[j] * sin_row[d0 + j];
}

// Persistent waves: wave w handles output rows w, w + W, ... (W = the grid's waves),
// so the LayerNorm parameters are staged in LDS once per work-group instead of
// being read for every row (8% faster at the frame blocks' 32 x 1,029 rows).
template <typename TI, typename TO>
__global__ __launch_bounds__(256) void qkv_epilogue_kernel(
    const TI* __restrict__ qkv, int64_t row_stride, int64_t n_in_rows,
    const int64_t* __restrict__ rows, int n_out, int t_in, int t_out, int heads,
    const float* __restrict__ qw, const float* __restrict__ qb, const float* __restrict__ kw,
    const float* __restrict__ kb, float eps, const float* __restrict__ rope_sin,
    const float* __restrict__ rope_cos, int rope_prefix, int rope_rows,
    TO* __restrict__ q_out, TO* __restrict__ k_out, TO* __restrict__ v_out) {
  __shared__ __attribute__((aligned(16))) float ln_lds[4][64];  // q weight, q bias, k weight, k bias
  for (int e = threadIdx.x; e < 256; e += blockDim.x) {
    const int a = e >> 6, j = e & 63;
    const float* p = a == 0 ? qw : a == 1 ? qb : a == 2 ? kw : kb;
    ln_lds[a][j] = p ? p[j] : 0.0f;
  }
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int C = heads * 64;
  const int d0 = (lane * 16) & 63;  // the same in every 1024-channel chunk
  for (int r = blockIdx.x * 4 + static_cast<int>(threadIdx.x >> 6); r < n_out; r += gridDim.x * 4) {
    const int64_t src = rows ? rows[r] : r;
    if (src < 0 || src >= n_in_rows) continue;
    const int seq = r / t_out;
    const int t = r - seq * t_out;
    const int pos = static_cast<int>(src % t_in) - rope_prefix;  // RoPE row of this token
    const bool rotate = rope_sin != nullptr && pos >= 0 && pos < rope_rows;
    const TI* row = qkv + src * row_stride;
    for (int c0 = lane * 16; c0 < C; c0 += 1024) {
      const int h = c0 >> 6;
      const int64_t o = ((static_cast<int64_t>(seq) * heads + h) * t_out + t) * 64 + d0;
      // The packed row always holds q, k and v, so the three loads are issued
      // together, whichever outputs are written, and wait once.
      float vq[16], vk[16], vv[16];
      load16(row + c0, vq);
      load16(row + C + c0, vk);
      load16(row + 2 * C + c0, vv);
      if (v_out) store16(v_out + o, vv);
      if (q_out) {
        if (qw) head_layer_norm(vq, ln_lds[0] + d0, ln_lds[1] + d0, eps);
        if (rotate) rope16(vq, rope_sin + static_cast<int64_t>(pos) * 64, rope_cos + static_cast<int64_t>(pos) * 64, d0);
        store16(q_out + o, vq);
      }
      if (k_out) {
        if (kw) head_layer_norm(vk, ln_lds[2] + d0, ln_lds[3] + d0, eps);
        if (rotate) rope16(vk, rope_sin + static_cast<int64_t>(pos) * 64, rope_cos + static_cast<int64_t>(pos) * 64, d0);
        store16(k_out + o, vk);
      }
    }
  }
}

template <typename TI, typename TO>
int launch_epilogue(const void* qkv, int64_t row_stride, int64_t n_in_rows, const int64_t* rows,
                    int n_out, int t_in, int t_out, int heads, const float* qw, const float* qb,
                    const float* kw, const float* kb, float eps, const float* rs, const float* rc,
                    int prefix, int rope_rows, void* q, void* k, void* v, hipStream_t s) {
  // Resident work-groups only (the kernel loops over its rows).
  int per_cu = 0, dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    cus = 256;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, qkv_epilogue_kernel<TI, TO>, 256, 0) != hipSuccess ||
      per_cu <= 0)
    per_cu = 1;
  const int64_t need = (static_cast<int64_t>(n_out) + 3) / 4;
  const dim3 grid(static_cast<unsigned>(std::min<int64_t>(need, static_cast<int64_t>(cus) * per_cu)));
  hipLaunchKernelGGL((qkv_epilogue_kernel<TI, TO>), grid, dim3(256), 0, s,
                     static_cast<const TI*>(qkv), row_stride, n_in_rows, rows, n_out, t_in, t_out,
                     heads, qw, qb, kw, kb, eps, rs, rc, prefix, rope_rows, static_cast<TO*>(q),
                     static_cast<TO*>(k), static_cast<TO*>(v));
  return check_launch("qkv_epilogue");
}

}  // namespace
}  // namespace vgo

using namespace vgo;

extern "C" int vgo_qkv_epilogue(const void* qkv, int64_t row_stride, int64_t n_in_rows, int in_dtype,
                                const int64_t* rows, int64_t n_out, int64_t tokens_in,
                                int64_t tokens_out, int64_t heads, const float* q_weight,
                                const float* q_bias, const float* k_weight, const float* k_bias,
                                float eps, const float* rope_sin, const float* rope_cos,
                                int64_t rope_prefix, int64_t rope_rows, void* q_out, void* k_out,
                                void* v_out, int out_dtype, void* stream) {
  VGO_REQUIRE(n_out >= 0 && heads > 0 && tokens_in > 0 && tokens_out > 0, "qkv_epilogue: bad size");
  if (n_out == 0) return VGO_OK;
  VGO_REQUIRE(qkv, "qkv_epilogue: null input");
  VGO_REQUIRE(n_out % tokens_out == 0, "qkv_epilogue: output rows must be whole sequences");
  VGO_REQUIRE(rows || n_out <= n_in_rows, "qkv_epilogue: more output rows than input rows");
  VGO_REQUIRE((q_weight == nullptr) == (q_bias == nullptr) && (k_weight == nullptr) == (k_bias == nullptr),
              "qkv_epilogue: LayerNorm weight and bias go together");
  VGO_REQUIRE((rope_sin == nullptr) == (rope_cos == nullptr), "qkv_epilogue: RoPE sin and cos go together");
  VGO_REQUIRE(n_out < (1LL << 31) && heads * 64 <= (1 << 16), "qkv_epilogue: size too large");
  const int64_t per = in_dtype == VGO_F32 ? 4 : 8;
  VGO_REQUIRE(row_stride % per == 0 && aligned(qkv, 16), "qkv_epilogue: misaligned projection rows");
  VGO_REQUIRE(row_stride >= 3 * heads * 64, "qkv_epilogue: row stride smaller than 3*C");
  hipStream_t s = as_stream(stream);
  const int no = static_cast<int>(n_out), ti = static_cast<int>(tokens_in), to = static_cast<int>(tokens_out);
  const int h = static_cast<int>(heads), pf = static_cast<int>(rope_prefix), rr = static_cast<int>(rope_rows);
#define VGO_EPI(TI, TO)                                                                              \
  return launch_epilogue<TI, TO>(qkv, row_stride, n_in_rows, rows, no, ti, to, h, q_weight, q_bias, \
                                 k_weight, k_bias, eps, rope_sin, rope_cos, pf, rr, q_out, k_out,   \
                                 v_out, s)
  if (in_dtype == VGO_BF16 && out_dtype == VGO_BF16) VGO_EPI(bf16_t, bf16_t);
  if (in_dtype == VGO_BF16 && out_dtype == VGO_F32) VGO_EPI(bf16_t, float);
  if (in_dtype == VGO_F32 && out_dtype == VGO_F32) VGO_EPI(float, float);
  if (in_dtype == VGO_F32 && out_dtype == VGO_BF16) VGO_EPI(float, bf16_t);
  if (in_dtype == VGO_F16 && out_dtype == VGO_F16) VGO_EPI(f16_t, f16_t);
#undef VGO_EPI
  return fail(VGO_EINVAL, "qkv_epilogue: unsupported dtype pair");
}
