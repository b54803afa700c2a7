// Mass-bias flash attention for gfx950: O = softmax(Q K^T / sqrt(64) + log m) V.
//
// Work of vggt_omega/models/mass_bias_attention.py:17-129 (Triton kernel and
// wrapper) and, with no bias, of the dense special-query SDPA at
// vggt_omega/models/layers/attention.py:406-422.
//
// bf16 / f16 path (the autocast path of the reference):
//  * A work-group of 4 waves owns 4*QB*32 queries of one (batch, head); each
//    wave keeps its Q rows in registers as MFMA B operands.
//  * Keys stream through LDS in tiles of 64: K row-major, V transposed (V^T, d
//    rows) so both feed v_mfma_f32_32x32x16 as A operands with one 16-byte LDS
//    read per lane.
//  * Scores are computed transposed, S^T = K' Q'^T, so a lane owns one query
//    and 16 keys of every 32-key sub-tile: the row max/sum of the online
//    softmax stay in registers except for one exchange with lane l^32, and the
//    exponentiated scores are already laid out as the B operand of O^T = V^T P^T.
//  * The per-key bias rides in the MFMA: a fifth k-step multiplies a Q-side
//    column of ones with a K-side column holding 8*log(m) (exact in bf16/f16),
//    so S'' = q.k + 8 log m and logit*log2(e) = S'' * log2(e)/8.  The reference
//    rounds log(m) to the input dtype first (mass_bias_attention.py:109); so do
//    we.  P is rounded to the input dtype before P.V (reference :74) and the row
//    sum is accumulated from those rounded values with v_dot2 (fp32 accumulate).
// fp32 path: exact fp32 arithmetic, one query row per lane, K/V tiles in LDS.
#include "vgo_common.h"

namespace vgo {
namespace {

constexpr int kD = 64;
constexpr int kBN = 64;                 // keys per LDS tile
constexpr int kWavesA = 4;              // waves per work-group
constexpr int kPad = 8;                 // elements of padding per LDS row
constexpr int kKRow = kD + kPad;        // K tile: [kBN keys][kKRow]
constexpr int kVRow = kBN + kPad;       // V^T tile: [kD dims][kVRow]
constexpr float kLog2e = 1.4426950408889634f;

template <typename T>
struct Mma;
template <>
struct Mma<bf16_t> {
  typedef bf16x8 op8;
  typedef bf16x2 op2;
  static __device__ __forceinline__ f32x16 mma(op8 a, op8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ float dot2(op2 a, op2 b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(a, b, c, false);
  }
};
template <>
struct Mma<f16_t> {
  typedef f16x8 op8;
  typedef f16x2 op2;
  static __device__ __forceinline__ f32x16 mma(op8 a, op8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ float dot2(op2 a, op2 b, float c) {
    return __builtin_amdgcn_fdot2(a, b, c, false);
  }
};

__device__ __forceinline__ float other_half(float x) { return __shfl_xor(x, 32); }

// Position of key `kk` (0..63) inside a V^T row.  Within every 16-key group the
// two middle quads are swapped, which is the order in which S^T's accumulator
// registers present keys to the P operand (see the header comment).
__device__ __forceinline__ int vt_pos(int kk) {
  return (kk & ~12) | ((kk & 4) << 1) | ((kk & 8) >> 1);
}

template <typename T, int QB>
__global__ __launch_bounds__(kWavesA * 64, 2) void attn_mfma_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    const T* __restrict__ bias, T* __restrict__ out, int heads, int nq, int nk, int n_qblocks,
    int64_t qsb, int64_t qsh, int64_t qsn, int64_t ksb, int64_t ksh, int64_t ksn, int64_t vsb,
    int64_t vsh, int64_t vsn, int64_t osb, int64_t osh, int64_t osn, float c) {
  typedef typename Mma<T>::op8 op8;
  typedef typename Mma<T>::op2 op2;
  constexpr int kQPerWave = QB * 32;
  constexpr int kQPerBlock = kWavesA * kQPerWave;
  __shared__ __attribute__((aligned(16))) T k_lds[kBN * kKRow];
  __shared__ __attribute__((aligned(16))) T vt_lds[kD * kVRow];
  __shared__ __attribute__((aligned(16))) T b_lds[kBN];

  const int task = xcd_remap(blockIdx.x, gridDim.x);
  const int bh = task / n_qblocks;
  const int qblk = task - bh * n_qblocks;
  const int b = bh / heads;
  const int h = bh - b * heads;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int l32 = lane & 31;
  const int hh = lane >> 5;
  const int qw0 = qblk * kQPerBlock + wave * kQPerWave;

  const T* qb_ptr = q + b * qsb + h * qsh;
  const T* kb_ptr = k + b * ksb + h * ksh;
  const T* vb_ptr = v + b * vsb + h * vsh;

  const op8 zero8 = {};
  op8 qreg[QB][4];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int row = qw0 + qb * 32 + l32;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      qreg[qb][t] = row < nq ? *reinterpret_cast<const op8*>(qb_ptr + row * qsn + 16 * t + 8 * hh)
                             : zero8;
    }
  }
  op8 qone = zero8;
  if (hh == 0) qone[0] = static_cast<T>(1.0f);

  float m[QB], lsum[QB];
  f32x16 o[QB][2];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    m[qb] = -__builtin_inff();
    lsum[qb] = 0.0f;
#pragma unroll
    for (int dt = 0; dt < 2; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[qb][dt][r] = 0.0f;
  }
  const op2 ones2 = {static_cast<T>(1.0f), static_cast<T>(1.0f)};

  // Staging roles: K rows (tid>>3) and (tid>>3)+32, V key pair 2*(tid>>3), 8 dims at dc.
  const int st_row = tid >> 3;
  const int dc = (tid & 7) * 8;

  for (int kt = 0; kt < nk; kt += kBN) {
    __syncthreads();
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int key = st_row + 32 * p;
      const op8 val =
          kt + key < nk ? *reinterpret_cast<const op8*>(kb_ptr + (kt + key) * ksn + dc) : zero8;
      *reinterpret_cast<op8*>(&k_lds[key * kKRow + dc]) = val;
    }
    {
      const int key0 = 2 * st_row;
      const op8 v0 =
          kt + key0 < nk ? *reinterpret_cast<const op8*>(vb_ptr + (kt + key0) * vsn + dc) : zero8;
      const op8 v1 = kt + key0 + 1 < nk
                         ? *reinterpret_cast<const op8*>(vb_ptr + (kt + key0 + 1) * vsn + dc)
                         : zero8;
      const int pos = vt_pos(key0);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const op2 pr = {v0[i], v1[i]};
        *reinterpret_cast<op2*>(&vt_lds[(dc + i) * kVRow + pos]) = pr;
      }
    }
    if (tid < kBN) {
      const int key = kt + tid;
      float bv = -__builtin_inff();
      if (key < nk) bv = bias ? 8.0f * to_f32(bias[key]) : 0.0f;
      b_lds[tid] = static_cast<T>(bv);
    }
    __syncthreads();

    // S^T = K' Q'^T for two 32-key sub-tiles.
    f32x16 s[QB][2];
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
#pragma unroll
      for (int qb = 0; qb < QB; ++qb)
#pragma unroll
        for (int r = 0; r < 16; ++r) s[qb][sub][r] = 0.0f;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const op8 a = *reinterpret_cast<const op8*>(&k_lds[(sub * 32 + l32) * kKRow + 16 * t + 8 * hh]);
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) s[qb][sub] = Mma<T>::mma(a, qreg[qb][t], s[qb][sub]);
      }
      op8 a = zero8;
      if (hh == 0) a[0] = b_lds[sub * 32 + l32];
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) s[qb][sub] = Mma<T>::mma(a, qone, s[qb][sub]);
    }

    // Online softmax in the exp2 domain; P rounded to T as the B operand.
    op8 pk[QB][4];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      float mx = s[qb][0][0];
#pragma unroll
      for (int sub = 0; sub < 2; ++sub)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[qb][sub][r]);
      mx = fmaxf(mx, other_half(mx));
      const float mnew = fmaxf(m[qb], mx);
      const float corr = __builtin_amdgcn_exp2f((m[qb] - mnew) * c);
      const float mc = mnew * c;
      float part = 0.0f;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float pv = __builtin_amdgcn_exp2f(fmaf(s[qb][t >> 1][(t & 1) * 8 + j], c, -mc));
          pk[qb][t][j] = static_cast<T>(pv);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const op2 pr = {pk[qb][t][2 * j], pk[qb][t][2 * j + 1]};
          part = Mma<T>::dot2(pr, ones2, part);
        }
      }
      lsum[qb] = lsum[qb] * corr + part;
      m[qb] = mnew;
#pragma unroll
      for (int dt = 0; dt < 2; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[qb][dt][r] *= corr;
    }

    // O^T += V^T P^T.
#pragma unroll
    for (int t = 0; t < 4; ++t) {
#pragma unroll
      for (int dt = 0; dt < 2; ++dt) {
        const op8 a =
            *reinterpret_cast<const op8*>(&vt_lds[(dt * 32 + l32) * kVRow + 16 * t + 8 * hh]);
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) o[qb][dt] = Mma<T>::mma(a, pk[qb][t], o[qb][dt]);
      }
    }
  }

  T* ob_ptr = out + b * osb + h * osh;
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const float ltot = lsum[qb] + other_half(lsum[qb]);
    const int row = qw0 + qb * 32 + l32;
    if (row < nq) {
#pragma unroll
      for (int dt = 0; dt < 2; ++dt) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int d = dt * 32 + 8 * g + 4 * hh;
          typedef __attribute__((__vector_size__(4 * sizeof(T)))) T t4;
          t4 val;
#pragma unroll
          for (int e = 0; e < 4; ++e) val[e] = static_cast<T>(o[qb][dt][4 * g + e] / ltot);
          *reinterpret_cast<t4*>(ob_ptr + row * osn + d) = val;
        }
      }
    }
  }
}

// fp32: one query per lane; 64 queries per work-group; K/V tiles of 64 keys.
constexpr int kF32Keys = 64;
__global__ __launch_bounds__(64) void attn_f32_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ bias, float* __restrict__ out, int heads, int nq, int nk,
    int n_qblocks, int64_t qsb, int64_t qsh, int64_t qsn, int64_t ksb, int64_t ksh, int64_t ksn,
    int64_t vsb, int64_t vsh, int64_t vsn, int64_t osb, int64_t osh, int64_t osn,
    float scale_log2) {
  __shared__ float k_lds[kF32Keys][kD + 1];
  __shared__ float v_lds[kF32Keys][kD];
  __shared__ float b_lds[kF32Keys];
  const int task = xcd_remap(blockIdx.x, gridDim.x);
  const int bh = task / n_qblocks;
  const int qblk = task - bh * n_qblocks;
  const int b = bh / heads;
  const int h = bh - b * heads;
  const int lane = threadIdx.x;
  const int row = qblk * 64 + lane;
  const float* kb_ptr = k + b * ksb + h * ksh;
  const float* vb_ptr = v + b * vsb + h * vsh;

  float qr[kD], acc[kD];
  const float* qrow = q + b * qsb + h * qsh + static_cast<int64_t>(row < nq ? row : 0) * qsn;
#pragma unroll
  for (int d = 0; d < kD; ++d) {
    qr[d] = row < nq ? qrow[d] : 0.0f;
    acc[d] = 0.0f;
  }
  float m = -__builtin_inff(), l = 0.0f;
  for (int kt = 0; kt < nk; kt += kF32Keys) {
    __syncthreads();
    for (int i = lane; i < kF32Keys * kD; i += 64) {
      const int key = i / kD, d = i % kD;
      const bool ok = kt + key < nk;
      k_lds[key][d] = ok ? kb_ptr[(kt + key) * ksn + d] : 0.0f;
      v_lds[key][d] = ok ? vb_ptr[(kt + key) * vsn + d] : 0.0f;
    }
    {
      const int key = kt + lane;
      b_lds[lane] = key < nk ? (bias ? bias[key] * kLog2e : 0.0f) : -__builtin_inff();
    }
    __syncthreads();
    float logit[kF32Keys];
    float mx = -__builtin_inff();
#pragma unroll
    for (int j = 0; j < kF32Keys; ++j) {
      float dot = 0.0f;
#pragma unroll
      for (int d = 0; d < kD; ++d) dot = fmaf(qr[d], k_lds[j][d], dot);
      logit[j] = dot * scale_log2 + b_lds[j];
      mx = fmaxf(mx, logit[j]);
    }
    const float mnew = fmaxf(m, mx);
    const float corr = exp2f(m - mnew);
    l *= corr;
#pragma unroll
    for (int d = 0; d < kD; ++d) acc[d] *= corr;
#pragma unroll
    for (int j = 0; j < kF32Keys; ++j) {
      const float p = exp2f(logit[j] - mnew);
      l += p;
#pragma unroll
      for (int d = 0; d < kD; ++d) acc[d] = fmaf(p, v_lds[j][d], acc[d]);
    }
    m = mnew;
  }
  if (row < nq) {
    float* orow = out + b * osb + h * osh + static_cast<int64_t>(row) * osn;
#pragma unroll
    for (int d = 0; d < kD; ++d) orow[d] = acc[d] / l;
  }
}

template <typename T>
int launch_mfma(const void* q, const void* k, const void* v, const void* bias, void* out,
                int64_t batch, int64_t heads, int64_t nq, int64_t nk, const int64_t* qs,
                const int64_t* ks, const int64_t* vs, const int64_t* os, hipStream_t stream) {
  constexpr int QB = 1;
  constexpr int kQPerBlock = kWavesA * QB * 32;
  const int64_t n_qblocks = (nq + kQPerBlock - 1) / kQPerBlock;
  const int64_t total = n_qblocks * batch * heads;
  VGO_REQUIRE(total <= 0x7fffffff, "mass_bias_attention: grid too large");
  const float c = kLog2e / 8.0f;
  hipLaunchKernelGGL((attn_mfma_kernel<T, QB>), dim3(static_cast<unsigned>(total)),
                     dim3(kWavesA * 64), 0, stream, static_cast<const T*>(q),
                     static_cast<const T*>(k), static_cast<const T*>(v),
                     static_cast<const T*>(bias), static_cast<T*>(out), static_cast<int>(heads),
                     static_cast<int>(nq), static_cast<int>(nk), static_cast<int>(n_qblocks), qs[0],
                     qs[1], qs[2], ks[0], ks[1], ks[2], vs[0], vs[1], vs[2], os[0], os[1], os[2], c);
  return check_launch("mass_bias_attention");
}

int launch_f32(const void* q, const void* k, const void* v, const void* bias, void* out,
               int64_t batch, int64_t heads, int64_t nq, int64_t nk, const int64_t* qs,
               const int64_t* ks, const int64_t* vs, const int64_t* os, hipStream_t stream) {
  const int64_t n_qblocks = (nq + 63) / 64;
  const int64_t total = n_qblocks * batch * heads;
  VGO_REQUIRE(total <= 0x7fffffff, "mass_bias_attention: grid too large");
  const float scale_log2 = 1.0f / 8.0f * kLog2e;
  hipLaunchKernelGGL(attn_f32_kernel, dim3(static_cast<unsigned>(total)), dim3(64), 0, stream,
                     static_cast<const float*>(q), static_cast<const float*>(k),
                     static_cast<const float*>(v), static_cast<const float*>(bias),
                     static_cast<float*>(out), static_cast<int>(heads), static_cast<int>(nq),
                     static_cast<int>(nk), static_cast<int>(n_qblocks), qs[0], qs[1], qs[2], ks[0],
                     ks[1], ks[2], vs[0], vs[1], vs[2], os[0], os[1], os[2], scale_log2);
  return check_launch("mass_bias_attention(f32)");
}

}  // namespace
}  // namespace vgo

extern "C" int vgo_mass_bias_attn_fwd(const void* q, const void* k, const void* v,
                                      const void* log_mass, void* out, int64_t batch,
                                      int64_t heads, int64_t n_query, int64_t n_key,
                                      int64_t head_dim, const int64_t q_stride[3],
                                      const int64_t k_stride[3], const int64_t v_stride[3],
                                      const int64_t o_stride[3], int dtype, void* stream) {
  using namespace vgo;
  VGO_REQUIRE(head_dim == 64, "the initial fused kernel supports head_dim=64 only");
  VGO_REQUIRE(batch >= 0 && heads >= 0 && n_query >= 0 && n_key >= 0,
              "mass_bias_attention: negative size");
  if (batch == 0 || heads == 0 || n_query == 0) return VGO_OK;
  VGO_REQUIRE(n_key > 0, "mass_bias_attention: no keys");
  VGO_REQUIRE(q && k && v && out, "mass_bias_attention: null pointer");
  VGO_REQUIRE(q_stride && k_stride && v_stride && o_stride, "mass_bias_attention: null strides");
  VGO_REQUIRE(n_query <= 0x7fffffff && n_key <= 0x7fffffff, "mass_bias_attention: too many tokens");
  hipStream_t s = as_stream(stream);
  if (dtype == VGO_BF16 || dtype == VGO_F16) {
    for (int i = 0; i < 3; ++i) {
      VGO_REQUIRE(q_stride[i] % 8 == 0 && k_stride[i] % 8 == 0 && v_stride[i] % 8 == 0 &&
                      o_stride[i] % 4 == 0,
                  "mass_bias_attention: token/head/batch strides must be multiples of 8 elements");
    }
    VGO_REQUIRE(aligned(q, 16) && aligned(k, 16) && aligned(v, 16) && aligned(out, 8),
                "mass_bias_attention: q/k/v must be 16-byte aligned");
    if (dtype == VGO_BF16)
      return launch_mfma<bf16_t>(q, k, v, log_mass, out, batch, heads, n_query, n_key, q_stride,
                                 k_stride, v_stride, o_stride, s);
    return launch_mfma<f16_t>(q, k, v, log_mass, out, batch, heads, n_query, n_key, q_stride,
                              k_stride, v_stride, o_stride, s);
  }
  if (dtype == VGO_F32)
    return launch_f32(q, k, v, log_mass, out, batch, heads, n_query, n_key, q_stride, k_stride,
                      v_stride, o_stride, s);
  return fail(VGO_EINVAL, "mass_bias_attention: unsupported dtype");
}
