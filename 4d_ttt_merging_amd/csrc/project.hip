// Top-4 convex projection (unmerge), the restore step of a merge plan:
//   out[i,:] = sum_{c<4} w[i,c] * table[index[i,c],:]
//
// Work of vggt_omega/models/token_merging.py:387-414 (WeightedBilinearTokenPlan.
// restore: `parent = value[:, parent]; (parent * w.to(value.dtype)).sum(2)`) and
// :193-196 (TokenPlan.restore, the one-hot case).  The reference materialises
// [M,4,C] and sums it; here one wave streams one output row: its four gathers
// are issued back to back (16 B per lane each), products are rounded to the
// value type exactly as the reference's elementwise multiply does, summed in
// fp32, and the row is written with non-temporal stores so the gathered table
// keeps the L2/MALL.  HBM-bound: per output row it moves dim*s bytes of output
// plus the 32 bytes of (index, weight); the table is compulsory traffic once.
#include "vgo_common.h"

namespace vgo {
namespace {

constexpr int kWaves = 4;  // waves per work-group; one output row per wave

template <typename T>
struct Vec16;  // 16 bytes of T
template <>
struct Vec16<float> {
  typedef f32x4 type;
  static constexpr int n = 4;
};
template <>
struct Vec16<bf16_t> {
  typedef bf16x8 type;
  static constexpr int n = 8;
};
template <>
struct Vec16<f16_t> {
  typedef f16x8 type;
  static constexpr int n = 8;
};


// Persistent waves: each wave owns R consecutive output rows per step and issues
// the gathers of all R rows (4 corners x CH 16-byte chunks per lane each) before
// reducing any of them, so a CU keeps hundreds of KB of gathers in flight.
//
// kRowSums (the gather probe, vgo_top4_gather_probe): the same gathers and
// arithmetic, but each row's output values are summed in fp32 (per lane, then over
// the wave) and only that sum is written, to row_sums[row]: the kernel's reads
// without its 2 GB of row writes, for measuring what the fabric gives the reads.
template <typename T, int R, int CH, bool kRowSums = false>
__global__ __launch_bounds__(kWaves * 64) void top4_project_kernel(
    const T* __restrict__ table, int64_t table_stride, const int32_t* __restrict__ index,
    const float* __restrict__ weight, const int32_t* __restrict__ order, T* __restrict__ out,
    int64_t out_stride, int64_t n_rows, int64_t table_rows, int dim, float* __restrict__ row_sums = nullptr) {
  typedef typename Vec16<T>::type V;
  constexpr int VN = Vec16<T>::n;
  const int lane = lane_id();
  const int64_t wave_gid = __builtin_amdgcn_readfirstlane(
      static_cast<int>(blockIdx.x) * kWaves + static_cast<int>(threadIdx.x >> 6));
  const int64_t step = static_cast<int64_t>(gridDim.x) * kWaves * R;

  for (int64_t r0 = wave_gid * R; r0 < n_rows; r0 += step) {
    int32_t id[R][4];
    float wq[R][4];
    bool use[R][4];
    bool bad[R];
    // Output row of each work position: the position itself, or order[position]
    // (positions whose order entry is out of range produce nothing).
    int64_t orow[R];
#pragma unroll
    for (int rr = 0; rr < R; ++rr) {
      const int64_t pos = r0 + rr;
      int64_t row = pos < n_rows ? pos : -1;
      if (order && row >= 0) {
        const int32_t o = order[pos];
        row = o >= 0 && o < n_rows ? o : -1;
      }
      orow[rr] = row;
    }
#pragma unroll
    for (int rr = 0; rr < R; ++rr) {
      const int64_t row = orow[rr];
      bad[rr] = false;
      i32x4 id4 = {0, 0, 0, 0};
      f32x4 w4 = {0.0f, 0.0f, 0.0f, 0.0f};
      if (row >= 0) {
        id4 = *reinterpret_cast<const i32x4*>(index + 4 * row);
        w4 = *reinterpret_cast<const f32x4*>(weight + 4 * row);
      }
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        id[rr][c] = id4[c];
        use[rr][c] = w4[c] != 0.0f;
        if (use[rr][c] && static_cast<uint32_t>(id4[c]) >= static_cast<uint64_t>(table_rows)) {
          bad[rr] = true;
          use[rr][c] = false;
        }
        wq[rr][c] = weight_as_value<T>(w4[c]);
      }
    }

    float lane_sum[R];
#pragma unroll
    for (int rr = 0; rr < R; ++rr) lane_sum[rr] = 0.0f;
    for (int base = 0; base < dim; base += CH * 64 * VN) {
      V y[R][4][CH];
#pragma unroll
      for (int rr = 0; rr < R; ++rr) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          if (use[rr][c]) {
            const T* trow = table + static_cast<int64_t>(id[rr][c]) * table_stride;
#pragma unroll
            for (int ch = 0; ch < CH; ++ch) {
              const int e = base + (ch * 64 + lane) * VN;
              if (e < dim) y[rr][c][ch] = *reinterpret_cast<const V*>(trow + e);
            }
          }
        }
      }
#pragma unroll
      for (int rr = 0; rr < R; ++rr) {
        const int64_t row = orow[rr];
        if (row < 0) continue;
        T* o_row = out + row * out_stride;
#pragma unroll
        for (int ch = 0; ch < CH; ++ch) {
          const int e = base + (ch * 64 + lane) * VN;
          if (e >= dim) continue;
          float acc[VN];
#pragma unroll
          for (int j = 0; j < VN; ++j) acc[j] = 0.0f;
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            if (use[rr][c]) {
#pragma unroll
              for (int j = 0; j < VN; ++j)
                acc[j] = acc[j] + rounded_product<T>(to_f32(y[rr][c][ch][j]), wq[rr][c]);
            }
          }
          V o;
#pragma unroll
          for (int j = 0; j < VN; ++j) o[j] = from_f32<T>(bad[rr] ? __builtin_nanf("") : acc[j]);
          if constexpr (kRowSums) {
#pragma unroll
            for (int j = 0; j < VN; ++j) lane_sum[rr] += to_f32(o[j]);
          } else {
            __builtin_nontemporal_store(o, reinterpret_cast<V*>(o_row + e));
          }
        }
      }
    }
    if constexpr (kRowSums) {
#pragma unroll
      for (int rr = 0; rr < R; ++rr) {
        float v = lane_sum[rr];
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
        if (lane == 0 && orow[rr] >= 0) row_sums[orow[rr]] = v;
      }
    }
  }
}

// Fallback for rows whose byte size is not a multiple of 16: one element per lane.
template <typename T>
__global__ __launch_bounds__(256) void top4_project_scalar_kernel(
    const T* __restrict__ table, int64_t table_stride, const int32_t* __restrict__ index,
    const float* __restrict__ weight, const int32_t* __restrict__ order, T* __restrict__ out,
    int64_t out_stride, int64_t n_rows, int64_t pos0, int64_t table_rows, int dim) {
  const int64_t pos = pos0 + blockIdx.y;
  const int e = blockIdx.x * 256 + threadIdx.x;
  if (pos >= n_rows || e >= dim) return;
  const int64_t row = order ? order[pos] : pos;
  if (row < 0 || row >= n_rows) return;
  float acc = 0.0f;
  bool bad = false;
  for (int c = 0; c < 4; ++c) {
    const float w = weight[4 * row + c];
    if (w == 0.0f) continue;
    const int32_t id = index[4 * row + c];
    if (static_cast<uint32_t>(id) >= static_cast<uint64_t>(table_rows)) {
      bad = true;
      continue;
    }
    acc = acc + (rounded_product<T>(to_f32(table[id * table_stride + e]),
                                            weight_as_value<T>(w)));
  }
  out[row * out_stride + e] = from_f32<T>(bad ? __builtin_nanf("") : acc);
}

template <typename T, int R, int CH>
void launch_vec(const T* tb, int64_t table_stride, const int32_t* index, const float* weight,
                const int32_t* order, T* ob, int64_t out_stride, int64_t n_rows, int64_t table_rows,
                int dim, int64_t blocks, hipStream_t stream, float* row_sums) {
  if (row_sums)
    hipLaunchKernelGGL((top4_project_kernel<T, R, CH, true>), dim3(static_cast<unsigned>(blocks)),
                       dim3(kWaves * 64), 0, stream, tb, table_stride, index, weight, order, ob,
                       out_stride, n_rows, table_rows, dim, row_sums);
  else
    hipLaunchKernelGGL((top4_project_kernel<T, R, CH>), dim3(static_cast<unsigned>(blocks)),
                       dim3(kWaves * 64), 0, stream, tb, table_stride, index, weight, order, ob,
                       out_stride, n_rows, table_rows, dim, nullptr);
}

// Work-groups resident per CU for the persistent launch (MI355X: 256 CUs).
constexpr int64_t kProjectBlocksPerCu = 8;

int device_cus() {
  static thread_local int cached = 0;
  if (cached > 0) return cached;
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus <= 0)
    cus = 256;
  cached = cus;
  return cached;
}

template <typename T>
int launch_project(const void* table, int64_t table_stride, const int32_t* index,
                   const float* weight, const int32_t* order, void* out, int64_t out_stride,
                   int64_t n_rows, int64_t table_rows, int64_t dim, hipStream_t stream,
                   float* row_sums = nullptr) {
  const T* tb = static_cast<const T*>(table);
  T* ob = static_cast<T*>(out);
  constexpr int VN = Vec16<T>::n;
  const bool vec_ok = (dim % VN == 0) && (table_stride % VN == 0) && (out_stride % VN == 0) &&
                      aligned(table, 16) && aligned(out, 16);
  if (vec_ok) {
    // 16-byte chunks per row per lane, and how many rows a wave gathers at once
    // (about 32 chunks = 512 B in flight per lane).
    const int row_chunks = static_cast<int>((dim + 64 * VN - 1) / (64 * VN));
    const int d = static_cast<int>(dim);
    const int64_t cap = static_cast<int64_t>(device_cus()) * kProjectBlocksPerCu;
    auto blocks_for = [&](int rows_per_wave) {
      const int64_t need = (n_rows + kWaves * rows_per_wave - 1) / (kWaves * rows_per_wave);
      return need < cap ? need : cap;
    };
    if (row_chunks >= 4) {
      launch_vec<T, 2, 4>(tb, table_stride, index, weight, order, ob, out_stride, n_rows, table_rows, d,
                          blocks_for(2), stream, row_sums);
    } else if (row_chunks >= 2) {
      launch_vec<T, 4, 2>(tb, table_stride, index, weight, order, ob, out_stride, n_rows, table_rows, d,
                          blocks_for(4), stream, row_sums);
    } else {
      launch_vec<T, 8, 1>(tb, table_stride, index, weight, order, ob, out_stride, n_rows, table_rows, d,
                          blocks_for(8), stream, row_sums);
    }
  } else {
    if (row_sums) return fail(VGO_EUNSUPPORTED, "top4_gather_probe: rows must be whole 16-byte chunks");
    dim3 grid(static_cast<unsigned>((dim + 255) / 256), 1, 1);
    // Rows go on grid.y in slabs of 65535 (the y limit).
    for (int64_t r0 = 0; r0 < n_rows; r0 += 65535) {
      const int64_t nr = (n_rows - r0) < 65535 ? (n_rows - r0) : 65535;
      grid.y = static_cast<unsigned>(nr);
      hipLaunchKernelGGL((top4_project_scalar_kernel<T>), grid, dim3(256), 0, stream, tb,
                         table_stride, index, weight, order, ob, out_stride, n_rows, r0, table_rows,
                         static_cast<int>(dim));
    }
  }
  return check_launch("top4_project");
}

}  // namespace
}  // namespace vgo

namespace {
int project_entry(const void* table, int64_t table_row_stride, const int32_t* index,
                  const float* weight, const int32_t* order, void* out, int64_t out_row_stride,
                  int64_t n_rows, int64_t table_rows, int64_t dim, int dtype, void* stream) {
  using namespace vgo;
  VGO_REQUIRE(n_rows >= 0 && table_rows >= 0 && dim >= 0, "top4_project: negative size");
  if (n_rows == 0 || dim == 0) return VGO_OK;
  VGO_REQUIRE(index && weight && out, "top4_project: null pointer");
  VGO_REQUIRE(table || table_rows == 0, "top4_project: null table");
  VGO_REQUIRE(dim <= 0x7fffffff && n_rows <= 0x7fffffff, "top4_project: size too large");
  VGO_REQUIRE(table_row_stride >= dim && out_row_stride >= dim, "top4_project: row stride < dim");
  VGO_REQUIRE(aligned(index, 16) && aligned(weight, 16),
              "top4_project: index/weight must be 16-byte aligned [n,4] arrays");
  hipStream_t s = as_stream(stream);
  switch (dtype) {
    case VGO_F32:
      return launch_project<float>(table, table_row_stride, index, weight, order, out, out_row_stride,
                                   n_rows, table_rows, dim, s);
    case VGO_BF16:
      return launch_project<bf16_t>(table, table_row_stride, index, weight, order, out, out_row_stride,
                                    n_rows, table_rows, dim, s);
    case VGO_F16:
      return launch_project<f16_t>(table, table_row_stride, index, weight, order, out, out_row_stride,
                                   n_rows, table_rows, dim, s);
    default:
      return fail(VGO_EINVAL, "top4_project: unknown dtype");
  }
}
}  // namespace

extern "C" int vgo_top4_project(const void* table, int64_t table_row_stride, const int32_t* index,
                                const float* weight, void* out, int64_t out_row_stride,
                                int64_t n_rows, int64_t table_rows, int64_t dim, int dtype,
                                void* stream) {
  return project_entry(table, table_row_stride, index, weight, nullptr, out, out_row_stride, n_rows,
                       table_rows, dim, dtype, stream);
}

extern "C" int vgo_top4_gather_probe(const void* table, int64_t table_row_stride,
                                     const int32_t* index, const float* weight, float* row_sums,
                                     int64_t n_rows, int64_t table_rows, int64_t dim, int dtype,
                                     void* stream) {
  using namespace vgo;
  VGO_REQUIRE(n_rows >= 0 && table_rows >= 0 && dim >= 0, "top4_gather_probe: negative size");
  if (n_rows == 0 || dim == 0) return VGO_OK;
  VGO_REQUIRE(table && index && weight && row_sums, "top4_gather_probe: null pointer");
  VGO_REQUIRE(dim <= 0x7fffffff && n_rows <= 0x7fffffff && table_row_stride >= dim,
              "top4_gather_probe: bad size or stride");
  VGO_REQUIRE(aligned(index, 16) && aligned(weight, 16),
              "top4_gather_probe: index/weight must be 16-byte aligned [n,4] arrays");
  hipStream_t s = as_stream(stream);
  switch (dtype) {
    case VGO_F32:
      return launch_project<float>(table, table_row_stride, index, weight, nullptr, nullptr, dim, n_rows,
                                   table_rows, dim, s, row_sums);
    case VGO_BF16:
      return launch_project<bf16_t>(table, table_row_stride, index, weight, nullptr, nullptr, dim, n_rows,
                                    table_rows, dim, s, row_sums);
    case VGO_F16:
      return launch_project<f16_t>(table, table_row_stride, index, weight, nullptr, nullptr, dim, n_rows,
                                   table_rows, dim, s, row_sums);
    default:
      return fail(VGO_EINVAL, "top4_gather_probe: unknown dtype");
  }
}

extern "C" int vgo_top4_project_ordered(const void* table, int64_t table_row_stride,
                                        const int32_t* index, const float* weight,
                                        const int32_t* order, void* out, int64_t out_row_stride,
                                        int64_t n_rows, int64_t table_rows, int64_t dim, int dtype,
                                        void* stream) {
  using namespace vgo;
  VGO_REQUIRE(order || n_rows == 0, "top4_project_ordered: null order");
  return project_entry(table, table_row_stride, index, weight, order, out, out_row_stride, n_rows,
                       table_rows, dim, dtype, stream);
}
