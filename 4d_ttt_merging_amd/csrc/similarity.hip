// Cosine-similarity matching with a per-row top-K epilogue (K = 1 or 4):
//   score[i, j] = bf16( src[i] . dict[j] )       (fp32 MFMA accumulation, one rounding)
//   out[i]      = the K largest (score, -j) over j, i.e. ties go to the lower j.
//
// Work of the FastVGGT match loop `bmm(src, dst^T).max(-1)` in
// vggt_omega/models/token_merging.py:1106-1111 (K = 1) and of the sparse-convex
// local/global `(src @ dict^T).topk(4)` in vggt_omega/models/sparse_convex.py:
// 2402-2404, 2430, whose rounding contract is spelled out by the Triton
// `_streaming_top4_kernel` (vggt_omega/models/sparse_convex_kernels.py:20-93):
// the fp32 dot product is rounded once to bf16 before ranking, and an equal
// score never displaces an earlier dictionary entry.
//
// The score matrix is never materialised.  A work-group computes 128 dict x 128
// source scores per step on v_mfma_f32_32x32x16_bf16 with both operands staged
// through LDS in 64-wide K chunks; the accumulators are laid out transposed
// (lane = source row, registers = dictionary rows) so each lane folds its 16
// scores per tile into a register-resident top-K of packed 64-bit keys
// (orderable bf16 score << 32 | ~j).  Work-groups split the dictionary into
// `parts`; a second kernel merges the per-part lists.  Keys make the result
// independent of evaluation order, so it is deterministic.
#include "vgo_common.h"

namespace vgo {
namespace {

constexpr int kTile = 128;       // dictionary rows and source rows per work-group step
constexpr int kKc = 64;          // K chunk staged in LDS
constexpr int kRowE = kKc + 8;   // padded LDS row (elements)

__device__ __forceinline__ uint32_t bf16_bits(float x) {
  const bf16_t b = static_cast<bf16_t>(x);
  return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, b));
}

// Monotone map of bf16 bit patterns to unsigned order; -0 is folded onto +0.
__device__ __forceinline__ uint32_t ord16(uint32_t b) {
  if (b == 0x8000u) b = 0;
  return (b & 0x8000u) ? (~b & 0xFFFFu) : (b | 0x8000u);
}
__host__ __device__ __forceinline__ uint32_t unord16(uint32_t o) {
  return (o & 0x8000u) ? (o & 0x7FFFu) : (~o & 0xFFFFu);
}

__device__ __forceinline__ uint64_t make_key(float score, int j) {
  return (static_cast<uint64_t>(ord16(bf16_bits(score))) << 32) |
         static_cast<uint64_t>(0xFFFFFFFFu - static_cast<uint32_t>(j));
}

template <int K>
struct TopK {
  uint64_t k[K];
  __device__ __forceinline__ void init() {
#pragma unroll
    for (int i = 0; i < K; ++i) k[i] = 0;
  }
  // Keeps k[] sorted descending; a key equal to one already held is dropped.
  __device__ __forceinline__ void insert(uint64_t key) {
    if (key <= k[K - 1]) return;
    uint64_t x = key;
#pragma unroll
    for (int i = 0; i < K; ++i) {
      const uint64_t hi = x > k[i] ? x : k[i];
      const uint64_t lo = x > k[i] ? k[i] : x;
      k[i] = hi;
      x = lo;
    }
  }
};

template <int K>
__global__ __launch_bounds__(256, 2) void sim_topk_kernel(
    const bf16_t* __restrict__ src, int64_t src_stride, int64_t src_capacity,
    const int64_t* __restrict__ src_rows, const int* __restrict__ n_src_dev, int n_src,
    const bf16_t* __restrict__ dict,
    int64_t dict_stride, int n0, int off1, int n_dict, int dim, int tiles_per_part,
    uint64_t* __restrict__ partial, int parts, bf16_t* __restrict__ scores,
    int64_t scores_stride) {
  __shared__ __attribute__((aligned(16))) bf16_t a_lds[kTile * kRowE];  // dictionary chunk
  __shared__ __attribute__((aligned(16))) bf16_t b_lds[kTile * kRowE];  // source chunk

  int ns = n_src;
  if (n_src_dev) ns = min(ns, *n_src_dev);
  const int s0 = blockIdx.x * kTile;
  if (s0 >= ns) return;
  const int part = blockIdx.y;
  const int d_begin = part * tiles_per_part * kTile;
  const int d_end = min(n_dict, d_begin + tiles_per_part * kTile);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wd = wave & 1;   // dictionary half of the tile
  const int ws = wave >> 1;  // source half of the tile
  const int l32 = lane & 31;
  const int hh = lane >> 5;
  const bf16x8 zero8 = {};

  // Staging: rows (tid>>3) + 32p, 8 columns at (tid&7)*8, for both operands.
  const int st_row = tid >> 3;
  const int st_col = (tid & 7) * 8;
  int64_t src_off[4];
  bool src_ok[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const int i = s0 + st_row + 32 * p;
    int64_t row = i < ns ? (src_rows ? src_rows[i] : i) : -1;
    src_ok[p] = row >= 0 && row < src_capacity;  // an invalid row id reads as zeros
    src_off[p] = (src_ok[p] ? row : 0) * src_stride;
  }

  TopK<K> best[2];
  best[0].init();
  best[1].init();

  for (int d0 = d_begin; d0 < d_end; d0 += kTile) {
    int64_t dict_off[4];
    bool dict_ok[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int j = d0 + st_row + 32 * p;
      dict_ok[p] = j < d_end;
      const int row = j < n0 ? j : off1 + (j - n0);
      dict_off[p] = static_cast<int64_t>(dict_ok[p] ? row : 0) * dict_stride;
    }
    f32x16 acc[2][2];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.0f;

    for (int kc = 0; kc < dim; kc += kKc) {
      const bool col_ok = kc + st_col < dim;
      bf16x8 av[4], bv[4];
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        av[p] = (dict_ok[p] && col_ok)
                    ? *reinterpret_cast<const bf16x8*>(dict + dict_off[p] + kc + st_col)
                    : zero8;
        bv[p] = (src_ok[p] && col_ok)
                    ? *reinterpret_cast<const bf16x8*>(src + src_off[p] + kc + st_col)
                    : zero8;
      }
      __syncthreads();
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        *reinterpret_cast<bf16x8*>(&a_lds[(st_row + 32 * p) * kRowE + st_col]) = av[p];
        *reinterpret_cast<bf16x8*>(&b_lds[(st_row + 32 * p) * kRowE + st_col]) = bv[p];
      }
      __syncthreads();
#pragma unroll
      for (int t = 0; t < kKc / 16; ++t) {
        bf16x8 a[2], b[2];
#pragma unroll
        for (int x = 0; x < 2; ++x) {
          a[x] = *reinterpret_cast<const bf16x8*>(
              &a_lds[(64 * wd + 32 * x + l32) * kRowE + 16 * t + 8 * hh]);
          b[x] = *reinterpret_cast<const bf16x8*>(
              &b_lds[(64 * ws + 32 * x + l32) * kRowE + 16 * t + 8 * hh]);
        }
#pragma unroll
        for (int x = 0; x < 2; ++x)
#pragma unroll
          for (int y = 0; y < 2; ++y)
            acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[x], b[y], acc[x][y], 0, 0, 0);
      }
    }

    // Epilogue: lane = source (64*ws + 32*sb + l32), registers = dictionary rows.
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
      const int i = s0 + 64 * ws + 32 * sb + l32;
#pragma unroll
      for (int db = 0; db < 2; ++db) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int j = d0 + 64 * wd + 32 * db + 8 * (r >> 2) + 4 * hh + (r & 3);
          if (j < d_end) {
            best[sb].insert(make_key(acc[db][sb][r], j));
            if (scores && i < ns)
              scores[static_cast<int64_t>(i) * scores_stride + j] = static_cast<bf16_t>(acc[db][sb][r]);
          }
        }
      }
    }
  }

  // Merge the four lists of every source row (two dictionary halves x two lane halves).
  __syncthreads();
  uint64_t* m_lds = reinterpret_cast<uint64_t*>(a_lds);  // [128 sources][4 lists][K]
#pragma unroll
  for (int sb = 0; sb < 2; ++sb) {
    const int local = 64 * ws + 32 * sb + l32;
#pragma unroll
    for (int t = 0; t < K; ++t) m_lds[(local * 4 + wd * 2 + hh) * K + t] = best[sb].k[t];
  }
  __syncthreads();
  if (tid < kTile) {
    const int i = s0 + tid;
    if (i < ns) {
      TopK<K> m;
      m.init();
#pragma unroll
      for (int l = 0; l < 4; ++l)
#pragma unroll
        for (int t = 0; t < K; ++t) m.insert(m_lds[(tid * 4 + l) * K + t]);
      uint64_t* out = partial + (static_cast<int64_t>(i) * parts + part) * K;
#pragma unroll
      for (int t = 0; t < K; ++t) out[t] = m.k[t];
    }
  }
}

// Merge `parts` partial lists per source row; decode keys into the bf16 score
// (as fp32) and the dictionary row (optionally mapped through index_map).
template <int K>
__global__ __launch_bounds__(256) void topk_finalize_kernel(
    const uint64_t* __restrict__ partial, int n_src, const int* __restrict__ n_src_dev, int parts,
    int n0, int off1, float* __restrict__ values, int64_t* __restrict__ index64,
    int32_t* __restrict__ index32, const int64_t* __restrict__ index_map) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  int ns = n_src;
  if (n_src_dev) ns = min(ns, *n_src_dev);
  if (i >= ns) return;
  TopK<K> m;
  m.init();
  const uint64_t* p = partial + static_cast<int64_t>(i) * parts * K;
  for (int q = 0; q < parts * K; ++q) m.insert(p[q]);
#pragma unroll
  for (int t = 0; t < K; ++t) {
    const uint64_t key = m.k[t];
    float v = -__builtin_inff();
    int64_t j = -1;
    if (key != 0) {
      const uint32_t bits = unord16(static_cast<uint32_t>(key >> 32));
      v = __builtin_bit_cast(float, bits << 16);
      j = static_cast<int64_t>(0xFFFFFFFFu - static_cast<uint32_t>(key & 0xFFFFFFFFu));
      j = j < n0 ? j : off1 + (j - n0);  // dictionary position -> dictionary row
      if (index_map) j = index_map[j];
    }
    if (values) values[static_cast<int64_t>(i) * K + t] = v;
    if (index64) index64[static_cast<int64_t>(i) * K + t] = j;
    if (index32) index32[static_cast<int64_t>(i) * K + t] = static_cast<int32_t>(j);
  }
}

int choose_parts(int64_t n_src, int64_t n_dict) {
  const int64_t src_tiles = (n_src + kTile - 1) / kTile;
  const int64_t dict_tiles = (n_dict + kTile - 1) / kTile;
  // Aim for about 1024 work-groups (4 per CU) without splitting below one tile.
  int64_t parts = (1024 + src_tiles - 1) / (src_tiles > 0 ? src_tiles : 1);
  if (parts > dict_tiles) parts = dict_tiles;
  if (parts < 1) parts = 1;
  return static_cast<int>(parts);
}

}  // namespace
}  // namespace vgo

extern "C" int vgo_similarity_topk_workspace(int64_t n_src, int64_t n_dict, int topk, int* parts,
                                             size_t* bytes) {
  using namespace vgo;
  VGO_REQUIRE(topk == 1 || topk == 4, "similarity_topk: topk must be 1 or 4");
  VGO_REQUIRE(n_src >= 0 && n_dict >= 0, "similarity_topk: negative size");
  const int p = choose_parts(n_src, n_dict);
  if (parts) *parts = p;
  if (bytes) *bytes = static_cast<size_t>(n_src) * p * topk * sizeof(uint64_t);
  return VGO_OK;
}

extern "C" int vgo_similarity_topk(const void* src, int64_t src_row_stride, int64_t src_capacity,
                                   const int64_t* src_rows, const int* n_src_device, int64_t n_src,
                                   const void* dict, int64_t dict_row_stride, int64_t dict_capacity,
                                   int64_t dict_n0, int64_t dict_off1, int64_t n_dict, int64_t dim, int topk, void* workspace,
                                   size_t workspace_bytes, float* values, int64_t* index64,
                                   int32_t* index32, const int64_t* index_map, void* scores,
                                   int64_t scores_row_stride, void* stream) {
  using namespace vgo;
  VGO_REQUIRE(topk == 1 || topk == 4, "similarity_topk: topk must be 1 or 4");
  VGO_REQUIRE(n_src >= 0 && n_dict >= 0 && dim > 0, "similarity_topk: bad size");
  if (n_src == 0) return VGO_OK;
  VGO_REQUIRE(n_dict >= topk, "similarity_topk: fewer dictionary rows than topk");
  VGO_REQUIRE(src && dict, "similarity_topk: null pointer");
  VGO_REQUIRE(dim % 8 == 0 && src_row_stride % 8 == 0 && dict_row_stride % 8 == 0,
              "similarity_topk: dim and row strides must be multiples of 8");
  VGO_REQUIRE(aligned(src, 16) && aligned(dict, 16), "similarity_topk: operands must be 16-byte aligned");
  VGO_REQUIRE(n_src < (1LL << 30) && n_dict < (1LL << 30) && dim < (1 << 20),
              "similarity_topk: size too large");
  VGO_REQUIRE(dict_n0 >= 0 && dict_n0 <= n_dict && dict_off1 >= 0 && dict_n0 <= dict_capacity &&
                  dict_off1 + (n_dict - dict_n0) <= dict_capacity,
              "similarity_topk: dictionary ranges exceed the dictionary");
  VGO_REQUIRE(src_rows || n_src <= src_capacity, "similarity_topk: more sources than rows");
  int parts = 0;
  size_t need = 0;
  vgo_similarity_topk_workspace(n_src, n_dict, topk, &parts, &need);
  VGO_REQUIRE(workspace && workspace_bytes >= need, "similarity_topk: workspace too small");
  VGO_REQUIRE(aligned(workspace, 8), "similarity_topk: workspace must be 8-byte aligned");
  const int64_t dict_tiles = (n_dict + kTile - 1) / kTile;
  const int tiles_per_part = static_cast<int>((dict_tiles + parts - 1) / parts);
  hipStream_t s = as_stream(stream);
  dim3 grid(static_cast<unsigned>((n_src + kTile - 1) / kTile), static_cast<unsigned>(parts));
  uint64_t* partial = static_cast<uint64_t*>(workspace);
  const bf16_t* sp = static_cast<const bf16_t*>(src);
  const bf16_t* dp = static_cast<const bf16_t*>(dict);
  bf16_t* sc = static_cast<bf16_t*>(scores);
  const int blocks2 = static_cast<int>((n_src + 255) / 256);
  if (topk == 1) {
    hipLaunchKernelGGL((sim_topk_kernel<1>), grid, dim3(256), 0, s, sp, src_row_stride, src_capacity, src_rows,
                       n_src_device, static_cast<int>(n_src), dp, dict_row_stride,
                       static_cast<int>(dict_n0), static_cast<int>(dict_off1),
                       static_cast<int>(n_dict), static_cast<int>(dim), tiles_per_part, partial,
                       parts, sc, scores_row_stride);
    hipLaunchKernelGGL((topk_finalize_kernel<1>), dim3(blocks2), dim3(256), 0, s, partial,
                       static_cast<int>(n_src), n_src_device, parts, static_cast<int>(dict_n0),
                       static_cast<int>(dict_off1), values, index64, index32, index_map);
  } else {
    hipLaunchKernelGGL((sim_topk_kernel<4>), grid, dim3(256), 0, s, sp, src_row_stride, src_capacity, src_rows,
                       n_src_device, static_cast<int>(n_src), dp, dict_row_stride,
                       static_cast<int>(dict_n0), static_cast<int>(dict_off1),
                       static_cast<int>(n_dict), static_cast<int>(dim), tiles_per_part, partial,
                       parts, sc, scores_row_stride);
    hipLaunchKernelGGL((topk_finalize_kernel<4>), dim3(blocks2), dim3(256), 0, s, partial,
                       static_cast<int>(n_src), n_src_device, parts, static_cast<int>(dict_n0),
                       static_cast<int>(dict_off1), values, index64, index32, index_map);
  }
  return check_launch("similarity_topk");
}
