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
// through double-buffered, XOR-swizzled LDS in 64-wide K chunks (the next
// chunk -- across dictionary tiles too -- is loaded into registers while the
// current one is multiplied; one barrier per chunk); the accumulators are laid out transposed
// (lane = source row, registers = dictionary rows) so each lane folds its 16
// scores per tile into a register-resident top-K of packed 64-bit keys
// (orderable bf16 score << 32 | ~j).  Work-groups split the dictionary into
// `parts`; a second kernel merges the per-part lists.  Keys make the result
// independent of evaluation order, so it is deterministic.
#include <algorithm>

#include "vgo_common.h"

namespace vgo {
namespace {

// Stream-K partition: work-group w of `groups` runs units [sk_begin(w), sk_begin(w + 1)).
__host__ __device__ __forceinline__ int64_t sk_begin(int64_t w, int64_t units, int64_t groups) {
  return w * units / groups;
}
// Work-group whose range holds unit u.
__host__ __device__ __forceinline__ int64_t sk_owner(int64_t u, int64_t units, int64_t groups) {
  return ((u + 1) * groups - 1) / units;
}

constexpr int kTile = 128;       // dictionary rows and source rows per work-group step
constexpr int kKc = 64;          // K chunk staged in LDS

__device__ __forceinline__ uint32_t bf16_bits(float x) {
  const bf16_t b = static_cast<bf16_t>(x);
  return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, b));
}

// Monotone map of bf16 bit patterns to unsigned order; -0 is folded onto +0
// and every NaN, whatever its sign (inf * 0 gives a negative one), onto the
// top, above +inf, as torch's descending sort ranks it.
__device__ __forceinline__ uint32_t ord16(uint32_t b) {
  if ((b & 0x7FFFu) > 0x7F80u) return 0xFFFFu;
  if (b == 0x8000u) b = 0;
  return (b & 0x8000u) ? (~b & 0xFFFFu) : (b | 0x8000u);
}
__host__ __device__ __forceinline__ uint32_t unord16(uint32_t o) {
  return (o & 0x8000u) ? (o & 0x7FFFu) : (~o & 0xFFFFu);
}

// fp32 value of x rounded to bf16 (round to nearest even, as the conversion).
__device__ __forceinline__ float bf16_round(float x) {
  return __builtin_bit_cast(float, bf16_bits(x) << 16);
}

// Smallest fp32 x whose bf16 rounding equals t (a bf16 value held in fp32, not
// NaN).  Rounding is to nearest even, so the midpoint below t belongs to t when
// t's last bf16 mantissa bit is 0.  Both zeros share the interval of -0 and +0;
// -inf is its own bound.  Rounding is monotone, so among values that are at
// most m, x rounds to bf16(m) exactly when x >= bf16_lower_bound(bf16(m)).
__device__ __forceinline__ float bf16_lower_bound(float t) {
  if (t == -__builtin_inff()) return t;
  const uint32_t b = __builtin_bit_cast(uint32_t, t);
  const uint32_t mag = b & 0x7FFFFFFFu;
  const uint32_t lsb = (mag >> 16) & 1u;
  if ((b >> 31) == 0u && mag != 0u) return __builtin_bit_cast(float, mag - 0x8000u + lsb);
  return __builtin_bit_cast(float, 0x80000000u | (mag + 0x8000u - lsb));
}

__device__ __forceinline__ uint64_t make_key(float score, int j) {
  return (static_cast<uint64_t>(ord16(bf16_bits(score))) << 32) |
         static_cast<uint64_t>(0xFFFFFFFFu - static_cast<uint32_t>(j));
}

// Key of a score at position pos (< 0x10000) of a lane's dictionary tile, for
// a score that is not NaN: ord16 of its bf16 rounding t in the high half (t
// with the sign bit set for t >= 0, which also folds -0 onto +0; t with its
// upper 16 bits inverted for t < 0) and 0xFFFF - pos in the low half.
__device__ __forceinline__ uint32_t tile_key(float score, int pos) {
  const float t = bf16_round(score);
  const uint32_t k = __builtin_bit_cast(uint32_t, t) | (0x80000000u | (0xFFFFu - static_cast<uint32_t>(pos)));
  return t < 0.0f ? k ^ 0xFFFF0000u : k;
}
// The make_key() key of a tile key whose lane's tile starts at row j0.
__device__ __forceinline__ uint64_t tile_key_to_key(uint32_t k, int j0) {
  const uint32_t j = static_cast<uint32_t>(j0) + (0xFFFFu - (k & 0xFFFFu));
  return (static_cast<uint64_t>(k >> 16) << 32) | static_cast<uint64_t>(0xFFFFFFFFu - j);
}
// Median of three unsigned integers (v_med3_u32; the compiler forms it from
// min/max only in some cases).
__device__ __forceinline__ uint32_t med3_u32(uint32_t a, uint32_t b, uint32_t c) {
  uint32_t d;
  asm("v_med3_u32 %0, %1, %2, %3" : "=v"(d) : "v"(a), "v"(b), "v"(c));
  return d;
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

// LDS operand tiles: 128 rows x 64 elements (128 B), no padding; the eight
// 16-byte chunks of a row are XOR-permuted by swz(row) so that the MFMA
// operand reads (eight consecutive rows at one logical chunk) and the staging
// stores (eight chunks of one row) fall in distinct banks.
__device__ __forceinline__ int swz(int row) { return (row & 7) ^ ((row >> 3) & 7); }
constexpr int kTileElems = kTile * kKc;

template <int K>
__global__ __launch_bounds__(256, 2) void sim_topk_kernel(
    const bf16_t* __restrict__ src, int64_t src_stride, int64_t src_capacity,
    const int64_t* __restrict__ src_rows, const int* __restrict__ n_src_dev, int n_src,
    const bf16_t* __restrict__ dict,
    int64_t dict_stride, int n0, int off1, int n_dict, int dim, int tiles_per_part,
    uint64_t* __restrict__ partial, int parts, bf16_t* __restrict__ scores,
    int64_t scores_stride) {
  // Double-buffered dictionary (a) and source (b) chunks.
  __shared__ __attribute__((aligned(16))) bf16_t a_lds[2 * kTileElems];
  __shared__ __attribute__((aligned(16))) bf16_t b_lds[2 * kTileElems];

  int ns = n_src;
  if (n_src_dev) ns = min(ns, *n_src_dev);
  // 1-D grid, dictionary part fastest, XCD-remapped: the work-groups resident
  // on one XCD at a time cover a few source tiles (kept in its L2 across their
  // dictionary tiles) against all dictionary parts.
  const int task = xcd_remap(blockIdx.x, gridDim.x);
  const int s0 = (task / parts) * kTile;
  if (s0 >= ns) return;
  const int part = task % parts;
  const int d_begin = part * tiles_per_part * kTile;
  const int d_end = min(n_dict, d_begin + tiles_per_part * kTile);  // may be empty: lists stay empty

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wd = wave & 1;   // dictionary half of the tile
  const int ws = wave >> 1;  // source half of the tile
  const int l32 = lane & 31;
  const int hh = lane >> 5;
  const bf16x8 zero8 = {};

  // Staging: rows st + 32p (p = 0..3), chunk sc of the 64-wide K chunk, both operands.
  const int st = tid >> 3;
  const int sc = tid & 7;
  int wr[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) wr[p] = (st + 32 * p) * kKc + ((sc ^ swz(st + 32 * p)) << 3);
  const bf16_t* src_ptr[4];
  bool src_ok[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const int i = s0 + st + 32 * p;
    const int64_t row = i < ns ? (src_rows ? src_rows[i] : i) : -1;
    src_ok[p] = row >= 0 && row < src_capacity;  // an invalid row id reads as zeros
    src_ptr[p] = src + (src_ok[p] ? row : 0) * src_stride + 8 * sc;
  }
  // Operand read offsets: row (x*32 + l32) of a 64-row half, logical chunk 2t+hh;
  // x = 1 uses off[t ^ 2] (swz flips bit 2 of the chunk there).
  int off[4];
  {
    const int s0w = swz(l32);
#pragma unroll
    for (int t = 0; t < 4; ++t) off[t] = l32 * kKc + (((2 * t + hh) ^ s0w) << 3);
  }

  const int n_chunks = (dim + kKc - 1) / kKc;
  const int n_dtiles = d_end > d_begin ? (d_end - d_begin + kTile - 1) / kTile : 0;

  // Global -> register staging.  Row pointers of the dictionary tile being
  // loaded are set once per tile; a chunk only adds its column offset.  Rows
  // and columns past the ends read a valid address and are zeroed when the
  // registers are stored to LDS, so the loads stay in flight across the MFMAs
  // of the current chunk.
  bf16x8 ga[4], gb[4];
  const bf16_t* dptr[4];
  unsigned row_mask = 0;  // bit p: dictionary row valid; bit 4+p: source row valid
  unsigned ok_mask = 0;   // row_mask of the loaded chunk, columns included
  int ld_dt = 0, ld_kc = 0;
  auto set_dtile = [&](int dt) {
    row_mask &= 0xF0u;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int jj = d_begin + dt * kTile + st + 32 * p;
      const bool ok = jj < d_end;
      const int row = jj < n0 ? jj : off1 + (jj - n0);
      dptr[p] = dict + static_cast<int64_t>(ok ? row : 0) * dict_stride + 8 * sc;
      row_mask |= (ok ? 1u : 0u) << p;
    }
  };
#pragma unroll
  for (int p = 0; p < 4; ++p) row_mask |= (src_ok[p] ? 1u : 0u) << (4 + p);
  set_dtile(0);
  auto load = [&]() {
    const int kc = ld_kc * kKc;
    const bool col_ok = kc + 8 * sc < dim;
    const int col = col_ok ? kc : 0;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      ga[p] = *reinterpret_cast<const bf16x8*>(dptr[p] + col);
      gb[p] = *reinterpret_cast<const bf16x8*>(src_ptr[p] + col);
    }
    ok_mask = col_ok ? row_mask : 0u;
    if (++ld_kc == n_chunks) {
      ld_kc = 0;
      if (++ld_dt < n_dtiles) set_dtile(ld_dt);
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      *reinterpret_cast<bf16x8*>(&a_lds[buf * kTileElems + wr[p]]) = (ok_mask >> p) & 1u ? ga[p] : zero8;
      *reinterpret_cast<bf16x8*>(&b_lds[buf * kTileElems + wr[p]]) = (ok_mask >> (4 + p)) & 1u ? gb[p] : zero8;
    }
  };

  TopK<K> best[2];
  best[0].init();
  best[1].init();
  float top_v[2] = {-__builtin_inff(), -__builtin_inff()};  // K == 1 running best
  int top_j[2] = {-1, -1};
  f32x16 acc[2][2];
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int y = 0; y < 2; ++y) acc[x][y] = f32x16{};

  const int n_steps = n_dtiles * n_chunks;
  load();
  store(0);
  __syncthreads();
  int dt = 0, kcs = 0;  // dictionary tile and K chunk of the step being computed
  for (int step = 0; step < n_steps; ++step) {
    const int buf = step & 1;
    const bool more = step + 1 < n_steps;
    if (more) load();
    const bf16_t* al = a_lds + buf * kTileElems + wd * 64 * kKc;
    const bf16_t* bl = b_lds + buf * kTileElems + ws * 64 * kKc;
    bf16x8 a[kKc / 16][2], b[kKc / 16][2];
#pragma unroll
    for (int t = 0; t < kKc / 16; ++t)
#pragma unroll
      for (int x = 0; x < 2; ++x) {
        a[t][x] = *reinterpret_cast<const bf16x8*>(al + x * 32 * kKc + off[t ^ (2 * x)]);
        b[t][x] = *reinterpret_cast<const bf16x8*>(bl + x * 32 * kKc + off[t ^ (2 * x)]);
      }
#pragma unroll
    for (int t = 0; t < kKc / 16; ++t)
#pragma unroll
      for (int x = 0; x < 2; ++x)
#pragma unroll
        for (int y = 0; y < 2; ++y)
          acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[t][x], b[t][y], acc[x][y], 0, 0, 0);
    if (kcs == n_chunks - 1) {
      // Epilogue of a dictionary tile: lane = source (64*ws + 32*sb + l32),
      // registers = dictionary rows in increasing order.
      const int d0 = d_begin + dt * kTile;
      if (scores) {
#pragma unroll
        for (int sb = 0; sb < 2; ++sb) {
          const int i = s0 + 64 * ws + 32 * sb + l32;
#pragma unroll
          for (int db = 0; db < 2; ++db)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int jj = d0 + 64 * wd + 32 * db + 8 * (r >> 2) + 4 * hh + (r & 3);
              if (jj < d_end && i < ns)
                scores[static_cast<int64_t>(i) * scores_stride + jj] = static_cast<bf16_t>(acc[db][sb][r]);
            }
        }
      }
      const int jl = d0 + 64 * wd + 4 * hh;  // this lane's first dictionary row
      if (K == 1) {
        // Running top-1 on the bf16-rounded score: a later (higher) j wins only
        // when strictly greater, which is the lower-index rule for ties; a NaN
        // wins over numbers and the first NaN is kept (ranking of the keys).
#pragma unroll
        for (int sb = 0; sb < 2; ++sb)
#pragma unroll
          for (int db = 0; db < 2; ++db)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int jj = jl + 32 * db + 8 * (r >> 2) + (r & 3);
              const float v = bf16_round(acc[db][sb][r]);
              const bool take = (jj < d_end) & ((v > top_v[sb]) | ((v != v) & (top_v[sb] == top_v[sb])));
              top_v[sb] = take ? v : top_v[sb];
              top_j[sb] = take ? jj : top_j[sb];
            }
      } else {
#pragma unroll
        for (int sb = 0; sb < 2; ++sb)
#pragma unroll
          for (int db = 0; db < 2; ++db)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int jj = jl + 32 * db + 8 * (r >> 2) + (r & 3);
              if (jj < d_end) best[sb].insert(make_key(acc[db][sb][r], jj));
            }
      }
#pragma unroll
      for (int sb = 0; sb < 2; ++sb)
#pragma unroll
        for (int db = 0; db < 2; ++db) acc[db][sb] = f32x16{};
      kcs = 0;
      ++dt;
    } else {
      ++kcs;
    }
    if (more) store(buf ^ 1);
    __syncthreads();
  }

  if (K == 1) {
#pragma unroll
    for (int sb = 0; sb < 2; ++sb)
      if (top_j[sb] >= 0) best[sb].k[0] = make_key(top_v[sb], top_j[sb]);
  }
  // Merge the four lists of every source row (two dictionary halves x two lane halves).
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

// ------------------------------------------------------ LDS-DMA ring ----
// Work-group tile 256 dictionary x 256 source rows, 8 waves of 128 x 64
// (four 32-row dictionary blocks by two 32-column source blocks, accumulators
// transposed as in the staged kernel), one work-group per CU.  A tile pair
// moves 1 MB for 134 MFLOP, twice the 128 x 128 tile's arithmetic per byte.
// Operands arrive by LDS DMA (global_load_lds_dwordx4) in 32-wide K chunks
// through a 5-stage ring (all 160 KB of the CU's LDS), up to four chunks
// ahead.  A step's first k-step operands are read from LDS during the
// previous step, its second k-step's during its first k-step's MFMAs, so the
// LDS reads (96 KB per step and CU) overlap the MFMAs instead of preceding
// them.  The CU's DMA path moves about 25 B per clock, a little slower than
// the MFMAs consume a step, and a DMA issue stalls its wave while that path
// is backed up; so the first k-step's MFMAs run before the step's barrier
// and the DMAs are issued between the second k-step's MFMAs, which keeps the
// matrix cores fed through barrier skew and issue stalls (with every wave
// issuing its DMAs right after the barrier, the transfer and the MFMAs
// mostly took turns).  LDS rows are 64 B; their four 16-byte chunks are
// XOR-permuted by sw4(row) = (row >> 2) & 3, so the operand reads (16 rows at
// one logical chunk per quarter-wave) are conflict-free.  Requires
// dim % 32 == 0.  Invalid source row ids read row 0 through the DMA and score
// 0 in the epilogue, as in the staged kernel.
//
// Two schedules.  kStreamK = false: work-group task t runs dictionary part
// t % parts (tiles_per_part tiles) of source tile t / parts and merges its four
// lists per source row through LDS into one.  kStreamK = true (top-1 without
// the score matrix): the `units` (source tile, dictionary tile) pairs, source
// tile major, are split evenly over the grid (stream-K: work-group w runs
// [sk_begin(w), sk_begin(w + 1))), so no round of the grid runs part-empty;
// the DMA ring runs on across source tiles, and at the end of its share of a
// source tile a work-group writes each lane's best key (four lists per source
// row) to slot w - (the tile's first owner) of `parts` slots, which
// topk_finalize_kernel merges.
constexpr int kRTile = 256;
constexpr int kRWaves = 8;
constexpr int kRKc = 32;
constexpr int kRStages = 5;                 // 5 x 32 KB: all of the CU's LDS
constexpr int kRAhead = kRStages - 1;       // steps in flight ahead of the one computed
constexpr int kRTileElems = kRTile * kRKc;
constexpr int kRDmaPerStep = 4;  // per wave: two 16-row blocks of each operand
__device__ __forceinline__ int sw4(int row) { return (row >> 2) & 3; }

template <int K, bool kStreamK>
__global__ __launch_bounds__(kRWaves * 64, 1) void sim_topk_ring_kernel(
    const bf16_t* __restrict__ src, int64_t src_stride, int64_t src_capacity,
    const int64_t* __restrict__ src_rows, const int* __restrict__ n_src_dev, int n_src,
    const bf16_t* __restrict__ dict,
    int64_t dict_stride, int n0, int off1, int n_dict, int dim, int tiles_per_part,
    uint64_t* __restrict__ partial, int parts, bf16_t* __restrict__ scores,
    int64_t scores_stride, int units) {
  static_assert(!kStreamK || K == 1, "the stream-K schedule is the top-1 kernel's");
  __shared__ __attribute__((aligned(16))) bf16_t a_lds[kRStages * kRTileElems];
  __shared__ __attribute__((aligned(16))) bf16_t b_lds[kRStages * kRTileElems];

  int ns = n_src;
  if (n_src_dev) ns = min(ns, *n_src_dev);
  const int task = xcd_remap(blockIdx.x, gridDim.x);
  // kStreamK: tiles_per_part is the dictionary's tile count; st_begin / dt_begin
  // are the first unit's tiles, slot_begin the first segment's slot (a later
  // segment starts its source tile, whose first owner is then this work-group).
  int s0, part, d_begin, d_end, st_begin = 0, dt_begin = 0, slot_begin = 0, n_units = 0;
  if constexpr (kStreamK) {
    const int u_begin = static_cast<int>(sk_begin(task, units, gridDim.x));
    n_units = static_cast<int>(sk_begin(task + 1, units, gridDim.x)) - u_begin;
    st_begin = u_begin / tiles_per_part;
    dt_begin = u_begin - st_begin * tiles_per_part;
    slot_begin = task - static_cast<int>(sk_owner(static_cast<int64_t>(st_begin) * tiles_per_part, units,
                                                   gridDim.x));
    s0 = st_begin * kRTile;
    part = 0;
    d_begin = 0;
    d_end = n_dict;
  } else {
    s0 = (task / parts) * kRTile;
    if (s0 >= ns) return;
    part = task % parts;
    d_begin = part * tiles_per_part * kRTile;
    d_end = min(n_dict, d_begin + tiles_per_part * kRTile);
  }

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wd = wave & 1;   // dictionary half (128 rows)
  const int ws = wave >> 1;  // source quarter (64 rows)
  const int l32 = lane & 31;
  const int hh = lane >> 5;

  // DMA lanes: a 1 KB block is 16 rows x 4 physical chunks; lane i fills row
  // i/4, physical chunk i%4 with logical chunk (i%4) ^ sw4(row).  This wave
  // loads rows 32*wave + 16*j + i/4 (j = 0, 1) of both operands.
  const int dr = lane >> 2;
  const int dpc = lane & 3;
  const bf16_t* src_p[2];
  auto set_stile = [&](int stile) {  // this wave's DMA rows of source tile stile
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int r = 32 * wave + 16 * j + dr;
      const int i = stile * kRTile + r;
      const int64_t row = i < ns ? (src_rows ? src_rows[i] : i) : 0;
      const bool ok = row >= 0 && row < src_capacity;
      src_p[j] = src + (ok ? row : 0) * src_stride + 8 * (dpc ^ sw4(r));
    }
  };
  set_stile(s0 / kRTile);
  // Epilogue sources of this lane (lane = source row): an invalid row id scores 0.
  bool src_ok[2];
  bool all_src_ok;
  auto set_epilogue_stile = [&](int stile) {
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
      const int i = stile * kRTile + 64 * ws + 32 * sb + l32;
      const int64_t row = i < ns ? (src_rows ? src_rows[i] : i) : 0;
      src_ok[sb] = row >= 0 && row < src_capacity;
    }
    all_src_ok = __ballot(!(src_ok[0] & src_ok[1])) == 0;
  };
  set_epilogue_stile(s0 / kRTile);

  const int n_chunks = dim / kRKc;
  const int n_dtiles = kStreamK ? n_units : d_end > d_begin ? (d_end - d_begin + kRTile - 1) / kRTile : 0;
  const int n_steps = n_dtiles * n_chunks;

  const bf16_t* dict_p[2] = {dict, dict};
  int cur_dt = -1;
  auto set_dtile = [&](int dt) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int r = 32 * wave + 16 * j + dr;
      const int jj = min(d_begin + dt * kRTile + r, d_end - 1);  // rows past the end repeat a valid row
      const int row = jj < n0 ? jj : off1 + (jj - n0);
      dict_p[j] = dict + static_cast<int64_t>(row) * dict_stride + 8 * (dpc ^ sw4(r));
    }
    cur_dt = dt;
  };
  // Issues the next step in order (iss_dt, iss_kc) into the next stage.  Past
  // the last step it re-issues the last one (valid rows, into a stage nobody
  // reads again): every call issues the same number of DMAs, which the
  // vmcnt waits below count on -- with fewer in flight, "at most N
  // outstanding" would no longer mean that the oldest step has landed.
  int iss_step = 0, iss_dt = dt_begin, iss_kc = 0, iss_stage = 0;
  int iss_st = st_begin;  // kStreamK: the issued step's source tile
  // DMA q (0..3) of the next step: block q >> 1 of the dictionary (q even) or
  // source (q odd) operand; the last one moves on to the following step.
  auto issue_one = [&](int q) {
    if (q == 0 && iss_dt != cur_dt) set_dtile(iss_dt);
    if constexpr (kStreamK)
      if (q == 0 && iss_dt == 0 && iss_kc == 0 && iss_step > 0) set_stile(iss_st);
    const int blk = (32 * wave + 16 * (q >> 1)) * kRKc;
    if ((q & 1) == 0)
      lds_dma16_addr(dict_p[q >> 1] + iss_kc, lds_offset(a_lds + iss_stage * kRTileElems + blk));
    else
      lds_dma16_addr(src_p[q >> 1] + iss_kc, lds_offset(b_lds + iss_stage * kRTileElems + blk));
    if (q == 3) {
      iss_stage = iss_stage == kRStages - 1 ? 0 : iss_stage + 1;
      if (++iss_step < n_steps) {
        iss_kc += kRKc;
        if (iss_kc == dim) {
          iss_kc = 0;
          ++iss_dt;
          if constexpr (kStreamK) {
            if (iss_dt == tiles_per_part) {
              iss_dt = 0;
              ++iss_st;
            }
          }
        }
      }
    }
  };
  auto issue_next = [&]() {
#pragma unroll
    for (int q = 0; q < 4; ++q) issue_one(q);
  };
  // Operand read offsets (elements) within a 32-row block: logical chunk 2t+hh
  // of row l32; sw4 of rows 32*x + l32 + base depends on l32 only.
  int off[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) off[t] = l32 * kRKc + (((2 * t + hh) ^ sw4(l32)) << 3);

  TopK<K> best[2];
  best[0].init();
  best[1].init();
  float top_v[2] = {-__builtin_inff(), -__builtin_inff()};
  int top_j[2] = {-1, -1};
  f32x16 acc[4][2];
#pragma unroll
  for (int x = 0; x < 4; ++x)
#pragma unroll
    for (int y = 0; y < 2; ++y) acc[x][y] = f32x16{};

  // Operands of one 16-wide k-step t of the step in stage `stg`: this wave's
  // 128 dictionary rows (4 blocks) and 64 source rows (2 blocks).
  auto read_half = [&](int stg, int t, bf16x8 (&a)[4], bf16x8 (&b)[2]) {
    const bf16_t* al = a_lds + stg * kRTileElems + wd * 128 * kRKc;
    const bf16_t* bl = b_lds + stg * kRTileElems + ws * 64 * kRKc;
#pragma unroll
    for (int x = 0; x < 4; ++x) a[x] = *reinterpret_cast<const bf16x8*>(al + x * 32 * kRKc + off[t]);
#pragma unroll
    for (int y = 0; y < 2; ++y) b[y] = *reinterpret_cast<const bf16x8*>(bl + y * 32 * kRKc + off[t]);
  };
  auto mma_half = [&](const bf16x8 (&a)[4], const bf16x8 (&b)[2]) {
#pragma unroll
    for (int x = 0; x < 4; ++x)
#pragma unroll
      for (int y = 0; y < 2; ++y)
        acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[x], b[y], acc[x][y], 0, 0, 0);
  };
  // k-step 0 operands of the current step (read a step ahead) and k-step 1
  // operands (read at the step's start, under k-step 0's MFMAs).
  bf16x8 a0[4], b0[2], a1[4], b1[2];
  if (n_steps > 0) {
    // The index loads above complete here, so no compiler-inserted wait for
    // them (which would count the untracked DMAs too) lands in the ring.
    wait_vmem<0>();
#pragma unroll
    for (int st = 0; st < kRAhead; ++st) issue_next();
    wait_vmem<(kRAhead - 1) * kRDmaPerStep>();  // step 0 has landed
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    read_half(0, 0, a0, b0);
  }
  int dt = dt_begin, kcs = 0, stage = 0;
  int st = st_begin;  // kStreamK: the computed unit's source tile
  for (int step = 0; step < n_steps; ++step) {
    const int next = stage == kRStages - 1 ? 0 : stage + 1;
    // Before the barrier: k-step 0's MFMAs (operands read in the previous
    // step) and the reads of k-step 1's operands, whose stage landed before
    // the previous barrier.  A wave arriving at the barrier leaves MFMAs in
    // the pipe, and the other wave of its SIMD keeps issuing them, so barrier
    // skew does not idle the matrix cores.
    if (K == 1) {
      // The compiler interleaves the reads with the MFMAs.
      read_half(stage, 1, a1, b1);
      mma_half(a0, b0);
    } else {
      // One read after each MFMA (the top-4 epilogue leaves the compiler
      // fewer registers to hoist the reads with).
      const bf16_t* al = a_lds + stage * kRTileElems + wd * 128 * kRKc;
      const bf16_t* bl = b_lds + stage * kRTileElems + ws * 64 * kRKc;
#pragma unroll
      for (int x = 0; x < 4; ++x)
#pragma unroll
        for (int y = 0; y < 2; ++y) {
          acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0[x], b0[y], acc[x][y], 0, 0, 0);
          const int q = 2 * x + y;
          if (q < 4) a1[q] = *reinterpret_cast<const bf16x8*>(al + q * 32 * kRKc + off[1]);
          else if (q < 6) b1[q - 4] = *reinterpret_cast<const bf16x8*>(bl + (q - 4) * 32 * kRKc + off[1]);
          __builtin_amdgcn_sched_barrier(0);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    // After this barrier step + 1 has landed for every wave and every wave
    // has finished step - 1, whose stage the DMAs below refill.  A wave's
    // reads of a stage are consumed by its MFMAs before its next barrier, so
    // the barrier need not wait for LDS reads in flight.
    wait_vmem<(kRAhead - 2) * kRDmaPerStep>();
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    // k-step 1's MFMAs with step + 4's four DMAs issued between them: a DMA
    // issue can stall the wave while the CU's DMA queue is full, and the
    // MFMAs issued before it keep the pipe busy meanwhile.  The reads of the
    // next step's k-step 0 operands are unconditional: after the last step
    // they read a stage nobody uses, and a branch here would make the wait
    // above cover them too.
    if (K == 1) {
      read_half(next, 0, a0, b0);
#pragma unroll
      for (int x = 0; x < 4; ++x) {
#pragma unroll
        for (int y = 0; y < 2; ++y)
          acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1[x], b1[y], acc[x][y], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        issue_one(x);
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
      const bf16_t* al = a_lds + next * kRTileElems + wd * 128 * kRKc;
      const bf16_t* bl = b_lds + next * kRTileElems + ws * 64 * kRKc;
#pragma unroll
      for (int x = 0; x < 4; ++x) {
#pragma unroll
        for (int y = 0; y < 2; ++y) {
          acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1[x], b1[y], acc[x][y], 0, 0, 0);
          const int q = 2 * x + y;
          if (q < 4) a0[q] = *reinterpret_cast<const bf16x8*>(al + q * 32 * kRKc + off[0]);
          else if (q < 6) b0[q - 4] = *reinterpret_cast<const bf16x8*>(bl + (q - 4) * 32 * kRKc + off[0]);
          __builtin_amdgcn_sched_barrier(0);
        }
        issue_one(x);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    stage = next;
    if (kcs == n_chunks - 1) {
      if (!all_src_ok) {
#pragma unroll
        for (int sb = 0; sb < 2; ++sb)
#pragma unroll
          for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[db][sb][r] = src_ok[sb] ? acc[db][sb][r] : 0.0f;
      }
      if constexpr (kStreamK) s0 = st * kRTile;
      const int d0 = d_begin + dt * kRTile;
      if (!kStreamK && scores) {  // the stream-K kernel never writes scores
#pragma unroll
        for (int sb = 0; sb < 2; ++sb) {
          const int i = s0 + 64 * ws + 32 * sb + l32;
#pragma unroll
          for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int jj = d0 + 128 * wd + 32 * db + 8 * (r >> 2) + 4 * hh + (r & 3);
              if (jj < d_end && i < ns)
                scores[static_cast<int64_t>(i) * scores_stride + jj] = static_cast<bf16_t>(acc[db][sb][r]);
            }
        }
      }
      const int jl = d0 + 128 * wd + 4 * hh;  // this lane's first dictionary row
      if (K == 1) {
        // Running top-1 on the bf16-rounded score: a later (higher) j wins only
        // when strictly greater, which is the lower-index rule for ties; a NaN
        // wins over numbers and the first NaN is kept (ranking of the keys).
        // A lane's rows jl + pos rise with pos, a compile-time constant per
        // element, so the tile's winner is tracked by pos and jl added once.
        // Rows past d_end exist only in a part's last, partial tile.
        //
        // Full tiles without a NaN take two cheap passes per source: the fp32
        // maximum m of the lane's 64 scores (NaN-propagating 3-input max), then
        // the first position whose score is at least the lower bound of
        // bf16(m)'s rounding interval -- the first score that rounds to the
        // tile's bf16 maximum -- by one compare and one select per score, where
        // the per-score loop below rounds and compares every score.
        const bool full = d0 + kRTile <= d_end;
        bool fast = false;
        float mx[2];
        if (full) {
#pragma unroll
          for (int sb = 0; sb < 2; ++sb) {
            float part[4];
#pragma unroll
            for (int db = 0; db < 4; ++db) {
              float m = acc[db][sb][0];
#pragma unroll
              for (int r = 1; r < 16; r += 2)
                m = __builtin_elementwise_maximum(__builtin_elementwise_maximum(m, acc[db][sb][r]),
                                                  r + 1 < 16 ? acc[db][sb][r + 1] : acc[db][sb][r]);
              part[db] = m;
            }
            mx[sb] = __builtin_elementwise_maximum(__builtin_elementwise_maximum(part[0], part[1]),
                                                   __builtin_elementwise_maximum(part[2], part[3]));
          }
          fast = __ballot((mx[0] != mx[0]) | (mx[1] != mx[1])) == 0;
        }
        if (fast) {
#pragma unroll
          for (int sb = 0; sb < 2; ++sb) {
            const float t = bf16_round(mx[sb]);
            const float lo = bf16_lower_bound(t);
            int tp = 0;  // some score reaches lo: the maximum itself
#pragma unroll
            for (int db = 3; db >= 0; --db)
#pragma unroll
              for (int r = 15; r >= 0; --r)
                tp = acc[db][sb][r] >= lo ? 32 * db + 8 * (r >> 2) + (r & 3) : tp;
            // Strictly greater: an equal maximum of an earlier tile keeps its
            // lower row, and a NaN kept from an earlier tile stays.
            if (t > top_v[sb]) {
              top_v[sb] = t;
              top_j[sb] = jl + tp;
            }
          }
        } else {
          const int lim = full ? kRTile : d_end - jl;
#pragma unroll
          for (int sb = 0; sb < 2; ++sb) {
            float tv = top_v[sb];
            int tp = -1;
#pragma unroll
            for (int db = 0; db < 4; ++db)
#pragma unroll
              for (int r = 0; r < 16; ++r) {
                const int pos = 32 * db + 8 * (r >> 2) + (r & 3);
                const float v = bf16_round(acc[db][sb][r]);
                const bool take = (pos < lim) & ((v > tv) | ((v != v) & (tv == tv)));
                tv = take ? v : tv;
                tp = take ? pos : tp;
              }
            top_j[sb] = tp >= 0 ? jl + tp : top_j[sb];
            top_v[sb] = tv;
          }
        }
      } else {
        // Full tiles without a NaN in the wave: a tile-local top-4 of 32-bit
        // keys per source, merged into the running list once.  tile_key()
        // puts ord16 of the bf16 score in the high half and 0xFFFF - position
        // in the low half, so a larger key is a larger score or, for equal
        // scores, the lower dictionary row; a sorted list takes a key with one
        // max and three medians.  Other tiles take the per-score inserts.
        const bool full = d0 + kRTile <= d_end;
        bool fast = false;
        if (full) {
          float m = acc[0][0][0];
#pragma unroll
          for (int sb = 0; sb < 2; ++sb)
#pragma unroll
            for (int db = 0; db < 4; ++db)
#pragma unroll
              for (int r = 0; r < 16; r += 2)
                m = __builtin_elementwise_maximum(__builtin_elementwise_maximum(m, acc[db][sb][r]),
                                                  acc[db][sb][r + 1]);
          fast = __ballot(m != m) == 0;
        }
        if (fast) {
#pragma unroll
          for (int sb = 0; sb < 2; ++sb) {
            uint32_t l0 = 0, l1 = 0, l2 = 0, l3 = 0;
#pragma unroll
            for (int db = 0; db < 4; ++db)
#pragma unroll
              for (int r = 0; r < 16; ++r) {
                const uint32_t key = tile_key(acc[db][sb][r], 32 * db + 8 * (r >> 2) + (r & 3));
                const uint32_t n1 = med3_u32(l0, l1, key);
                const uint32_t n2 = med3_u32(l1, l2, key);
                l3 = med3_u32(l2, l3, key);
                l0 = max(l0, key);
                l1 = n1;
                l2 = n2;
              }
            // 64 keys went in, so all four slots hold scores.
            best[sb].insert(tile_key_to_key(l0, jl));
            best[sb].insert(tile_key_to_key(l1, jl));
            best[sb].insert(tile_key_to_key(l2, jl));
            best[sb].insert(tile_key_to_key(l3, jl));
          }
        } else {
#pragma unroll
          for (int sb = 0; sb < 2; ++sb)
#pragma unroll
            for (int db = 0; db < 4; ++db)
#pragma unroll
              for (int r = 0; r < 16; ++r) {
                const int jj = jl + 32 * db + 8 * (r >> 2) + (r & 3);
                if (jj < d_end) best[sb].insert(make_key(acc[db][sb][r], jj));
              }
        }
      }
#pragma unroll
      for (int sb = 0; sb < 2; ++sb)
#pragma unroll
        for (int db = 0; db < 4; ++db) acc[db][sb] = f32x16{};
      kcs = 0;
      ++dt;
      if constexpr (kStreamK) {
        const bool tile_done = dt == tiles_per_part;
        const bool last = step == n_steps - 1;
        if (tile_done || last) {
          // End of this work-group's share of source tile st: every lane writes
          // its two sources' best keys (list wd * 2 + hh) to the share's slot.
          const int slot = st == st_begin ? slot_begin : 0;
#pragma unroll
          for (int sb = 0; sb < 2; ++sb) {
            const int i = s0 + 64 * ws + 32 * sb + l32;
            if (i < ns)
              partial[static_cast<int64_t>(i) * parts + slot * 4 + wd * 2 + hh] =
                  top_j[sb] >= 0 ? make_key(top_v[sb], top_j[sb]) : 0ull;
            top_v[sb] = -__builtin_inff();
            top_j[sb] = -1;
          }
        }
        if (tile_done) {
          dt = 0;
          ++st;
          if (!last) set_epilogue_stile(st);
        }
      }
    } else {
      ++kcs;
    }
  }
  // The look-ahead DMAs land before the ring's LDS is reused for the merge.
  wait_vmem<0>();
  if constexpr (kStreamK) return;
  __syncthreads();

  if (K == 1) {
#pragma unroll
    for (int sb = 0; sb < 2; ++sb)
      if (top_j[sb] >= 0) best[sb].k[0] = make_key(top_v[sb], top_j[sb]);
  }
  // Merge the four lists of every source row (two dictionary halves x two lane halves).
  uint64_t* m_lds = reinterpret_cast<uint64_t*>(a_lds);  // [256 sources][4 lists][K]
#pragma unroll
  for (int sb = 0; sb < 2; ++sb) {
    const int local = 64 * ws + 32 * sb + l32;
#pragma unroll
    for (int t = 0; t < K; ++t) m_lds[(local * 4 + wd * 2 + hh) * K + t] = best[sb].k[t];
  }
  __syncthreads();
  if (tid < kRTile) {
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
// With sk_groups > 0 the lists come from the stream-K top-1 ring kernel: row i's
// source tile was split over work-groups first..last of the schedule, which
// wrote four lists each into slots 0 .. last - first of the row's `parts`.
template <int K>
__global__ __launch_bounds__(256) void topk_finalize_kernel(
    const uint64_t* __restrict__ partial, int n_src, const int* __restrict__ n_src_dev, int parts,
    int n0, int off1, float* __restrict__ values, int64_t* __restrict__ index64,
    int32_t* __restrict__ index32, const int64_t* __restrict__ index_map, int sk_units, int sk_groups,
    int sk_dict_tiles) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  int ns = n_src;
  if (n_src_dev) ns = min(ns, *n_src_dev);
  if (i >= ns) return;
  int used = parts;
  if (sk_groups > 0) {
    const int64_t u0 = static_cast<int64_t>(i / kRTile) * sk_dict_tiles;
    const int64_t u1 = u0 + sk_dict_tiles - 1;
    used = 4 * static_cast<int>(sk_owner(u1, sk_units, sk_groups) - sk_owner(u0, sk_units, sk_groups) + 1);
  }
  TopK<K> m;
  m.init();
  const uint64_t* p = partial + static_cast<int64_t>(i) * parts * K;
  for (int q = 0; q < used * K; ++q) m.insert(p[q]);
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


// Resident work-groups of the similarity kernel on the current device, cached.
template <int K>
int64_t resident_groups(bool ring) {
  static int cache[2][64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return ring ? 256 : 512;
  if (cache[ring][dev] == 0) {
    int cus = 0, per_cu = 0;
    const hipError_t occ =
        ring ? hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, sim_topk_ring_kernel<K, false>, kRWaves * 64, 0)
             : hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, sim_topk_kernel<K>, 256, 0);
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        occ != hipSuccess)
      return ring ? 256 : 512;
    cache[ring][dev] = cus * (per_cu > 0 ? per_cu : 1);
  }
  return cache[ring][dev];
}

// The ring kernel runs when the dimension is a whole number of its K chunks.
inline bool use_ring(int64_t dim) { return dim % kRKc == 0; }

// Dictionary split for a kernel with `tile` x `tile` steps: the number of parts
// that minimises (rounds of resident work-groups) x (dictionary tiles per
// work-group + a half-tile fixed cost).
int choose_parts(int64_t n_src, int64_t n_dict, int topk, bool ring) {
  const int64_t tile = ring ? kRTile : kTile;
  const int64_t src_tiles = (n_src + tile - 1) / tile;
  const int64_t dict_tiles = (n_dict + tile - 1) / tile;
  if (src_tiles <= 0 || dict_tiles <= 0) return 1;
  const int64_t slots = topk == 1 ? resident_groups<1>(ring) : resident_groups<4>(ring);
  int best = 1;
  double best_cost = 1e300;
  for (int64_t p = 1; p <= dict_tiles && p <= 4096; ++p) {
    const int64_t rounds = (src_tiles * p + slots - 1) / slots;
    const int64_t tpp = (dict_tiles + p - 1) / p;
    const double cost = static_cast<double>(rounds) * (static_cast<double>(tpp) + 0.5);
    if (cost < best_cost) {
      best_cost = cost;
      best = static_cast<int>(p);
    }
  }
  return best;
}

// Stream-K schedule of the top-1 ring kernel over units = source tiles x
// dictionary tiles on as many work-groups as are resident.  It removes the
// split schedule's last-round waste but gives up its cache locality (the
// resident tasks of a round read a few dictionary tiles and source tiles
// together; a stream-K share walks its own), so it is taken only where that
// waste is large and a share spans few source tiles: when the longest share,
// ceil(units / groups) tiles, is at least 5% below the split's rounds x tiles
// per part, and a share is at most two dictionaries long.  At C4 (93 x 35
// units, 256 work-groups) 13 against 2 x 7 tiles: 431 -> 393 us in a same-box
// A/B; at 372 x 140 units (1.9% waste) stream-K ran 19% slower, at 47 x 18 units
// (4 tiles either way) no faster.  `lists` = 4 x the most work-groups one source
// tile is split over; groups = 0 when the split schedule is kept.
struct StreamK {
  int units = 0, groups = 0, dict_tiles = 0, lists = 0;
};
StreamK stream_k_schedule(int64_t n_src, int64_t n_dict) {
  StreamK r;
  const int64_t src_tiles = (n_src + kRTile - 1) / kRTile;
  const int64_t dict_tiles = (n_dict + kRTile - 1) / kRTile;
  if (src_tiles <= 0 || dict_tiles <= 0 || src_tiles * dict_tiles >= (1LL << 31)) return r;
  const int64_t slots = resident_groups<1>(true);
  const int p = choose_parts(n_src, n_dict, 1, true);
  const int64_t tpp = (dict_tiles + p - 1) / p;
  const int64_t split = (src_tiles * p + slots - 1) / slots * tpp;
  const int64_t units = src_tiles * dict_tiles;
  const int64_t share = (units + slots - 1) / slots;
  if (static_cast<double>(share) > 0.95 * static_cast<double>(split) || share > 2 * dict_tiles) return r;
  r.units = static_cast<int>(units);
  r.groups = static_cast<int>(std::min(slots, units));
  r.dict_tiles = static_cast<int>(dict_tiles);
  int64_t most = 1;
  for (int64_t st = 0; st < src_tiles; ++st)
    most = std::max(most, sk_owner((st + 1) * dict_tiles - 1, units, r.groups) -
                              sk_owner(st * dict_tiles, units, r.groups) + 1);
  r.lists = static_cast<int>(4 * most);
  return r;
}

}  // namespace
}  // namespace vgo

extern "C" int vgo_similarity_topk_workspace(int64_t n_src, int64_t n_dict, int topk, int* parts,
                                             size_t* bytes) {
  using namespace vgo;
  VGO_REQUIRE(topk == 1 || topk == 4, "similarity_topk: topk must be 1 or 4");
  VGO_REQUIRE(n_src >= 0 && n_dict >= 0, "similarity_topk: negative size");
  // Sized for whichever kernel and schedule the dimension selects.
  int p = std::max(choose_parts(n_src, n_dict, topk, true), choose_parts(n_src, n_dict, topk, false));
  if (topk == 1) p = std::max(p, stream_k_schedule(n_src, n_dict).lists);
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
  const bool ring = use_ring(dim);
  const StreamK sk = ring && topk == 1 && !scores ? stream_k_schedule(n_src, n_dict) : StreamK{};
  const int parts = sk.groups > 0 ? sk.lists : choose_parts(n_src, n_dict, topk, ring);
  const size_t need = static_cast<size_t>(n_src) * parts * topk * sizeof(uint64_t);
  VGO_REQUIRE(workspace && workspace_bytes >= need, "similarity_topk: workspace too small");
  VGO_REQUIRE(aligned(workspace, 8), "similarity_topk: workspace must be 8-byte aligned");
  const int64_t tile = ring ? kRTile : kTile;
  const int64_t dict_tiles = (n_dict + tile - 1) / tile;
  const int tiles_per_part = sk.groups > 0 ? sk.dict_tiles : static_cast<int>((dict_tiles + parts - 1) / parts);
  hipStream_t s = as_stream(stream);
  const int64_t src_tiles = (n_src + tile - 1) / tile;
  VGO_REQUIRE(src_tiles * parts < (1LL << 31), "similarity_topk: grid too large");
  dim3 grid(static_cast<unsigned>(sk.groups > 0 ? sk.groups : src_tiles * parts));
  uint64_t* partial = static_cast<uint64_t*>(workspace);
  const bf16_t* sp = static_cast<const bf16_t*>(src);
  const bf16_t* dp = static_cast<const bf16_t*>(dict);
  bf16_t* sc = static_cast<bf16_t*>(scores);
  const int blocks2 = static_cast<int>((n_src + 255) / 256);
  if (ring) {
    // 64-bit row addresses per lane; the DMA reads stay inside the buffers
    // (rows are clamped, dim is a multiple of the chunk).
    auto launch = [&](auto kernel) {
      hipLaunchKernelGGL(kernel, grid, dim3(kRWaves * 64), 0, s, sp, src_row_stride, src_capacity, src_rows,
                         n_src_device, static_cast<int>(n_src), dp, dict_row_stride, static_cast<int>(dict_n0),
                         static_cast<int>(dict_off1), static_cast<int>(n_dict), static_cast<int>(dim),
                         tiles_per_part, partial, parts, sc, scores_row_stride, sk.units);
    };
    if (sk.groups > 0)
      launch(sim_topk_ring_kernel<1, true>);
    else if (topk == 1)
      launch(sim_topk_ring_kernel<1, false>);
    else
      launch(sim_topk_ring_kernel<4, false>);
  } else if (topk == 1) {
    hipLaunchKernelGGL((sim_topk_kernel<1>), grid, dim3(256), 0, s, sp, src_row_stride, src_capacity, src_rows,
                       n_src_device, static_cast<int>(n_src), dp, dict_row_stride,
                       static_cast<int>(dict_n0), static_cast<int>(dict_off1),
                       static_cast<int>(n_dict), static_cast<int>(dim), tiles_per_part, partial,
                       parts, sc, scores_row_stride);
  } else {
    hipLaunchKernelGGL((sim_topk_kernel<4>), grid, dim3(256), 0, s, sp, src_row_stride, src_capacity, src_rows,
                       n_src_device, static_cast<int>(n_src), dp, dict_row_stride,
                       static_cast<int>(dict_n0), static_cast<int>(dict_off1),
                       static_cast<int>(n_dict), static_cast<int>(dim), tiles_per_part, partial,
                       parts, sc, scores_row_stride);
  }
  if (topk == 1)
    hipLaunchKernelGGL((topk_finalize_kernel<1>), dim3(blocks2), dim3(256), 0, s, partial,
                       static_cast<int>(n_src), n_src_device, parts, static_cast<int>(dict_n0),
                       static_cast<int>(dict_off1), values, index64, index32, index_map, sk.units, sk.groups,
                       sk.dict_tiles);
  else
    hipLaunchKernelGGL((topk_finalize_kernel<4>), dim3(blocks2), dim3(256), 0, s, partial,
                       static_cast<int>(n_src), n_src_device, parts, static_cast<int>(dict_n0),
                       static_cast<int>(dict_off1), values, index64, index32, index_map, 0, 0, 0);
  return check_launch("similarity_topk");
}
