// Mass-bias flash attention for gfx950: O = softmax(Q K^T / sqrt(64) + log m) V.
//
// Work of vggt_omega/models/mass_bias_attention.py:17-129 (Triton kernel and
// wrapper) and, with no bias, of the dense special-query SDPA at
// vggt_omega/models/layers/attention.py:406-422.
//
// bf16 / f16 path (the autocast path of the reference):
//  * A task is 256 queries of one (batch, head): 4 waves x 64 queries, each
//    wave holding its Q rows in registers as MFMA B operands (2 x 32 columns).
//  * Keys stream through LDS in tiles of 64, double-buffered: the next tile's
//    K/V rows are loaded into registers while the current tile is computed,
//    then stored to the other buffer -- one barrier per tile.  K is stored
//    row-major, V transposed (V^T, one row per dim) so both feed
//    v_mfma_f32_32x32x16 as A operands with one 16-byte LDS read per lane;
//    rows are 128 B with XOR-permuted 16-byte chunks (no padding, no bank
//    conflicts for the reads or for the transposing V stores).
//  * Scores are computed transposed, S^T = K' Q'^T, so a lane owns one query
//    and 16 keys of every 32-key sub-tile: the row max/sum of the online
//    softmax stay in registers except for one v_permlane32_swap, and the
//    exponentiated scores are already laid out as the B operand of O^T = V^T P^T.
//  * Q is scaled by 1/8 = 1/sqrt(64) as it is loaded, which is exact in the
//    input dtype, so the MFMA yields the reference's logits q.k/8 from the
//    inputs as given; log2(e) multiplies them in fp32 before v_exp_f32, as
//    the reference multiplies its fp32 dot products (mass_bias_attention.py:
//    56-58).  (Rounding Q*log2(e)/8 to the input dtype instead saves that
//    multiply but adds a logit error of up to 2^-9 of each product, which
//    grows with the logit scale: 7e-2 of the output at q, k of 3x unit scale
//    in bf16.)  Sub-tile 0's multiplies run under sub-tile 1's MFMAs.  The
//    per-key bias enters as the accumulator the score MFMAs start from: in
//    S^T a register holds one key for all 32 queries of its lane half, so the
//    tile's fp32 biases (log m in the input dtype, as the reference rounds it
//    first, mass_bias_attention.py:109; -inf past n_key) are four 16-byte LDS
//    broadcast reads per 32-key sub-tile, shared by both query blocks.  The
//    softmax offset -mref joins the log2(e) multiply as the addend of an fma,
//    so neither takes an MFMA k-step (an 8-deep v_mfma_f32_32x32x8 holds the
//    matrix pipe as long as a 16-deep one).
//  * Lazy online softmax: P = e^S straight from the accumulator while no
//    logit exceeds the reference max mref by more than 15 ln 2 (checked through the
//    per-lane sums); only then, and on a segment's first tile, are the tile's
//    logits recomputed, mref moved and O / the row sum rescaled.  P is rounded
//    to the input dtype before P.V (reference :74); the row sum adds the
//    unrounded fp32 values, as the reference's does (:62).
//  * Scheduling: with G work-groups resident at once, every work-group runs
//    whole tasks w, w+G, ... for floor(tasks/G) rounds (neighbouring groups,
//    i.e. one XCD's, share a head's K/V in L2), and the (task, key tile)
//    units of the remaining tasks are split evenly over all G (stream-K on
//    the last round only); tasks cut between work-groups are finished by
//    attn_merge_kernel from fp32 partial states.
// fp32 path: exact fp32 arithmetic, one query row per lane, K/V tiles in LDS.
#include <algorithm>
#include <mutex>
#include <string>
#include <type_traits>
#include <vector>

#include "vgo_common.h"

namespace vgo {
namespace {

constexpr int kD = 64;
constexpr int kBN = 64;                      // keys per LDS tile
constexpr int kWaves = 4;                    // waves per work-group
constexpr int kQB = 2;                       // 32-query MFMA column blocks per wave
constexpr int kQPerWave = 32 * kQB;          // 64
constexpr int kQBlock = kWaves * kQPerWave;  // 256 queries per work-group task
constexpr int kTileElems = kBN * kD;         // one K (or V^T) tile, elements
constexpr float kLog2e = 1.4426950408889634f;

template <typename T>
struct Mma;
template <>
struct Mma<bf16_t> {
  typedef bf16x8 op8;
  typedef bf16x2 op2;
  typedef bf16x4 op4;
  static __device__ __forceinline__ f32x16 mma(op8 a, op8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};
template <>
struct Mma<f16_t> {
  typedef f16x8 op8;
  typedef f16x2 op2;
  typedef f16x4 op4;
  static __device__ __forceinline__ f32x16 mma(op8 a, op8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

// (x[l], x[l ^ 32]) for every lane l in one VALU op: v_permlane32_swap
// exchanges the upper half of one register with the lower half of another.
__device__ __forceinline__ void both_halves(float x, float& a, float& b) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  a = __uint_as_float(r[0]);
  b = __uint_as_float(r[1]);
}
__device__ __forceinline__ float half_max(float x) {
  float a, b;
  both_halves(x, a, b);
  return fmaxf(a, b);
}
__device__ __forceinline__ float half_sum(float x) {
  float a, b;
  both_halves(x, a, b);
  return a + b;  // identical in both halves: IEEE addition commutes
}

// Position of key `kk` (0..63) inside a V^T row.  Within every 16-key group the
// two middle quads are swapped, which is the order in which S^T's accumulator
// registers present keys to the P operand (see the header comment).
__device__ __forceinline__ int vt_pos(int kk) {
  return (kk & ~12) | ((kk & 4) << 1) | ((kk & 8) >> 1);
}

// LDS tiles are 64 rows x 64 elements (128 B) with no padding; the eight
// 16-byte chunks of a row are XOR-permuted by swz(row), so that eight
// consecutive rows read at one logical chunk, and eight chunks of eight rows
// written by one store, all fall in distinct banks.
__device__ __forceinline__ int swz(int row) { return (row & 7) ^ ((row >> 3) & 7); }

template <typename T>
struct AttnArgs {
  const T* q;
  const T* k;
  const T* v;
  const T* bias;
  T* out;
  int heads, nq, nk, n_qblocks, ntiles;
  int64_t qsb, qsh, qsn, ksb, ksh, ksn, vsb, vsh, vsn, osb, osh, osn;
  float c;  // 1/8, folded into Q (exact)
  // LDS-DMA kernel only: V^T packed per (batch*head) as [64][npad] in the MFMA
  // key order, and per key the bias as fp32 (the input dtype's value; -inf past
  // n_key), npad long.
  const T* vt;
  const float* kbias;
  int npad;
};

// Schedule of one attn_pp_kernel launch over one or two problems (the second:
// the dense special-query pass, run in the merged attention's launch).  With
// `groups` work-groups, work-group w first runs problem 0's whole tasks w,
// w + groups, ... (`full_rounds` of them), then its share of the (task, key
// tile) units of problem 0's remaining tasks tail_task0.. (units [0, units0),
// `tail_tasks0` tasks) followed by every task of problem 1 (units [units0,
// units)), split evenly over the first `tail_groups` work-groups: stream-K on
// the last round only.
struct PPSchedule {
  float* partial;  // stream-K partial states, 2 per work-group (may be null)
  // Clock samples of the kernel-timing record (null unless sampled): work-group
  // b's wave 0 stores its shader-clock and constant-clock counters at its start
  // (stamps[4b], stamps[4b + 1]) and end (stamps[4b + 2], stamps[4b + 3]).
  unsigned long long* stamps;
  int64_t groups, full_rounds, tail_task0, tail_tasks0, units0, units, tail_groups;
};
template <typename T>
struct PPLaunch {
  AttnArgs<T> p[2];
  PPSchedule s;
};

// First unit of work-group w under the static stream-K partition.
__host__ __device__ __forceinline__ int64_t sk_begin(int64_t w, int64_t units, int64_t groups) {
  return w * units / groups;
}
// Work-group whose range holds unit u.
__host__ __device__ __forceinline__ int64_t sk_owner(int64_t u, int64_t units, int64_t groups) {
  return ((u + 1) * groups - 1) / units;
}

// LDS stages: 2 (register-staged kernel) or 4 (DMA kernel); a stage holds a
// K tile, a V^T tile and the tile's 64 key biases (fp32).
// Largest per-lane sum of 32 probabilities the lazy softmax accepts without
// moving its reference max.  It bounds every P by 2^15, below the largest
// finite f16 (65,504), so the rounded P operands of either type stay finite;
// the bound exists only for that.  P's relative rounding error is the same at
// any magnitude, and a higher bound takes the rescaling path less often when
// logits spread widely (q, k at 2-3x unit scale: 16-19% faster at C4 than a
// bound of 2^8; at unit scale and below the path is never taken and the
// results are the same bit for bit).
constexpr float kLazyLimit = 32768.0f;

// Per-wave state of the bf16/f16 kernels: QB 32-column MFMA blocks of queries
// (two, 64 queries; one where the wave's second block would hold only rows past
// n_query) -- their scaled Q operands, the online-softmax state and the O^T
// accumulators -- and the tile-level steps on LDS-resident K / V^T / bias.
template <typename T, int QB = kQB>
struct WaveAttn {
  typedef typename Mma<T>::op8 op8;
  typedef typename Mma<T>::op2 op2;
  typedef typename Mma<T>::op4 op4;

  op8 qreg[QB][4];  // Q' = Q / 8 (exact), B operands
  // Reference max per query (a T value; -inf until a finite logit is seen);
  // the running sum and O are relative to e^mref.  nm = -mref log2(e), the
  // offset of the exp2 argument (+inf while mref = -inf).
  float mref[QB], lsum[QB], nm[QB];
  f32x16 o[QB][2];
  int off[4];  // LDS element offsets of logical chunk pair t of row l32
  int l32, hh;

  // Q' = Q * c for the wave's rows qw0.. (rows past n_query read a valid row;
  // never stored); c = 1/8 keeps Q' exact, so K Q'^T holds the logits.
  __device__ __forceinline__ void init(const T* qb_ptr, int64_t qsn, int qw0, int nq, float c) {
    const int lane = threadIdx.x & 63;
    l32 = lane & 31;
    hh = lane >> 5;
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      const int row = min(qw0 + qb * 32 + l32, nq - 1);
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const op8 raw = *reinterpret_cast<const op8*>(qb_ptr + row * qsn + 16 * t + 8 * hh);
#pragma unroll
        for (int e = 0; e < 8; ++e) qreg[qb][t][e] = static_cast<T>(to_f32(raw[e]) * c);
      }
    }
    // Row l32 + 32 uses off[t ^ 2] (swz flips bit 2 of the chunk there).
    const int s0 = swz(l32);
#pragma unroll
    for (int t = 0; t < 4; ++t) off[t] = l32 * kD + (((2 * t + hh) ^ s0) << 3);
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      mref[qb] = -__builtin_inff();
      nm[qb] = exp_offset(mref[qb]);
      lsum[qb] = 0.0f;
#pragma unroll
      for (int dt = 0; dt < 2; ++dt) o[qb][dt] = f32x16{};
    }
  }

  // Offset of the exp2 argument for reference max m: -m log2(e), +inf while
  // m = -inf (every P then non-finite, which takes the rescaling path).
  static __device__ __forceinline__ float exp_offset(float m) {
    return m == -__builtin_inff() ? __builtin_inff() : -m * kLog2e;
  }
  // The key biases of sub-tile sub in the accumulator layout: register r of
  // lane l holds key 32 sub + 8 (r / 4) + 4 (l / 32) + r % 4, so each group of
  // four registers is one 16-byte LDS read (the same address in every lane of a
  // half: a broadcast).  The score MFMAs start from it.
  __device__ __forceinline__ f32x16 key_bias(const float* bl, int sub) const {
    f32x16 c;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const f32x4 x = *reinterpret_cast<const f32x4*>(bl + 32 * sub + 8 * g + 4 * hh);
#pragma unroll
      for (int e = 0; e < 4; ++e) c[4 * g + e] = x[e];
    }
    return c;
  }
  // A operand of rows 32*half.. of a K or V^T tile, k-chunk pair t.
  __device__ __forceinline__ op8 tile_op(const T* tl, int half, int t) const {
    return *reinterpret_cast<const op8*>(tl + half * 32 * kD + off[t ^ (2 * half)]);
  }

  // Operands of one tile, read from LDS in one batch ahead of their MFMAs (so
  // the reads overlap each other rather than each MFMA waiting for its own).
  struct KOps {
    op8 k[2][4];  // K rows 32*sub.., k-chunk pair t
  };
  struct VOps {
    op8 v[4][2];  // V^T rows (dims) 32*dt.., key chunk pair t
  };
  __device__ __forceinline__ void load_k(const T* kl, KOps& ops) const {
#pragma unroll
    for (int sub = 0; sub < 2; ++sub)
#pragma unroll
      for (int t = 0; t < 4; ++t) ops.k[sub][t] = tile_op(kl, sub, t);
  }
  __device__ __forceinline__ void load_v(const T* vl, VOps& ops) const {
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int dt = 0; dt < 2; ++dt) ops.v[t][dt] = tile_op(vl, dt, t);
  }

  // S^T = K Q'^T + bias for the tile's two 32-key sub-tiles (the MFMAs start
  // from the key biases); sub-tile 0 then leaves in the exp2 domain,
  // S log2(e) - mref log2(e), as pv_scores leaves it.
  // kRaw: both sub-tiles stay raw logits (tile 0 of a register-staged task,
  // whose softmax_first takes their maximum before any offset exists).
  template <bool kRaw = false>
  __device__ __forceinline__ void scores(const KOps& ops, const float* bl, f32x16 (&s)[QB][2]) const {
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
      const f32x16 c = key_bias(bl, sub);
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) s[qb][sub] = Mma<T>::mma(ops.k[sub][0], qreg[qb][0], c);
#pragma unroll
      for (int t = 1; t < 4; ++t)
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) s[qb][sub] = Mma<T>::mma(ops.k[sub][t], qreg[qb][t], s[qb][sub]);
    }
    if constexpr (!kRaw) {
#pragma unroll
      for (int qb = 0; qb < QB; ++qb)
#pragma unroll
        for (int r = 0; r < 16; ++r) s[qb][0][r] = fmaf(s[qb][0][r], kLog2e, nm[qb]);
    }
  }
  template <bool kRaw = false>
  __device__ __forceinline__ void scores(const T* kl, const float* bl, f32x16 (&s)[QB][2]) const {
    KOps ops;
    load_k(kl, ops);
    __builtin_amdgcn_sched_barrier(0);
    scores<kRaw>(ops, bl, s);
  }

  // P = e^(x - m) = exp2(x log2(e) + nmv) with nmv = -m log2(e), for one
  // 32-key sub-tile (x; kScaled: x is already x log2(e) + nmv), rounded to T and
  // packed into B operands p[2*sub], p[2*sub+1] of O^T += V^T P^T.  The
  // unrounded values are summed into part[4] (started by sub 0), as the
  // reference sums its fp32 probabilities; the sum uses fp32 adds because dot
  // instructions would share the matrix pipe with the other wave's MFMAs.
  template <bool kScaled = false>
  __device__ __forceinline__ void exp_pack(const f32x16& x, int sub, float nmv, op8 (&p)[4],
                                           float (&part)[4]) const {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      i32x4 packed;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r = u * 8 + 2 * j;
        const float e0 = __builtin_amdgcn_exp2f(kScaled ? x[r] : fmaf(x[r], kLog2e, nmv));
        const float e1 = __builtin_amdgcn_exp2f(kScaled ? x[r + 1] : fmaf(x[r + 1], kLog2e, nmv));
        part[j] = sub == 0 && u == 0 ? e0 : part[j] + e0;
        part[j] += e1;
        const op2 pr = {static_cast<T>(e0), static_cast<T>(e1)};
        packed[j] = __builtin_bit_cast(int, pr);
      }
      p[2 * sub + u] = __builtin_bit_cast(op8, packed);
    }
  }
  __device__ __forceinline__ static float sum4(const float (&part)[4]) {
    return (part[0] + part[1]) + (part[2] + part[3]);
  }

  // Logits (with the key bias) of query block qb against the sub-tile's 32 keys.
  __device__ __forceinline__ f32x16 logits(const T* kl, const float* bl, int qb, int sub) const {
    f32x16 x = key_bias(bl, sub);
#pragma unroll
    for (int t = 0; t < 4; ++t) x = Mma<T>::mma(tile_op(kl, sub, t), qreg[qb][t], x);
    return x;
  }

  // Lazy online softmax of one tile's scores.  P = e^S directly while every
  // lane's sum of its 32 probabilities stays <= kLazyLimit (so no logit
  // exceeds mref by more than 15 ln 2): the reference max then need not move.
  // Otherwise (and on a segment's first tile, when mref = -inf makes S
  // non-finite) the tile's logits are recomputed without the offset from K
  // (at kl, bias at bl), mref moves to the T value nearest the running max,
  // O and the sum are rescaled, and P is recomputed.  That path works one
  // 32-key sub-tile at a time (logits computed twice) to stay within the
  // registers the fast path leaves free.
  //
  // In three steps, so that a caller can take the rare branch away from the
  // work that feeds it: softmax_fast computes P and the per-lane sums and
  // returns whether any lane of the wave failed the check, rescale redoes
  // the tile, and commit adds the sums.
  __device__ __forceinline__ bool softmax_fast(const f32x16 (&s)[QB][2], op8 (&p)[QB][4],
                                               float (&part)[QB]) const {
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      float acc[4];
      exp_pack<true>(s[qb][0], 0, 0.0f, p[qb], acc);
      exp_pack(s[qb][1], 1, nm[qb], p[qb], acc);
      part[qb] = sum4(acc);
    }
    bool over = false;
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) over |= !(part[qb] <= kLazyLimit);
    return __ballot(over) != 0;
  }
  __device__ __forceinline__ void rescale(const T* kl, const float* bl, op8 (&p)[QB][4], float (&part)[QB]) {
    // Reload K here rather than keep the score operands alive.
    asm volatile("" ::: "memory");
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      float mx = -__builtin_inff();
#pragma unroll
      for (int sub = 0; sub < 2; ++sub) {
        const f32x16 x = logits(kl, bl, qb, sub);
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, x[r]);
      }
      // Rounding is monotone and mref is a T value, so mnew >= mref.
      const float mnew = to_f32(static_cast<T>(fmaxf(mref[qb], half_max(mx))));
      if (__ballot(mnew != mref[qb])) {
        const float corr = mnew == -__builtin_inff() ? 1.0f : __builtin_amdgcn_exp2f((mref[qb] - mnew) * kLog2e);
        lsum[qb] *= corr;
#pragma unroll
        for (int dt = 0; dt < 2; ++dt)
#pragma unroll
          for (int r = 0; r < 16; ++r) o[qb][dt][r] *= corr;
        mref[qb] = mnew;
        nm[qb] = exp_offset(mnew);
      }
      // No finite logit yet: every P is 0 (x = -inf).
      const float nmv = mref[qb] == -__builtin_inff() ? 0.0f : nm[qb];
      asm volatile("" ::: "memory");
      float acc[4];
      exp_pack(logits(kl, bl, qb, 0), 0, nmv, p[qb], acc);
      exp_pack(logits(kl, bl, qb, 1), 1, nmv, p[qb], acc);
      part[qb] = sum4(acc);
    }
  }
  __device__ __forceinline__ void commit(const float (&part)[QB]) {
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) lsum[qb] += part[qb];
  }
  __device__ __forceinline__ void softmax(const f32x16 (&s)[QB][2], const T* kl, const float* bl,
                                          op8 (&p)[QB][4]) {
    float part[QB];
    if (__builtin_expect(softmax_fast(s, p, part), 0)) rescale(kl, bl, p, part);
    commit(part);
  }

  // The softmax of a task's first tile from its raw logits (scores<true>):
  // the reference max moves from -inf to the T value nearest the tile's
  // maximum and P is computed once with that offset -- the values the
  // rescaling path would give, without recomputing the logits from K.  The
  // state is the one init leaves (O and the sums zero), so nothing rescales.
  __device__ __forceinline__ void softmax_first(const f32x16 (&s)[QB][2], op8 (&p)[QB][4]) {
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      float mx = -__builtin_inff();
#pragma unroll
      for (int sub = 0; sub < 2; ++sub)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[qb][sub][r]);
      mref[qb] = to_f32(static_cast<T>(fmaxf(mref[qb], half_max(mx))));
      nm[qb] = exp_offset(mref[qb]);
      // No finite logit yet: every P is 0 (x = -inf).
      const float nmv = mref[qb] == -__builtin_inff() ? 0.0f : nm[qb];
      float acc[4];
      exp_pack(s[qb][0], 0, nmv, p[qb], acc);
      exp_pack(s[qb][1], 1, nmv, p[qb], acc);
      lsum[qb] += sum4(acc);
    }
  }

  // O^T += V^T P^T.
  __device__ __forceinline__ void pv(const VOps& ops, const op8 (&p)[QB][4]) {
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int dt = 0; dt < 2; ++dt)
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) o[qb][dt] = Mma<T>::mma(ops.v[t][dt], p[qb][t], o[qb][dt]);
  }
  __device__ __forceinline__ void pv(const T* vl, const op8 (&p)[QB][4]) {
    VOps ops;
    load_v(vl, ops);
    __builtin_amdgcn_sched_barrier(0);
    pv(ops, p);
  }

  // O^T += V^T P^T with the tile at vl, then the scores of the tile at kl / bl.
  // K reads go out in two halves (one per 32-key sub-tile), each while MFMAs
  // of the previous step run: their latency is hidden and at most about half
  // of the operands are held at once.
  __device__ __forceinline__ void pv_scores(const T* vl, const op8 (&p)[QB][4], const T* kl,
                                            const float* bl, f32x16 (&s)[QB][2]) {
    VOps vops;
    load_v(vl, vops);
    __builtin_amdgcn_sched_barrier(0);
    pv_scores(vops, p, kl, bl, s);
  }
  // The same with the V^T operands already requested (vops).
  __device__ __forceinline__ void pv_scores(const VOps& vops, const op8 (&p)[QB][4], const T* kl,
                                            const float* bl, f32x16 (&s)[QB][2]) {
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int dt = 0; dt < 2; ++dt)
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) o[qb][dt] = Mma<T>::mma(vops.v[t][dt], p[qb][t], o[qb][dt]);
    __builtin_amdgcn_sched_barrier(0);
    op8 ka[4], kb[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) ka[t] = tile_op(kl, 0, t);
    const f32x16 ca = key_bias(bl, 0);
    __builtin_amdgcn_sched_barrier(0);
    // The second half's K reads go out between the last two P.V k-steps and
    // ahead of every score MFMA (left to itself the scheduler sinks them
    // below the first score MFMAs to reuse ka's registers, four MFMAs before
    // their use); issuing ka earlier than this, under the V^T reads still in
    // flight, is slower.
#pragma unroll
    for (int dt = 0; dt < 2; ++dt)
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) o[qb][dt] = Mma<T>::mma(vops.v[2][dt], p[qb][2], o[qb][dt]);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int t = 0; t < 4; ++t) kb[t] = tile_op(kl, 1, t);
    const f32x16 cb = key_bias(bl, 1);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int dt = 0; dt < 2; ++dt)
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) o[qb][dt] = Mma<T>::mma(vops.v[3][dt], p[qb][3], o[qb][dt]);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      s[qb][0] = Mma<T>::mma(ka[0], qreg[qb][0], ca);
#pragma unroll
      for (int t = 1; t < 4; ++t) s[qb][0] = Mma<T>::mma(ka[t], qreg[qb][t], s[qb][0]);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      s[qb][1] = Mma<T>::mma(kb[0], qreg[qb][0], cb);
#pragma unroll
      for (int t = 1; t < 4; ++t) s[qb][1] = Mma<T>::mma(kb[t], qreg[qb][t], s[qb][1]);
    }
    // Sub-tile 0's scores into the exp2 domain under sub-tile 1's MFMAs.
#pragma unroll
    for (int qb = 0; qb < QB; ++qb)
#pragma unroll
      for (int r = 0; r < 16; ++r) s[qb][0][r] = fmaf(s[qb][0][r], kLog2e, nm[qb]);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
      __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);  // four VALU
    }
  }

  // Normalised output rows qw0.. (rows past n_query are not stored).
  __device__ __forceinline__ void store_out(T* ob_ptr, int64_t osn, int qw0, int nq) const {
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      const float ltot = half_sum(lsum[qb]);
      const int row = qw0 + qb * 32 + l32;
      if (row < nq) {
#pragma unroll
        for (int dt = 0; dt < 2; ++dt) {
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            op4 val;
#pragma unroll
            for (int e = 0; e < 4; ++e) val[e] = static_cast<T>(o[qb][dt][4 * g + e] / ltot);
            *reinterpret_cast<op4*>(ob_ptr + row * osn + dt * 32 + 8 * g + 4 * hh) = val;
          }
        }
      }
    }
  }

  // Partial state of a task of `qblock` queries (O unnormalised, then mref,
  // then the sum of every query); this wave's queries start at ql0.
  __device__ __forceinline__ void store_partial(float* partial, int qblock, int ql0) const {
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      const int ql = ql0 + qb * 32 + l32;
      float* po = partial + ql * kD;
#pragma unroll
      for (int dt = 0; dt < 2; ++dt)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const f32x4 val = {o[qb][dt][4 * g], o[qb][dt][4 * g + 1], o[qb][dt][4 * g + 2],
                             o[qb][dt][4 * g + 3]};
          *reinterpret_cast<f32x4*>(po + dt * 32 + 8 * g + 4 * hh) = val;
        }
      const float ltot = half_sum(lsum[qb]);
      if (hh == 0) {
        partial[qblock * kD + ql] = mref[qb];
        partial[qblock * kD + qblock + ql] = ltot;
      }
    }
  }
};

// ------------------------------------------- register-staged kernel -------
// One work-group (4 waves x 64 queries) per 256-query task of one (batch,
// head), no workspace.  K/V tiles are double-buffered in LDS: the next tile's
// rows are loaded into registers while the current tile is computed, then
// stored to the other buffer (K row-major, V transposed into V^T in the MFMA
// key order) -- one barrier per tile.
template <typename T>
__global__ __launch_bounds__(kWaves * 64, 2) void attn_reg_kernel(AttnArgs<T> a) {
  typedef typename Mma<T>::op8 op8;
  typedef typename Mma<T>::op2 op2;
  __shared__ __attribute__((aligned(16))) T k_lds[2 * kTileElems];
  __shared__ __attribute__((aligned(16))) T vt_lds[2 * kTileElems];
  __shared__ __attribute__((aligned(16))) float b_lds[2 * kBN];
  const int task = static_cast<int>(xcd_remap(blockIdx.x, gridDim.x));
  const int bh = task / a.n_qblocks;
  const int qblk = task - bh * a.n_qblocks;
  const int b = bh / a.heads;
  const int h = bh - b * a.heads;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // Wave-uniform (scalar): the loop variants below hold barriers, so the
  // branch between them must be a plain branch that each wave takes one way.
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int qw0 = qblk * kQBlock + wave * kQPerWave;
  const T* kb_ptr = a.k + b * a.ksb + h * a.ksh;
  const T* vb_ptr = a.v + b * a.vsb + h * a.vsh;

  // K: rows st and st+32, chunk sc.  V: keys 2st, 2st+1, dims 8sc..8sc+7.
  // Row offsets fit in 32 bits (checked on the host).
  const int last_key = a.nk - 1;
  const int ksn = static_cast<int>(a.ksn), vsn = static_cast<int>(a.vsn);
  const int st = tid >> 3;
  const int sc = tid & 7;
  const int kw0 = st * kD + ((sc ^ swz(st)) << 3);
  const int kw1 = (st + 32) * kD + ((sc ^ swz(st + 32)) << 3);
  const int vpos = vt_pos(2 * st);
  const int vphys = (vpos >> 3) ^ sc;  // chunk of dim 8sc+i is vphys ^ i
  const int vbase = 8 * sc * kD + (vpos & 7);
  const T* kcol = kb_ptr + 8 * sc;
  const T* vcol = vb_ptr + 8 * sc;

  // Rows past n_key read a valid row; their bias is -inf.
  op8 pk0, pk1, pv0, pv1;
  T pb = static_cast<T>(0.0f);
  auto stage_load = [&](int tile) {
    const int kt = tile * kBN;
    pk0 = *reinterpret_cast<const op8*>(kcol + min(kt + st, last_key) * ksn);
    pk1 = *reinterpret_cast<const op8*>(kcol + min(kt + st + 32, last_key) * ksn);
    pv0 = *reinterpret_cast<const op8*>(vcol + min(kt + 2 * st, last_key) * vsn);
    pv1 = *reinterpret_cast<const op8*>(vcol + min(kt + 2 * st + 1, last_key) * vsn);
    if (a.bias) pb = a.bias[min(kt + lane, last_key)];
  };
  // Every wave writes the same 64 key biases (branch-free; identical data).
  auto stage_store = [&](int tile, int buf) {
    T* kl = k_lds + buf * kTileElems;
    T* vl = vt_lds + buf * kTileElems;
    *reinterpret_cast<op8*>(kl + kw0) = pk0;
    *reinterpret_cast<op8*>(kl + kw1) = pk1;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const op2 pr = {pv0[i], pv1[i]};
      *reinterpret_cast<op2*>(vl + vbase + i * kD + ((vphys ^ i) << 3)) = pr;
    }
    const bool valid = tile * kBN + lane < a.nk;
    b_lds[buf * kBN + lane] = valid ? (a.bias ? to_f32(pb) : 0.0f) : -__builtin_inff();
  };

  // The tile loop with qbs::value query blocks per wave; every variant meets
  // the same ntiles + 1 barriers.
  auto run = [&](auto qbs) {
    constexpr int QB = decltype(qbs)::value;
    WaveAttn<T, QB> w;
    w.init(a.q + b * a.qsb + h * a.qsh, a.qsn, qw0, a.nq, a.c);
    stage_load(0);
    stage_store(0, 0);
    __syncthreads();
    // Tile `tile` (first: tile 0, whose softmax starts from its raw logits).
    auto step = [&](auto first, int tile) {
      const int buf = tile & 1;
      const bool more = tile + 1 < a.ntiles;
      if (more) stage_load(tile + 1);
      const T* kl = k_lds + buf * kTileElems;
      const float* bl = b_lds + buf * kBN;
      // A wave whose 64 queries all lie past n_query (the short last block of
      // a problem) only stages tiles and meets the barriers; its SIMD is then
      // free for the other work-group resident on the CU.
      if (qw0 < a.nq) {
        f32x16 s[QB][2];
        op8 p[QB][4];
        if constexpr (decltype(first)::value) {
          w.template scores<true>(kl, bl, s);
          w.softmax_first(s, p);
        } else {
          w.scores(kl, bl, s);
          w.softmax(s, kl, bl, p);
        }
        w.pv(vt_lds + buf * kTileElems, p);
      }
      if (more) stage_store(tile + 1, buf ^ 1);
      __syncthreads();
    };
    step(std::true_type{}, 0);
    for (int tile = 1; tile < a.ntiles; ++tile) step(std::false_type{}, tile);
    w.store_out(a.out + b * a.osb + h * a.osh, a.osn, qw0, a.nq);
  };
  // A wave whose second 32-query block lies wholly past n_query (the 5 queries
  // past 4 x 256 of a frame's 1,029) computes its first block only.
  if (qw0 < a.nq && qw0 + 32 >= a.nq)
    run(std::integral_constant<int, 1>{});
  else
    run(std::integral_constant<int, kQB>{});
}

// ------------------------------------------------- ping-pong kernel -------
// Workspace path.  A task is 512 queries of one (batch, head): 8 waves x 64
// queries in two groups of four; a SIMD holds one wave of each group (waves w
// and w + 4).  Half-periods end at work-group barriers, and in each one group
// runs its softmax (VALU) while the other runs its MFMAs, so both pipes of
// every SIMD stay busy:
//   H0:   group 0 S(0)                group 1 --
//   A_j:  group 0 softmax(j)          group 1 P.V(j-1), S(j)
//   B_j:  group 0 P.V(j), S(j+1)      group 1 softmax(j)
//   H_n:  group 0 --                  group 1 P.V(n-1)
// K/V^T/bias tiles arrive by LDS DMA in a 4-stage ring (tile j in stage
// j & 3), tile j + 3 issued by group 0 at the start of B_j (under its
// MFMAs); tile j is read from B_{j-1} to A_{j+1}.  Only group 0 issues DMAs: the compiler does not
// see them, and a wait it inserts for its own memory operations (a register
// reload, say) would also wait for every DMA in flight; group 0's loop has
// none, group 1 then has no DMA to wait for.
constexpr int kPPWaves = 8;
constexpr int kPPQBlock = kPPWaves * kQPerWave;  // 512 queries per task
constexpr int kPPStages = 4;
// Per group-0 wave and tile: two K blocks, two V^T blocks, the bias.
constexpr int kPPDmaPerTile = 5;
// Partial state of one stream-K segment: O (fp32, unnormalised), then the
// reference max and the sum of every query of the task.
constexpr int kPartialFloats = kPPQBlock * kD + 2 * kPPQBlock;

// Keep x computed before this point / treat it as redefined after it: holds
// each phase's work on its side of a barrier.
template <typename V>
__device__ __forceinline__ void pin_in(const V& x) {
#if __HIP_DEVICE_COMPILE__
  asm volatile("" ::"v"(x));
#endif
}
template <typename V>
__device__ __forceinline__ void pin_out(V& x) {
#if __HIP_DEVICE_COMPILE__
  asm volatile("" : "+v"(x));
#endif
}

// Work-group barrier of the DMA ring: this wave's LDS reads are complete (a
// stage is overwritten only after every wave has passed a later barrier), at
// most N of its DMAs are outstanding (N < 0: no wait; the wave issues none),
// and no memory access moves across.
template <int N>
__device__ __forceinline__ void ring_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  if constexpr (N >= 0) wait_vmem<N>();
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// The same barrier without waiting for this wave's LDS reads: V^T operands
// requested at the end of a softmax phase for the next MFMA phase stay in
// flight across it.  They read a stage that the DMA overwrites only two
// barriers later, and the compiler waits for them before their first use.
template <int N>
__device__ __forceinline__ void ring_barrier_reads_in_flight() {
  asm volatile("" ::: "memory");
  if constexpr (N >= 0) wait_vmem<N>();
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

template <typename T>
__device__ __forceinline__ void attn_pp_segment(const AttnArgs<T>& a, T* k_lds, T* vt_lds, float* b_lds,
                                                int bh, int qblk, int tile0, int tile1, float* partial) {
  typedef typename Mma<T>::op8 op8;
  const int b = bh / a.heads;
  const int h = bh - b * a.heads;
  const int lane = threadIdx.x & 63;
  // Wave-uniform (scalar) so the two groups' paths are plain branches.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int group = wave >> 2;
  const int qw0 = qblk * kPPQBlock + wave * kQPerWave;
  const T* kb_ptr = a.k + b * a.ksb + h * a.ksh;
  const T* vt_head = a.vt + static_cast<int64_t>(bh) * kD * a.npad;
  const int last_key = a.nk - 1;
  const int ksn = static_cast<int>(a.ksn);

  WaveAttn<T> w;
  w.init(a.q + b * a.qsb + h * a.qsh, a.qsn, qw0, a.nq, a.c);
  // The Q loads complete here, so no compiler-inserted wait for them (which
  // would count the untracked DMAs too) lands inside the ring.
  wait_vmem<0>();

  // Per tile each group-0 wave issues rows 16*wave.. 16*wave+15 of K and of
  // V^T as two 8-row blocks (lane i: row i/8, physical chunk i%8, i.e. the
  // global chunk (i%8) ^ swz(row)) and the tile's 64 key biases (every wave
  // the same, so the count is uniform).
  const int dr = lane >> 3;
  const int dc = lane & 7;
  const int row0 = 16 * wave + dr;
  const int lc0 = dc ^ swz(row0), lc1 = dc ^ swz(row0 + 8);
  // Byte offsets of the lane's rows from the tile's first key; the tile's base
  // moves in scalar registers, so a full tile's DMAs take no VALU work (which
  // would run between the MFMAs, waiting for the VALU issue that the other
  // group's softmax holds).  The offsets fit in 32 bits (checked on the host).
  const uint32_t k_off0 = (static_cast<uint32_t>(row0) * ksn + lc0 * 8) * sizeof(T);
  const uint32_t k_off1 = (static_cast<uint32_t>(row0 + 8) * ksn + lc1 * 8) * sizeof(T);
  const uint32_t v_off0 = (static_cast<uint32_t>(row0) * a.npad + lc0 * 8) * sizeof(T);
  const uint32_t v_off1 = (static_cast<uint32_t>(row0 + 8) * a.npad + lc1 * 8) * sizeof(T);
  const uint32_t b_off = lane * sizeof(float);
  auto issue = [&](int tile) {
    const int stage = tile & (kPPStages - 1);
    const int kt = min(tile, a.ntiles - 1) * kBN;
    T* kst = k_lds + stage * kTileElems + 16 * wave * kD;
    T* vst = vt_lds + stage * kTileElems + 16 * wave * kD;
    if (kt + kBN <= a.nk) {
      const T* kbase = kb_ptr + static_cast<int64_t>(kt) * ksn;
      lds_dma16(kbase, k_off0, lds_offset(kst));
      lds_dma16(kbase, k_off1, lds_offset(kst + 8 * kD));
    } else {  // the last tile: rows past n_key read the last key (their bias is -inf)
      lds_dma16(kb_ptr, (static_cast<uint32_t>(min(kt + row0, last_key) * ksn) + lc0 * 8) * sizeof(T),
                lds_offset(kst));
      lds_dma16(kb_ptr, (static_cast<uint32_t>(min(kt + row0 + 8, last_key) * ksn) + lc1 * 8) * sizeof(T),
                lds_offset(kst + 8 * kD));
    }
    lds_dma16(vt_head + kt, v_off0, lds_offset(vst));
    lds_dma16(vt_head + kt, v_off1, lds_offset(vst + 8 * kD));
    lds_dma4(a.kbias + kt, b_off, lds_offset(b_lds + stage * kBN));
  };
  auto kl = [&](int tile) { return k_lds + (tile & (kPPStages - 1)) * kTileElems; };
  auto vl = [&](int tile) { return vt_lds + (tile & (kPPStages - 1)) * kTileElems; };
  auto bl = [&](int tile) { return b_lds + (tile & (kPPStages - 1)) * kBN; };

  f32x16 s[kQB][2];
  op8 p[kQB][4];
  auto pin_scores = [&]() {
#pragma unroll
    for (int qb = 0; qb < kQB; ++qb)
#pragma unroll
      for (int sub = 0; sub < 2; ++sub) {
        pin_in(s[qb][sub]);
        pin_in(w.o[qb][sub]);
      }
  };
  auto pin_probs = [&]() {
#pragma unroll
    for (int qb = 0; qb < kQB; ++qb) {
#pragma unroll
      for (int t = 0; t < 4; ++t) pin_in(p[qb][t]);
      pin_in(w.lsum[qb]);
    }
  };
  auto pin_sums = [&](const float (&part)[kQB]) {
#pragma unroll
    for (int qb = 0; qb < kQB; ++qb) pin_in(part[qb]);
  };
  // The rescaling path of the lazy softmax for tile `tile`, taken at the
  // start of the MFMA phase after the softmax phase that found the tile's
  // probabilities out of range (a branch at the end of that phase would
  // hold the wave until the check's whole dependency chain has drained).
  // The tile's V^T operands in flight are dropped and read again, so their
  // registers are free meanwhile.
  auto redo = [&](int tile, float (&part)[kQB], typename WaveAttn<T>::VOps& vops) {
    w.rescale(kl(tile), bl(tile), p, part);
    w.load_v(vl(tile), vops);
  };
  auto renew_scores = [&]() {
#pragma unroll
    for (int qb = 0; qb < kQB; ++qb)
#pragma unroll
      for (int sub = 0; sub < 2; ++sub) pin_out(s[qb][sub]);
  };
  auto renew_probs = [&]() {
#pragma unroll
    for (int qb = 0; qb < kQB; ++qb)
#pragma unroll
      for (int t = 0; t < 4; ++t) pin_out(p[qb][t]);
  };

  // A wave whose 64 queries all lie past the problem's end (the last task of
  // a problem whose query count is not a multiple of 512, e.g. the special
  // queries' 160) computes nothing: it issues its share of the DMAs (group 0)
  // and meets the same 2 n + 3 barriers, and its SIMD's other wave runs its
  // phases alone.  Its rows are never stored or merged.
  if (qw0 >= a.nq) {
    const int n = tile1 - tile0;
    if (group == 0) {
      issue(tile0);
      issue(tile0 + 1);
      issue(tile0 + 2);
      ring_barrier<2 * kPPDmaPerTile>();
      ring_barrier<2 * kPPDmaPerTile>();
      for (int tile = tile0; tile < tile1; ++tile) {
        ring_barrier_reads_in_flight<kPPDmaPerTile>();
        issue(tile + 3);
        ring_barrier<2 * kPPDmaPerTile>();
      }
      ring_barrier<0>();
    } else {
      for (int i = 0; i < 2 * n + 3; ++i) ring_barrier<-1>();
    }
    return;
  }

  if (group == 0) {
    issue(tile0);
    issue(tile0 + 1);
    issue(tile0 + 2);
    ring_barrier<2 * kPPDmaPerTile>();  // tile0 has landed
    w.scores(kl(tile0), bl(tile0), s);  // H0
    pin_scores();
    ring_barrier<2 * kPPDmaPerTile>();
    renew_scores();
    for (int tile = tile0; tile < tile1; ++tile) {
      float part[kQB];
      const bool over = w.softmax_fast(s, p, part);  // A_j
      pin_probs();
      pin_sums(part);
      __builtin_amdgcn_sched_barrier(0);
      typename WaveAttn<T>::VOps vops;
      w.load_v(vl(tile), vops);  // B_j's first operands, in flight across the barrier
      ring_barrier_reads_in_flight<kPPDmaPerTile>();  // tile + 1 has landed
      renew_probs();
      // B_j.  A tile that failed the lazy check is redone first (its stage
      // stays valid until A_{j+1}).
      if (__builtin_expect(over, 0)) redo(tile, part, vops);
      w.commit(part);
      // Tile j + 3 refills the stage of tile j - 1, whose last reads
      // (group 1's, in A_j) completed before the barrier just passed; the
      // DMA issue runs under this phase's MFMAs rather than the softmax.
      // After the last tile the scores of the look-ahead tile go unused.
      issue(tile + 3);
      w.pv_scores(vops, p, kl(tile + 1), bl(tile + 1), s);
      pin_scores();
      ring_barrier<2 * kPPDmaPerTile>();
      renew_scores();
    }
    ring_barrier<0>();  // H_n; the look-ahead DMAs have landed
  } else {
    ring_barrier<-1>();  // tile0 has landed
    ring_barrier<-1>();  // H0
    w.scores(kl(tile0), bl(tile0), s);  // A_0 (no P.V yet)
    pin_scores();
    ring_barrier<-1>();
    renew_scores();
    float part[kQB];
    bool over = w.softmax_fast(s, p, part);  // B_0
    pin_probs();
    pin_sums(part);
    __builtin_amdgcn_sched_barrier(0);
    typename WaveAttn<T>::VOps vops;
    w.load_v(vl(tile0), vops);
    ring_barrier_reads_in_flight<-1>();
    for (int tile = tile0 + 1; tile < tile1; ++tile) {
      renew_probs();
      // A_j: tile j - 1 redone if it failed the lazy check, its P.V, S(j).
      if (__builtin_expect(over, 0)) redo(tile - 1, part, vops);
      w.commit(part);
      w.pv_scores(vops, p, kl(tile), bl(tile), s);
      pin_scores();
      ring_barrier<-1>();
      renew_scores();
      over = w.softmax_fast(s, p, part);  // B_j
      pin_probs();
      pin_sums(part);
      __builtin_amdgcn_sched_barrier(0);
      w.load_v(vl(tile), vops);
      ring_barrier_reads_in_flight<-1>();
    }
    renew_probs();
    if (__builtin_expect(over, 0)) redo(tile1 - 1, part, vops);
    w.commit(part);
    w.pv(vops, p);  // H_n
    pin_scores();
    ring_barrier<-1>();
  }

  if (partial == nullptr)
    w.store_out(a.out + b * a.osb + h * a.osh, a.osn, qw0, a.nq);
  else
    w.store_partial(partial, kPPQBlock, wave * kQPerWave);
}

// One work-group walks the units [sk_begin(w), sk_begin(w+1)) of the flattened
// (task, key tile) space; a task is a (batch*head, 512-query block) pair of
// one problem.  A segment that covers a whole task writes the output; a
// segment that covers a part writes its partial state (slot 0: the
// work-group's first segment, slot 1: its last), which attn_merge_kernel
// combines.  Only a range's first and last segments can be partial: the
// units of a task are contiguous and problem 1's start at a task boundary.
template <typename T>
__global__ __launch_bounds__(kPPWaves * 64, 1) void attn_pp_kernel(PPLaunch<T> L) {
  __shared__ __attribute__((aligned(16))) T k_lds[kPPStages * kTileElems];
  __shared__ __attribute__((aligned(16))) T vt_lds[kPPStages * kTileElems];
  __shared__ __attribute__((aligned(16))) float b_lds[kPPStages * kBN];
  const PPSchedule& sc = L.s;
  // Clock samples: read here, stored after the last segment (a store before the
  // segments would have to be assumed to alias the kernel arguments they read).
  const unsigned long long clock0 = sc.stamps != nullptr ? __builtin_amdgcn_s_memtime() : 0;
  const unsigned long long const0 = sc.stamps != nullptr ? __builtin_amdgcn_s_memrealtime() : 0;
  const int64_t w = xcd_remap(blockIdx.x, gridDim.x);
  // Whole tasks first: consecutive work-groups (one XCD's, after the remap)
  // take consecutive tasks of a round, so they stream one head's K/V in step
  // and share it in that XCD's L2.  Then the stream-K range.  One call site
  // for both keeps a single copy of the segment code.
  int64_t r = 0;
  int64_t u = 0, u_end = 0;
  if (w < sc.tail_groups) {
    u = sk_begin(w, sc.units, sc.tail_groups);
    u_end = sk_begin(w + 1, sc.units, sc.tail_groups);
  }
  bool first = true;
  for (;;) {
    int second, bh, qblk, tile0, tile1;
    float* partial = nullptr;
    if (r < sc.full_rounds) {
      const int64_t task = w + r * sc.groups;
      ++r;
      second = 0;
      bh = static_cast<int>(task / L.p[0].n_qblocks);
      qblk = static_cast<int>(task - static_cast<int64_t>(bh) * L.p[0].n_qblocks);
      tile0 = 0;
      tile1 = L.p[0].ntiles;
    } else if (u < u_end) {
      second = u >= sc.units0 ? 1 : 0;
      const int ntiles = L.p[second].ntiles;
      const int64_t base = second ? sc.units0 : 0;
      const int64_t tt = (u - base) / ntiles;  // tail task of the problem
      tile0 = static_cast<int>(u - base - tt * ntiles);
      const int64_t seg_end = min(u_end, base + (tt + 1) * ntiles);
      tile1 = static_cast<int>(seg_end - base - tt * ntiles);
      const int64_t task = (second ? 0 : sc.tail_task0) + tt;
      const int n_qblocks = L.p[second].n_qblocks;
      bh = static_cast<int>(task / n_qblocks);
      qblk = static_cast<int>(task - static_cast<int64_t>(bh) * n_qblocks);
      if (tile0 != 0 || tile1 != ntiles)
        partial = sc.partial + (2 * w + (first ? 0 : 1)) * static_cast<int64_t>(kPartialFloats);
      u = seg_end;
      first = false;
    } else {
      break;
    }
    attn_pp_segment<T>(L.p[second], k_lds, vt_lds, b_lds, bh, qblk, tile0, tile1, partial);
  }
  if (sc.stamps != nullptr && threadIdx.x == 0) {
    const unsigned long long clock1 = __builtin_amdgcn_s_memtime();
    const unsigned long long const1 = __builtin_amdgcn_s_memrealtime();
    sc.stamps[4 * blockIdx.x] = clock0;
    sc.stamps[4 * blockIdx.x + 1] = const0;
    sc.stamps[4 * blockIdx.x + 2] = clock1;
    sc.stamps[4 * blockIdx.x + 3] = const1;
  }
}

// Combines the partial states of every tail task split across work-groups.
// Block b handles tail task b / kMergeSplit (problem 0's tail tasks, then
// problem 1's tasks), queries (b % kMergeSplit) * kPPQBlock / kMergeSplit
// onwards; 16 threads per query, 4 dims each.  Partial states are read eight
// at a time so their loads overlap.  32 blocks per task (16 queries each):
// with 16 tail tasks at C4 that is 512 work-groups, two per CU (8 per task
// left half the CUs idle: 6 us more per launch).
constexpr int kMergeSplit = 32;
template <typename T>
__global__ __launch_bounds__(256) void attn_merge_kernel(PPLaunch<T> L) {
  const PPSchedule& sc = L.s;
  const int64_t tt_all = blockIdx.x / kMergeSplit;
  const int qpart = blockIdx.x % kMergeSplit;
  const int second = tt_all >= sc.tail_tasks0 ? 1 : 0;
  const AttnArgs<T>& a = L.p[second];
  const int64_t tt = second ? tt_all - sc.tail_tasks0 : tt_all;
  const int64_t t0 = (second ? sc.units0 : 0) + tt * a.ntiles;
  const int64_t w0 = sk_owner(t0, sc.units, sc.tail_groups);
  const int64_t w1 = sk_owner(t0 + a.ntiles - 1, sc.units, sc.tail_groups);
  if (w1 == w0) return;  // whole inside one work-group: already written
  const int first_slot = sk_begin(w0, sc.units, sc.tail_groups) < t0 ? 1 : 0;
  const int64_t task = (second ? 0 : sc.tail_task0) + tt;
  const int bh = static_cast<int>(task / a.n_qblocks);
  const int qblk = static_cast<int>(task - static_cast<int64_t>(bh) * a.n_qblocks);
  const int b = bh / a.heads;
  const int h = bh - b * a.heads;
  T* ob_ptr = a.out + b * a.osb + h * a.osh;
  const int d0 = (threadIdx.x & 15) * 4;
  auto slot_ptr = [&](int64_t w) {
    const int slot = w == w0 ? first_slot : 0;
    return sc.partial + (2 * w + slot) * static_cast<int64_t>(kPartialFloats);
  };
  for (int ql = qpart * (kPPQBlock / kMergeSplit) + (threadIdx.x >> 4);
       ql < (qpart + 1) * (kPPQBlock / kMergeSplit); ql += 16) {
    const int row = qblk * kPPQBlock + ql;
    if (row >= a.nq) break;
    float mmax = -__builtin_inff();
    for (int64_t wb = w0; wb <= w1; wb += 8) {
      float mv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) mv[e] = wb + e <= w1 ? slot_ptr(wb + e)[kPPQBlock * kD + ql] : -__builtin_inff();
#pragma unroll
      for (int e = 0; e < 8; ++e) mmax = fmaxf(mmax, mv[e]);
    }
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    float l = 0.0f;
    for (int64_t wb = w0; wb <= w1; wb += 8) {
      float mv[8], lv[8];
      f32x4 xv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        if (wb + e <= w1) {
          const float* p = slot_ptr(wb + e);
          mv[e] = p[kPPQBlock * kD + ql];
          lv[e] = p[kPPQBlock * kD + kPPQBlock + ql];
          xv[e] = *reinterpret_cast<const f32x4*>(p + ql * kD + d0);
        }
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        if (wb + e <= w1) {
          const float f = __builtin_amdgcn_exp2f((mv[e] - mmax) * kLog2e);
#pragma unroll
          for (int q = 0; q < 4; ++q) acc[q] = fmaf(xv[e][q], f, acc[q]);
          l = fmaf(lv[e], f, l);
        }
      }
    }
    typedef typename Mma<T>::op4 op4;
    op4 val;
#pragma unroll
    for (int q = 0; q < 4; ++q) val[q] = static_cast<T>(acc[q] / l);
    *reinterpret_cast<op4*>(ob_ptr + row * a.osn + d0) = val;
  }
}

// fp32: one query per lane; 64 queries per work-group; K/V tiles of 64 keys.
constexpr int kF32Keys = 64;
constexpr int kF32Chunk = 32;  // keys summed on their own before joining the running sums
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
    // 32 keys at a time, each chunk's P and P.V summed on their own and then added to
    // the running totals: the rounding of the sums grows with sqrt(32) + sqrt(nk / 32)
    // instead of sqrt(nk), which keeps the output within 1e-5 of the exact result at
    // tens of thousands of keys.
#pragma unroll
    for (int j0 = 0; j0 < kF32Keys; j0 += kF32Chunk) {
      float logit[kF32Chunk];
      float mx = -__builtin_inff();
#pragma unroll
      for (int j = 0; j < kF32Chunk; ++j) {
        float dot = 0.0f;
#pragma unroll
        for (int d = 0; d < kD; ++d) dot = fmaf(qr[d], k_lds[j0 + j][d], dot);
        logit[j] = dot * scale_log2 + b_lds[j0 + j];
        mx = fmaxf(mx, logit[j]);
      }
      const float mnew = fmaxf(m, mx);
      // No finite logit yet (every key so far of mass 0): every P is 0 and the
      // sums stay 0, where -inf - -inf would make them NaN.
      const float base = mnew == -__builtin_inff() ? 0.0f : mnew;
      const float corr = exp2f(m - base);
      float lc = 0.0f, accc[kD];
#pragma unroll
      for (int d = 0; d < kD; ++d) accc[d] = 0.0f;
#pragma unroll
      for (int j = 0; j < kF32Chunk; ++j) {
        const float p = exp2f(logit[j] - base);
        lc += p;
#pragma unroll
        for (int d = 0; d < kD; ++d) accc[d] = fmaf(p, v_lds[j0 + j][d], accc[d]);
      }
      l = fmaf(l, corr, lc);
#pragma unroll
      for (int d = 0; d < kD; ++d) acc[d] = fmaf(acc[d], corr, accc[d]);
      m = mnew;
    }
  }
  if (row < nq) {
    float* orow = out + b * osb + h * osh + static_cast<int64_t>(row) * osn;
#pragma unroll
    for (int d = 0; d < kD; ++d) orow[d] = acc[d] / l;
  }
}

// Packs V of every (batch, head) into V^T tiles for the DMA kernel:
// vt[bh][d][j'] = V[bh][key j][d] with j' = vt_pos(j) inside each 16-key group
// (the key order of the P operand), zeros past n_key, npad = ntiles * 64
// columns; and kbias[j] = bias[j] as fp32 (0 without a bias) for j < n_key,
// -inf up to npad.  One block per (64-key tile, bh).
template <typename T>
__global__ __launch_bounds__(256) void vt_pack_kernel(const T* __restrict__ v, int heads, int nk,
                                                      int ntiles, int npad, int64_t vsb, int64_t vsh,
                                                      int64_t vsn, const T* __restrict__ bias,
                                                      T* __restrict__ vt, float* __restrict__ kbias) {
  typedef typename Mma<T>::op8 op8;
  constexpr int kRow = kD + 2;  // padded LDS row
  __shared__ T tile[kBN * kRow];
  const int tix = blockIdx.x;
  const int bh = blockIdx.y;
  const int b = bh / heads;
  const int h = bh - b * heads;
  const int kt = tix * kBN;
  const int tid = threadIdx.x;
  const T* vb = v + b * vsb + h * vsh;
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const int r = (tid >> 3) + 32 * p;
    const int c0 = (tid & 7) * 8;
    op8 x = {};
    if (kt + r < nk) x = *reinterpret_cast<const op8*>(vb + static_cast<int64_t>(kt + r) * vsn + c0);
#pragma unroll
    for (int e = 0; e < 8; ++e) tile[r * kRow + c0 + e] = x[e];
  }
  __syncthreads();
  {
    const int d = tid >> 2;
    const int g = (tid & 3) * 16;  // 16 positions g..g+15 of row d
    op8 lo, hi;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      lo[e] = tile[vt_pos(g + e) * kRow + d];
      hi[e] = tile[vt_pos(g + 8 + e) * kRow + d];
    }
    T* dst = vt + (static_cast<int64_t>(bh) * kD + d) * npad + kt + g;
    *reinterpret_cast<op8*>(dst) = lo;
    *reinterpret_cast<op8*>(dst + 8) = hi;
  }
  if (bh == 0 && tid < kBN) {
    const int j = kt + tid;
    kbias[j] = j < nk ? (bias ? to_f32(bias[j]) : 0.0f) : -__builtin_inff();
  }
}

// Resident work-groups of attn_pp_kernel<T> on the current device (CUs x
// blocks per CU), cached per device.
template <typename T>
int64_t resident_groups() {
  static int cache[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (cache[dev] == 0) {
    int cus = 0, per_cu = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      return 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, attn_pp_kernel<T>, kPPWaves * 64, 0) !=
        hipSuccess)
      return 0;
    cache[dev] = cus * (per_cu > 0 ? per_cu : 1);
  }
  return cache[dev];
}

constexpr int64_t kMinUnitsPerGroup = 8;  // key tiles per work-group, at least

// A split tail task is cut into at most about this many pieces, which bounds
// the partial states attn_merge_kernel reads per query.
constexpr int64_t kMaxPieces = 32;

// One attention problem of a call, as the C ABI describes it.
struct Problem {
  const void* q;
  const void* k;
  const void* v;
  const void* bias;
  void* out;
  int64_t batch, heads, nq, nk;
  const int64_t* qs;
  const int64_t* ks;
  const int64_t* vs;
  const int64_t* os;
};

// The stream-K schedule of an attn_pp_kernel launch over `count` problems;
// the workspace query and the launch compute the same one on one device.
struct PPPlan {
  int count;
  int64_t tasks[2], ntiles[2];
  PPSchedule s;
};

template <typename T>
PPPlan pp_plan(const Problem* pr, int count) {
  PPPlan plan{};
  plan.count = count;
  int64_t units_all = 0, max_tiles = 1;
  for (int i = 0; i < count; ++i) {
    plan.tasks[i] = (pr[i].nq + kPPQBlock - 1) / kPPQBlock * pr[i].batch * pr[i].heads;
    plan.ntiles[i] = (pr[i].nk + kBN - 1) / kBN;
    units_all += plan.tasks[i] * plan.ntiles[i];
    max_tiles = std::max(max_tiles, plan.ntiles[i]);
  }
  const int64_t slots = resident_groups<T>();
  int64_t groups = std::min<int64_t>(slots, (units_all + kMinUnitsPerGroup - 1) / kMinUnitsPerGroup);
  if (groups <= 0) groups = plan.tasks[0] + (count > 1 ? plan.tasks[1] : 0);  // one task per group
  PPSchedule& sc = plan.s;
  sc.partial = nullptr;
  sc.groups = groups;
  sc.full_rounds = plan.tasks[0] / groups;
  sc.tail_task0 = sc.full_rounds * groups;
  sc.tail_tasks0 = plan.tasks[0] - sc.tail_task0;
  sc.units0 = sc.tail_tasks0 * plan.ntiles[0];
  sc.units = sc.units0 + (count > 1 ? plan.tasks[1] * plan.ntiles[1] : 0);
  const int64_t min_units = std::max<int64_t>(kMinUnitsPerGroup, (max_tiles + kMaxPieces - 1) / kMaxPieces);
  sc.tail_groups = sc.units > 0 ? std::min<int64_t>(groups, std::max<int64_t>(1, sc.units / min_units)) : 0;
  return plan;
}

// Workspace of the DMA path: per problem V^T and the fp32 key biases, then the
// partial states (each part 256-byte aligned).
struct AttnWorkspace {
  size_t vt[2], kbias[2], partial, total;
};
inline size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }
inline AttnWorkspace attn_workspace(const PPPlan& plan, const Problem* pr, size_t elem) {
  AttnWorkspace w{};
  size_t at = 0;
  for (int i = 0; i < plan.count; ++i) {
    const int64_t npad = plan.ntiles[i] * kBN;
    w.vt[i] = at;
    at += align256(static_cast<size_t>(pr[i].batch * pr[i].heads) * kD * npad * elem);
    w.kbias[i] = at;
    at += align256(static_cast<size_t>(npad) * sizeof(float));
  }
  w.partial = at;
  w.total = at + (plan.s.units > 0 ? static_cast<size_t>(plan.s.groups) * 2 * kPartialFloats * sizeof(float) : 0);
  return w;
}

template <typename T>
AttnArgs<T> make_args(const Problem& pr, int64_t qblock) {
  AttnArgs<T> a;
  a.q = static_cast<const T*>(pr.q);
  a.k = static_cast<const T*>(pr.k);
  a.v = static_cast<const T*>(pr.v);
  a.bias = static_cast<const T*>(pr.bias);
  a.out = static_cast<T*>(pr.out);
  a.heads = static_cast<int>(pr.heads);
  a.nq = static_cast<int>(pr.nq);
  a.nk = static_cast<int>(pr.nk);
  a.n_qblocks = static_cast<int>((pr.nq + qblock - 1) / qblock);
  a.ntiles = static_cast<int>((pr.nk + kBN - 1) / kBN);
  a.qsb = pr.qs[0], a.qsh = pr.qs[1], a.qsn = pr.qs[2];
  a.ksb = pr.ks[0], a.ksh = pr.ks[1], a.ksn = pr.ks[2];
  a.vsb = pr.vs[0], a.vsh = pr.vs[1], a.vsn = pr.vs[2];
  a.osb = pr.os[0], a.osh = pr.os[1], a.osn = pr.os[2];
  a.c = 0.125f;
  a.vt = nullptr;
  a.kbias = nullptr;
  a.npad = a.ntiles * kBN;
  return a;
}

// No workspace: one 256-query task per work-group of attn_reg_kernel.
template <typename T>
int launch_reg(const Problem& pr, hipStream_t stream) {
  const int64_t tasks = (pr.nq + kQBlock - 1) / kQBlock * pr.batch * pr.heads;
  const int64_t ntiles = (pr.nk + kBN - 1) / kBN;
  VGO_REQUIRE(tasks <= 0x7fffffff && pr.batch * pr.heads <= 0xffff && ntiles < 0x7fffffff / kBN,
              "mass_bias_attention: grid too large");
  const AttnArgs<T> a = make_args<T>(pr, kQBlock);
  hipLaunchKernelGGL((attn_reg_kernel<T>), dim3(static_cast<unsigned>(tasks)), dim3(kWaves * 64), 0,
                     stream, a);
  return check_launch("mass_bias_attention");
}

// Kernel timing (vgo_attn_kernel_timing): while it is on, every attn_pp_kernel
// launch made outside stream capture on the device it was switched on for is
// bracketed by a pair of HIP events from a fixed pool, so the kernel's own
// duration can be read without the V^T pack and the merge around it.
// The first kClockSlots timed launches of up to kClockGroups work-groups also
// carry clock samples (PPSchedule::stamps), in a buffer allocated on the device
// when timing is switched on there.
constexpr int kTimingSlots = 4096;
constexpr int kClockSlots = 512;
constexpr int64_t kClockGroups = 1024;
struct KernelTiming {
  std::mutex mutex;
  bool on = false;
  int device = -1;
  int used = 0;
  int64_t dropped = 0;
  hipEvent_t start[kTimingSlots] = {};
  hipEvent_t stop[kTimingSlots] = {};
  unsigned long long* stamps = nullptr;  // kClockSlots x kClockGroups x 4, on `device`
  int64_t clock_groups[kClockSlots] = {};  // work-groups of each sampled launch (0: none)
};
KernelTiming& kernel_timing() {
  static KernelTiming t;
  return t;
}

// The event pair for the next launch on `stream` (and, for one of the first
// kClockSlots launches with at most kClockGroups work-groups, its clock-sample
// slice in *stamps, else null), or false when timing is off, the stream is being
// captured or belongs to another device, or the pool is full.
bool timing_slot(hipStream_t stream, int64_t groups, hipEvent_t* start, hipEvent_t* stop,
                 unsigned long long** stamps) {
  *stamps = nullptr;
  KernelTiming& t = kernel_timing();
  std::lock_guard<std::mutex> lock(t.mutex);
  if (!t.on) return false;
  int dev = -1;
  hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
  if (hipGetDevice(&dev) != hipSuccess || dev != t.device ||
      hipStreamIsCapturing(stream, &capture) != hipSuccess || capture != hipStreamCaptureStatusNone)
    return false;
  if (t.used == kTimingSlots) {
    ++t.dropped;
    return false;
  }
  const int i = t.used;
  if (t.start[i] == nullptr && hipEventCreate(&t.start[i]) != hipSuccess) return false;
  if (t.stop[i] == nullptr && hipEventCreate(&t.stop[i]) != hipSuccess) return false;
  ++t.used;
  *start = t.start[i];
  *stop = t.stop[i];
  if (i < kClockSlots) {
    t.clock_groups[i] = 0;
    if (t.stamps != nullptr && groups <= kClockGroups) {
      t.clock_groups[i] = groups;
      *stamps = t.stamps + static_cast<int64_t>(i) * kClockGroups * 4;
    }
  }
  return true;
}

// Workspace path over one or two problems: pack V^T and the bias of each,
// then the ping-pong LDS-DMA kernel, then the merge of split tasks.
template <typename T>
int launch_pp(const Problem* pr, int count, void* workspace, size_t workspace_bytes,
              hipStream_t stream) {
  for (int i = 0; i < count; ++i) {
    const int64_t tasks = (pr[i].nq + kPPQBlock - 1) / kPPQBlock * pr[i].batch * pr[i].heads;
    const int64_t ntiles = (pr[i].nk + kBN - 1) / kBN;
    VGO_REQUIRE(tasks <= 0x7fffffff && pr[i].batch * pr[i].heads <= 0xffff &&
                    ntiles < 0x7fffffff / kBN,
                "mass_bias_attention: grid too large");
  }
  PPPlan plan = pp_plan<T>(pr, count);
  VGO_REQUIRE(plan.s.groups <= 0x7fffffff, "mass_bias_attention: grid too large");
  const AttnWorkspace ws = attn_workspace(plan, pr, sizeof(T));
  if (workspace == nullptr || workspace_bytes < ws.total)
    return fail(VGO_EWORKSPACE, "mass_bias_attention: workspace too small");
  VGO_REQUIRE(aligned(workspace, 256), "mass_bias_attention: workspace must be 256-byte aligned");
  char* base = static_cast<char*>(workspace);
  PPLaunch<T> L{};
  for (int i = 0; i < count; ++i) {
    AttnArgs<T>& a = L.p[i];
    a = make_args<T>(pr[i], kPPQBlock);
    a.vt = reinterpret_cast<T*>(base + ws.vt[i]);
    a.kbias = reinterpret_cast<float*>(base + ws.kbias[i]);
    hipLaunchKernelGGL((vt_pack_kernel<T>),
                       dim3(static_cast<unsigned>(a.ntiles), static_cast<unsigned>(pr[i].batch * pr[i].heads)),
                       dim3(256), 0, stream, a.v, a.heads, a.nk, a.ntiles, a.npad, a.vsb, a.vsh, a.vsn,
                       a.bias, const_cast<T*>(a.vt), const_cast<float*>(a.kbias));
    const int status = check_launch("mass_bias_attention(pack)");
    if (status != VGO_OK) return status;
  }
  if (count == 1) L.p[1] = L.p[0];  // never selected: problem 1 has no units
  L.s = plan.s;
  if (plan.s.units > 0) L.s.partial = reinterpret_cast<float*>(base + ws.partial);
  hipEvent_t t_start = nullptr, t_stop = nullptr;
  const bool timed = timing_slot(stream, plan.s.groups, &t_start, &t_stop, &L.s.stamps);
  if (timed) (void)hipEventRecord(t_start, stream);
  hipLaunchKernelGGL((attn_pp_kernel<T>), dim3(static_cast<unsigned>(plan.s.groups)),
                     dim3(kPPWaves * 64), 0, stream, L);
  int status = check_launch("mass_bias_attention");
  if (timed) (void)hipEventRecord(t_stop, stream);
  if (status != VGO_OK || plan.s.units == 0) return status;
  const int64_t tail_tasks = plan.s.tail_tasks0 + (count > 1 ? plan.tasks[1] : 0);
  hipLaunchKernelGGL((attn_merge_kernel<T>), dim3(static_cast<unsigned>(tail_tasks * kMergeSplit)),
                     dim3(256), 0, stream, L);
  return check_launch("mass_bias_attention(merge)");
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

namespace {

using vgo::Problem;

// Checks one problem; sets *empty when it has no output rows.
int check_problem(const Problem& p, int64_t head_dim, int dtype, bool* empty) {
  using namespace vgo;
  VGO_REQUIRE(head_dim == 64, "mass_bias_attention: only head_dim=64 is supported");
  VGO_REQUIRE(p.batch >= 0 && p.heads >= 0 && p.nq >= 0 && p.nk >= 0,
              "mass_bias_attention: negative size");
  *empty = p.batch == 0 || p.heads == 0 || p.nq == 0;
  if (*empty) return VGO_OK;
  VGO_REQUIRE(p.nk > 0, "mass_bias_attention: no keys");
  VGO_REQUIRE(p.q && p.k && p.v && p.out, "mass_bias_attention: null pointer");
  VGO_REQUIRE(p.qs && p.ks && p.vs && p.os, "mass_bias_attention: null strides");
  VGO_REQUIRE(p.nq <= 0x7fffffff && p.nk <= 0x7fffffff, "mass_bias_attention: too many tokens");
  if (dtype == VGO_BF16 || dtype == VGO_F16) {
    for (int i = 0; i < 3; ++i) {
      VGO_REQUIRE(p.qs[i] % 8 == 0 && p.ks[i] % 8 == 0 && p.vs[i] % 8 == 0 && p.os[i] % 4 == 0,
                  "mass_bias_attention: token/head/batch strides must be multiples of 8 elements");
    }
    VGO_REQUIRE(aligned(p.q, 16) && aligned(p.k, 16) && aligned(p.v, 16) && aligned(p.out, 8),
                "mass_bias_attention: q/k/v must be 16-byte aligned");
    // Token offsets inside one (batch, head) plane are 32-bit in the kernel.
    const int64_t lim = int64_t(1) << 31;
    if (p.nk * std::max<int64_t>(p.ks[2], p.vs[2]) >= lim || p.nq * std::max<int64_t>(p.qs[2], p.os[2]) >= lim)
      return fail(VGO_EUNSUPPORTED, "mass_bias_attention: token stride x tokens exceeds 2^31 elements");
    return VGO_OK;
  }
  if (dtype == VGO_F32) return VGO_OK;
  return fail(VGO_EINVAL, "mass_bias_attention: unsupported dtype");
}

// Runs the non-empty problems of `problems` (count 1 or 2) in one launch of
// the workspace kernel (split) or one launch each of the kernel without one.
int attn_run(const Problem* problems, const int64_t* head_dims, int count, int dtype,
             void* workspace, size_t workspace_bytes, bool split, void* stream) {
  using namespace vgo;
  Problem live[2];
  int n = 0;
  for (int i = 0; i < count; ++i) {
    bool empty = false;
    const int status = check_problem(problems[i], head_dims[i], dtype, &empty);
    if (status != VGO_OK) return status;
    if (!empty) live[n++] = problems[i];
  }
  if (n == 0) return VGO_OK;
  hipStream_t s = as_stream(stream);
  if (dtype == VGO_F32) {
    for (int i = 0; i < n; ++i) {
      const Problem& p = live[i];
      const int status = launch_f32(p.q, p.k, p.v, p.bias, p.out, p.batch, p.heads, p.nq, p.nk, p.qs,
                                    p.ks, p.vs, p.os, s);
      if (status != VGO_OK) return status;
    }
    return VGO_OK;
  }
  if (split)
    return dtype == VGO_BF16 ? launch_pp<bf16_t>(live, n, workspace, workspace_bytes, s)
                             : launch_pp<f16_t>(live, n, workspace, workspace_bytes, s);
  for (int i = 0; i < n; ++i) {
    const int status = dtype == VGO_BF16 ? launch_reg<bf16_t>(live[i], s) : launch_reg<f16_t>(live[i], s);
    if (status != VGO_OK) return status;
  }
  return VGO_OK;
}

// Workspace bytes of the split path (0 for fp32 or when every problem is empty).
int attn_workspace_bytes(const Problem* problems, int count, int dtype, size_t* bytes) {
  using namespace vgo;
  VGO_REQUIRE(bytes, "mass_bias_attention: null size pointer");
  *bytes = 0;
  Problem live[2];
  int n = 0;
  for (int i = 0; i < count; ++i) {
    const Problem& p = problems[i];
    VGO_REQUIRE(p.batch >= 0 && p.heads >= 0 && p.nq >= 0 && p.nk >= 0,
                "mass_bias_attention: negative size");
    if (p.batch == 0 || p.heads == 0 || p.nq == 0 || p.nk == 0) continue;
    live[n++] = p;
  }
  if (n == 0 || dtype == VGO_F32) return VGO_OK;
  VGO_REQUIRE(dtype == VGO_BF16 || dtype == VGO_F16, "mass_bias_attention: unsupported dtype");
  const PPPlan plan = dtype == VGO_BF16 ? pp_plan<bf16_t>(live, n) : pp_plan<f16_t>(live, n);
  *bytes = attn_workspace(plan, live, 2).total;
  return VGO_OK;
}

Problem single_problem(const void* q, const void* k, const void* v, const void* log_mass, void* out,
                       int64_t batch, int64_t heads, int64_t n_query, int64_t n_key,
                       const int64_t* q_stride, const int64_t* k_stride, const int64_t* v_stride,
                       const int64_t* o_stride) {
  return Problem{q, k, v, log_mass, out, batch, heads, n_query, n_key, q_stride, k_stride, v_stride, o_stride};
}

Problem from_c(const vgo_attn_problem& p) {
  return Problem{p.q, p.k, p.v, p.log_mass, p.out, p.batch, p.heads, p.n_query, p.n_key,
                 p.q_stride, p.k_stride, p.v_stride, p.o_stride};
}

}  // namespace

extern "C" int vgo_mass_bias_attn_fwd(const void* q, const void* k, const void* v,
                                      const void* log_mass, void* out, int64_t batch,
                                      int64_t heads, int64_t n_query, int64_t n_key,
                                      int64_t head_dim, const int64_t q_stride[3],
                                      const int64_t k_stride[3], const int64_t v_stride[3],
                                      const int64_t o_stride[3], int dtype, void* stream) {
  const Problem p = single_problem(q, k, v, log_mass, out, batch, heads, n_query, n_key, q_stride,
                                   k_stride, v_stride, o_stride);
  return attn_run(&p, &head_dim, 1, dtype, nullptr, 0, false, stream);
}

extern "C" int vgo_mass_bias_attn_workspace(int64_t batch, int64_t heads, int64_t n_query,
                                            int64_t n_key, int dtype, size_t* bytes) {
  const Problem p = single_problem(nullptr, nullptr, nullptr, nullptr, nullptr, batch, heads, n_query,
                                   n_key, nullptr, nullptr, nullptr, nullptr);
  return attn_workspace_bytes(&p, 1, dtype, bytes);
}

extern "C" int vgo_mass_bias_attn_fwd_ws(const void* q, const void* k, const void* v,
                                         const void* log_mass, void* out, int64_t batch,
                                         int64_t heads, int64_t n_query, int64_t n_key,
                                         int64_t head_dim, const int64_t q_stride[3],
                                         const int64_t k_stride[3], const int64_t v_stride[3],
                                         const int64_t o_stride[3], int dtype, void* workspace,
                                         size_t workspace_bytes, void* stream) {
  const Problem p = single_problem(q, k, v, log_mass, out, batch, heads, n_query, n_key, q_stride,
                                   k_stride, v_stride, o_stride);
  return attn_run(&p, &head_dim, 1, dtype, workspace, workspace_bytes, true, stream);
}

extern "C" int vgo_mass_bias_attn_fwd_static(const void* q, const void* k, const void* v,
                                             const void* log_mass, void* out, int64_t batch,
                                             int64_t heads, int64_t n_query, int64_t n_key,
                                             int64_t head_dim, const int64_t q_stride[3],
                                             const int64_t k_stride[3], const int64_t v_stride[3],
                                             const int64_t o_stride[3], int dtype, void* stream) {
  using namespace vgo;
  const Problem p = single_problem(q, k, v, log_mass, out, batch, heads, n_query, n_key, q_stride,
                                   k_stride, v_stride, o_stride);
  size_t need = 0;
  const int status = attn_workspace_bytes(&p, 1, dtype, &need);
  if (status != VGO_OK) return status;
  if (need > VGO_ATTN_STATIC_SCRATCH_BYTES)
    return fail(VGO_EWORKSPACE,
                "mass_bias_attention(static): the problem needs " + std::to_string(need) +
                    " bytes of scratch, more than the static " +
                    std::to_string(static_cast<size_t>(VGO_ATTN_STATIC_SCRATCH_BYTES)) +
                    "; use vgo_mass_bias_attn_fwd_ws with a workspace");
  void* ptr = nullptr;
  if (need > 0) {
    const int found = static_scratch(&ptr);
    if (found != VGO_OK) return found;
  }
  return attn_run(&p, &head_dim, 1, dtype, ptr, VGO_ATTN_STATIC_SCRATCH_BYTES, true, stream);
}

extern "C" int vgo_mass_bias_attn_pair_workspace(const vgo_attn_problem* problems, int count,
                                                 int dtype, size_t* bytes) {
  using namespace vgo;
  VGO_REQUIRE(problems && (count == 1 || count == 2), "mass_bias_attention: 1 or 2 problems");
  Problem p[2];
  for (int i = 0; i < count; ++i) p[i] = from_c(problems[i]);
  return attn_workspace_bytes(p, count, dtype, bytes);
}

extern "C" int vgo_mass_bias_attn_pair_fwd_ws(const vgo_attn_problem* problems, int count, int dtype,
                                              void* workspace, size_t workspace_bytes, void* stream) {
  using namespace vgo;
  VGO_REQUIRE(problems && (count == 1 || count == 2), "mass_bias_attention: 1 or 2 problems");
  Problem p[2];
  int64_t head_dims[2];
  for (int i = 0; i < count; ++i) {
    p[i] = from_c(problems[i]);
    head_dims[i] = problems[i].head_dim;
  }
  return attn_run(p, head_dims, count, dtype, workspace, workspace_bytes, true, stream);
}

extern "C" int vgo_attn_kernel_timing(int enable) {
  using namespace vgo;
  KernelTiming& t = kernel_timing();
  std::lock_guard<std::mutex> lock(t.mutex);
  if (!enable) {
    t.on = false;
    return VGO_OK;
  }
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0)
    return fail(VGO_ELAUNCH, "vgo_attn_kernel_timing: no current device");
  if (t.device >= 0 && t.device != dev && t.used > 0)
    return fail(VGO_EINVAL, "vgo_attn_kernel_timing: read the launches recorded on device " +
                                std::to_string(t.device) + " first");
  if (t.device != dev) {
    // Events belong to the device they were created on: the old device's pool is
    // destroyed there, and the new device starts a new one.
    if (t.device >= 0) {
      if (hipSetDevice(t.device) == hipSuccess) {
        for (int i = 0; i < kTimingSlots; ++i) {
          if (t.start[i]) (void)hipEventDestroy(t.start[i]);
          if (t.stop[i]) (void)hipEventDestroy(t.stop[i]);
        }
        if (t.stamps) (void)hipFree(t.stamps);
      }
      if (hipSetDevice(dev) != hipSuccess)
        return fail(VGO_ELAUNCH, "vgo_attn_kernel_timing: cannot return to the current device");
    }
    for (int i = 0; i < kTimingSlots; ++i) t.start[i] = t.stop[i] = nullptr;
    t.stamps = nullptr;
  }
  if (t.stamps == nullptr) {
    void* buf = nullptr;
    const hipError_t err = hipMalloc(&buf, sizeof(unsigned long long) * kClockSlots * kClockGroups * 4);
    if (err != hipSuccess)
      return fail(VGO_ELAUNCH, std::string("vgo_attn_kernel_timing: ") + hipGetErrorString(err));
    t.stamps = static_cast<unsigned long long*>(buf);
  }
  t.device = dev;
  t.on = true;
  return VGO_OK;
}

extern "C" int vgo_attn_kernel_clock_read(double* shader_cycles, double* const_ticks,
                                          double* span_ticks, double* span_ms, int64_t* launches) {
  using namespace vgo;
  VGO_REQUIRE(shader_cycles && const_ticks && span_ticks && span_ms && launches,
              "vgo_attn_kernel_clock_read: null output");
  KernelTiming& t = kernel_timing();
  std::lock_guard<std::mutex> lock(t.mutex);
  *shader_cycles = *const_ticks = *span_ticks = *span_ms = 0.0;
  *launches = 0;
  const int n = std::min(t.used, kClockSlots);
  if (n == 0 || t.stamps == nullptr) return VGO_OK;
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev != t.device)
    return fail(VGO_EINVAL, "vgo_attn_kernel_clock_read: call it on the device the launches ran on");
  std::vector<unsigned long long> host(static_cast<size_t>(kClockGroups) * 4);
  for (int i = 0; i < n; ++i) {
    hipError_t err = hipEventSynchronize(t.stop[i]);
    float ms = 0.0f;
    if (err == hipSuccess) err = hipEventElapsedTime(&ms, t.start[i], t.stop[i]);
    const int64_t groups = t.clock_groups[i];
    if (err == hipSuccess && groups > 0)
      err = hipMemcpy(host.data(), t.stamps + static_cast<int64_t>(i) * kClockGroups * 4,
                      sizeof(unsigned long long) * 4 * groups, hipMemcpyDeviceToHost);
    if (err != hipSuccess)
      return fail(VGO_ELAUNCH, std::string("vgo_attn_kernel_clock_read: ") + hipGetErrorString(err));
    if (groups == 0) continue;
    unsigned long long first = ~0ull, last = 0;
    for (int64_t b = 0; b < groups; ++b) {
      const unsigned long long* g = host.data() + 4 * b;
      *shader_cycles += static_cast<double>(g[2] - g[0]);
      *const_ticks += static_cast<double>(g[3] - g[1]);
      first = std::min(first, g[1]);
      last = std::max(last, g[3]);
    }
    *span_ticks += static_cast<double>(last - first);
    *span_ms += ms;
    ++*launches;
  }
  return VGO_OK;
}

extern "C" int vgo_attn_kernel_timing_read(double* total_ms, int64_t* launches, int64_t* dropped) {
  using namespace vgo;
  VGO_REQUIRE(total_ms && launches, "vgo_attn_kernel_timing_read: null output");
  KernelTiming& t = kernel_timing();
  std::lock_guard<std::mutex> lock(t.mutex);
  double sum = 0.0;
  for (int i = 0; i < t.used; ++i) {
    hipError_t err = hipEventSynchronize(t.stop[i]);
    float ms = 0.0f;
    if (err == hipSuccess) err = hipEventElapsedTime(&ms, t.start[i], t.stop[i]);
    if (err != hipSuccess)
      return fail(VGO_ELAUNCH, std::string("vgo_attn_kernel_timing_read: ") + hipGetErrorString(err));
    sum += ms;
  }
  *total_ms = sum;
  *launches = t.used;
  if (dropped) *dropped = t.dropped;
  t.used = 0;
  t.dropped = 0;
  return VGO_OK;
}
