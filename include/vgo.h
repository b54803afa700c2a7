/*
 * vgo.h — C ABI of the MI355X (gfx950) merged-token global-attention library.
 *
 * Every entry point is stateless and re-entrant: device pointers in, device
 * pointers out, launches only on the stream passed in (`void*` is a
 * hipStream_t; NULL is the null stream), no host synchronisation and no device
 * allocation inside.  Callers own every buffer, including workspaces whose size
 * is reported by the matching `*_workspace_bytes` query.
 *
 * Return value: VGO_OK (0) or a negative status.  `vgo_last_error()` returns a
 * thread-local, human-readable message for the most recent failure on the
 * calling thread.
 *
 * The reference (shuang-yang18/4D_TTT_merging, package `vggt_omega`) is pure
 * Python + Triton and exposes no FFI; each entry point below names the Python
 * function or Triton kernel whose work it replaces (paths relative to the
 * reference root).
 */
#ifndef VGO_H_
#define VGO_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VGO_ABI_VERSION 1

#define VGO_OK 0
#define VGO_EINVAL (-1)       /* bad shape, stride, dtype, size or null pointer */
#define VGO_ELAUNCH (-2)      /* the HIP runtime rejected a launch */
#define VGO_EUNSUPPORTED (-3) /* valid request outside what the kernels implement */
#define VGO_EWORKSPACE (-4)   /* workspace missing or too small */

/* Element types (values fixed by this ABI). */
#define VGO_F32 0
#define VGO_BF16 1
#define VGO_F16 2

const char* vgo_last_error(void);
int vgo_abi_version(void);

/*
 * Mass-bias attention, O = softmax(Q K^T / sqrt(64) + log_mass) V, head_dim 64.
 *
 * Replaces `mass_bias_attention` (vggt_omega/models/mass_bias_attention.py:85-129,
 * Triton kernel :17-82) and, with log_mass == NULL, the dense special-query SDPA
 * of vggt_omega/models/layers/attention.py:406-422.
 *
 * q [batch, heads, n_query, 64], k/v [batch, heads, n_key, 64]; strides are in
 * elements for (batch, head, token); the channel stride must be 1.  log_mass
 * holds n_key elements of `dtype` (the reference rounds log(mass) to q's dtype,
 * mass_bias_attention.py:109) shared by every batch and head, or NULL for no
 * bias.  out uses o_stride and `dtype`.  dtype: VGO_BF16 / VGO_F16 run on bf16/
 * f16 MFMA with fp32 softmax state; VGO_F32 runs in fp32 throughout.
 */
int vgo_mass_bias_attn_fwd(const void* q, const void* k, const void* v, const void* log_mass,
                           void* out, int64_t batch, int64_t heads, int64_t n_query,
                           int64_t n_key, int64_t head_dim, const int64_t q_stride[3],
                           const int64_t k_stride[3], const int64_t v_stride[3],
                           const int64_t o_stride[3], int dtype, void* stream);

/*
 * Top-4 convex projection (unmerge): out[i,:] = sum_c w[i,c] * table[index[i,c],:].
 *
 * Replaces the restore of WeightedBilinearTokenPlan / TokenPlan
 * (vggt_omega/models/token_merging.py:387-414 and :193-196), whose caller is
 * vggt_omega/models/layers/attention.py:303.  table [table_rows, dim], out
 * [n_rows, dim], both row-major with the given row strides (elements); index and
 * weight are [n_rows, 4] int32 / fp32.  For bf16/f16 the weight is rounded to
 * the value type and each product is rounded before an fp32 sum, as the
 * reference's `(parent * w.to(value.dtype)).sum(2)` does.  Zero weights skip
 * their gather.  An index outside [0, table_rows) with a non-zero weight writes
 * NaN to that output row instead of reading out of bounds.
 */
int vgo_top4_project(const void* table, int64_t table_row_stride, const int32_t* index,
                     const float* weight, void* out, int64_t out_row_stride, int64_t n_rows,
                     int64_t table_rows, int64_t dim, int dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* VGO_H_ */
