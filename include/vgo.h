/*
 * vgo.h — C ABI of the MI355X (gfx950) merged-token global-attention library.
 *
 * Every entry point is stateless and re-entrant (except
 * vgo_mass_bias_attn_fwd_static, which uses a static device scratch): device
 * pointers in, device pointers out, launches only on the stream passed in
 * (`void*` is a hipStream_t; NULL is the null stream), no host synchronisation
 * and no device allocation inside.  Callers own every buffer, including workspaces whose size
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
 * Workspace variant of vgo_mass_bias_attn_fwd, same arguments and result.
 * `workspace` receives V transposed per head and the key bias (packed by a
 * first small kernel) and the fp32 partial states of split blocks.  The
 * library schedules the call's 512-query blocks over the G work-groups the
 * device holds resident at once: whole blocks for floor(blocks / G) rounds,
 * then the (block, 64-key tile) units of the remaining blocks split evenly
 * (stream-K); a block whose key range is shared by several work-groups is
 * finished by a third, small kernel from those partial states.  Query the
 * size with vgo_mass_bias_attn_workspace on the device that will run the
 * call; it is 0 bytes only for empty inputs and fp32 (workspace may then be
 * NULL).  Replaces the same reference function as vgo_mass_bias_attn_fwd.
 */
int vgo_mass_bias_attn_workspace(int64_t batch, int64_t heads, int64_t n_query, int64_t n_key,
                                 int dtype, size_t* bytes);
int vgo_mass_bias_attn_fwd_ws(const void* q, const void* k, const void* v, const void* log_mass,
                              void* out, int64_t batch, int64_t heads, int64_t n_query,
                              int64_t n_key, int64_t head_dim, const int64_t q_stride[3],
                              const int64_t k_stride[3], const int64_t v_stride[3],
                              const int64_t o_stride[3], int dtype, void* workspace,
                              size_t workspace_bytes, void* stream);

/*
 * Allocation-free variant of vgo_mass_bias_attn_fwd_ws: same arguments (minus
 * the workspace), kernels and result, bit for bit.  It has no counterpart in
 * the reference; it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  The scratch is a static device array of
 * VGO_ATTN_STATIC_SCRATCH_BYTES in a code object of its own: a GPU holds it from
 * the first call of this entry on that device (which looks up its address)
 * until the process ends; processes that never call it do not hold it.  A
 * problem whose workspace (vgo_mass_bias_attn_workspace) exceeds it returns
 * VGO_EWORKSPACE before launching anything.  Calls on one GPU share that
 * array: calls that overlap on one GPU (different streams, or host threads)
 * race and must be serialised by the caller.  Nothing in the scratch needs
 * clearing between calls; each call writes what it reads.
 */
#define VGO_ATTN_STATIC_SCRATCH_BYTES (192u * 1024u * 1024u)
int vgo_mass_bias_attn_fwd_static(const void* q, const void* k, const void* v,
                                  const void* log_mass, void* out, int64_t batch, int64_t heads,
                                  int64_t n_query, int64_t n_key, int64_t head_dim,
                                  const int64_t q_stride[3], const int64_t k_stride[3],
                                  const int64_t v_stride[3], const int64_t o_stride[3], int dtype,
                                  void* stream);

/*
 * One attention problem of vgo_mass_bias_attn_pair_fwd_ws, with the meaning of
 * vgo_mass_bias_attn_fwd's arguments of the same names (log_mass NULL: no bias).
 */
typedef struct vgo_attn_problem {
  const void* q;
  const void* k;
  const void* v;
  const void* log_mass;
  void* out;
  int64_t batch, heads, n_query, n_key, head_dim;
  int64_t q_stride[3], k_stride[3], v_stride[3], o_stride[3];
} vgo_attn_problem;

/*
 * Merged global attention and its dense special-query pass in one launch.
 * problems[0] is the mass-bias attention over merged keys; problems[1]
 * (count == 2) is the exact pass of the special-token queries over every
 * original key, without bias.  Together they replace the two calls of
 * vggt_omega/models/layers/attention.py:386-405 (mass_bias_attention) and
 * :406-422 (the special queries' dense SDPA), which run one after the other.
 * The two problems' (512-query block, 64-key tile) units share one stream-K
 * schedule, so the short special pass fills the merged attention's last round
 * instead of running alone on a few work-groups.  Each problem writes its own
 * `out`; the reference then copies the special rows over the merged result
 * (attention.py:420), which the caller still does.  Same dtypes, checks and
 * workspace rules as vgo_mass_bias_attn_fwd_ws; count == 1 equals that call.
 */
int vgo_mass_bias_attn_pair_workspace(const vgo_attn_problem* problems, int count, int dtype,
                                      size_t* bytes);
int vgo_mass_bias_attn_pair_fwd_ws(const vgo_attn_problem* problems, int count, int dtype,
                                   void* workspace, size_t workspace_bytes, void* stream);

/*
 * Kernel timing of the workspace attention path.  No counterpart in the
 * reference, whose profiling timers (vggt_omega/models/layers/attention.py:25-63)
 * bracket labelled spans of a layer, not single kernels; it serves callers that
 * measure the attention kernel against its roofline.
 *
 * vgo_attn_kernel_timing(1) records a HIP event pair around every
 * attn_pp_kernel launch that vgo_mass_bias_attn_fwd_ws / _fwd_static /
 * _pair_fwd_ws make afterwards on the device current at the call, outside
 * stream capture, up to 4096 launches (later ones are counted in `dropped`);
 * vgo_attn_kernel_timing(0) stops recording.  vgo_attn_kernel_timing_read
 * waits for the recorded launches, returns their summed duration in
 * milliseconds and their count, and empties the record.  The V^T pack and
 * the merge of split tasks that the same calls launch are not included.
 */
int vgo_attn_kernel_timing(int enable);
int vgo_attn_kernel_timing_read(double* total_ms, int64_t* launches, int64_t* dropped);

/*
 * Clock of the timed attention launches.  No counterpart in the reference; it
 * serves callers that state the kernel's fraction of the MFMA peak at the
 * clock the chip held under it.  Of the launches timed since the last
 * vgo_attn_kernel_timing_read, the first 512 with at most 1,024 work-groups
 * also record, per work-group, the shader-clock counter and the constant
 * 100 MHz counter at its start and end (wave 0).  This call returns, summed
 * over those launches, the work-groups' shader-clock cycles, their
 * constant-clock ticks, each launch's constant-clock span (its last
 * work-group's end less its first one's start), the HIP-event duration of
 * the same launches in milliseconds, and their count.  Mean clock =
 * shader_cycles / const_ticks x the constant clock's rate; span_ticks /
 * span_ms checks that rate.  Call it before vgo_attn_kernel_timing_read,
 * which empties the record; it waits for the launches and leaves the
 * record as it is.
 */
int vgo_attn_kernel_clock_read(double* shader_cycles, double* const_ticks, double* span_ticks,
                               double* span_ms, int64_t* launches);

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

/*
 * vgo_top4_project with the output rows taken in a given order: work position i
 * computes output row order[i] (order is int32 [n_rows], normally a permutation
 * of 0..n_rows-1; entries outside that range compute nothing).  Each output row
 * is computed exactly as by vgo_top4_project, so any order gives the same
 * result.  An order that groups rows by a shared parent (the stable sort of
 * index[:, 0] that vgo_csr_build gives) lets the repeated gathers of that parent
 * hit the L2 cache.  Same restore as vgo_top4_project (token_merging.py:387-414).
 */
int vgo_top4_project_ordered(const void* table, int64_t table_row_stride, const int32_t* index,
                             const float* weight, const int32_t* order, void* out,
                             int64_t out_row_stride, int64_t n_rows, int64_t table_rows,
                             int64_t dim, int dtype, void* stream);

/*
 * Gather probe: vgo_top4_project's gathers and arithmetic with each output row
 * summed (fp32, over its elements) into row_sums[n_rows] instead of being
 * written, i.e. the projection's reads without its row writes.  No reference
 * counterpart: a measurement of what the memory fabric gives the restore's
 * random-row reads (bench.py --only gather).  Rows must be whole 16-byte chunks
 * (else VGO_EUNSUPPORTED).
 */
int vgo_top4_gather_probe(const void* table, int64_t table_row_stride, const int32_t* index,
                          const float* weight, float* row_sums, int64_t n_rows, int64_t table_rows,
                          int64_t dim, int dtype, void* stream);


/*
 * Row gather + L2 normalisation: out[r] = x[rows[r]] / max(||x[rows[r]]||, eps),
 * fp32 accumulation, one rounding to out_dtype.  rows == NULL means rows[r] = r;
 * a row id outside [0, x_rows) yields a NaN row.  Replaces the
 * `F.normalize(...).to(bfloat16)` front end of the matchers
 * (vggt_omega/models/token_merging.py:1102-1103; sparse_convex.py:2384, 2403).
 */
int vgo_normalize_rows(const void* x, int64_t x_row_stride, int64_t x_rows, int x_dtype,
                       const int64_t* rows, int64_t n_rows, int64_t dim, float eps, void* out,
                       int64_t out_row_stride, int out_dtype, void* stream);

/*
 * Cosine matching with a per-source top-K (K = 1 or 4) over bf16 operands:
 * score[i,j] = bf16(src[i] . dict[j]) (fp32 accumulation), ties to the lower j.
 * Replaces the FastVGGT match loop `bmm(...).max(-1)`
 * (vggt_omega/models/token_merging.py:1106-1111), the sparse-convex local and
 * global `(...).topk(4)` (vggt_omega/models/sparse_convex.py:2402-2404, 2430) and
 * the Triton `streaming_top4` (vggt_omega/models/sparse_convex_kernels.py:20-93,
 * 309-329).
 *   src: bf16 rows, source i reads row src_rows ? src_rows[i] : i (< src_capacity);
 *        n_src_device (nullable) caps the source count on the device.
 *   dict: bf16 rows; dictionary position j < dict_n0 reads row j, else row
 *        dict_off1 + (j - dict_n0) (two contiguous ranges, e.g. frame-0 patches
 *        plus a window of anchors).
 *   values [n_src, K] fp32 (bf16-exact), index64/index32 [n_src, K] (either may
 *        be NULL): the dictionary row of each match, mapped through
 *        index_map[row] when index_map != NULL.  Ties break on the position j.
 *   scores (nullable): also store the bf16 score matrix (test/debug use).
 * Workspace size: vgo_similarity_topk_workspace.
 */
int vgo_similarity_topk_workspace(int64_t n_src, int64_t n_dict, int topk, int* parts,
                                  size_t* bytes);
int vgo_similarity_topk(const void* src, int64_t src_row_stride, int64_t src_capacity,
                        const int64_t* src_rows, const int* n_src_device, int64_t n_src,
                        const void* dict, int64_t dict_row_stride, int64_t dict_capacity,
                        int64_t dict_n0, int64_t dict_off1, int64_t n_dict, int64_t dim, int topk,
                        void* workspace, size_t workspace_bytes, float* values, int64_t* index64,
                        int32_t* index32, const int64_t* index_map, void* scores,
                        int64_t scores_row_stride, void* stream);

/*
 * FastVGGT plan assembly from match scores: removes the `removed` sources with
 * the largest (best, -position) -- the set `argsort(best, descending=True,
 * stable=True)[:removed]` selects -- and builds keep [batch, total-removed]
 * (ascending ids) and inverse [batch, total] (compact id; removed sources get
 * their target's).  Replaces vggt_omega/models/token_merging.py:1112-1121.
 * removed_flag [batch, n_sources] receives 1 for removed sources.
 */
int vgo_fastvggt_assemble(const float* best, const int32_t* target, const int64_t* source_ids,
                          const int64_t* dest_ids, int64_t batch, int64_t n_sources,
                          int64_t n_dest, int64_t total_tokens, int64_t removed, int64_t* keep,
                          int64_t* inverse, uint8_t* removed_flag, void* stream);

/*
 * Workspace variant of vgo_fastvggt_assemble, same arguments and result (bit
 * for bit).  The selection, marking, compaction and inverse steps run as a
 * chain of short kernels over many work-groups instead of one; `workspace`
 * (size from vgo_fastvggt_assemble_workspace, 4-byte aligned, any contents)
 * holds the digit histograms and per-group counts.  Replaces the same
 * reference lines (vggt_omega/models/token_merging.py:1112-1121).
 */
int vgo_fastvggt_assemble_workspace(int64_t batch, int64_t n_sources, int64_t total_tokens,
                                    size_t* bytes);
int vgo_fastvggt_assemble_ws(const float* best, const int32_t* target, const int64_t* source_ids,
                             const int64_t* dest_ids, int64_t batch, int64_t n_sources,
                             int64_t n_dest, int64_t total_tokens, int64_t removed, int64_t* keep,
                             int64_t* inverse, uint8_t* removed_flag, void* workspace,
                             size_t workspace_bytes, void* stream);

/*
 * Sparse-convex plan assembly (vggt_omega/models/sparse_convex.py:2435-2455):
 * sources = candidates with fit >= threshold (ascending), keep = the rest,
 * original_to_compact, parent = original_to_compact[support], weight = alpha.
 * Outputs are sized for the worst case (n_candidates sources / total_tokens
 * kept); stats[4] = {sources M, hard candidates, fallback candidates, sum of
 * selected fits} lets the caller size the plan with one small device->host copy.
 */
int vgo_sparse_convex_assemble(const float* fit, const float* alpha, const int64_t* support,
                               const int64_t* candidate, const float* top1, float easy_threshold,
                               const int* failed_count, int64_t n_candidates,
                               int64_t total_tokens, float threshold, int64_t* keep,
                               int64_t* original_to_compact, int64_t* source, int64_t* parent,
                               float* weight, float* stats, void* stream);

/*
 * Stable bucket order (CSR): order = item ids sorted by key, equal keys in item
 * order; offsets[k] .. offsets[k+1] delimit bucket k; keys >= n_buckets are
 * dropped.  Replaces the per-corner `argsort(stable=True)` + `bincount` of
 * vggt_omega/models/token_merging.py:323-333 and :51-54.
 */
int vgo_csr_workspace(int64_t n_items, int64_t n_buckets, size_t* bytes);
int vgo_csr_build(const uint32_t* keys, int64_t n_items, int64_t n_buckets, void* workspace,
                  size_t workspace_bytes, uint32_t* order, int32_t* offsets, void* stream);

/*
 * Per-row mass: mass[k] = (((start + S_0) + S_1) + ...), S_c = sequential sum of
 * weights[p] over the items p of segment (k, c) in CSR order (weights == NULL
 * counts items); log_mass (nullable) = log(mass).  With start = 1 and one
 * segment per corner this is `deterministic_weighted_normalizer`
 * (vggt_omega/models/token_merging.py:40-59) and the sparse-convex mass
 * (vggt_omega/models/sparse_convex.py:2448-2450, 2468).  items may be NULL
 * when every segment is empty (a plan without merged sources).
 */
int vgo_segment_mass(const int32_t* offsets, int64_t segs_per_row, const uint32_t* items,
                     const float* weights, int64_t n_weights, int64_t rows, float start,
                     float* mass, float* log_mass, void* stream);

/*
 * Plan compaction (Q/K/V pooling): out[k] = (f(x[base_rows[k]]) + sum_c sum_{p in
 * segment (k,c)} f(x[item_rows[p >> item_shift]]) * weights[p]) / normalizer[k] in
 * fp32, rounded once to out_dtype.  f is the identity, or with ln_weight != NULL a
 * per-head LayerNorm over 64 channels (eps ln_eps, shared affine) -- the q_norm /
 * k_norm of vggt_omega/models/layers/attention.py:337-339 fused into the pooling.
 * Channel c of token t lives at t*token_stride + (c/64)*head_stride + c%64 for
 * input and output, so the packed qkv projection ([N, 3C] rows) is read and
 * head-major [H, K, 64] attention operands are written without copies.
 * Replaces WeightedBilinearTokenPlan.compact / compact_key / compact_query and
 * TokenPlan.compact (vggt_omega/models/token_merging.py:343-385, 176-191), whose
 * caller is vggt_omega/models/layers/attention.py:346-375.
 */
int vgo_compact(const void* x, int64_t x_token_stride, int64_t x_head_stride, int64_t x_rows,
                const int64_t* base_rows, const int32_t* offsets, int64_t segs_per_row,
                const uint32_t* items, int item_shift, const int64_t* item_rows,
                const float* weights, int64_t n_weights, const float* normalizer, int64_t rows,
                int64_t dim, const float* ln_weight, const float* ln_bias, float ln_eps, void* out,
                int64_t out_token_stride, int64_t out_head_stride, int in_dtype, int out_dtype,
                void* stream);

/*
 * vgo_compact for up to three outputs that share one segment structure, in one
 * launch: output g pools the channels at element offset x_offsets[g] of every
 * member row (LayerNorm per head with ln_weights[g] / ln_biases[g] when given;
 * either array may be NULL) into outs[g] with its own token / head strides.
 * Same arithmetic and order as vgo_compact per output; in and out share
 * `dtype`; needs the vector layout (dim % 64 == 0, 16-byte aligned rows and
 * offsets).  Replaces the three compact calls over q, k and v of one plan
 * (vggt_omega/models/layers/attention.py:346-375).
 */
int vgo_compact_multi(const void* x, int64_t x_token_stride, int64_t x_head_stride, int64_t x_rows,
                      const int64_t* base_rows, const int32_t* offsets, int64_t segs_per_row,
                      const uint32_t* items, int item_shift, const int64_t* item_rows,
                      const float* weights, int64_t n_weights, const float* normalizer, int64_t rows,
                      int64_t dim, int n_outputs, const int64_t* x_offsets,
                      const float* const* ln_weights, const float* const* ln_biases, float ln_eps,
                      void* const* outs, const int64_t* out_token_strides,
                      const int64_t* out_head_strides, int dtype, void* stream);

/*
 * Fused QKV epilogue: from packed projection rows qkv[src] = [q | k | v] (each
 * heads*64 channels), write head-major q/k/v [seq, heads, tokens_out, 64] for
 * output rows r (src = rows ? rows[r] : r; seq = r / tokens_out), applying the
 * per-head LayerNorm(64) to q and k (when weights are given) and axial RoPE
 * (when rope_sin/cos are given) to tokens whose position within their
 * tokens_in-long sequence is >= rope_prefix, in fp32, one rounding to
 * out_dtype.  Any of q_out/k_out/v_out may be NULL; all 3*heads*64 channels of
 * every selected row are read whichever outputs are written.  Replaces the reshape,
 * q_norm/k_norm, apply_rope and transposes of
 * vggt_omega/models/layers/attention.py:243-262, 334-341.
 */
int vgo_qkv_epilogue(const void* qkv, int64_t row_stride, int64_t n_in_rows, int in_dtype,
                     const int64_t* rows, int64_t n_out, int64_t tokens_in, int64_t tokens_out,
                     int64_t heads, const float* q_weight, const float* q_bias,
                     const float* k_weight, const float* k_bias, float eps, const float* rope_sin,
                     const float* rope_cos, int64_t rope_prefix, int64_t rope_rows, void* q_out,
                     void* k_out, void* v_out, int out_dtype, void* stream);

/*
 * Dense [total, 4] restore map for vgo_top4_project: kept token keep[k] ->
 * (k,k,k,k)/(1,0,0,0); source token source[i] -> parent[i,:]/weight[i,:]; with
 * inverse != NULL (TokenPlan) token t -> inverse[t] one-hot.  Rows covered by
 * neither stay as the caller initialised them (zero weights give zero rows, as
 * the reference's `new_zeros` output does, token_merging.py:405-413).
 */
int vgo_restore_map(const int64_t* keep, int64_t n_keep, const int64_t* source,
                    const int64_t* parent, const float* weight, int64_t n_source,
                    const int64_t* inverse, int64_t total, int32_t* index_out, float* weight_out,
                    void* stream);

/*
 * Exact four-support simplex fit (15 active sets, 5x5 KKT systems by Gaussian
 * elimination with partial pivoting): `_convex_fit`
 * (vggt_omega/models/sparse_convex.py:2260-2304) with the easy-accept rule of
 * :2415-2418 (top1 >= easy_threshold keeps the one-hot fit).  Source rows[r] and
 * supports[r,0..3] are token ids into `tokens` (normalised twice, eps).  With
 * row_list != NULL only rows row_list[0 .. *n_list_device) are solved; with
 * list_supports != NULL as well, list entry w takes its supports from
 * list_supports[w,0..3] and writes them into supports[row_list[w],:] (the global
 * fallback of :2424-2434).
 */
int vgo_convex_fit(const void* tokens, int64_t token_row_stride, int64_t n_tokens, int dtype,
                   const int64_t* rows, int64_t* supports, const int64_t* list_supports,
                   const float* top1,
                   float easy_threshold, const int32_t* row_list, const int* n_list_device,
                   int64_t n, int64_t dim, float eps, float ridge, float* fit, float* alpha,
                   void* stream);

/*
 * Exact 15-active-set simplex least squares on given inputs: for each row,
 * min_a a^T G a - 2 r^T a over the probability simplex with G + ridge I in the
 * reduced solves, the one-hot (1,0,0,0) when r_0 beats the fit's cosine.
 * gram [rows,4,4], rhs [rows,4], out [rows,4]: contiguous fp32, 16-byte
 * aligned.  Replaces `four_support_active_set`
 * (vggt_omega/models/sparse_convex_kernels.py:332-353; kernels :102-212).
 */
int vgo_four_support_active_set(const float* gram, const float* rhs, int64_t rows, float ridge,
                                float* out, void* stream);

/*
 * `steps` projected-gradient iterations of the same problem (no ridge) from
 * (1,0,0,0), step 0.95 / max(max_i sum_j |G_ij|, 1e-4), simplex projection by a
 * four-value sorting network.  Same layouts.  Replaces
 * `four_support_projected_gradient` (sparse_convex_kernels.py:283-296; kernel
 * :214-280).
 */
int vgo_four_support_projected_gradient(const float* gram, const float* rhs, int64_t rows,
                                        int steps, float* out, void* stream);

/* Stable list of hard rows with fit < threshold and its length (sparse_convex.py:2424). */
int vgo_failed_rows(const float* fit, const float* top1, float easy_threshold, int64_t n,
                    float threshold, int32_t* list, int* count, void* stream);

/*
 * Residual-stream rows of a transformer block, one pass per row of dim fp32
 * values (dim a multiple of 4, at most 2048):
 *   s = x + gamma * branch   (branch == NULL: s = x; gamma == NULL: gamma = 1),
 *   written to x_out (NULL: not written; may equal x),
 *   LN(s) = (s - mean) / sqrt(var + eps) * ln_weight + ln_bias (either affine
 *   pointer may be NULL), written to norm_out in norm_dtype (bf16 or f16) and/or
 *   to norm_f32 (either may be NULL),
 *   LN(s) / max(||LN(s)||_2, unit_eps), written to unit_out in norm_dtype (NULL:
 *   not written; needs norm_out), bit-identical to vgo_normalize_rows of the
 *   fp32 LN(s) rows (the planners' F.normalize front end).
 * s is bit-identical to torch's `x + branch * gamma` in fp32 (branch widened
 * first, separate roundings).  Pointers are 4-element aligned and row strides
 * are multiples of 4 elements.  Replaces the LayerScale multiply, residual add,
 * LayerNorm and autocast cast of SelfAttentionBlock.forward /
 * forward_compacted (vggt_omega/models/layers/block.py:126-127, 219-226;
 * layer_scale.py:38).
 */
int vgo_residual_layer_norm(const float* x, int64_t x_row_stride, const void* branch,
                            int64_t branch_row_stride, int branch_dtype, const float* gamma,
                            const float* ln_weight, const float* ln_bias, float eps, int64_t rows,
                            int64_t dim, float* x_out, int64_t x_out_row_stride, void* norm_out,
                            int64_t norm_row_stride, int norm_dtype, float* norm_f32,
                            int64_t norm_f32_row_stride, void* unit_out, int64_t unit_row_stride,
                            float unit_eps, void* stream);

/*
 * The same row pass with the branch row restored from a merge plan's output
 * in the pass itself (the restored rows never go to memory):
 *   branch[r,:] = sum_{c<4} weight[r,c] * table[index[r,c],:]
 * rounded as vgo_top4_project rounds it (weight and each product in the table
 * dtype, fp32 sum in corner order, result in the table dtype; zero weights
 * skip their row; an out-of-range index with a non-zero weight gives a NaN
 * row), then s = x + gamma * branch and LN(s) as in vgo_residual_layer_norm.
 * table: [table_rows, dim] rows of table_dtype (bf16, f16 or fp32) with
 * table_row_stride; index int32 [rows, 4] and weight fp32 [rows, 4], contiguous
 * and 16-byte aligned (the plan's restore map, vgo_restore_map).  With weight
 * == NULL the map is one-hot: index is int32 [rows] (4-byte aligned) and
 * branch[r,:] = table[index[r],:] as the map row (index[r] x 4, (1, 0, 0, 0))
 * gives it, a zero row for index[r] < 0 -- a token plan's inverse.  x_out and
 * norm_out as above (at least one).  Replaces the plan restore
 * (vggt_omega/models/token_merging.py:387-414, 193-196) together with the
 * LayerScale, residual add and norm2 that follow it in forward_compacted
 * (layers/block.py:219-226, layers/attention.py:303).
 */
int vgo_restore_residual_layer_norm(const float* x, int64_t x_row_stride, const void* table,
                                    int64_t table_row_stride, int64_t table_rows, int table_dtype,
                                    const int32_t* index, const float* weight, const float* gamma,
                                    const float* ln_weight, const float* ln_bias, float eps,
                                    int64_t rows, int64_t dim, float* x_out,
                                    int64_t x_out_row_stride, void* norm_out,
                                    int64_t norm_row_stride, int norm_dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* VGO_H_ */
