/*
 * grm_hip.h - C ABI of the MI355X (gfx950) GRM hot-path library, libgrm_hip.so.
 *
 * Every entry point takes raw device pointers, int64 sizes, dtype codes and a
 * hipStream_t (passed as void*; NULL is the null stream).  It enqueues its
 * kernels on that stream and returns without synchronising.  Nothing here
 * allocates device memory, and nothing reads or writes torch objects.
 *
 * Return value: GRM_HIP_OK (0) on success.  A negative GRM_HIP_E* code means
 * the arguments were rejected before any launch.  A positive value is the
 * hipError_t of a failed launch.  grm_hip_last_error() returns a
 * thread-local message describing the last failure.
 *
 * Layouts follow the reference op schemas (grm/csrc/bindings.cpp:6-10):
 *   keys, queries   [batch, seq_len, key_dim]       row-major, contiguous
 *   values, hidden  [batch, seq_len, value_dim]
 *   memory          [batch, value_dim, key_dim]     (row = value index)
 * Mixed precision: keys/values/queries share one dtype; memory may be that
 * dtype or float32.  All accumulation is float32.
 */
#ifndef GRM_HIP_H
#define GRM_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype codes */
#define GRM_HIP_F32 0
#define GRM_HIP_F16 1
#define GRM_HIP_BF16 2

/* status codes */
#define GRM_HIP_OK 0
#define GRM_HIP_EINVAL (-1)      /* bad pointer, size or dtype */
#define GRM_HIP_EUNSUPPORTED (-2) /* valid for the reference, not for this kernel (e.g. key_dim > 256) */

/* Library ABI version (major * 100 + minor). */
int grm_hip_abi_version(void);

/* Thread-local text of the last error returned by any entry point. */
const char* grm_hip_last_error(void);

/* Number of kernels this library has launched in the process.  Lets a caller
 * prove that a call ran on the native path. */
uint64_t grm_hip_launch_count(void);

/*
 * Chunked linear-memory update fused with query application.
 *   M_t = decay * M_{t-1} + (1 - decay) / sqrt(key_dim) * v_t k_t^T
 *   h_t = M_t q_t
 * Replaces grm_cuda::chunk_update_forward
 *   (reference grm/csrc/bindings.cpp:6, chunk_update.cu:523-586, grm_cuda.cpp:46-90,
 *    Python fallback grm/core/cuda_ops.py:218-254).
 * hidden:     [batch, seq_len, value_dim] in the input dtype, or NULL to skip it.
 * memory_out: [batch, value_dim, key_dim] in mem_dtype (may not alias memory), or
 *             NULL to skip it when snapshots are requested.
 * snapshots:  NULL, or float32 [batch, ceil(seq_len / snapshot_len), value_dim, key_dim]
 *             holding the state after every snapshot_len tokens (the last one
 *             is the final state).  This is the whole-sequence form of the op:
 *             one call covers every segment of a sequence.
 * snapshot_len: tokens per snapshot (> 0) when snapshots != NULL, ignored otherwise.
 * workspace:  optional device scratch of workspace_bytes (16-byte aligned).  With
 *             at least grm_hip_chunk_update_fwd_workspace() bytes, long sequences
 *             are split into time parts scanned in parallel (two launches);
 *             with less (or NULL) each sequence is scanned by one workgroup chain.
 *             Results are the same either way up to float rounding.
 * Limits: 1 <= key_dim <= 256 (<= 128 for float32 inputs), value_dim >= 1;
 * seq_len >= 0; batch >= 0.
 */
int grm_hip_chunk_update_fwd(const void* keys, const void* values, const void* queries,
                             const void* memory, void* hidden, void* memory_out, float* snapshots,
                             void* workspace, int64_t workspace_bytes, int64_t batch,
                             int64_t seq_len, int64_t key_dim, int64_t value_dim, int in_dtype,
                             int mem_dtype, double memory_decay, int64_t snapshot_len, void* stream);

/* Workspace bytes grm_hip_chunk_update_fwd can use for these sizes (0: none).
 * No counterpart in the reference (its kernel walks each sequence serially). */
int64_t grm_hip_chunk_update_fwd_workspace(int64_t batch, int64_t seq_len, int64_t key_dim,
                                           int64_t value_dim, int64_t snapshot_len);

/*
 * grm_hip_chunk_update_fwd without any device allocation, for callers that
 * cannot allocate (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  No counterpart in the reference.
 * Same arguments and results as grm_hip_chunk_update_fwd minus the workspace:
 * the time-split scratch is a fixed device array inside the library of
 * GRM_HIP_NOALLOC_SCRATCH_BYTES per GPU, resident on every GPU where the
 * library's scan kernels are loaded (whether or not this entry point is ever
 * called) until the process ends.  Calls whose sizes need more time-split scratch than
 * that (grm_hip_chunk_update_fwd_workspace() above the limit) are rejected with
 * GRM_HIP_EINVAL and a message.  Every call on one GPU shares that GPU's
 * scratch, so calls take it in turn: a call on a different stream than the
 * previous call on that GPU first makes its stream wait for the previous
 * call's kernels (an event the library records after each call; the event
 * and the scratch's address are set up at the first call on a device and
 * kept), and calls from several host threads hold a lock while they launch.
 * Under stream capture nothing is recorded or waited for: replays of a
 * captured call must not overlap other calls on the same GPU.  The scratch
 * needs no clearing between calls.
 */
#define GRM_HIP_NOALLOC_SCRATCH_BYTES (32ll << 20)
int64_t grm_hip_chunk_update_fwd_noalloc_limit(void);
int grm_hip_chunk_update_fwd_noalloc(const void* keys, const void* values, const void* queries,
                                     const void* memory, void* hidden, void* memory_out, float* snapshots,
                                     int64_t batch, int64_t seq_len, int64_t key_dim, int64_t value_dim,
                                     int in_dtype, int mem_dtype, double memory_decay, int64_t snapshot_len,
                                     void* stream);

/*
 * Gradient of grm_hip_chunk_update_fwd.
 * Replaces grm_cuda::chunk_update_backward
 *   (reference grm/csrc/bindings.cpp:7, chunk_update.cu:588-716, grm_cuda.cpp:92-126).
 * grad_hidden [batch, seq_len, value_dim] and grad_memory_out [batch, value_dim, key_dim]
 * come in the input dtype and mem_dtype; the four gradients are written in the
 * dtype of the tensor they belong to.
 * chunk_states: float32 [batch, ceil(seq_len / 64), value_dim, key_dim], the state after
 *   each 64-token chunk.  states_given != 0: the caller filled it (the forward's
 *   64-token snapshots, grm_hip_chunk_update_fwd with snapshot_len 64, passed from the
 *   forward as the op's aux); otherwise it is a workspace that the backward fills by
 *   running the forward again.
 * dkq_partial: float32 workspace [2, batch, ceil(value_dim / 16), seq_len, key_dim]
 *   (caller-provided).  The scalar kernel keeps per 16-column value tile partial sums of
 *   grad_keys and grad_queries there; the MFMA kernels for 16-bit inputs keep the adjoint
 *   dL/dM at every 64-token chunk end, [batch, ceil(seq_len / 64), value_dim, key_dim], at
 *   its front (they run when that fits, from about ten tokens on), followed, when the walk
 *   over the chunks runs in parts, by each part's adjoint at its start
 *   [batch, parts, value_dim, key_dim].
 */
int grm_hip_chunk_update_bwd(const void* grad_hidden, const void* grad_memory_out, const void* keys,
                             const void* values, const void* queries, const void* memory,
                             void* grad_keys, void* grad_values, void* grad_queries,
                             void* grad_memory, float* chunk_states, int states_given, float* dkq_partial,
                             int64_t batch, int64_t seq_len, int64_t key_dim, int64_t value_dim,
                             int in_dtype, int mem_dtype, double memory_decay, void* stream);

/*
 * Query application against stacked memories, float32 accumulation.
 *   hidden[b, q, r, h] = sum_k memories[b, q, r, h, k] * queries[b, q, k]
 * Rank 4 of the reference (memories [B, R, H, K], queries [B, K]) is n_query = 1.
 * Replaces grm_cuda::apply_query_forward
 *   (reference grm/csrc/bindings.cpp:8, apply_query.cu:186-254, grm_cuda.cpp:128-134).
 * memories, queries and hidden share dtype.
 */
int grm_hip_apply_query_fwd(const void* memories, const void* queries, void* hidden,
                            int64_t batch, int64_t n_query, int64_t routes, int64_t hidden_size,
                            int64_t key_dim, int dtype, void* stream);

/*
 * Gradient of grm_hip_apply_query_fwd:
 *   grad_memories[b, q, r, h, k] = grad_hidden[b, q, r, h] * queries[b, q, k]
 *   grad_queries[b, q, k]        = sum_{r, h} grad_hidden[b, q, r, h] * memories[b, q, r, h, k]
 * Replaces grm_cuda::apply_query_backward
 *   (reference grm/csrc/bindings.cpp:9, apply_query.cu:256-330, grm_cuda.cpp:136-154).
 * grad_memories may be NULL: only grad_queries is computed (a retrieved archive
 * needs no gradient; the reference always writes both).
 */
int grm_hip_apply_query_bwd(const void* grad_hidden, const void* memories, const void* queries,
                            void* grad_memories, void* grad_queries, int64_t batch,
                            int64_t n_query, int64_t routes, int64_t hidden_size, int64_t key_dim,
                            int dtype, void* stream);

/*
 * Batched gather of archived segment states:
 *   out[b, i, :] = memories[b, indices[b, i], :]      i < n_index, row of row_elems elements
 * The reference's [B, R] and [B, Q, R] index shapes are n_index = R and Q * R.
 * Replaces grm_cuda::batched_memory_gather
 *   (reference grm/csrc/bindings.cpp:10, batched_gather.cu:91-181, grm_cuda.cpp:156-179).
 * An index outside [0, segments) yields a zero row and, when bad_index_count is
 * not NULL, increments that device int32 counter (the reference's CUDA kernel
 * does not check; its CPU path raises).
 */
int grm_hip_batched_gather(const void* memories, const int64_t* indices, void* out, int64_t batch,
                           int64_t segments, int64_t n_index, int64_t row_elems, int elem_bytes,
                           int32_t* bad_index_count, void* stream);

/*
 * Gather + query application without materialising the gathered states:
 *   out[b, q, r, h] = sum_k memories'[b, indices[b, q, r], h, k] * queries'[b, q, k]
 * equal to grm_hip_apply_query_fwd over grm_hip_batched_gather(memories, indices), i.e.
 * the reference's apply_query_forward(batched_memory_gather(memories, indices), queries)
 *   (grm/core/cuda_ops.py:370-402, composed by the retriever in grm/core/paper_grm.py:229,301-313).
 * The arithmetic type is out_dtype: either mem_dtype, or float32 for 16-bit
 * memories, which is the retriever's widening of the fp16 archive with
 * .to(torch.float32) (paper_grm.py:227) done on load.  memories' and queries' are
 * memories and queries cast to that type, as the reference's caller does
 * (paper_grm.py:301).  memories [batch, segments, hidden_size, key_dim] are
 * mem_dtype; out [batch, n_query, routes, hidden_size] is out_dtype; queries
 * [batch, n_query, key_dim] are q_dtype.  Every archived state is read from HBM
 * once and applied to all the queries that selected it; accumulation is float32.
 * An index outside [0, segments) yields a zero row and, when bad_index_count is
 * not NULL, increments that device int32 counter.
 * workspace: at least grm_hip_gather_apply_workspace(batch, segments, n_query * routes)
 * bytes of device memory (the pairs sorted by segment); contents need not be initialised.
 * Limits: key_dim <= 128, segments <= 16384.
 */
int64_t grm_hip_gather_apply_workspace(int64_t batch, int64_t segments, int64_t n_index);
int grm_hip_gather_apply(const void* memories, const int64_t* indices, const void* queries, void* out,
                         void* workspace, int64_t workspace_bytes, int64_t batch, int64_t segments,
                         int64_t n_query, int64_t routes, int64_t hidden_size, int64_t key_dim,
                         int mem_dtype, int q_dtype, int out_dtype, int32_t* bad_index_count, void* stream);

/*
 * The queries' gradient of gather_apply (float32 out), per pair:
 *   grad_pairs[b, q, r, :] = memories[b, indices[b, q, r]]^T grad_out[b, q, r, :]
 * grad_out [batch, n_query, routes, hidden_size] and grad_pairs [batch, n_query,
 * routes, key_dim] are float32; the caller sums over routes (grad of q'[b, q] is
 * sum_r grad_pairs[b, q, r]).  This is the backward of the reference's
 * apply_query_forward(batched_memory_gather(M, idx), q) with respect to q
 * (grm/core/cuda_ops.py:324-344,388-402; apply_query.cu:256-330) without the
 * gathered states; the memories get no gradient (the archive is detached, as the
 * reference's native gather has no backward).  Pairs with an index outside
 * [0, segments) get zero rows and, when bad_index_count is not NULL, are counted.
 * workspace: grm_hip_gather_apply_workspace(batch, segments, n_query * routes) bytes.
 * Limits: key_dim <= 128, segments <= 16384, (hidden_size rounded up to 16) x
 * (key_dim rounded up to 16/32/64/128, + 4) x 4 bytes within 160 KB (the float32
 * state in LDS).
 */
int grm_hip_gather_apply_bwd_queries(const void* memories, const int64_t* indices, const float* grad_out,
                                     float* grad_pairs, void* workspace, int64_t workspace_bytes, int64_t batch,
                                     int64_t segments, int64_t n_query, int64_t routes, int64_t hidden_size,
                                     int64_t key_dim, int mem_dtype, int32_t* bad_index_count, void* stream);

/*
 * grm_hip_gather_apply_bwd_queries with one gradient row per query, shared by
 * its routes (float32 grad_tokens [batch, n_query, hidden_size]):
 *   grad_pairs[b, q, r, :] = memories[b, indices[b, q, r]]^T grad_tokens[b, q, :]
 * For x = h + sum_r gates_r M[idx_r] q and g = dL/dx this is u_r, from which the
 * queries' gradient is sum_r gates_r u_r and the gates' u_r . q, with no
 * [batch, n_query, routes, hidden_size] tensor.  The reference differentiates the
 * same composition through its gathered states (paper_grm.py:229,301-313,
 * aggregator.py:67-145 under autograd).  Workspace, index handling and limits as
 * grm_hip_gather_apply_bwd_queries.  ABI 105.
 */
int grm_hip_gather_apply_bwd_tokens(const void* memories, const int64_t* indices, const float* grad_tokens,
                                    float* grad_pairs, void* workspace, int64_t workspace_bytes, int64_t batch,
                                    int64_t segments, int64_t n_query, int64_t routes, int64_t hidden_size,
                                    int64_t key_dim, int mem_dtype, int32_t* bad_index_count, void* stream);

/*
 * Fused retrieval: gather + query application + gate-weighted sum + residual +
 * LayerNorm, without the per-(query, route) rows of gather_apply in float32:
 *   out[b, q, :] = LN(h_online[b, q, :] + sum_r gates[b, q, r] * M[b, idx[b, q, r]] q[b, q])
 * the composition fuse_residual(h_online, gather_apply(memories, indices, queries,
 * float32), gates, ln_weight, ln_bias), i.e. the reference's retriever followed by its
 * aggregator (grm/core/paper_grm.py:229,301-313,604-611; grm/core/aggregator.py:67-145).
 * The state products are the exact 16-bit MFMA products of gather_apply with float32
 * accumulation; each gate-weighted row g * M q is kept in the workspace as float16
 * scaled by a power of two per (pair, 128-value tile) so that its largest magnitude
 * lies in [2^14, 2^15) (relative rounding 2^-11 of the tile's largest value, no
 * overflow), and the sum over routes runs in float32 in route order 0 .. R-1: no
 * atomics, deterministic.  Indices outside [0, segments) contribute nothing and,
 * when bad_index_count is not NULL, increment that device int32 counter.
 * memories [batch, segments, value_dim, key_dim] mem_dtype (float32 with bf16 queries,
 * or 16-bit); queries [batch, n_query, key_dim] bf16 (f16 with f16 memories); gates
 * [batch, n_query, routes] float32; h_online and out [batch, n_query, value_dim] are
 * h_dtype (the sum and the LayerNorm run in float32, out is rounded once);
 * ln_weight / ln_bias [value_dim] are float32, ln_weight NULL for no LayerNorm,
 * ln_bias NULL for none; 16-byte aligned.
 * workspace: grm_hip_retrieve_fuse_workspace(batch, segments, n_query * routes,
 * value_dim) bytes, contents need not be initialised.
 * Limits: key_dim <= 128 with 16-byte key rows, value_dim a multiple of 8 and <= 2048,
 * segments <= 16384; otherwise GRM_HIP_EUNSUPPORTED (use gather_apply + fuse_residual).
 */
int64_t grm_hip_retrieve_fuse_workspace(int64_t batch, int64_t segments, int64_t n_index, int64_t value_dim);
int grm_hip_retrieve_fuse(const void* memories, const int64_t* indices, const void* queries, const float* gates,
                          const void* h_online, const void* ln_weight, const void* ln_bias, void* out,
                          void* workspace, int64_t workspace_bytes, int64_t batch, int64_t segments,
                          int64_t n_query, int64_t routes, int64_t value_dim, int64_t key_dim, int mem_dtype,
                          int q_dtype, int h_dtype, float eps, int32_t* bad_index_count, void* stream);

/*
 * Split of the concatenated projection rows of LinearMemoryCell.project,
 * proj [rows, key_dim | value_dim | key_dim | extra_dim] (one GEMM over the
 * key, value, query and an extra projection's weights), into contiguous
 * keys / queries [rows, key_dim], L2-normalised as F.normalize(p=2, eps)
 * (reference grm/core/paper_grm.py:491-493; the norm and its eps clamp are
 * rounded to dtype before the division, as F.normalize does on a 16-bit row),
 * values [rows, value_dim] and extra [rows, extra_dim] (the gating query
 * projection of paper_grm.py:570-574; NULL when extra_dim is 0), copied.
 * One pass over the rows in place of the split views' copies and two
 * normalisations of several launches each.  dtype for every buffer.
 * Limits: dims multiples of 8, 16-byte aligned buffers.
 */
int grm_hip_project_split(const void* proj, void* keys, void* values, void* queries, void* extra, int64_t rows,
                          int64_t key_dim, int64_t value_dim, int64_t extra_dim, int dtype, float eps,
                          void* stream);

/*
 * out = LayerNorm(x + residual) over rows of hidden_size: the block output of
 * SegmentRecurrentMemoryLayer, layer_norm(outputs + x)
 * (reference grm/core/multilayer_grm.py:92-97), in one pass.  x, residual and out
 * are dtype; x + residual is rounded to dtype first (the torch add), then the
 * statistics and the affine map run in float32.  weight / bias [hidden_size] are
 * param_dtype; weight NULL for no affine map, bias NULL for none.
 * Limits: hidden_size a multiple of 8 and <= 2048, 16-byte aligned buffers.
 */
int grm_hip_residual_layer_norm(const void* x, const void* residual, const void* weight, const void* bias,
                                void* out, int64_t rows, int64_t hidden_size, int dtype, int param_dtype,
                                float eps, void* stream);

/*
 * LinearMemoryCell.project in one kernel: proj = x weight^T + bias over the
 * concatenated [key | value | query | extra] projection weights, rounded to
 * the input dtype (F.linear's output), then split as grm_hip_project_split
 * does: keys and queries L2-normalised (norm and eps clamp rounded to the
 * dtype), every part written contiguous.  x [rows, in_dim], weight
 * [2 key_dim + value_dim + extra_dim, in_dim], bias [that] or NULL, all in
 * dtype (f16 or bf16).
 *   (reference grm/core/paper_grm.py:491-493: key_proj / value_proj /
 *   query_proj and F.normalize; 570-574: the gating query projection; torch
 *   ops in the reference.)
 * Limits: key_dim 64, value_dim and extra_dim multiples of 64, in_dim a
 * multiple of 64, x and weight under 2 GiB, 16-byte aligned buffers.  ABI 107.
 */
int grm_hip_project_gemm(const void* x, const void* weight, const void* bias, void* keys, void* values,
                         void* queries, void* extra, int64_t rows, int64_t in_dim, int64_t key_dim,
                         int64_t value_dim, int64_t extra_dim, int dtype, float eps, void* stream);

/*
 * The layer's output side in one kernel:
 *   y   = x weight^T + bias, rounded to dtype (F.linear's output);
 *   s   = y + residual, rounded to dtype (the torch add);
 *   out = LayerNorm(s) over the out_dim columns, statistics in float32,
 *         times ln_weight plus ln_bias (param_dtype; NULL for none).
 *   (reference grm/core/paper_grm.py:709: output_proj, then
 *   grm/core/multilayer_grm.py:92-97: layer_norm(outputs + x); a library GEMM
 *   and torch ops in the reference.)
 * x [rows, in_dim], weight [out_dim, in_dim], bias [out_dim] or NULL, residual
 * and out [rows, out_dim], all dtype (f16 or bf16).  For the backward, pre
 * (NULL: not written) receives s, and mean / rstd (float32 [rows], both or
 * neither) the LayerNorm's row statistics, as aten's native_layer_norm saves
 * them.
 * Limits: in_dim a positive multiple of 64, out_dim a positive multiple of 64
 * and at most 512, weight under 2 GiB, 16-byte aligned buffers.  ABI 108.
 */
int grm_hip_linear_residual_layer_norm(const void* x, const void* weight, const void* bias, const void* residual,
                                       const void* ln_weight, const void* ln_bias, void* out, void* pre,
                                       float* mean, float* rstd, int64_t rows, int64_t in_dim, int64_t out_dim,
                                       int dtype, int param_dtype, float eps, void* stream);

/*
 * Archive form of float32 states: out[i] = storage(model(states[i])), each
 * value rounded (to nearest even) to model_dtype and then to storage_dtype,
 * which is what push() stores for a state the model computed
 *   (reference grm/core/paper_grm.py:139-140: the model's state, then
 *   .to(memory_storage_dtype)); the reference runs it as two torch casts.
 * n elements, any dtype pair; a float32 model dtype is the identity step.
 * Limits: 16-byte aligned buffers.  ABI 106.
 */
int grm_hip_archive_cast(const float* states, void* out, int64_t n, int model_dtype, int storage_dtype,
                         void* stream);

/*
 * Segment routing: dot-product score, top-k and softmax gates.
 *   score[b, q, s] = scale * sum_d queries[b, q, d] * keys[b, s, d]
 * Each score is one float32 fused multiply-add chain over d = 0 .. dim-1 in
 * order, so it is reproducible bit for bit on any IEEE machine.
 * With k = min(top_k, n_keys) < n_keys: the k best scores, descending, ties to
 * the lower index.  With k == n_keys: every score in index order (indices
 * 0 .. n_keys-1), the reference's arange branch.
 * gates = softmax(selected scores / temperature).
 * Outputs are [batch, n_query, k]: indices int64, scores and gates float32.
 * Replaces the routing of SegmentRecurrentMemoryModel._route_chunk
 *   (reference grm/core/paper_grm.py:566-589) and TopKMemoryRetriever.forward
 *   (grm/core/gating_unit.py:54-91); the reference runs it as torch ops.
 * Limits: 1 <= top_k <= 128 when top_k < n_keys (top_k > 32 runs a slower per-row list).
 */
int grm_hip_topk_route(const void* queries, const void* keys, int64_t* topk_indices,
                       float* topk_scores, float* gates, int64_t batch, int64_t n_query,
                       int64_t n_keys, int64_t dim, int dtype, int64_t top_k, float scale,
                       float temperature, void* stream);

/*
 * Segment routing over a growing archive, every segment of a sequence in one
 * call (the whole-sequence form of the per-segment routing above).
 * Query row t belongs to segment s = t / segment_len and is routed over the
 * keys [lo, hi) with hi = base + s and lo = max(0, hi - capacity): the
 * archive of at most `capacity` summaries as it stood when segment s ran,
 * `base` entries having been archived before this sequence.  Within a window
 * of n keys the rule is grm_hip_topk_route's: n > top_k selects the top_k best
 * (descending, ties to the lower index); n <= top_k takes all n in index
 * order and leaves slots n .. top_k-1 empty (index -1, score -inf, gate 0).
 * Indices are absolute key positions (key j of the window is index lo + j).
 * Outputs are [batch, n_query, top_k].
 * Replaces the per-segment routing calls of the reference's segment loop
 *   (grm/core/paper_grm.py:702-728 -> _route_chunk, :566-589) with one launch.
 * Limits: 1 <= top_k <= 128; base + (n_query - 1) / segment_len <= n_keys.
 */
int grm_hip_segment_route(const void* queries, const void* keys, int64_t* topk_indices,
                          float* topk_scores, float* gates, int64_t batch, int64_t n_query,
                          int64_t n_keys, int64_t dim, int dtype, int64_t top_k, int64_t segment_len,
                          int64_t base, int64_t capacity, float scale, float temperature, void* stream);

/*
 * Segment-window retrieval: retrieve_fuse for the indices of grm_hip_segment_route,
 * summing each query's routes without one row per (query, route):
 *   out[b, t, :] = LN(h_online[b, t, :] + sum_r gates[b, t, r] * M[b, idx[b, t, r]] q[b, t])
 * Query t sees the entries [lo(t), hi(t)), hi(t) = base + t / segment_len,
 * lo(t) = max(0, hi(t) - capacity), as in grm_hip_segment_route.  A negative
 * index is an empty slot.  An index outside the query's window, or repeating an
 * earlier route of the same query, contributes nothing and, when
 * bad_index_count is not NULL, increments that device int32 counter.
 * The products are retrieve_fuse's exact 16-bit MFMA products; each query's
 * float32 sum runs in index order over the entries, then leaves as float16
 * scaled by a power of two per (query, 128-value tile) (relative rounding 2^-11
 * of the tile's largest value) for the residual + LayerNorm pass, as one route
 * of retrieve_fuse.  Deterministic, no atomics in the sums.
 * Dtypes, layouts and LayerNorm parameters as grm_hip_retrieve_fuse (float16
 * memories with bf16 queries use float16 MFMA with each query scaled by a power of
 * two: its components within 2^-29 of its largest magnitude are exact, smaller
 * ones kept to 2^-40 of it).  Workspace: grm_hip_segment_retrieve_fuse_workspace(
 * batch, n_query, value_dim, key_dim, segment_len, base, capacity, mem_dtype) bytes
 * (the scaled sums and a copy of the windows' entries in MMA fragment order).
 * Replaces, for the reference's segment loop (grm/core/paper_grm.py:702-728),
 * the retriever and the aggregator's residual fusion it runs per segment
 *   (paper_grm.py:229,301-313,604-611; grm/core/aggregator.py:67-145).
 * Limits: key_dim <= 128 and a multiple of 8, value_dim a multiple of 8 and
 * <= 2048, routes <= 32, min(capacity, base + (n_query - 1) / segment_len) +
 * 95 / segment_len + 1 <= 256, base + (n_query - 1) / segment_len <= segments;
 * otherwise GRM_HIP_EUNSUPPORTED or GRM_HIP_EINVAL.  ABI 109.
 */
int64_t grm_hip_segment_retrieve_fuse_workspace(int64_t batch, int64_t n_query, int64_t value_dim, int64_t key_dim,
                                                int64_t segment_len, int64_t base, int64_t capacity, int mem_dtype);
int grm_hip_segment_retrieve_fuse(const void* memories, const int64_t* indices, const void* queries,
                                  const float* gates, const void* h_online, const void* ln_weight,
                                  const void* ln_bias, void* out, void* workspace, int64_t workspace_bytes,
                                  int64_t batch, int64_t segments, int64_t n_query, int64_t routes,
                                  int64_t value_dim, int64_t key_dim, int64_t segment_len, int64_t base,
                                  int64_t capacity, int mem_dtype, int q_dtype, int h_dtype, float eps,
                                  int32_t* bad_index_count, void* stream);

/*
 * Residual fusion of the online state with gated retrieved states:
 *   x = h_online[n] + sum_r gates[n, r] * retrieved[n, r]
 *   out[n] = layer_norm(x) * weight + bias      (ln_weight == NULL: no LayerNorm)
 * Replaces RetrievedStateFusion residual mode
 *   (reference grm/core/aggregator.py:67-145); the reference runs it as torch ops.
 * h_online, retrieved, out, ln_weight and ln_bias share dtype; gates are float32.
 */
int grm_hip_fuse_residual(const void* h_online, const void* retrieved, const float* gates,
                          const void* ln_weight, const void* ln_bias, void* out, int64_t rows,
                          int64_t routes, int64_t hidden_size, int dtype, float eps, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* GRM_HIP_H */
