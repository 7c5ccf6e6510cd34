/*
 * tris_moe_hip.h — C ABI of the MI355X (gfx950) TriS-MoE grouped expert
 * dequant-GEMM library (libtris_moe_hip.so).
 *
 * Every entry point takes plain device pointers (fp16 data as uint16_t bit
 * patterns), sizes and a hipStream_t passed as void*; nothing here depends on
 * torch.  All kernels run on the given stream and no entry point
 * synchronises the device.  Return value: 0 on success, a negative
 * TRIS_ERR_* code otherwise; tris_last_error() then describes the failure
 * (thread-local, valid until the next failing call on the same thread).
 *
 * Each declaration names the reference interface it replaces
 * (paths relative to the TriS-MoE checkout):
 *   TriSMoE_cuda.cpp  = AutoGPTQ/autogptq_extension/TriSMoE/TriSMoE_cuda.cpp
 *   kernel.cu         = AutoGPTQ/autogptq_extension/TriSMoE/TriSMoE_cuda_kernel.cu
 *   qlinear_cuda.py   = AutoGPTQ/auto_gptq/nn_modules/qlinear/qlinear_cuda.py
 */
#ifndef TRIS_MOE_HIP_H_
#define TRIS_MOE_HIP_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TRIS_COMPACT3_KERNEL_ABI_VERSION 2

#define TRIS_OK 0
#define TRIS_ERR_INVALID (-1) /* argument / shape contract violated (the reference's TORCH_CHECK) */
#define TRIS_ERR_HIP (-2)     /* a HIP runtime call or kernel launch failed */

/*
 * One projection's stacked grouped compact3 payload, as produced by
 * build_grouped_precomputed_payload (qlinear_cuda.py:1512-1636); shapes
 * (E experts, K = rank, N = outfeatures, G groups):
 *   qweight1               int32 [E, ceil(K/32), N]
 *   qweight2_sparse        int32 [E, qweight2_sparse_rows, N]   (zero padded)
 *   qweight2_sparse_prefix int32 [E, ceil(K/32)+1]
 *   q_gmap_gr_words        int32 [E, gr_words_stride]           (zero padded)
 *   q_gmap_gr_offsets      int32 [E, nblk+1]
 *   q_gmap_gr_meta         int32 [E, nblk], nblk = ceil(ceil(K/32)/2)*ceil(N/64)
 *   c_map                  int32 [E, ceil(K/32)]
 *   g_idx                  int32 [E, K]
 *   col_pack3              int64 [E, K]
 *   row_pack3              int64 [E, N, G]
 *   output_scale           fp16  [E, N]  (read only if has_output_scale)
 *   bias                   fp16  [E, N]  (read only if has_bias)
 * The q_gmap_gr_* pointers may be NULL for the *_predecoded entry points.
 */
typedef struct tris_compact3_payload {
  int32_t num_experts;
  int32_t rank;
  int32_t outfeatures;
  int32_t num_groups;
  int32_t qweight2_sparse_rows;
  int32_t gr_words_stride;
  const int32_t* qweight1;
  const int32_t* qweight2_sparse;
  const int32_t* qweight2_sparse_prefix;
  const int32_t* q_gmap_gr_words;
  const int32_t* q_gmap_gr_offsets;
  const int32_t* q_gmap_gr_meta;
  const int32_t* c_map;
  const int32_t* g_idx;
  const int64_t* col_pack3;
  const int64_t* row_pack3;
  const uint16_t* output_scale;
  const uint16_t* bias;
  int32_t has_output_scale;
  int32_t has_bias;
  int32_t use_uniform_k64_groups; /* every 64-column tile lies in one group (kernel.cu:830-853) */
} tris_compact3_payload;

/* Module attribute TRIS_COMPACT3_KERNEL_ABI_VERSION (TriSMoE_cuda.cpp:1139). Returns 2. */
int tris_abi_version(void);

/* Message of the last failing call on this thread ("" if none). */
const char* tris_last_error(void);

/*
 * Offline block-GR encoder (host, CPU): replaces QuantLinear._pack_block_gr_gmap_tensor
 * (qlinear_cuda.py:3793-3859) and tools/rewrite_runtime_min_checkpoint.py:252-347
 * (pack_block_gr_gmap_tensor with k_min/k_max bounds, force_raw).
 * packed: host int32 [packed_rows, outfeatures]; words_out capacity must be
 * >= nblk*128 (words_capacity); offsets_out [nblk+1]; meta_out [nblk].
 * Returns the number of words written (>= 0) or a negative error code.
 */
int64_t tris_gr_encode(const int32_t* packed, int32_t packed_rows, int32_t outfeatures, int32_t k_min,
                       int32_t k_max, int32_t force_raw, int32_t* words_out, int64_t words_capacity,
                       int32_t* offsets_out, int32_t* meta_out);

/*
 * Device route builder: replaces build_grouped_route (TriSMoE_cuda.cpp:741-793;
 * Python fallback qlinear_cuda.py:1301-1378) without its device->host sync.
 * selected_experts int64 [num_tokens, top_k].  Outputs (device):
 *   perm, grouped_token_indices, grouped_slots  int64 [R], R = num_tokens*top_k
 *     (perm is the stable argsort of the flattened expert ids)
 *   grouped_expert_ids int32 [R]
 *   expert_ids         int32 [num_experts]   active experts ascending, then -1
 *   segment_offsets    int32 [num_experts+1] valid prefix [num_active+1], rest = R
 *   problem_offsets    int32 [num_experts+1] prefix of ceil(len/m_tile), rest = total
 *   counts             int32 [2] = {num_active, total_problem_tiles}
 *   inverse_perm       int32 [R] or NULL: grouped row of flat slot t*top_k + s
 * Expert ids outside [0, num_experts) are an error reported through counts[0] = -1 (no host
 * synchronisation); the route stays memory-safe for callers that do not check it: the valid entries keep
 * their segments, and the invalid ones fill grouped rows [segment_offsets[num_experts], R) in flat order
 * with their own token index and slot, grouped_expert_ids -1 and inverse_perm -1 (no segment covers them,
 * and tris_moe_combine skips them).
 */
int tris_build_grouped_route(const int64_t* selected_experts, int32_t num_tokens, int32_t top_k,
                             int32_t num_experts, int32_t m_tile, int64_t* perm,
                             int64_t* grouped_token_indices, int64_t* grouped_slots,
                             int32_t* grouped_expert_ids, int32_t* expert_ids, int32_t* segment_offsets,
                             int32_t* problem_offsets, int32_t* counts, int32_t* inverse_perm, void* stream);

/*
 * Router softmax, top-k and optional renormalisation for any batch: replaces route_topk with the fp16 cast
 * of the routing weights (modeling_mixtral.py:548-555: F.softmax(dtype=float), torch.topk, weights /
 * weights.sum, .to(fp16)), one wavefront per token, picks in descending probability with ties to the lower
 * expert, the renormalising sum added in pick order.  routing_weights_f32 may be NULL.  Outputs
 * [num_tokens, top_k]; num_experts <= 1024, top_k <= 16.  For batches past tris_route_topk_grouped's limit;
 * tris_build_grouped_route then builds the route from selected_experts.
 */
int tris_route_topk(const float* router_logits, int32_t num_tokens, int32_t num_experts, int32_t top_k,
                    int32_t renormalize, uint16_t* routing_weights_f16, float* routing_weights_f32,
                    int64_t* selected_experts, void* stream);

/*
 * Router softmax + top-k fused with the grouped route for decode-sized batches
 * (no reference counterpart: fuses F.softmax(router_logits, dtype=float),
 * torch.topk, the optional renormalisation and the routing-weight cast of
 * modeling_mixtral.py:548-555 with tris_build_grouped_route).  One launch.
 * router_logits fp32 [num_tokens, num_experts]; top-k by probability with ties
 * to the lower expert id; weights renormalised over the k picks when
 * renormalize != 0.  routing_weights_f16 fp16 [num_tokens, top_k] (required),
 * routing_weights_f32 / selected_experts optional (NULL to skip); the route
 * outputs are those of tris_build_grouped_route (padded to num_experts
 * segments).  Limits: num_tokens * top_k <= 2048, num_experts <= 1024,
 * top_k <= 16 (else TRIS_ERR_INVALID: use tris_build_grouped_route).
 */
int tris_route_topk_grouped(const float* router_logits, int32_t num_tokens, int32_t num_experts, int32_t top_k,
                            int32_t renormalize, int32_t m_tile, uint16_t* routing_weights_f16,
                            float* routing_weights_f32, int64_t* selected_experts, int64_t* perm,
                            int64_t* grouped_token_indices, int64_t* grouped_slots, int32_t* grouped_expert_ids,
                            int32_t* expert_ids, int32_t* segment_offsets, int32_t* problem_offsets, int32_t* counts,
                            int32_t* inverse_perm, void* stream);

/*
 * Grouped expert GEMM with in-kernel block-GR decode: replaces
 * compact3_tris_precomputed_grouped_forward_block_gr (TriSMoE_cuda.cpp:1018-1063,
 * kernel.cu:9768-10213).  output[r, n] = fp16(sum_k hidden[r,k] * W_e[n,k]
 * (* output_scale[e,n]) (+ bias[e,n])) for row r of segment s, e = expert_ids[s]
 * (e < 0, and e >= num_experts, give zero rows).  hidden fp16 [batch, rank];
 * output fp16 [batch, N]: rows inside segments are written, others untouched.  total_problem_tiles is the host copy of the route's
 * tile count (m_tile 4); it only bounds the launch.
 */
int tris_grouped_forward_block_gr(const uint16_t* hidden, int32_t batch, const int32_t* expert_ids,
                                  const int32_t* segment_offsets, const int32_t* problem_offsets,
                                  int32_t num_segments, int64_t total_problem_tiles,
                                  const tris_compact3_payload* payload, uint16_t* output, void* stream);

/*
 * Sparse split-bitmap variant: replaces compact3_tris_precomputed_grouped_forward (TriSMoE_cuda.cpp:795-832,
 * bound at :1263; host kernel.cu:8777-8975, kernels :3908-4498, split-bit lookups :619-637), the payload
 * format of TRIS_COMPACT3_BLOCK_GR=0 checkpoints.  q_gmap_sparse int32 [E, q_gmap_sparse_rows, N]: the j-th
 * non-salient column of an expert (k order) has its split bits in row j / 32, bit j % 32;
 * q_gmap_sparse_prefix int32 [E, ceil(K/32)+1]: the non-salient columns before each packed row.  The
 * payload's q_gmap_gr_* are not read.  As in the reference's sparse kernels, output_scale is always applied
 * (has_output_scale is ignored) and bias when has_bias.
 */
int tris_grouped_forward_sparse(const uint16_t* hidden, int32_t batch, const int32_t* expert_ids,
                                const int32_t* segment_offsets, const int32_t* problem_offsets, int32_t num_segments,
                                int64_t total_problem_tiles, const tris_compact3_payload* payload,
                                const int32_t* q_gmap_sparse, const int32_t* q_gmap_sparse_prefix,
                                int32_t q_gmap_sparse_rows, uint16_t* output, void* stream);

/* Gate/up pair in one launch: replaces compact3_tris_precomputed_grouped_dual_forward_block_gr
 * (TriSMoE_cuda.cpp:1065-1136, kernel.cu:10214-10779). */
int tris_grouped_dual_forward_block_gr(const uint16_t* hidden_a, const uint16_t* hidden_b, int32_t batch,
                                       const int32_t* expert_ids, const int32_t* segment_offsets,
                                       const int32_t* problem_offsets, int32_t num_segments,
                                       int64_t total_problem_tiles, const tris_compact3_payload* payload_a,
                                       const tris_compact3_payload* payload_b, uint16_t* output_a,
                                       uint16_t* output_b, void* stream);

/*
 * Grouped expert GEMM for decode-sized row tiles with the block-GR split bitmap decoded inside the kernel, on
 * MFMA: the reference's compact3_tris_precomputed_grouped_forward_block_gr (TriSMoE_cuda.cpp:1018-1063) for
 * rows gathered through an index (no reference counterpart as one call: the reference gathers with
 * index_select first, modeling_mixtral.py:475-476).  output[r, n] = fp16(sum_k hidden[row(r), k] * W_e[n, k]
 * (* output_scale[e, n]) (+ bias[e, n])) for every row r of segment s, e = expert_ids[s] (e outside
 * [0, num_experts): zero rows); row(r) = row_index[r] when row_index is given (an index outside
 * [0, hidden_rows) reads row 0), else r.  hidden fp16 [hidden_rows, rank], 16-byte aligned; output fp16
 * [batch, N]: rows inside segments are written, others untouched.  The payload needs the GR stream, uniform
 * 64-column groups and rank a multiple of 256 up to 512 (else TRIS_ERR_INVALID).  Rows are taken in tiles of
 * 16 per segment, so the kernel suits decode (few rows per segment); prefill-sized segments belong to the
 * predecoded MFMA entries.
 */
int tris_grouped_decode_forward_block_gr(const uint16_t* hidden, const int64_t* row_index, int32_t hidden_rows,
                                         int32_t batch, const int32_t* expert_ids, const int32_t* segment_offsets,
                                         int32_t num_segments, const tris_compact3_payload* payload, uint16_t* output,
                                         void* stream);

/*
 * Gate and up projections of the same routed rows in one launch with in-kernel GR decode: replaces
 * compact3_tris_precomputed_grouped_dual_forward_block_gr (TriSMoE_cuda.cpp:1065-1136) for decode-sized row
 * tiles.  swiglu == 0: output_a / output_b receive the two projections as tris_grouped_decode_forward_block_gr
 * would; swiglu != 0: output_a receives fp16(fp16(silu(g)) * u) of the two fp16 outputs (act_fn(gate_out) *
 * up_out, modeling_mixtral.py:496) and output_b is not used.  Both payloads must have one shape.
 */
int tris_grouped_decode_pair_forward_block_gr(const uint16_t* hidden_a, const uint16_t* hidden_b,
                                              const int64_t* row_index, int32_t hidden_rows, int32_t batch,
                                              const int32_t* expert_ids, const int32_t* segment_offsets,
                                              int32_t num_segments, const tris_compact3_payload* payload_a,
                                              const tris_compact3_payload* payload_b, uint16_t* output_a,
                                              uint16_t* output_b, int32_t swiglu, void* stream);

/*
 * Decode every GR block of the listed experts: replaces
 * compact3_tris_precomputed_grouped_block_gr_predecode (TriSMoE_cuda.cpp:836-853,
 * kernel.cu:4683-4718, host :8980-9029).  decoded int32 [num_active, nblk, 128];
 * an expert id outside [0, num_experts) gives zero blocks.
 */
int tris_grouped_block_gr_predecode(int32_t* decoded, const int32_t* expert_ids, int32_t num_active,
                                    const int32_t* q_gmap_gr_words, const int32_t* q_gmap_gr_offsets,
                                    const int32_t* q_gmap_gr_meta, int32_t num_experts, int32_t words_stride,
                                    int32_t packed_rows, int32_t outfeatures, void* stream);

/* One projection's GR stream for tris_grouped_block_gr_predecode_multi. */
typedef struct tris_gr_predecode_job {
  int32_t* decoded;              /* int32 [num_active, nblk, 128] */
  const int32_t* q_gmap_gr_words;
  const int32_t* q_gmap_gr_offsets;
  const int32_t* q_gmap_gr_meta;
  int32_t num_experts;
  int32_t words_stride;
  int32_t packed_rows;
  int32_t outfeatures;
} tris_gr_predecode_job;

#define TRIS_MAX_PREDECODE_JOBS 4

/* Predecode of up to TRIS_MAX_PREDECODE_JOBS projections (e.g. gate, up and
 * down of one layer) for the same routed experts in one launch (no reference
 * counterpart: batches the per-projection predecode calls, TriSMoE_cuda.cpp:836-853).
 * Each job's output is what tris_grouped_block_gr_predecode would write. */
int tris_grouped_block_gr_predecode_multi(const tris_gr_predecode_job* jobs, int32_t num_jobs,
                                          const int32_t* expert_ids, int32_t num_active, void* stream);

/*
 * One or two fp16 backbone projections of the same token rows, as tris_backbone_linear_pair takes them
 * (row_index NULL): out_a = fp16(x * in_scale_a) . sv_a^T [tokens, rank], out_b likewise (sv_b NULL: one
 * projection); workspace of tris_backbone_pair_workspace_bytes(tokens, in_features, rank) bytes.
 */
typedef struct tris_backbone_pair_job {
  const uint16_t* x;           /* fp16 [tokens, in_features], 16-byte aligned */
  int32_t tokens;
  int32_t in_features;
  const uint16_t* sv_a;        /* fp16 [rank, in_features] */
  const uint16_t* sv_b;        /* fp16 [rank, in_features] or NULL */
  int32_t rank;
  const uint16_t* in_scale_a;  /* fp16 [in_features] or NULL */
  const uint16_t* in_scale_b;
  uint16_t* out_a;             /* fp16 [tokens, rank], or [tokens, split] with a column split */
  uint16_t* out_b;
  void* workspace;
  int64_t workspace_bytes;
  /* Column split (0: none).  With split in (0, rank) each projection is two stacked ones: out_a / out_b hold
   * columns [0, split) as [tokens, split] and out_a_hi / out_b_hi columns [split, rank) as [tokens, rank - split]
   * (the same values the whole projection gives in those columns).  Decode-size launches only. */
  uint16_t* out_a_hi;
  uint16_t* out_b_hi;
  int32_t split;
} tris_backbone_pair_job;

/*
 * The router of tris_route_topk_grouped and the gate/up backbone projections of the same tokens in one
 * launch (no reference counterpart: the router, modeling_mixtral.py:548-555, and compute_shared_hidden,
 * qlinear_cuda.py:4454-4502, do not depend on each other, so one launch runs both).  The route outputs are
 * tris_route_topk_grouped's and the backbone outputs tris_backbone_linear_pair's (row_index NULL), bit
 * for bit.  bb->tokens == num_tokens <= 64.  When the projection is split over K and defer_reduce != 0,
 * the partial sums stay in bb->workspace and out_a / out_b are written by a later
 * tris_grouped_block_gr_predecode_multi_reduce with the same job; otherwise a second launch reduces them.
 */
int tris_route_topk_backbone(const float* router_logits, int32_t num_tokens, int32_t num_experts, int32_t top_k,
                             int32_t renormalize, int32_t m_tile, uint16_t* routing_weights_f16,
                             float* routing_weights_f32, int64_t* selected_experts, int64_t* perm,
                             int64_t* grouped_token_indices, int64_t* grouped_slots, int32_t* grouped_expert_ids,
                             int32_t* expert_ids, int32_t* segment_offsets, int32_t* problem_offsets,
                             int32_t* counts, int32_t* inverse_perm, const tris_backbone_pair_job* bb,
                             int32_t defer_reduce, void* stream);

/*
 * tris_grouped_block_gr_predecode_multi with the deferred slice reduction of a tris_route_topk_backbone
 * launch (defer_reduce != 0, the same job) in the same launch (no reference counterpart: the two do not
 * depend on each other).  bb NULL: the plain predecode.  The backbone outputs are the bits
 * tris_backbone_linear_pair writes.
 */
int tris_grouped_block_gr_predecode_multi_reduce(const tris_gr_predecode_job* jobs, int32_t num_jobs,
                                                 const int32_t* expert_ids, int32_t num_active,
                                                 const tris_backbone_pair_job* bb, void* stream);

/*
 * Grouped GEMM reading predecoded split bitmaps: replaces
 * compact3_tris_precomputed_grouped_forward_block_gr_predecoded (TriSMoE_cuda.cpp:855-889,
 * kernel.cu:4720-4885).  decoded is indexed by segment (the predecode of
 * expert_ids).  As in the reference, no output scale or bias is applied.
 */
int tris_grouped_forward_block_gr_predecoded(const uint16_t* hidden, int32_t batch, const int32_t* expert_ids,
                                             const int32_t* segment_offsets, const int32_t* problem_offsets,
                                             int32_t num_segments, int64_t total_problem_tiles,
                                             const int32_t* decoded, const tris_compact3_payload* payload,
                                             uint16_t* output, void* stream);

/* Dual variant: replaces compact3_tris_precomputed_grouped_dual_forward_block_gr_predecoded
 * (TriSMoE_cuda.cpp:922-974, kernel.cu:5094-5380). */
int tris_grouped_dual_forward_block_gr_predecoded(const uint16_t* hidden_a, const uint16_t* hidden_b,
                                                  int32_t batch, const int32_t* expert_ids,
                                                  const int32_t* segment_offsets, const int32_t* problem_offsets,
                                                  int32_t num_segments, int64_t total_problem_tiles,
                                                  const int32_t* decoded_a, const int32_t* decoded_b,
                                                  const tris_compact3_payload* payload_a,
                                                  const tris_compact3_payload* payload_b, uint16_t* output_a,
                                                  uint16_t* output_b, void* stream);

/*
 * Gate/up grouped GEMM over predecoded bitmaps with the SwiGLU product fused
 * (no reference counterpart: fuses tris_grouped_dual_forward_block_gr_predecoded,
 * TriSMoE_cuda.cpp:922-974, with act_fn(gate_out) * up_out of
 * modeling_mixtral.py:496 so the gate and up outputs never reach HBM).
 * output fp16 [batch, N] = fp16(fp16(silu(g)) * u) with g, u the fp16 outputs
 * the dual entry point would return.  Requires uniform 64-column groups,
 * rank % 64 == 0 and 16-byte aligned hidden rows (else TRIS_ERR_INVALID).
 */
int tris_grouped_swiglu_forward_block_gr_predecoded(
    const uint16_t* hidden_gate, const uint16_t* hidden_up, int32_t batch, const int32_t* expert_ids,
    const int32_t* segment_offsets, const int32_t* problem_offsets, int32_t num_segments, int64_t total_problem_tiles,
    const int32_t* decoded_gate, const int32_t* decoded_up, const tris_compact3_payload* payload_gate,
    const tris_compact3_payload* payload_up, uint16_t* output, void* stream);

/*
 * The dual and SwiGLU predecoded entries above with the routed rows gathered from per-token activations
 * (no reference counterpart: fuses the row gather of the reference's grouped forward,
 * modeling_mixtral.py:467-470, where the shared backbone output is indexed by the route's token indices,
 * into the GEMM's activation staging).  Grouped row r reads hidden row row_index[r] of hidden_* fp16
 * [hidden_rows, rank]; row_index is the route's int64 grouped_token_indices [batch].  An index outside
 * [0, hidden_rows) reads zeros.  Requires the MFMA kernel's payload conditions (uniform 64-column groups,
 * rank % 64 == 0, 16-byte aligned rows) and hidden_rows * rank * 2 < 2 GiB, else TRIS_ERR_INVALID.
 * problem_offsets is not needed (the kernels map their tiles from segment_offsets).
 */
int tris_grouped_dual_forward_block_gr_predecoded_rows(
    const uint16_t* hidden_a, const uint16_t* hidden_b, const int64_t* row_index, int32_t hidden_rows, int32_t batch,
    const int32_t* expert_ids, const int32_t* segment_offsets, int32_t num_segments, int64_t total_problem_tiles,
    const int32_t* decoded_a, const int32_t* decoded_b, const tris_compact3_payload* payload_a,
    const tris_compact3_payload* payload_b, uint16_t* output_a, uint16_t* output_b, void* stream);
int tris_grouped_swiglu_forward_block_gr_predecoded_rows(
    const uint16_t* hidden_gate, const uint16_t* hidden_up, const int64_t* row_index, int32_t hidden_rows,
    int32_t batch, const int32_t* expert_ids, const int32_t* segment_offsets, int32_t num_segments,
    int64_t total_problem_tiles, const int32_t* decoded_gate, const int32_t* decoded_up,
    const tris_compact3_payload* payload_gate, const tris_compact3_payload* payload_up, uint16_t* output,
    void* stream);

/*
 * The predecoded grouped GEMM (one projection, or two as the dual entry point) over bitmaps decoded for every
 * expert (no reference counterpart: TriSMoE_cuda.cpp:855-889 and 922-974 read one slot per routed segment).
 * decoded_* [num_experts, blocks, 128] (tris_route_predecode_all_reduce): segment s reads slot expert_ids[s].
 * row_index (or NULL) as in the _rows entry points.  hidden_b, decoded_b, payload_b and output_b are all NULL
 * for one projection.  Requires the MFMA kernel's payload conditions (else TRIS_ERR_INVALID); no output scale
 * or bias is applied.
 */
int tris_grouped_forward_block_gr_predecoded_experts(
    const uint16_t* hidden_a, const uint16_t* hidden_b, const int64_t* row_index, int32_t hidden_rows, int32_t batch,
    const int32_t* expert_ids, const int32_t* segment_offsets, int32_t num_segments, int64_t total_problem_tiles,
    const int32_t* decoded_a, const int32_t* decoded_b, const tris_compact3_payload* payload_a,
    const tris_compact3_payload* payload_b, uint16_t* output_a, uint16_t* output_b, void* stream);

/*
 * The predecoded grouped GEMM of one projection (TriSMoE_cuda.cpp:855-889) whose activation rows are taken from
 * the fp32 split-K partial sums of the backbone that produced them (no reference counterpart: the reference
 * projects the shared hidden with F.linear, qlinear_cuda.py:4454-4502, and reads it back).  partials
 * [slices][batch][rank] as tris_backbone_linear_deferred leaves them; row r of the GEMM is fp16 of the slices'
 * sum added in slice order, the bits tris_backbone_linear writes, so the output equals the predecoded GEMM over
 * that projection's output bit for bit.  decoded: one slot per segment, or with decoded_by_expert != 0 one per
 * expert (as tris_grouped_forward_block_gr_predecoded_experts).  Requires the MFMA kernel's payload conditions,
 * rank <= 512 and batch <= 4 (the decode batches after the fused gate/up GEMM; else TRIS_ERR_INVALID); no output
 * scale or bias is applied.
 */
int tris_grouped_forward_block_gr_predecoded_partials(
    const float* partials, int32_t slices, int32_t batch, const int32_t* expert_ids, const int32_t* segment_offsets,
    int32_t num_segments, int64_t total_problem_tiles, const int32_t* decoded, const tris_compact3_payload* payload,
    uint16_t* output, int32_t decoded_by_expert, void* stream);

/*
 * tris_grouped_forward_block_gr_predecoded_partials for one token routed to two experts, with the routed combine
 * (tris_moe_combine, modeling_mixtral.py:529-536) in the same launch (no reference counterpart): partials
 * [slices][2][rank] are the two routed rows' down backbone, segments 0 and 1 one row each (a top-2 route of one
 * token); inverse_perm [2] and routing_weights_f16 [2] are the route's.  out [1, N] in bf16 (out_bf16 != 0) or
 * fp16 receives dt(fp16(y_r0 * w_r0) + fp16(y_r1 * w_r1)) with y the GEMM's rows rounded to fp16: tris_moe_combine's
 * output over the GEMM's, bit for bit.  A route that is not one token on two valid experts gives zeros.
 */
int tris_grouped_forward_block_gr_predecoded_partials_combine(
    const float* partials, int32_t slices, const int32_t* expert_ids, const int32_t* segment_offsets,
    int64_t total_problem_tiles, const int32_t* decoded, const tris_compact3_payload* payload,
    const int32_t* inverse_perm, const uint16_t* routing_weights_f16, int32_t out_bf16, uint16_t* out,
    int32_t decoded_by_expert, void* stream);

/*
 * Dequantise the listed experts to dense fp16 weights [num, N, rank]
 * (verification kernel; the product GEMMs never write weights).  Replaces the
 * reference's CPU dequant QuantLinear._dequantize_compact3_matrix
 * (qlinear_cuda.py:4200-4236) with the GPU per-weight formula of
 * kernel.cu:665-774 and row-pack selection :830-853.  Uses the GR bitmap.
 */
int tris_compact3_dequant(const tris_compact3_payload* payload, const int32_t* expert_ids, int32_t num,
                          uint16_t* weights, void* stream);

/*
 * Decode the listed experts' GR bitmaps into the dense packed layout
 * int32 [num, ceil(rank/32), N] (verification kernel; inverse of the encoder's
 * block gather, qlinear_cuda.py:3810-3822 / kernel.cu:481-502).
 */
int tris_gr_decode_dense(const int32_t* q_gmap_gr_words, const int32_t* q_gmap_gr_offsets,
                         const int32_t* q_gmap_gr_meta, int32_t num_experts, int32_t words_stride,
                         const int32_t* expert_ids, int32_t num, int32_t packed_rows, int32_t outfeatures,
                         int32_t* dense, void* stream);

/*
 * Shared backbone projection: replaces QuantLinear.compute_shared_hidden's fp16
 * branch (qlinear_cuda.py:4454-4502: F.linear(x * s_in, SV)).  x fp16 [tokens, in];
 * sv fp16 [rank, in]; in_scale fp16 [in] or NULL (applied as fp16(x*s) when
 * ns_mode == 1, :4477-4480); out fp16 [tokens, rank]; fp32 accumulation.
 * row_index int64 [tokens] or NULL gathers x rows (x[row_index[t]]), fusing the
 * reference's index_select (modeling_mixtral.py:467).  x, sv and in_scale must
 * be 16-byte aligned.  workspace: device scratch of
 * tris_backbone_workspace_bytes(tokens, in, rank) bytes (fp32 split-K partial
 * sums; no initial contents needed; may be NULL when that size is 0).  Calls
 * sharing a workspace on different streams must not overlap.  Deterministic:
 * the same inputs give the same bits.
 */
int tris_backbone_linear(const uint16_t* x, int32_t tokens, int32_t in_features, const int64_t* row_index,
                         const uint16_t* sv, int32_t rank, const uint16_t* in_scale, uint16_t* out,
                         void* workspace, int64_t workspace_bytes, void* stream);

/*
 * tris_backbone_linear with its split-K reduction left to the consumer (no reference counterpart; an extension of
 * compute_shared_hidden, qlinear_cuda.py:4454-4502).  *slices is set to the plan's slice count: with one slice out
 * holds the projection, as tris_backbone_linear writes it; with more, out is not written and workspace holds the
 * fp32 partial sums [slices][tokens][rank] that tris_grouped_forward_block_gr_predecoded_partials adds.  Shapes
 * that take the tiled GEMM (prefill-size batches) are rejected with TRIS_ERR_INVALID.
 */
int tris_backbone_linear_deferred(const uint16_t* x, int32_t tokens, int32_t in_features, const int64_t* row_index,
                                  const uint16_t* sv, int32_t rank, const uint16_t* in_scale, uint16_t* out,
                                  void* workspace, int64_t workspace_bytes, int32_t* slices, void* stream);

/* Two backbone projections of the same gathered rows in one launch (no
 * reference counterpart: batches the gate and up compute_shared_hidden calls
 * of a grouped SwiGLU layer, modeling_mixtral.py:467-476, each with its own
 * ns_mode == 1 input scale, qlinear_cuda.py:4477-4480).
 * out_a = fp16(x[row_index] * in_scale_a) . sv_a^T, out_b likewise with
 * in_scale_b (either scale may be NULL), as two calls of tris_backbone_linear
 * would give.  workspace: see tris_backbone_pair_workspace_bytes. */
int tris_backbone_linear_pair(const uint16_t* x, int32_t tokens, int32_t in_features, const int64_t* row_index,
                              const uint16_t* sv_a, const uint16_t* sv_b, int32_t rank, const uint16_t* in_scale_a,
                              const uint16_t* in_scale_b, uint16_t* out_a, uint16_t* out_b, void* workspace,
                              int64_t workspace_bytes, void* stream);

/* The gate/up backbones of prefill-size batches written straight to the routed rows (no reference
 * counterpart: the reference projects the gathered rows, compute_shared_hidden on x[perm],
 * qlinear_cuda.py:4454-4502 with modeling_mixtral.py:467-476; this projects each token once and stores the
 * result to every row the route sends it to, so the gather of the rows is never materialised).
 * out_a[inverse_perm[t * top_k + j]] = fp16(x[t] * in_scale_a) . sv_a^T for every token t and slot j (slots
 * holding -1 or a row >= out_rows are skipped; rows no slot names are left as they are), out_b likewise (sv_b
 * NULL: one projection).  inverse_perm int32 [tokens * top_k] as tris_build_grouped_route writes it; out
 * fp16 [out_rows, rank].  Needs tokens >= 512, rank a multiple of 128 and in_features a multiple of 32 (the
 * tiled GEMM; else TRIS_ERR_INVALID); the values are the bits tris_backbone_linear_pair gives for the token
 * rows.  workspace: tris_backbone_scatter_workspace_bytes(tokens, in_features, rank, 1 or 2). */
int tris_backbone_linear_pair_scatter(const uint16_t* x, int32_t tokens, int32_t in_features, const uint16_t* sv_a,
                                      const uint16_t* sv_b, int32_t rank, const uint16_t* in_scale_a,
                                      const uint16_t* in_scale_b, const int32_t* inverse_perm, int32_t top_k,
                                      int32_t out_rows, uint16_t* out_a, uint16_t* out_b, void* workspace,
                                      int64_t workspace_bytes, void* stream);
int64_t tris_backbone_scatter_workspace_bytes(int32_t tokens, int32_t in_features, int32_t rank, int32_t nproj);

/*
 * tris_backbone_linear with no workspace argument and no allocation (no reference counterpart: for
 * callers that cannot allocate, such as code under HIP graph capture or tight serving loops).  The split-K
 * partial sums live in a file-scope device array of tris_backbone_noalloc_scratch_bytes() bytes (4 MiB,
 * held by every GPU the library runs on until the process ends); its address is looked up once per device
 * on the first call.  Every call on one GPU shares that GPU's array: calls that overlap on one GPU (on
 * different streams, or from different threads) race.  Each launch writes every partial sum it reads, so
 * no clearing is needed.  It runs tris_backbone_linear's plan (the same kernel and split-K slice count), so
 * every shape it accepts gives tris_backbone_linear's results bit for bit.  Shapes whose partial sums
 * (tris_backbone_workspace_bytes) exceed the array are rejected with TRIS_ERR_INVALID: decode-sized batches
 * always fit (below 4 MiB), prefill-size ones (512 rows on, rank a multiple of 128, in_features of 64) may
 * not.
 */
int tris_backbone_linear_noalloc(const uint16_t* x, int32_t tokens, int32_t in_features, const int64_t* row_index,
                                 const uint16_t* sv, int32_t rank, const uint16_t* in_scale, uint16_t* out,
                                 void* stream);

/* Size of the static scratch array of tris_backbone_linear_noalloc, in bytes. */
int64_t tris_backbone_noalloc_scratch_bytes(void);

/* Workspace sizes for tris_backbone_linear / _pair (no reference counterpart:
 * cuBLAS owns its workspace). */
int64_t tris_backbone_pair_workspace_bytes(int32_t tokens, int32_t in_features, int32_t rank);
int64_t tris_backbone_workspace_bytes(int32_t tokens, int32_t in_features, int32_t rank);

/*
 * The down projection's shared backbone with the SwiGLU product of its input fused (no reference
 * counterpart: act_fn(gate_out) * up_out of modeling_mixtral.py:496 formed inside compute_shared_hidden's
 * projection, qlinear_cuda.py:4454-4502, so the product never reaches HBM).  in[r][k] =
 * fp16(fp16(silu(gate[r][k])) * up[r][k]), the bits tris_swiglu_mul writes, times in_scale[k] (an fp16
 * product, the ns_mode == 1 input scale) when in_scale is not NULL; out fp16 [rows, rank] = in . sv^T with
 * fp32 accumulation, split over K and the slices added in fixed order (deterministic).  gate, up fp16
 * [rows, in_features], sv fp16 [rank, in_features]; in_features a multiple of 32; above 128 rows the decode kernel
 * runs in row groups of 128 up to 512 rows for a rank that is not a multiple of 512, and otherwise the tiled
 * prefill GEMM, which needs a rank that is a multiple of 128; 16-byte aligned pointers (else TRIS_ERR_INVALID);
 * workspace of tris_backbone_swiglu_workspace_bytes(rows, in_features, rank).
 */
int tris_backbone_swiglu_linear(const uint16_t* gate, const uint16_t* up, int32_t rows, int32_t in_features,
                                const uint16_t* sv, int32_t rank, const uint16_t* in_scale, uint16_t* out,
                                void* workspace, int64_t workspace_bytes, void* stream);
int64_t tris_backbone_swiglu_workspace_bytes(int32_t rows, int32_t in_features, int32_t rank);

/*
 * tris_backbone_swiglu_linear of two stacked projections with its output split by columns (no reference
 * counterpart: it runs the routed experts' down backbone, compute_shared_hidden of qlinear_cuda.py:4454-4502, and
 * the always-on shared expert's down projection, modeling_qwen2_moe.py:815-818, as one projection of the stacked
 * weights over the stacked rows).  out fp16 [rows, split] gets columns [0, split), out_hi fp16
 * [rows, rank - split] columns [split, rank), each the value the whole projection gives there.  0 < split < rank;
 * the decode kernel only (at most 128 rows, or 512 for a rank that is not a multiple of 512; else TRIS_ERR_INVALID);
 * workspace as tris_backbone_swiglu_linear's.
 */
int tris_backbone_swiglu_linear_split(const uint16_t* gate, const uint16_t* up, int32_t rows, int32_t in_features,
                                      const uint16_t* sv, int32_t rank, const uint16_t* in_scale, uint16_t* out,
                                      uint16_t* out_hi, int32_t split, void* workspace, int64_t workspace_bytes,
                                      void* stream);

/*
 * 4-bit packed backbone matrix (PackedQuantMatrix4bit buffers, qlinear_cuda.py:2637-2786):
 * SV[r][c] = fp16((q - z) * s) with q = nibble c % 8 (bits 4*(c%8)) of qweight[c / 8][r],
 * z = nibble r % 8 of qzeros[g][r / 8] plus one, s = scales[g][r], g = g_idx[c]
 * (the reference's dequantize, :2761-2786).
 */
typedef struct tris_packed4_matrix {
  const int32_t* qweight;  /* int32 [ceil(cols / 8), rows] */
  const int32_t* qzeros;   /* int32 [num_groups, ceil(rows / 8)] */
  const uint16_t* scales;  /* fp16 [num_groups, rows] */
  const int32_t* g_idx;    /* int32 [cols] (may be NULL for the fused projection) */
  int32_t rows;            /* out features (the backbone rank) */
  int32_t cols;            /* in features */
  int32_t num_groups;
  int32_t group_size;      /* > 0 when g_idx[c] == c / group_size for every c, else 0 */
} tris_packed4_matrix;

/* Dequantise to fp16 out [rows, cols] (any g_idx): the reference's
 * PackedQuantMatrix4bit.dequantize (qlinear_cuda.py:2761-2786), bit for bit. */
int tris_packed4_dequant(const tris_packed4_matrix* w, uint16_t* out, void* stream);

/*
 * hidden = x[row_index] (* in_scale) . SV^T from the packed matrix without materialising SV: replaces
 * packed4_linear_forward (TriSMoE_cuda_kernel.cu:8023-8137, called by compute_shared_hidden through
 * _run_packed_4bit_linear_cuda, qlinear_cuda.py:4487-4494).  Same tiling, split-K and workspace
 * (tris_backbone_workspace_bytes(tokens, cols, rows)) as tris_backbone_linear; exact fp16 weights
 * and products, fp32 accumulation (the reference's kernels round products or partial sums to fp16;
 * results agree within the fp16 tolerance).  Needs uniform groups: group_size > 0, a multiple of 8.
 */
int tris_packed4_backbone_linear(const uint16_t* x, int32_t tokens, const int64_t* row_index,
                                 const tris_packed4_matrix* w, const uint16_t* in_scale, uint16_t* out,
                                 void* workspace, int64_t workspace_bytes, void* stream);

/* Gate and up packed backbones of the same rows in one launch, each with its own input scale or NULL
 * (no reference counterpart; see tris_backbone_linear_pair).  Workspace: tris_backbone_pair_workspace_bytes. */
int tris_packed4_backbone_linear_pair(const uint16_t* x, int32_t tokens, const int64_t* row_index,
                                      const tris_packed4_matrix* wa, const tris_packed4_matrix* wb,
                                      const uint16_t* in_scale_a, const uint16_t* in_scale_b, uint16_t* out_a,
                                      uint16_t* out_b, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Matrix-mode null-space compensation payload of one projection (build_grouped_ns_compensation_payload,
 * qlinear_cuda.py:1734-1872): per expert e two 4-bit packed matrices (PackedQuantMatrix4bit layout),
 * C2_e [rank_e, in] and C1_e [out, rank_e], concatenated over the experts:
 *   C2: qweight int32 [ceil(in/8), total_rank], qzeros int32 [ceil(in/group_size), total_rank_words],
 *       scales fp16 [ceil(in/group_size), total_rank]; expert e's rows start at column
 *       ns_c2_rank_offsets[e] (qzeros: ns_c2_rank_word_offsets[e]); experts may share a C2.
 *   C1: qweight int32 [sum ceil(rank_e/8), out] from row ns_c1_rank_word_offsets[e], qzeros int32
 *       [sum groups_e, ceil(out/8)] and scales fp16 [sum groups_e, out] from row ns_c1_group_offsets[e];
 *       groups of min(rank_e, group_size) columns.
 * ns_rank_per_expert[e] == 0: no compensation for expert e.
 */
typedef struct tris_ns_payload {
  const int32_t* ns_rank_per_expert;       /* int32 [E] */
  const int32_t* ns_c2_rank_offsets;       /* int32 [E] */
  const int32_t* ns_c2_rank_word_offsets;  /* int32 [E] */
  const int32_t* ns_c1_rank_word_offsets;  /* int32 [E] */
  const int32_t* ns_c1_group_offsets;      /* int32 [E] */
  const int32_t* ns_c2_qweight;
  const int32_t* ns_c2_qzeros;
  const uint16_t* ns_c2_scales;
  const int32_t* ns_c1_qweight;
  const int32_t* ns_c1_qzeros;
  const uint16_t* ns_c1_scales;
  int32_t num_experts;
  int32_t infeatures;
  int32_t outfeatures;
  int32_t max_ns_rank;                     /* <= 512 */
  int32_t group_size;
  int32_t total_rank;                      /* ns_c2_qweight / ns_c2_scales columns */
  int32_t total_rank_words;                /* ns_c2_qzeros columns */
} tris_ns_payload;

/*
 * comp[r] = fp16(C1_e . fp16(C2_e . x_grouped[r])) for the rows r of every segment (e = its expert):
 * replaces grouped_ns_compensation_forward (TriSMoE_cuda_kernel.cu:1208-2145) and, with accumulate != 0,
 * the caller's out.add_(compensation) (qlinear_cuda.py:2322-2334): out[r] = fp16(out[r] + comp[r]);
 * with accumulate == 0, out = comp.  x_grouped fp16 [batch, in] (16-byte aligned, in % 8 == 0); out fp16
 * [batch, out].  The scale and zero point of element c come from group c / group_size (C2) and
 * j / min(rank_e, group_size) (C1).  workspace: device scratch of
 * tris_grouped_ns_workspace_bytes(batch, num_segments, in, max_ns_rank) bytes (fp32 split-K partial sums
 * of C2 . x, added in a fixed order; no initial contents).  Exact fp16 weights, fp32 sums, fp16 between
 * the two products.  Calls sharing a workspace on different streams must not overlap.
 */
int tris_grouped_ns_compensation_forward(const uint16_t* x_grouped, int32_t batch, const int32_t* expert_ids,
                                         const int32_t* segment_offsets, int32_t num_segments,
                                         const tris_ns_payload* ns, void* workspace, int64_t workspace_bytes,
                                         uint16_t* out, int32_t accumulate, void* stream);

/* Workspace size for tris_grouped_ns_compensation_forward (no reference counterpart). */
int64_t tris_grouped_ns_workspace_bytes(int32_t batch, int32_t num_segments, int32_t infeatures,
                                        int32_t max_ns_rank);

/*
 * Two payloads over the same input rows and routing in one pair of launches: the gate and up
 * projections' compensation terms, which the reference computes with two
 * grouped_ns_compensation_forward calls on the same x_grouped (qlinear_cuda.py:2322-2334, once per
 * projection).  ns_a and ns_b share infeatures; out_a / out_b [batch, out] as out above.  Input rows:
 * with row_index NULL, x is x_grouped [batch, in]; else grouped row r is x[row_index[r]] of x fp16
 * [x_rows, in], row_index int64 [batch] (the route's grouped_token_indices: the gather
 * x.index_select(0, grouped_token_indices) done inside; an index outside [0, x_rows) reads row 0).
 * workspace: tris_grouped_ns_pair_workspace_bytes(...) bytes.
 */
int tris_grouped_ns_compensation_pair_forward(const uint16_t* x, int32_t x_rows, const int64_t* row_index,
                                              int32_t batch, const int32_t* expert_ids,
                                              const int32_t* segment_offsets, int32_t num_segments,
                                              const tris_ns_payload* ns_a, const tris_ns_payload* ns_b,
                                              void* workspace, int64_t workspace_bytes, uint16_t* out_a,
                                              uint16_t* out_b, int32_t accumulate, void* stream);

/*
 * The C1 half alone, on a given hidden: replaces grouped_ns_c1_forward (TriSMoE_cuda.cpp:423-455,
 * kernel.cu:8526-8674; called by run_grouped_ns_c1_forward, qlinear_cuda.py:1964-2025, when every expert
 * shares one cached C2 projection).  comp[r] = fp16(C1_e . hidden[r][0:rank_e]) for the rows of each
 * segment, with accumulate as in tris_grouped_ns_compensation_forward.  hidden fp16 [batch, max_ns_rank];
 * only the C1 fields of ns are read (the C2 pointers may be NULL).
 */
int tris_grouped_ns_c1_forward(const uint16_t* hidden, int32_t batch, const int32_t* expert_ids,
                               const int32_t* segment_offsets, int32_t num_segments, const tris_ns_payload* ns,
                               uint16_t* out, int32_t accumulate, void* stream);

/* Workspace size for tris_grouped_ns_compensation_pair_forward (no reference counterpart). */
int64_t tris_grouped_ns_pair_workspace_bytes(int32_t batch, int32_t num_segments, int32_t infeatures,
                                             int32_t max_ns_rank_a, int32_t max_ns_rank_b);

/*
 * Non-expert compact3 linear: replaces compact3_linear_forward (TriSMoE_cuda.cpp:497-563,
 * kernel.cu:10781-11191, kernels :2146-3130) for block-GR payloads.  The module's matrix is a one-expert
 * payload (num_experts == 1, rank = in_features); output[b][n] = fp16((sum_k x'[b][k] * W[n][k] (+
 * addend[b][n])) (* output_scale[n]) (+ bias[n])) with x' = fp16(input * input_scale) per column when
 * input_scale is given (__hmul), else input.  input fp16 [batch, rank]; addend fp32 [batch, out] or NULL
 * (the module's null-space term C1 . (C2 . x), which the reference adds to the fp32 accumulator before
 * the output scale); output fp16 [batch, out] (every row written).  The exact-weight VALU kernel over one
 * segment of all rows.
 */
int tris_compact3_linear_forward(const uint16_t* input, int32_t batch, const tris_compact3_payload* payload,
                                 const uint16_t* input_scale, const float* addend, uint16_t* output, void* stream);

/*
 * Two non-expert compact3 linears on the same input in one launch (no scale, no bias): replaces
 * compact3_dual_linear_forward (TriSMoE_cuda.cpp:641-700, kernel.cu:11192-11456; the reference returns
 * them stacked [2, batch, out]).  The same bits as two tris_compact3_linear_forward calls.
 */
int tris_compact3_dual_linear_forward(const uint16_t* input, int32_t batch, const tris_compact3_payload* payload_a,
                                      const tris_compact3_payload* payload_b, uint16_t* output_a, uint16_t* output_b,
                                      void* stream);

/*
 * output[b][n] = sum_k input[b][k] * weight[n][k] in fp32, no rounding; input fp16 (input_f16) or fp32
 * (input_f32, exactly one non-NULL), weight fp16 [out, in].  The non-expert linear's null-space term
 * C1 . (C2 . x) from the dequantised packed matrices, kept in fp32 as the reference's kernel does
 * (kernel.cu:2252-2316).  No reference counterpart as a call.
 */
int tris_dense_linear_f32(const uint16_t* input_f16, const float* input_f32, int32_t batch, int32_t in_features,
                          const uint16_t* weight, int32_t out_features, float* output, void* stream);

/*
 * Routing-weighted combine: replaces final.index_add_(0, grouped_token_indices,
 * (down_out * routing).to(output_dtype)) (modeling_mixtral.py:529-536).
 * out[t, :] = bf16( sum_s fp16(expert_out[inverse_perm[t*top_k+s], :] * weights[t, s])
 *                   (+ shared[t, :]) ), summed in fp32 and rounded once.
 * expert_out fp16 [R, hidden] (16-byte aligned when hidden % 8 == 0);
 * inverse_perm int32 [tokens*top_k] (entries < 0 are skipped: picks the route left out); weights fp16
 * [tokens, top_k];
 * shared fp16 [tokens, hidden] or NULL; out bf16 [tokens, hidden].
 */
int tris_moe_combine(const uint16_t* expert_out, const int32_t* inverse_perm, const uint16_t* weights,
                     const uint16_t* shared, int32_t tokens, int32_t top_k, int32_t hidden, uint16_t* out,
                     void* stream);

/*
 * out = act_fn(gate) * up for fp16 tensors of `count` elements (16-byte aligned): SiLU in fp32 rounded
 * to fp16, then the fp16 product, as the reference's MixtralBlockSparseTop2MLP.forward
 * (modeling_mixtral.py:496) computes act_fn(w1(x)) * w3(x) on the two fp16 GEMM outputs.  Used after
 * tris_grouped_dual_forward_block_gr_predecoded; gives the same bits as the fused
 * tris_grouped_swiglu_forward_block_gr_predecoded.
 */
int tris_swiglu_mul(const uint16_t* gate, const uint16_t* up, int64_t count, uint16_t* out, void* stream);

/*
 * tris_swiglu_mul after the null-space compensation of each projection: out = act_fn(fp16(gate + comp_gate))
 * * fp16(up + comp_up), the reference's out.add_(compensation) on each GEMM output (qlinear_cuda.py:2322-2334)
 * followed by act_fn(w1(x)) * w3(x) (modeling_mixtral.py:496), in one pass.  comp_gate / comp_up: fp16
 * like gate, or NULL for no term.  Lets the compensation be computed beside the GEMMs (no reference
 * counterpart as one call).
 */
int tris_swiglu_mul_compensated(const uint16_t* gate, const uint16_t* up, const uint16_t* comp_gate,
                                const uint16_t* comp_up, int64_t count, uint16_t* out, void* stream);

/*
 * tris_moe_combine with expert_out[r] replaced by fp16(expert_out[r] + expert_comp[r]): the down
 * projection's out.add_(compensation) (qlinear_cuda.py:2322-2334) folded into the combine.  expert_comp:
 * fp16 [R, hidden] like expert_out (16-byte aligned when hidden % 8 == 0), or NULL (no reference
 * counterpart as one call).
 */
int tris_moe_combine_compensated(const uint16_t* expert_out, const uint16_t* expert_comp, const int32_t* inverse_perm,
                                 const uint16_t* weights, const uint16_t* shared, int32_t tokens, int32_t top_k,
                                 int32_t hidden, uint16_t* out, void* stream);

/*
 * The block's output with a gated shared expert: replaces the end of the Qwen MoE blocks' forward
 * (modeling_qwen2_moe.py:815-818, modeling_qwen3_5_moe.py:186-188):
 *   shared_expert_output = shared_expert(h).to(dt)
 *   shared_expert_gate   = sigmoid(shared_expert_gate(h)).to(dt)      (Linear(hidden, 1, bias=False))
 *   final = final + shared_expert_gate * shared_expert_output
 * with final = the routed combine of tris_moe_combine_compensated in the output dtype dt (bf16 when
 * out_bf16, else fp16).  Per token t and feature h, every step rounded to dt as torch rounds it:
 *   g = dt(sigmoid(dt(shared_gate_input[t] . shared_gate_weight)))    (fp32 sum of exact products)
 *   out[t, h] = dt(dt(routed[t, h]) + dt(g * dt(shared[t, h])))
 * shared_gate_input [tokens, hidden] and shared_gate_weight [hidden] are in dt (the block's model dtype,
 * as h and the gate Linear are); shared fp16 [tokens, hidden]; out dt [tokens, hidden].  With
 * shared_gate_weight NULL the shared output (or none, with shared NULL) is added ungated before the one
 * rounding, as tris_moe_combine does, in dt.  Tensors are 16-byte aligned when hidden % 8 == 0.
 */
int tris_moe_combine_gated(const uint16_t* expert_out, const uint16_t* expert_comp, const int32_t* inverse_perm,
                           const uint16_t* weights, const uint16_t* shared, const uint16_t* shared_gate_input,
                           const uint16_t* shared_gate_weight, int32_t tokens, int32_t top_k, int32_t hidden,
                           int32_t out_bf16, uint16_t* out, void* stream);

/*
 * The block's router Linear and the expert kernels' input cast in one launch: replaces router_logits =
 * self.gate(hidden_states) (nn.Linear(hidden, num_experts, bias=False) in the model dtype) and the fp16 cast
 * of the kernel input (modeling_mixtral.py:83-90, 546-553).  x [tokens, hidden] and router_weight
 * [num_experts, hidden] in the model dtype (bf16 when model_bf16, else fp16).  Outputs:
 *   router_logits [tokens, num_experts], model dtype: dt(sum_k x[t][k] * w[e][k]), the fp32 sum of the exact
 *     products (on MFMA) rounded once, the block's second output;
 *   logits_f32 [tokens, num_experts]: the same values widened (the softmax input, F.softmax(..., dtype=float));
 *   x16 [tokens, hidden] fp16(x) (round to nearest even) when model_bf16 and x16 is not NULL.
 * hidden a multiple of 8; x, router_weight and x16 16-byte aligned.  No reference counterpart as one call.
 */
int tris_router_linear(const uint16_t* x, const uint16_t* router_weight, int32_t tokens, int32_t hidden,
                       int32_t num_experts, int32_t model_bf16, uint16_t* router_logits, float* logits_f32,
                       uint16_t* x16, void* stream);

/*
 * The block's first launch at decode: tris_router_linear (bf16 model) and the gate/up backbone projections of
 * the same tokens side by side (no reference counterpart as one call: the router Linear and
 * compute_shared_hidden, modeling_mixtral.py:546 and qlinear_cuda.py:4454-4502, do not depend on each
 * other).  x [tokens, hidden] bf16; router_weight [num_experts, hidden] bf16; router_logits bf16 and logits_f32
 * [tokens, num_experts] and x16 [tokens, hidden] as tris_router_linear writes them.  bb projects the same
 * input: bb->x == x (its bf16 values converted to fp16 on load, the bits x16 holds), bb->tokens == tokens
 * <= 64, bb->in_features == hidden.  When the projection is split over K its partial sums stay in
 * bb->workspace for tris_route_predecode_multi_reduce (or tris_grouped_block_gr_predecode_multi_reduce) to
 * add with the same job; the outputs then equal tris_backbone_linear_pair's on x16, bit for bit.
 * hidden a multiple of 8 and at most 8192; 16-byte aligned pointers.
 */
int tris_router_backbone(const uint16_t* x, const uint16_t* router_weight, int32_t tokens, int32_t hidden,
                         int32_t num_experts, uint16_t* router_logits, float* logits_f32, uint16_t* x16,
                         const tris_backbone_pair_job* bb, void* stream);

/*
 * The decode route and the predecode of its experts' split bitmaps in one launch (no reference counterpart as
 * one call: build_grouped_route with the router, TriSMoE_cuda.cpp:741-793 and modeling_mixtral.py:548-555,
 * and the per-projection predecode, TriSMoE_cuda.cpp:836-853).  One workgroup writes the route outputs
 * exactly as tris_route_topk_grouped does; every decode workgroup derives the routed experts from the same
 * router_logits with the same selection, and fills the jobs' buffers as tris_grouped_block_gr_predecode_multi
 * does for that route's expert_ids (num_slots = min(num_experts, num_tokens * top_k) slots, the active experts
 * first).  bb (or NULL): a backbone job whose deferred partial sums are reduced in the same launch, as
 * tris_grouped_block_gr_predecode_multi_reduce does.  num_jobs may be 0 (jobs NULL): the route and bb's reduction
 * alone, for GEMMs that decode the bitmaps themselves.  The one-wavefront route only: num_tokens * top_k <= 64,
 * num_experts <= 8.
 */
int tris_route_predecode_multi_reduce(const float* router_logits, int32_t num_tokens, int32_t num_experts,
                                      int32_t top_k, int32_t renormalize, int32_t m_tile,
                                      uint16_t* routing_weights_f16, float* routing_weights_f32,
                                      int64_t* selected_experts, int64_t* perm, int64_t* grouped_token_indices,
                                      int64_t* grouped_slots, int32_t* grouped_expert_ids, int32_t* expert_ids,
                                      int32_t* segment_offsets, int32_t* problem_offsets, int32_t* counts,
                                      int32_t* inverse_perm, const tris_gr_predecode_job* jobs, int32_t num_jobs,
                                      int32_t num_slots, const tris_backbone_pair_job* bb, void* stream);

/*
 * tris_route_predecode_multi_reduce that decodes every expert's split bitmaps, slot e for expert e (no reference
 * counterpart: the reference predecodes the routed experts, TriSMoE_cuda.cpp:836-853).  The decoders then need
 * nothing from the route, so they start without reading the router logits; at decode batches that route rows to
 * nearly every expert this costs little extra work.  The route outputs are tris_route_predecode_multi_reduce's;
 * each job's buffer holds num_experts slots [num_experts, blocks, 128].  Read them with
 * tris_grouped_forward_block_gr_predecoded_experts.
 */
int tris_route_predecode_all_reduce(const float* router_logits, int32_t num_tokens, int32_t num_experts,
                                    int32_t top_k, int32_t renormalize, int32_t m_tile, uint16_t* routing_weights_f16,
                                    float* routing_weights_f32, int64_t* selected_experts, int64_t* perm,
                                    int64_t* grouped_token_indices, int64_t* grouped_slots,
                                    int32_t* grouped_expert_ids, int32_t* expert_ids, int32_t* segment_offsets,
                                    int32_t* problem_offsets, int32_t* counts, int32_t* inverse_perm,
                                    const tris_gr_predecode_job* jobs, int32_t num_jobs,
                                    const tris_backbone_pair_job* bb, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TRIS_MOE_HIP_H_ */
