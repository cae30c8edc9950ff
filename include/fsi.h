/*
 * fsi.h — C ABI of the MI355X (gfx950) routed sparse path of the foveal sparse indexer.
 *
 * Conventions (every entry point):
 *   - Plain pointers to device memory, element counts, leading dimensions in
 *     elements, and a hipStream_t (passed as void*; NULL = default stream).
 *   - Outputs and workspaces are caller-allocated.  The library never allocates
 *     or frees device memory.  Launches are asynchronous on `stream`.
 *   - Return value: FSI_OK (0) or a negative fsi_status.  No C++ exception
 *     crosses this boundary.  fsi_last_error() gives a per-thread message.
 *   - Workspaces: the first FSI_WORKSPACE_COUNTER_BYTES bytes are an arrival
 *     counter area that must be zero before the first call; every entry point
 *     leaves it zero again and keeps its scratch data after it.  A workspace
 *     zeroed once at allocation can therefore be shared by any number of
 *     stream-ordered calls of any entry points.  Calls that overlap in time
 *     must not share a workspace.
 *   - Kernels never read outside the given arrays: out-of-range block / page
 *     indices are skipped and reported through the optional device error word
 *     `err` (first error code wins; caller zeroes it).
 */
#ifndef FSI_H_
#define FSI_H_

#include <stddef.h>
#include <stdint.h>

#if defined(__GNUC__) || defined(__clang__)
#define FSI_API __attribute__((visibility("default")))
#else
#define FSI_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

typedef enum fsi_status {
  FSI_OK = 0,
  FSI_ERR_INVALID_ARG = -1,  /* null pointer, bad enum, non-positive size        */
  FSI_ERR_SHAPE = -2,        /* inconsistent or unsupported dimensions            */
  FSI_ERR_INDEX_RANGE = -3,  /* block / page index outside [0, n)                 */
  FSI_ERR_CAPACITY = -4,     /* count or size beyond a documented maximum         */
  FSI_ERR_DTYPE = -5,        /* dtype not supported by this entry point           */
  FSI_ERR_HIP = -6,          /* HIP runtime reported an error at launch           */
  FSI_ERR_ALIGN = -7,        /* pointer / leading dimension not suitably aligned  */
  FSI_ERR_WORKSPACE = -8     /* workspace missing or smaller than required        */
} fsi_status;

/* FSI_DTYPE_F16 is accepted only where an entry point says so
 * (fsi_sram_indexer_attention). */
typedef enum fsi_dtype { FSI_DTYPE_F32 = 0, FSI_DTYPE_BF16 = 1, FSI_DTYPE_F16 = 2 } fsi_dtype;

/* Size of the zero-initialised arrival-counter area at the start of every workspace. */
#define FSI_WORKSPACE_COUNTER_BYTES 65536

/* Activation codes of the fused non-softmax Pattention
 * (foveal_indexer/pattention_triton.py:121,245). */
typedef enum fsi_activation {
  FSI_ACT_SWIGLU = 0,
  FSI_ACT_SILU = 1,
  FSI_ACT_GELU = 2, /* exact erf GeLU, as the reference's PyTorch path (pattention_triton.py:300) */
  FSI_ACT_RELU = 3,
  FSI_ACT_RELU2 = 4
} fsi_activation;

/* Where bf16 rounding happens in the activation (bf16 only; fp32 never rounds).
 *   EAGER: g,u rounded; silu(g) rounded; product rounded
 *          (foveal_pattention.py:284,334 CPU branch `F.silu(kg)*ku`; pattention_triton.py:292-308)
 *   FUSED: g,u rounded; silu(g)*u computed in fp32, rounded once
 *          (foveal_pattention.py:282,332 -> pattention_triton.py:40-47 `_swiglu_fwd_kernel`)
 *   FP32 : act from the fp32 accumulators, rounded once before the V contraction
 *          (pattention_triton.py:172-197 `_pattention_fused_kernel`) */
typedef enum fsi_rounding { FSI_ROUND_EAGER = 0, FSI_ROUND_FUSED = 1, FSI_ROUND_FP32 = 2 } fsi_rounding;

FSI_API int fsi_abi_version(void);
FSI_API const char* fsi_status_string(int status);
FSI_API const char* fsi_last_error(void);

/* ------------------------------------------------------------------------- *
 * Block-sparse non-softmax Pattention forward
 *   out[M, D_out] = act(x K_gate[S]^T [, x K_up[S]^T]) V[S]
 * where S is the channel set { active_blocks[i]*block_n + j : j < block_n } in
 * list order (or all N_p channels when active_blocks == NULL).
 *
 * Replaces:
 *   triton_pattention + _pattention_fused_kernel   foveal_indexer/pattention_triton.py:108-277
 *   _pytorch_pattention_fallback                   foveal_indexer/pattention_triton.py:280-311
 *   FovealPattentionMLP 3x F.linear + SwiGLU body  foveal_indexer/foveal_pattention.py:278-288,328-335
 *
 * x: [M, K] (row stride ldx); k_gate, k_up: [N_p, K] (row stride ldk);
 * v: [N_p, D_out] (row stride ldv), or with v_transposed != 0 stored as
 * [D_out, N_p] (row stride ldv) — the layout of a dense MLP's down_proj weight,
 * which the bf16 decode kernels read with full-line loads (fastest path);
 * out: [M, D_out] (row stride ldo).
 * dtype: FSI_DTYPE_BF16 (fp32 accumulate) or FSI_DTYPE_F32.  k_up may be NULL
 * unless activation == SWIGLU.  block_n: power of two.  Channels whose row is
 * >= N_p contribute zero (the reference kernel's mask, pattention_triton.py:151).
 * M, K, D_out: any size; bf16 requires K % 8 == 0 and 16-byte aligned
 * x / k_gate / k_up rows, and each tensor smaller than 4 GiB.
 * ------------------------------------------------------------------------- */
FSI_API size_t fsi_pattention_workspace_size(int64_t M, int64_t K, int64_t D_out, int64_t n_channels, int dtype);

FSI_API int fsi_pattention_fwd(const void* x, int64_t ldx, const void* k_gate, const void* k_up, int64_t ldk,
                       const void* v, int64_t ldv, int v_transposed, const int32_t* active_blocks, int64_t n_active,
                       int64_t block_n, int64_t M, int64_t K, int64_t N_p, int64_t D_out, int dtype,
                       int activation, int rounding, void* out, int64_t ldo, void* workspace,
                       size_t workspace_bytes, int* err, void* stream);

/* ------------------------------------------------------------------------- *
 * Decode Pattention over weights repacked into the MFMA operand layout (bf16,
 * SwiGLU).  The reference streams k_gate / k_up / v rows of the active blocks
 * after copying them (foveal_pattention.py:115-122, 278-288); here the three
 * weights are repacked once per weight version, and each decode step streams
 * the active blocks' 1 KiB operand tiles.
 *
 * fsi_pattention_pack: k_gate, k_up [N_p, K] (row stride ldk); v as in
 * fsi_pattention_fwd ([N_p, D_out], or [D_out, N_p] storage with v_transposed).
 * packed: fsi_pattention_packed_size(N_p, K, D_out) bytes, 256-byte aligned.
 * Requires block_n a power of two >= 32 dividing N_p, K % 32 == 0,
 * D_out % 16 == 0.
 *
 * fsi_pattention_fwd_packed: out[M, D_out] = (silu(x K_g,S^T) * (x K_u,S^T)) V_S
 * for K = 256 * {1, 2, 4, 8, 16, 32} and either 1 <= M <= 64 tokens (decode
 * kernels, at most 8192 active channels) or M >= 256 (prefill: the 256 x 256
 * GEMMs reading the same packed tiles, at most 2048 active blocks); rounding as
 * fsi_pattention_fwd.  Out-of-range block ids contribute zero and are reported
 * through err.  Workspace: fsi_pattention_packed_workspace_size(M, K, D_out,
 * n_channels, block_n) (for prefill it holds H [M, n_channels]).
 * ------------------------------------------------------------------------- */
FSI_API size_t fsi_pattention_packed_size(int64_t N_p, int64_t K, int64_t D_out);

FSI_API int fsi_pattention_pack(const void* k_gate, const void* k_up, int64_t ldk, const void* v, int64_t ldv,
                                int v_transposed, int64_t N_p, int64_t K, int64_t D_out, int64_t block_n, int dtype,
                                void* packed, size_t packed_bytes, void* stream);

FSI_API size_t fsi_pattention_packed_workspace_size(int64_t M, int64_t K, int64_t D_out, int64_t n_channels,
                                                    int64_t block_n);

FSI_API int fsi_pattention_fwd_packed(const void* x, int64_t ldx, const void* packed, const int32_t* active_blocks,
                                      int64_t n_active, int64_t block_n, int64_t M, int64_t K, int64_t N_p,
                                      int64_t D_out, int dtype, int rounding, void* out, int64_t ldo,
                                      void* workspace, size_t workspace_bytes, int* err, void* stream);

/* Elementwise SwiGLU: out = silu(g) * u, computed in fp32 and rounded once to
 * the storage dtype (rounding = FUSED) or with torch-eager rounding points
 * (rounding = EAGER).  Replaces triton_fused_swiglu / _swiglu_fwd_kernel
 * (foveal_indexer/pattention_triton.py:30-47,98-104). */
FSI_API int fsi_swiglu(const void* g, const void* u, void* out, int64_t n, int dtype, int rounding, void* stream);

/* SwiGLU backward: with s = sigmoid(g), du = dout * g * s and
 * dg = dout * u * s * (1 + g * (1 - s)), computed in fp32 and rounded once to the
 * storage dtype.  Replaces _swiglu_bwd_kernel / TritonFusedSwiGLUFunction.backward
 * (foveal_indexer/pattention_triton.py:49-71, 86-96). */
FSI_API int fsi_swiglu_bwd(const void* dout, const void* g, const void* u, void* dg, void* du, int64_t n, int dtype,
                           void* stream);

/* ------------------------------------------------------------------------- *
 * Pooled 16-D router of FovealPattentionMLP in eval mode
 * (foveal_indexer/foveal_pattention.py:310-322):
 *   q = rms_norm(q_proj(mean_tokens(x))); s = q . block_keys^T * score_scale
 *   out_active = [0..base) ++ (topk(s[base:], remote_blocks) + base)
 * Top-k order is descending score, ties broken by the lower block index.
 * x: [M, D] (row stride ldx); q_proj_w: [index_dim, D]; block_keys:
 * [n_blocks, index_dim]; all of `dtype`.  out_active: base + remote int32.
 * out_scores (optional): n_blocks fp32 (the bf16-rounded scores for bf16).
 * Workspace: fsi_mlp_router_workspace_size(D, n_blocks) bytes (no counters).
 * ------------------------------------------------------------------------- */
FSI_API size_t fsi_mlp_router_workspace_size(int64_t D, int64_t n_blocks);

FSI_API int fsi_mlp_router(const void* x, int64_t ldx, int64_t M, int64_t D, const void* q_proj_w,
                           int64_t index_dim, const void* block_keys, int64_t n_blocks, int64_t base_blocks,
                           int64_t remote_blocks, float score_scale, int dtype, int32_t* out_active,
                           float* out_scores, void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------- *
 * 16-D indexer routing.
 * Selection semantics (every entry point below): fp32 masked softmax over the
 * complete entries, remote candidates ranked by probability (equal
 * probabilities: lower index first), running mass accumulated in fp64 and
 * rounded to fp32 per rank, and
 *   target = max(top_p - local_mass, 0)
 *   needed = #(cum < target) + (target > 0); max(needed, K_min) if any remote
 *   count  = min(needed, available, K_max)
 * ------------------------------------------------------------------------- */
#define FSI_ROUTE_MAX_BLOCKS 65536     /* blocks (or pages) per routed row           */
#define FSI_SCORE_ROUTE_MAX_KEYS 65536 /* keys per row of fsi_score_and_route        */
#define FSI_ROUTE_MAX_RANKED 256       /* bound on min(max(K_max, capacity), blocks) */

/* masked_softmax (foveal_indexer/core.py:36-43): fp32 softmax of scores over
 * the entries where mask != 0, masked entries exactly 0, rows without a valid
 * entry all 0, written in the scores' dtype.  scores/out: contiguous (B, Q, N);
 * mask: uint8 with element strides over (B, Q, N) (0 = broadcast). */
FSI_API int fsi_masked_softmax(const void* scores, int dtype, int64_t B, int64_t Q, int64_t N, const uint8_t* mask,
                               int64_t mask_stride_b, int64_t mask_stride_q, int64_t mask_stride_n, void* out,
                               void* stream);

/* Backward of masked_softmax (autograd of core.py:36-43): dscores = p (dp - sum p dp)
 * on masked-in entries, 0 elsewhere, with p recomputed in fp32 from scores.
 * scores/dprobs/dscores: contiguous (B, Q, N); mask as in fsi_masked_softmax. */
FSI_API int fsi_masked_softmax_bwd(const void* scores, const void* dprobs, int dtype, int64_t B, int64_t Q, int64_t N,
                                   const uint8_t* mask, int64_t mask_stride_b, int64_t mask_stride_q,
                                   int64_t mask_stride_n, void* dscores, void* stream);

/* select_blocks on materialised scores
 * (foveal_indexer/core.py:46-160, via FovealIndexer.route core.py:268-286).
 * scores: (B, Qb, Nb) contiguous fp32 or bf16 (upcast to fp32 first).
 * Masks: causal -> complete = p < q, local = the local_window_blocks blocks
 * before q; non-causal -> every block complete, local = p < local_window_blocks.
 * top_p / k_min / k_max apply to every row unless the matching *_rows array
 * (B*Qb values, device memory) is given; with k_max_rows, k_max_bound must be
 * >= every value in it.
 * out_indices (B, Qb, capacity) int32: remote blocks in rank order, then the
 * non-remote blocks in index order, then zeros past Nb (core.py:121-123).
 * out_counts (B, Qb) int32; out_mass (optional, B*Qb fp32) = local mass +
 * cumulative remote mass of the selected blocks. */
FSI_API int fsi_route_from_scores(const void* scores, int dtype, int64_t B, int64_t Qb, int64_t Nb, int causal,
                                  int local_window_blocks, float top_p, int k_min, int k_max, int capacity,
                                  const float* top_p_rows, const int32_t* k_min_rows, const int32_t* k_max_rows,
                                  int k_max_bound, int32_t* out_indices, int32_t* out_counts, float* out_mass,
                                  void* stream);

/* Fused cosine scoring + select_blocks: scores = normalize(q) . normalize(k) /
 * sqrt(index_dim), all in fp32 (the fp32 form of FovealIndexer.compute_block_scores,
 * foveal_indexer/core.py:254-266), never materialised.  q: (B, Q, 16) and k: (N, 16)
 * per batch entry at element offset b * k_batch_stride (0 = shared keys), both
 * of `dtype`, k 16-byte aligned.  Outputs as fsi_route_from_scores; the query
 * row index is the query block index of the causal mask. */
FSI_API int fsi_score_and_route(const void* q, const void* k, int dtype, int64_t B, int64_t Q,
                                int64_t N, int64_t index_dim, int64_t k_batch_stride, int causal,
                                int local_window_blocks, float top_p, int k_min, int k_max, int capacity,
                                int32_t* out_indices, int32_t* out_counts, float* out_mass, void* stream);

/* decode_step remote-page routing and additive-stream context
 * (foveal_indexer/attention.py:313-337,369-376), one sequence per row.
 * qi: (B, 16) in dtype; kp: (B, P, 16) fp32 page keys; vp: (B, P, 16) in dtype.
 * Position per sequence: pos_rows[b] (device int32) or pos for all.
 * first_local_page = max(0, pos + 1 - window) / page_size; routes only when
 * completed_pages > first_local_page > 0, over pages [0, first_local_page):
 * count = min(max(K_min, min(#(cum < top_p) + 1, min(K_max, first_local_page))),
 * first_local_page).  out_pages (B, capacity) int32: page ids in rank order, -1
 * past count (capacity >= max(K_max, K_min) returns every selected page).
 * out_context (optional, (B, 16) in dtype): softmax over all completed pages
 * (probabilities cast to dtype) times vp. */
FSI_API int fsi_decode_route(const void* qi, const float* kp, const void* vp, int dtype, int64_t B, int64_t P,
                             int64_t index_dim, const int32_t* pos_rows, int64_t pos, int64_t page_size,
                             int64_t window, int64_t completed_pages, float top_p, int k_min, int k_max,
                             int capacity, int32_t* out_pages, int32_t* out_counts, void* out_context,
                             void* stream);

/* ------------------------------------------------------------------------- *
 * FovealIndexer representations (foveal_indexer/core.py:214-312), index_dim 16.
 * The D -> 16 projections are plain GEMMs done by the caller; these entry
 * points apply everything after them with the reference's bf16 rounding points.
 * All tensors contiguous and of `dtype`.
 * ------------------------------------------------------------------------- */
/* F.rms_norm over the 16 components (eps = FLT_EPSILON), x/out: (M, 16).
 * Replaces the norm of compute_query_16d (core.py:221-222) and of decode_step's
 * index key (attention.py:305). */
FSI_API int fsi_index_rms_norm(const void* x, int dtype, int64_t M, int64_t index_dim, void* out, void* stream);

/* compute_kv_blocks_16d after the projections (core.py:241-250):
 * k_blocks = normalize(mean_block(rms_norm(k_lin))), v_blocks = mean_block(v_lin).
 * k_lin/v_lin: (B, N, 16); k_blocks/v_blocks: (B, N / block_size, 16). */
FSI_API int fsi_index_pool_kv(const void* k_lin, const void* v_lin, int dtype, int64_t B, int64_t N,
                              int64_t index_dim, int64_t block_size, void* k_blocks, void* v_blocks, void* stream);

/* FovealKVCache page pooling at the end of a page (attention.py:84-91):
 * kp = normalize(mean(partial_k)) in fp32, vp = mean(partial_v) in dtype.
 * partial_k/partial_v: (B, page_size, 16) contiguous; kp_out (fp32) and vp_out
 * (dtype) rows are written at element offset b * out_batch_stride. */
FSI_API int fsi_kv_page_pool(const void* partial_k, const void* partial_v, int dtype, int64_t B, int64_t page_size,
                             int64_t index_dim, float* kp_out, void* vp_out, int64_t out_batch_stride,
                             void* stream);

/* compute_block_scores (core.py:254-266): normalize(q) . normalize(k) / sqrt(16)
 * with the operands rounded to dtype after normalising and the product rounded
 * before the division.  q: (B, Q, 16); k: (B, N, 16); out: (B, Q, N). */
FSI_API int fsi_block_scores(const void* q, const void* k, int dtype, int64_t B, int64_t Q, int64_t N,
                             int64_t index_dim, void* out, void* stream);

/* additive_stream up to the output projection (core.py:288-310):
 * context = masked_softmax(scores, causal ? p < q : all) . v_blocks, probabilities
 * rounded to dtype.  scores: (B, Q, N); v_blocks: (B, N, 16); context: (B, Q, 16). */
FSI_API int fsi_additive_context(const void* scores, const void* v_blocks, int dtype, int64_t B, int64_t Q,
                                 int64_t N, int64_t index_dim, int causal, void* context, void* stream);

/* ------------------------------------------------------------------------- *
 * Dense teacher block targets for KL distillation
 * (archive/hy_mt2/llm_pattention/train_foveal_pattention_speedrun.py:154-189,
 * compute_teacher_dense_block_targets): with act = silu(h W_gate^T) * (h W_up^T)
 * over all I channels (bf16 roundings of eager SwiGLU), dw[b] = block mean of
 * W_down's column norms, out[m, b] = softmax_b(bf16(bf16(mean_b |act[m]|) * dw[b]) / T).
 * h: (M, D) bf16 rows (stride ldh); w_gate, w_up: (I, D) bf16 (stride ld_gu);
 * w_down: (D, I) bf16 (stride ld_down); out: (M, I / block_size) fp32 (stride ldo).
 * block_size a multiple of 32 dividing I; D % 8 == 0; 16-byte aligned h and
 * gate/up rows.  Workspace (256-byte aligned, need not be zeroed) from
 * fsi_dense_block_targets_workspace_size. */
FSI_API size_t fsi_dense_block_targets_workspace_size(int64_t M, int64_t D, int64_t I, int64_t block_size);
FSI_API int fsi_dense_block_targets(const void* h, int64_t ldh, const void* w_gate, const void* w_up, int64_t ld_gu,
                                    const void* w_down, int64_t ld_down, int64_t M, int64_t D, int64_t I,
                                    int64_t block_size, float temperature, float* out, int64_t ldo, void* workspace,
                                    size_t workspace_bytes, void* stream);

/* Backward passes of the four entry points above: the autograd of
 * compute_query_16d, compute_kv_blocks_16d, compute_block_scores and
 * additive_stream (core.py:214-310, exercised by tests/test_indexer.py:63-101).
 * Gradients are computed in fp32 from the forward inputs (intermediates
 * recomputed) and rounded to dtype where the reference's graph holds a tensor
 * of that dtype.  Shapes as in the forward; gradient tensors have the shapes
 * of the tensors they belong to. */
FSI_API int fsi_index_rms_norm_bwd(const void* x, const void* dy, int dtype, int64_t M, int64_t index_dim, void* dx,
                                   void* stream);
FSI_API int fsi_index_pool_kv_bwd(const void* k_lin, const void* dk_blocks, const void* dv_blocks, int dtype, int64_t B,
                                  int64_t N, int64_t index_dim, int64_t block_size, void* dk_lin, void* dv_lin,
                                  void* stream);
FSI_API int fsi_block_scores_bwd(const void* q, const void* k, const void* dscores, int dtype, int64_t B, int64_t Q,
                                 int64_t N, int64_t index_dim, void* dq, void* dk, void* stream);
/* Workspace: per-row softmax statistics, written before they are read (need
 * not be zeroed), 8-byte aligned. */
FSI_API size_t fsi_additive_context_bwd_workspace_size(int64_t B, int64_t Q);
FSI_API int fsi_additive_context_bwd(const void* scores, const void* v_blocks, const void* dcontext, int dtype,
                                     int64_t B, int64_t Q, int64_t N, int64_t index_dim, int causal, void* dscores,
                                     void* dv_blocks, void* workspace, size_t workspace_bytes, void* stream);

/* Block-level KL distillation loss, FovealIndexer.distillation_loss
 * (foveal_indexer/core.py:315-353).  Per row (b, q) with valid set V
 * (mask_mode 0: every entry; 1: the causal set p < q; 2: mask[b, q, p] != 0,
 * uint8 with element strides, 0 = broadcast):
 *   target = max(t, 0) / sum_V max(t, 0) if that sum > 1e-12, else 1 / |V|;
 *   row loss = -sum_V target * log_softmax_V(s / temperature).
 * loss[0] (fp32, device) = mean of the row losses over rows with |V| > 0 (0 if
 * none); n_rows[0] (device) = that row count.  scores, teacher: contiguous
 * (B, Q, N) fp32 or bf16.  Workspace: fsi_distill_kl_workspace_size(B, Q) bytes. */
FSI_API size_t fsi_distill_kl_workspace_size(int64_t B, int64_t Q);
FSI_API int fsi_distill_kl_fwd(const void* scores, int s_dtype, const void* teacher, int t_dtype, int64_t B,
                               int64_t Q, int64_t N, int mask_mode, const uint8_t* mask, int64_t mask_stride_b,
                               int64_t mask_stride_q, int64_t mask_stride_n, float temperature, float* loss,
                               int32_t* n_rows, void* workspace, size_t workspace_bytes, void* stream);
/* Gradient of that loss with respect to the scores (the teacher takes none):
 * dscores = dloss[0] / n_rows[0] * (softmax_V(z) * sum_V target - target) / temperature
 * on valid entries of valid rows, 0 elsewhere, written in the scores' dtype.
 * dloss and n_rows are device scalars (n_rows as the forward wrote it). */
FSI_API int fsi_distill_kl_bwd(const void* scores, int s_dtype, const void* teacher, int t_dtype, int64_t B,
                               int64_t Q, int64_t N, int mask_mode, const uint8_t* mask, int64_t mask_stride_b,
                               int64_t mask_stride_q, int64_t mask_stride_n, float temperature, const float* dloss,
                               const int32_t* n_rows, void* dscores, void* stream);

/* ------------------------------------------------------------------------- *
 * Foveal paged-KV decode attention (foveal_indexer/attention.py:284-367).
 * Paged pools (bf16), page = 64 tokens of one sequence for all KV heads:
 *   K pool: [n_phys_pages][Hkv][head_dim/32][64][32]
 *   V pool: [n_phys_pages][Hkv][2][head_dim][32], each 32-token half stored
 *           dim-major with token tau at slot 8*((tau%16)/4) + 4*(tau/16) + tau%4
 * page_table: (B, max_pages) int32 logical page -> physical page.
 * head_dim: 64 or 128.
 * ------------------------------------------------------------------------- */
/* Write tokens start .. start + n_tok - 1 (start_rows[b] per sequence, or start)
 * of K and V given as (B, Hkv, n_tok, head_dim) bf16 with element strides
 * (16-byte aligned rows) into the pools.  Replaces the slice writes of
 * FovealKVCache.update (attention.py:72-73).  Positions outside the page table
 * or pages outside the pool are skipped and reported through err. */
FSI_API int fsi_kv_write(const void* k, const void* v, int64_t k_stride_b, int64_t k_stride_h, int64_t k_stride_t,
                         int64_t v_stride_b, int64_t v_stride_h, int64_t v_stride_t, int64_t B, int64_t Hkv,
                         int64_t n_tok, int64_t head_dim, const int32_t* start_rows, int64_t start,
                         const int32_t* page_table, int64_t max_pages, int64_t n_phys_pages, void* k_pool,
                         void* v_pool, int* err, void* stream);

/* Read tokens [0, n_tok) of every sequence back to contiguous (B, Hkv, n_tok,
 * head_dim) K and V (the reference cache layout, attention.py:48-49). */
FSI_API int fsi_kv_read(const void* k_pool, const void* v_pool, int64_t B, int64_t Hkv, int64_t n_tok,
                        int64_t head_dim, const int32_t* page_table, int64_t max_pages, int64_t n_phys_pages,
                        void* k_out, void* v_out, void* stream);

FSI_API size_t fsi_decode_attn_workspace_size(int64_t B, int64_t Hq, int64_t Hkv, int64_t head_dim, int64_t window,
                                              int64_t capacity, int64_t max_pages);

/* out (B, Hq, head_dim) bf16 = softmax(scale * q K^T) V over each sequence's
 * support: tokens [max(0, pos + 1 - window), pos] followed by the pages
 * remote_pages[b, :remote_counts[b]] (logical ids, as fsi_decode_route returns
 * them).  Query head h uses KV head h / (Hq / Hkv); Hq / Hkv <= 16.
 * Replaces the gather + repeat_interleave + SDPA of decode_step
 * (attention.py:339-365).  remote_pages/remote_counts may be NULL when
 * capacity == 0.  Invalid page ids are skipped and reported through err. */
FSI_API int fsi_decode_attn(const void* q, const void* k_pool, const void* v_pool, const int32_t* page_table,
                            int64_t max_pages, int64_t n_phys_pages, const int32_t* pos_rows, int64_t pos,
                            int64_t window, const int32_t* remote_pages, const int32_t* remote_counts,
                            int64_t capacity, int64_t B, int64_t Hq, int64_t Hkv, int64_t head_dim, float scale,
                            void* out, void* workspace, size_t workspace_bytes, int* err, void* stream);

/* Fused decode step: fsi_decode_route (bf16 index query and page values, page
 * size 64, index_dim 16) and fsi_decode_attn (bf16 paged pools).  With at least
 * one (sequence, KV head) pair per compute unit and at most 2048 complete pages,
 * one launch: per pair, four waves route the sequence while four stream the
 * local window, then all stream the selected pages and merge.  Otherwise two
 * launches: workgroups routing each sequence beside the local-window partials,
 * then the selected pages' partials and the merge.  Outputs as the two calls:
 * pages / counts (context optional) and out, bit-identical routing either way.  batch0 != 0: every sequence attends sequence 0's pages,
 * as the reference's decode_step does (attention.py:348).  Workspace:
 * fsi_decode_attn_workspace_size(B, Hq, Hkv, head_dim, window, capacity,
 * max_pages).  Replaces decode_step's routing + attention
 * (attention.py:313-365). */
FSI_API int fsi_decode_step_attn(const void* qi, const float* kp, const void* vp, int64_t P, int64_t completed_pages,
                                 float top_p, int k_min, int k_max, int capacity, int32_t* out_pages,
                                 int32_t* out_counts, void* out_context, const void* q, const void* k_pool,
                                 const void* v_pool, const int32_t* page_table, int64_t max_pages,
                                 int64_t n_phys_pages, const int32_t* pos_rows, int64_t pos, int64_t window,
                                 int64_t B, int64_t Hq, int64_t Hkv, int64_t head_dim, float scale, int batch0,
                                 void* out, void* workspace, size_t workspace_bytes, int* err, void* stream);

/* Decode attention over the reference's contiguous cache layout
 * (FovealKVCache k_cache / v_cache (B, Hkv, max_seq, head_dim), attention.py:45-57),
 * fp32 or bf16, any page size, head_dim 1..256: the same support as
 * fsi_decode_attn (tokens [max(0, pos + 1 - window), pos], then every token of
 * each page remote_pages[b, :remote_counts[b]], concatenated as attention.py:341-352
 * gathers them) and the same result, computed in fp32.  Cache strides in
 * elements (unit stride over head_dim); q and out contiguous (B, Hq, head_dim)
 * of `dtype`.  Tokens beyond max_seq are skipped and reported through err.
 * Replaces the gather + repeat_interleave + SDPA of attention.py:339-365.
 * With a workspace of fsi_decode_attn_dense_workspace_size(B, Hq, head_dim,
 * window, capacity, page_size, max_seq) bytes, fp32 caches with head_dim 64 or
 * 128 and 16-byte aligned K rows run split over the keys on MFMA (partials in
 * the workspace, then a merge); otherwise (workspace NULL, bf16, other head
 * dims) one wave per query head. */
FSI_API size_t fsi_decode_attn_dense_workspace_size(int64_t B, int64_t Hq, int64_t head_dim, int64_t window,
                                                    int64_t capacity, int64_t page_size, int64_t max_seq);
FSI_API int fsi_decode_attn_dense(const void* q, const void* k_cache, const void* v_cache, int64_t ks_b, int64_t ks_h,
                                  int64_t ks_t, int64_t vs_b, int64_t vs_h, int64_t vs_t, int64_t max_seq,
                                  const int32_t* pos_rows, int64_t pos, int64_t window, int64_t page_size,
                                  const int32_t* remote_pages, const int32_t* remote_counts, int64_t capacity,
                                  int64_t B, int64_t Hq, int64_t Hkv, int64_t head_dim, float scale, int dtype,
                                  void* out, void* workspace, size_t workspace_bytes, int* err, void* stream);

/* fsi_decode_attn without a workspace argument and without any allocation.
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  The partials live in a file-scope device array of
 * FSI_DECODE_ATTN_NOALLOC_MAX_BYTES per GPU, held until the process ends; a
 * call needing more (fsi_decode_attn_workspace_size(...) -
 * FSI_WORKSPACE_COUNTER_BYTES - 256 bytes, about 4.5 MB for 32 sequences x 32
 * heads x head_dim 128) returns FSI_ERR_CAPACITY.  Every call on one GPU shares
 * that array: calls that overlap in time on one GPU (different streams, or
 * different host threads without ordering) race and must not be issued.
 * Arguments and results are those of fsi_decode_attn. */
#define FSI_DECODE_ATTN_NOALLOC_MAX_BYTES (16u << 20)
FSI_API int fsi_decode_attn_noalloc(const void* q, const void* k_pool, const void* v_pool, const int32_t* page_table,
                                    int64_t max_pages, int64_t n_phys_pages, const int32_t* pos_rows, int64_t pos,
                                    int64_t window, const int32_t* remote_pages, const int32_t* remote_counts,
                                    int64_t capacity, int64_t B, int64_t Hq, int64_t Hkv, int64_t head_dim,
                                    float scale, void* out, int* err, void* stream);

/* Query gradient of decode attention (autograd of attention.py:339-367 in q;
 * the cache is a constant): dq = scale sum_t p_t (dout . v_t - dout . o) k_t over
 * each sequence's support, fp32 math, written to dq (B, Hq, head_dim) fp32.  q,
 * dout: contiguous (B, Hq, head_dim) of dtype.  With page_table (paged bf16
 * pools of fsi_decode_attn: page 64, head_dim 64 or 128) the pools are read
 * through it; without, k_cache / v_cache are the contiguous (B, Hkv, max_seq,
 * head_dim) cache given by element strides (any page_size, head_dim <= 256).
 * Other arguments as fsi_decode_attn / fsi_decode_attn_dense. */
FSI_API int fsi_decode_attn_bwd_q(const void* q, const void* dout, const void* k_cache, const void* v_cache,
                                  int64_t ks_b, int64_t ks_h, int64_t ks_t, int64_t vs_b, int64_t vs_h, int64_t vs_t,
                                  int64_t max_seq, const int32_t* page_table, int64_t max_pages, int64_t n_phys_pages,
                                  const int32_t* pos_rows, int64_t pos, int64_t window, int64_t page_size,
                                  const int32_t* remote_pages, const int32_t* remote_counts, int64_t capacity,
                                  int64_t B, int64_t Hq, int64_t Hkv, int64_t head_dim, float scale, int dtype,
                                  float* dq, int* err, void* stream);

/* ------------------------------------------------------------------------- *
 * Block-sparse prefill attention (bf16 in, fp32 softmax and accumulate, bf16 out).
 * q: (B, Hq, T, head_dim), k and v: (B, Hkv, T, head_dim), out: (B, Hq, T,
 * head_dim), each given by element strides (s_b, s_h, s_t; unit stride over
 * head_dim).  Query head h uses KV head h / (Hq / Hkv).  Query block qb holds
 * queries [qb * block, (qb + 1) * block); lists: (B, ceil(T / block), capacity)
 * int32 key-block ids (strides ls_b, ls_q), counts: (B, ceil(T / block)) int32
 * (strides cs_b, cs_q; values clamped to [0, capacity]).  Key block j holds keys
 * [j * block, min((j + 1) * block, T)).  Ids outside [0, ceil(T / block)) are
 * skipped and reported through err.  A query with no key gets 0.
 * ------------------------------------------------------------------------- */
typedef enum fsi_sattn_mode {
  /* FovealSparseAttention.forward with _build_sparse_mask (attention.py:148-227):
   * query t sees keys s with t - window < s <= t, plus every key of the listed
   * remote pages of its block (a union: a key in both, or in a page listed
   * twice, counts once). */
  FSI_SATTN_LOCAL_REMOTE = 0,
  /* triton_foveal_sparse_attention (foveal_indexer/triton_ops.py:26-93,256-313):
   * query block qb sees every key of each listed block, no causal mask (a block
   * listed twice counts twice). */
  FSI_SATTN_BLOCK_LIST = 1
} fsi_sattn_mode;

FSI_API size_t fsi_sparse_attn_workspace_size(int64_t B, int64_t Hkv, int64_t T, int64_t head_dim);

/* dtype FSI_DTYPE_BF16 or FSI_DTYPE_F32 (fp32 math either way, output in dtype);
 * head_dim 1..256; any block; capacity <= 4096; window > 0 for
 * FSI_SATTN_LOCAL_REMOTE.  bf16 with head_dim 16, 32, 64 or 128, block a
 * multiple of 16, strides multiples of 8 elements (out: 4) and q, k, v 16-byte
 * aligned runs the MFMA kernels; everything else the generic fp32-math kernel.
 * Replaces the dense masked SDPA of attention.py:211-218 and the Triton kernel
 * launch of triton_ops.py:298-312. */
FSI_API int fsi_sparse_attn(const void* q, int64_t qs_b, int64_t qs_h, int64_t qs_t, const void* k, int64_t ks_b,
                            int64_t ks_h, int64_t ks_t, const void* v, int64_t vs_b, int64_t vs_h, int64_t vs_t,
                            int64_t B, int64_t Hq, int64_t Hkv, int64_t T, int64_t head_dim, int64_t block, int mode,
                            int64_t window, const int32_t* lists, int64_t ls_b, int64_t ls_q, int64_t capacity,
                            const int32_t* counts, int64_t cs_b, int64_t cs_q, float scale, int dtype, void* out,
                            int64_t os_b, int64_t os_h, int64_t os_t, void* workspace, size_t workspace_bytes,
                            int* err, void* stream);

/* Backward of fsi_sparse_attn (autograd of the masked SDPA of attention.py:211-218
 * and of triton_ops.py:26-93): dq (B, Hq, T, head_dim), dk and dv (B, Hkv, T,
 * head_dim), contiguous fp32, written, from q, k, v, the forward's out and dout
 * (element strides as in fsi_sparse_attn, unit stride over head_dim) and the same
 * pattern arguments.  fp32 math on 64 x 64 LDS tiles; no (T, T) tensor: the
 * workspace (fsi_sparse_attn_bwd_workspace_size bytes) holds the counter area, a
 * (B, ceil(T / block)^2) int32 block map and three fp32 (B, Hq, T) row
 * statistics.  head_dim 1..128, dtype FSI_DTYPE_BF16 or FSI_DTYPE_F32. */
FSI_API size_t fsi_sparse_attn_bwd_workspace_size(int64_t B, int64_t Hq, int64_t T, int64_t block);
FSI_API int fsi_sparse_attn_bwd(const void* q, int64_t qs_b, int64_t qs_h, int64_t qs_t, const void* k, int64_t ks_b,
                                int64_t ks_h, int64_t ks_t, const void* v, int64_t vs_b, int64_t vs_h, int64_t vs_t,
                                const void* out, int64_t os_b, int64_t os_h, int64_t os_t, const void* dout,
                                int64_t ds_b, int64_t ds_h, int64_t ds_t, int64_t B, int64_t Hq, int64_t Hkv,
                                int64_t T, int64_t head_dim, int64_t block, int mode, int64_t window,
                                const int32_t* lists, int64_t ls_b, int64_t ls_q, int64_t capacity,
                                const int32_t* counts, int64_t cs_b, int64_t cs_q, float scale, int dtype, float* dq,
                                float* dk, float* dv, void* workspace, size_t workspace_bytes, int* err,
                                void* stream);

/* Fused 16-D block indexer + greedy block selection + block attention
 * (triton_fused_sram_indexer_attention, foveal_indexer/triton_ops.py:142-249,373-435).
 * q, k, v, out: contiguous (B, H, N, head_dim) of `dtype` (F32, BF16 or F16;
 * fp32 math); q16, k16: contiguous (B, N / block_size, 16), shared by the heads,
 * of idx_dtype (`dtype` or F32).  Query block m scores every block j by <q16[m], k16[j]> / 4,
 * softmaxes over j != m (sum + 1e-6), then takes max_remote greedy picks (largest
 * remaining probability, lowest index on ties); a pick is attended iff the mass
 * of the picks before it is < top_p and its probability > 1e-4.  The block's
 * queries attend the self block then the attended picks (no causal mask).
 * selected (optional, int32 [B, N / block_size, max_remote]) receives each
 * pick's block, or -1 where the pick is not attended.  Limits: block_size <= 64,
 * head_dim <= 256, block_size * head_dim <= 8192, N / block_size <= 8192,
 * max_remote <= 64, B * H <= 65535 (FSI_ERR_CAPACITY). */
FSI_API int fsi_sram_indexer_attention(const void* q, const void* k, const void* v, int dtype, const void* q16,
                                       const void* k16, int idx_dtype, int64_t B, int64_t H, int64_t N, int64_t head_dim,
                                       int64_t block_size, int64_t max_remote, float scale, float top_p, void* out,
                                       int32_t* selected, void* stream);

/* ------------------------------------------------------------------------- *
 * Block-sparse GEMMs (bf16 in, fp32 accumulate, bf16 out) on 128 x 128 MFMA
 * tiles.  x: (M, K) row stride ldx; w: (N, K) row stride ldw (the nn.Linear
 * weight layout); out: (M, N) row stride ldo.  K, N and leading dimensions
 * multiples of 8, base pointers 16-byte aligned.
 * ------------------------------------------------------------------------- */
FSI_API size_t fsi_block_sparse_linear_workspace_size(int64_t N, int64_t block_size);

/* Column-block sparse linear (triton_block_sparse_linear, foveal_indexer/triton_ops.py:316-370):
 * out[:, b*bs:(b+1)*bs] = x w[b*bs:(b+1)*bs]^T (+ bias[b*bs:(b+1)*bs]) for every
 * active block b, all other columns 0.  block_size: multiple of 32 dividing N.
 * Block ids outside [0, N / block_size) are skipped and reported through err. */
FSI_API int fsi_block_sparse_linear(const void* x, int64_t ldx, const void* w, int64_t ldw, const void* bias,
                                    const int32_t* active_blocks, int64_t n_active, int64_t block_size, int64_t M,
                                    int64_t N, int64_t K, int dtype, void* out, int64_t ldo, void* workspace,
                                    size_t workspace_bytes, int* err, void* stream);

FSI_API size_t fsi_blockwise_matmul_workspace_size(int64_t M, int64_t N, int64_t K, int64_t block_k);

/* 2-D tile-sparse matmul (BlockwiseMatMul2D, foveal_indexer/block_matmul.py:335-392):
 * out = x (w o T)^T where T expands tile_mask to elements: tile (k_b, n_b) of
 * size block_k x block_n is active iff tile_mask[g][k_b * (N / block_n) + n_b],
 * with g the row group of the output row (rows_per_group rows each; groups = 1
 * applies one mask to every row; with groups > 1 they must cover all M rows,
 * groups * rows_per_group >= M, else FSI_ERR_SHAPE).  block_k divides K, block_n divides N.  The
 * MFMA kernel takes bf16 with block_k a multiple of 32, block_n a multiple of
 * 128 or one of 16, 32, 64, K / block_k <= 2048, rows_per_group a multiple of
 * 128 (or groups = 1) and 16-byte aligned x, w rows; other problems and fp32
 * run on a generic kernel.  Rows of a group whose tiles are all inactive get 0.
 * Every tile builds its k-block list on chip.  The workspace
 * (fsi_blockwise_matmul_workspace_size bytes: one int32 per 128 x 128 output
 * tile after the counter area) receives the tile order from a pre-pass when
 * the grid spans several rounds of workgroups: inside each 128-row band of
 * output tiles, heaviest k-block list first.  With a null or smaller workspace
 * tiles run in dispatch order.  Results do not depend on the order. */
FSI_API int fsi_blockwise_matmul(const void* x, int64_t ldx, const void* w, int64_t ldw,
                                 const uint8_t* tile_mask, int64_t groups, int64_t rows_per_group, int64_t block_k,
                                 int64_t block_n, int64_t M, int64_t N, int64_t K, int dtype, void* out, int64_t ldo,
                                 void* workspace, size_t workspace_bytes, void* stream);

/* 2-D tile routing of BlockwiseMatMul2D (foveal_indexer/block_matmul.py:355-377).
 * Per row r of scores (rows x n_tiles, row stride ld_scores, fp32 or bf16):
 * p = softmax(row) (rounded to bf16 for bf16 rows), tiles ranked by p
 * descending (equal p: lower tile id first), running mass summed in fp64 and
 * compared after rounding to the row dtype, needed = min(#(cum < top_p) + 1,
 * n_tiles) (no K_min, no K_max).  out_mask (groups x n_tiles uint8,
 * groups = ceil(rows / rows_per_group)): 1 for tiles [0, base_tiles) and for
 * every tile some row of the group selects, 0 elsewhere (rows_per_group >= rows
 * gives the reference's single union mask).  out_needed (optional, rows
 * int32) and out_probs (optional, rows x n_tiles contiguous, row dtype).
 * n_tiles <= 4096. */
FSI_API int fsi_tile_route(const void* scores, int dtype, int64_t rows, int64_t n_tiles, int64_t ld_scores,
                           int64_t rows_per_group, int64_t base_tiles, float top_p, uint8_t* out_mask,
                           int32_t* out_needed, void* out_probs, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FSI_H_ */
