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

typedef enum fsi_dtype { FSI_DTYPE_F32 = 0, FSI_DTYPE_BF16 = 1 } fsi_dtype;

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

/* Elementwise SwiGLU: out = silu(g) * u, computed in fp32 and rounded once to
 * the storage dtype (rounding = FUSED) or with torch-eager rounding points
 * (rounding = EAGER).  Replaces triton_fused_swiglu / _swiglu_fwd_kernel
 * (foveal_indexer/pattention_triton.py:30-47,98-104). */
FSI_API int fsi_swiglu(const void* g, const void* u, void* out, int64_t n, int dtype, int rounding, void* stream);

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

#ifdef __cplusplus
}
#endif

#endif /* FSI_H_ */
