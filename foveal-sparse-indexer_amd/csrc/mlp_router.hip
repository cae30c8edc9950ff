// Pooled 16-D router of FovealPattentionMLP in eval mode
// (foveal_indexer/foveal_pattention.py:310-322):
//
//   q      = rms_norm(q_proj_16d(mean_over_tokens(x)))         (bf16 rounding after each op)
//   s[b]   = q . block_keys_16d[b]                              (no 1/sqrt(16) in eval)
//   top    = topk(s[base:], remote_blocks)                      (descending; ties -> lower index)
//   active = [0, 1, ..., base-1] ++ (top + base)
//
// Rounding points mirror torch's CPU bf16 ops: the token mean accumulates in
// fp32 (chunked, fixed order) and rounds once;
// the projection and scores accumulate in fp32 and round once; rms_norm runs in
// fp32 with eps = FLT_EPSILON and rounds once.
#include "fsi_common.h"

using namespace fsi;

namespace {

constexpr int MAX_INDEX_DIM = 64;

// Mean of x[:, d] over the tokens, rounded to the storage dtype.  The tokens
// are cut into at most MEAN_CHUNKS chunks; each chunk is summed sequentially in
// fp32 (one thread per column, coalesced across the wave), then the chunk sums
// are added in chunk order (deterministic).  The order differs from torch's
// CPU reduction only in fp32 rounding, below one bf16 ulp of the mean.
constexpr int MEAN_CHUNKS = 64;

template <bool BF16>
__global__ __launch_bounds__(256) void token_partial(const void* __restrict__ x, int64_t ldx, int M, int D,
                                                     int rows_per_chunk, float* __restrict__ part) {
  const int d = blockIdx.x * 256 + threadIdx.x;
  if (d >= D) return;
  const int m0 = blockIdx.y * rows_per_chunk;
  const int m1 = min(M, m0 + rows_per_chunk);
  float acc = 0.f;
#pragma unroll 16
  for (int m = m0; m < m1; ++m) {
    const int64_t i = static_cast<int64_t>(m) * ldx + d;
    acc += BF16 ? bf16_to_f32(static_cast<const bf16_t*>(x)[i]) : static_cast<const float*>(x)[i];
  }
  part[static_cast<int64_t>(blockIdx.y) * D + d] = acc;
}

template <bool BF16>
__global__ __launch_bounds__(256) void token_mean(const float* __restrict__ part, int n_chunks, int M, int D,
                                                  float* __restrict__ xm) {
  const int d = blockIdx.x * 256 + threadIdx.x;
  if (d >= D) return;
  // chunk order kept; the loads are issued 16 at a time (a dependent chain of
  // L2 round trips otherwise)
  float acc = 0.f;
  int c = 0;
  for (; c + 16 <= n_chunks; c += 16) {
    float v[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) v[e] = part[static_cast<int64_t>(c + e) * D + d];
#pragma unroll
    for (int e = 0; e < 16; ++e) acc += v[e];
  }
  for (; c < n_chunks; ++c) acc += part[static_cast<int64_t>(c) * D + d];
  const float mean = acc / static_cast<float>(M);
  xm[d] = BF16 ? round_bf16(mean) : mean;
}

template <bool BF16>
__device__ __forceinline__ float ldval(const void* p, int64_t i) {
  return BF16 ? bf16_to_f32(static_cast<const bf16_t*>(p)[i]) : static_cast<const float*>(p)[i];
}

// One workgroup of 16 waves: projection, rms_norm, scores and top-k selection.
constexpr int PR_THREADS = 1024;
constexpr int PR_LDS_SCORES = 8192;

// Order-preserving 32-bit key of a float for ranking: NaN -> 0xffffffff (above
// +inf), -0 -> the key of +0, otherwise larger floats get larger keys.
__device__ __forceinline__ uint32_t rank_key(float f) {
  if (f != f) return 0xffffffffu;
  if (f == 0.0f) f = 0.0f;
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

template <bool BF16>
__global__ __launch_bounds__(PR_THREADS) void pooled_route(const float* __restrict__ xm, int D,
                                                           const void* __restrict__ wq, int index_dim,
                                                           const void* __restrict__ keys, int n_blocks,
                                                           int base_blocks, int remote_blocks, float score_scale,
                                                           int32_t* __restrict__ active,
                                                           float* __restrict__ scores_out,
                                                           float* __restrict__ scratch) {
  __shared__ float q[MAX_INDEX_DIM];
  __shared__ float lds_scores[PR_LDS_SCORES];
  // the ranking re-reads every score once per candidate: keep them in LDS
  float* sc = n_blocks <= PR_LDS_SCORES ? lds_scores : scratch;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // q_j = x_mean . Wq[j]  (wave w handles j = w, w + 16, ...); eight independent
  // partial sums per lane keep eight loads in flight
  for (int j = wave; j < index_dim; j += PR_THREADS / 64) {
    float part[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    const int64_t row = static_cast<int64_t>(j) * D;
    int d = lane;
    for (; d + 7 * 64 < D; d += 8 * 64) {
#pragma unroll
      for (int e = 0; e < 8; ++e) part[e] = fmaf(xm[d + 64 * e], ldval<BF16>(wq, row + d + 64 * e), part[e]);
    }
    for (; d < D; d += 64) part[0] = fmaf(xm[d], ldval<BF16>(wq, row + d), part[0]);
    float acc = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc += part[e];
    acc = wave_sum(acc);
    if (lane == 0) q[j] = BF16 ? round_bf16(acc) : acc;
  }
  __syncthreads();
  if (tid == 0) {
    float ss = 0.f;
    for (int j = 0; j < index_dim; ++j) ss += q[j] * q[j];
    const float r = 1.0f / sqrtf(ss / static_cast<float>(index_dim) + 1.1920928955078125e-07f);
    for (int j = 0; j < index_dim; ++j) q[j] = BF16 ? round_bf16(q[j] * r) : q[j] * r;
  }
  __syncthreads();
  // scores
  for (int b = tid; b < n_blocks; b += PR_THREADS) {
    float acc = 0.f;
    if (index_dim == 16) {  // the module's index_dim: the 16 loads issued together
      float kv[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) kv[j] = ldval<BF16>(keys, static_cast<int64_t>(b) * 16 + j);
#pragma unroll
      for (int j = 0; j < 16; ++j) acc = fmaf(q[j], kv[j], acc);
    } else {
      for (int j = 0; j < index_dim; ++j)
        acc = fmaf(q[j], ldval<BF16>(keys, static_cast<int64_t>(b) * index_dim + j), acc);
    }
    if (score_scale != 1.0f) {
      if (BF16) acc = round_bf16(acc);
      acc = acc * score_scale;
    }
    const float s = BF16 ? round_bf16(acc) : acc;
    sc[b] = s;
    if (scores_out) scores_out[b] = s;
  }
  __syncthreads();
  // Rank among remote candidates: larger score first, ties broken by lower index.
  // Scores compare through an order-preserving integer key in which NaN sorts
  // above +inf (torch.topk ranks NaN largest) and -0 equals +0, so the ranks
  // are a permutation and every output slot is written.
  for (int b = base_blocks + tid; b < n_blocks; b += PR_THREADS) {
    const uint32_t s = rank_key(sc[b]);
    int rank = 0;
    for (int o = base_blocks; o < n_blocks; ++o) {
      const uint32_t t = rank_key(sc[o]);
      rank += (t > s) || (t == s && o < b);
    }
    if (rank < remote_blocks) active[base_blocks + rank] = b;
  }
  for (int b = tid; b < base_blocks; b += PR_THREADS) active[b] = b;
}

}  // namespace

extern "C" {

FSI_API size_t fsi_mlp_router_workspace_size(int64_t D, int64_t n_blocks) {
  return FSI_WORKSPACE_COUNTER_BYTES + fsi_host::align_up(sizeof(float) * D, 256) +
         fsi_host::align_up(sizeof(float) * n_blocks, 256) + fsi_host::align_up(sizeof(float) * MEAN_CHUNKS * D, 256);
}

FSI_API int fsi_mlp_router(const void* x, int64_t ldx, int64_t M, int64_t D, const void* q_proj_w, int64_t index_dim,
                           const void* block_keys, int64_t n_blocks, int64_t base_blocks, int64_t remote_blocks,
                           float score_scale, int dtype, int32_t* out_active, float* out_scores, void* workspace,
                           size_t workspace_bytes, void* stream) {
  FSI_CHECK_ARG(dtype == FSI_DTYPE_BF16 || dtype == FSI_DTYPE_F32, FSI_ERR_DTYPE, "mlp_router: dtype %d", dtype);
  FSI_CHECK_ARG(x && q_proj_w && block_keys && out_active, FSI_ERR_INVALID_ARG, "mlp_router: null pointer");
  FSI_CHECK_ARG(M > 0 && D > 0 && ldx >= D && n_blocks > 0, FSI_ERR_SHAPE, "mlp_router: M=%lld D=%lld n_blocks=%lld",
                (long long)M, (long long)D, (long long)n_blocks);
  FSI_CHECK_ARG(index_dim > 0 && index_dim <= MAX_INDEX_DIM, FSI_ERR_SHAPE, "mlp_router: index_dim %lld > %d",
                (long long)index_dim, MAX_INDEX_DIM);
  FSI_CHECK_ARG(base_blocks >= 0 && remote_blocks >= 0 && base_blocks <= n_blocks, FSI_ERR_SHAPE,
                "mlp_router: base=%lld remote=%lld", (long long)base_blocks, (long long)remote_blocks);
  // torch.topk raises when k exceeds the candidate count (foveal_pattention.py:314).
  FSI_CHECK_ARG(remote_blocks <= n_blocks - base_blocks, FSI_ERR_CAPACITY,
                "mlp_router: remote_blocks=%lld > candidates=%lld", (long long)remote_blocks,
                (long long)(n_blocks - base_blocks));
  const size_t need = fsi_mlp_router_workspace_size(D, n_blocks);
  FSI_CHECK_ARG(workspace && workspace_bytes >= need, FSI_ERR_WORKSPACE, "mlp_router: workspace %zu < %zu",
                workspace_bytes, need);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  float* xm = reinterpret_cast<float*>(static_cast<char*>(workspace) + FSI_WORKSPACE_COUNTER_BYTES);
  float* scratch = reinterpret_cast<float*>(reinterpret_cast<char*>(xm) + fsi_host::align_up(sizeof(float) * D, 256));
  float* part = reinterpret_cast<float*>(reinterpret_cast<char*>(scratch) + fsi_host::align_up(sizeof(float) * n_blocks, 256));
  const int rows = static_cast<int>((M + MEAN_CHUNKS - 1) / MEAN_CHUNKS);
  const int n_chunks = static_cast<int>((M + rows - 1) / rows);
  const dim3 gp((unsigned)((D + 255) / 256), (unsigned)n_chunks);
  const dim3 g1((unsigned)((D + 255) / 256));
  if (dtype == FSI_DTYPE_BF16) {
    token_partial<true><<<gp, 256, 0, st>>>(x, ldx, (int)M, (int)D, rows, part);
    token_mean<true><<<g1, 256, 0, st>>>(part, n_chunks, (int)M, (int)D, xm);
    FSI_HIP_LAUNCH_CHECK("mlp_router mean");
    pooled_route<true><<<1, PR_THREADS, 0, st>>>(xm, (int)D, q_proj_w, (int)index_dim, block_keys, (int)n_blocks,
                                          (int)base_blocks, (int)remote_blocks, score_scale, out_active, out_scores,
                                          scratch);
  } else {
    token_partial<false><<<gp, 256, 0, st>>>(x, ldx, (int)M, (int)D, rows, part);
    token_mean<false><<<g1, 256, 0, st>>>(part, n_chunks, (int)M, (int)D, xm);
    FSI_HIP_LAUNCH_CHECK("mlp_router mean");
    pooled_route<false><<<1, PR_THREADS, 0, st>>>(xm, (int)D, q_proj_w, (int)index_dim, block_keys, (int)n_blocks,
                                           (int)base_blocks, (int)remote_blocks, score_scale, out_active, out_scores,
                                           scratch);
  }
  FSI_HIP_LAUNCH_CHECK("mlp_router route");
  return FSI_OK;
}

}  // extern "C"
