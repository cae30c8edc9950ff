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

// Token mean for small batches (M <= MEAN_DIRECT_ROWS) in one kernel: one
// thread per column sums the rows in order, 16 loads in flight; the same
// additions as token_partial + token_mean with one row per chunk.
constexpr int MEAN_DIRECT_ROWS = 64;

template <bool BF16>
__global__ __launch_bounds__(64) void token_mean_direct(const void* __restrict__ x, int64_t ldx, int M, int D,
                                                        float* __restrict__ xm) {
  const int d = blockIdx.x * 64 + threadIdx.x;
  if (d >= D) return;
  float acc = 0.f;
  int m = 0;
  for (; m + 16 <= M; m += 16) {
    float v[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int64_t i = static_cast<int64_t>(m + e) * ldx + d;
      v[e] = BF16 ? bf16_to_f32(static_cast<const bf16_t*>(x)[i]) : static_cast<const float*>(x)[i];
    }
#pragma unroll
    for (int e = 0; e < 16; ++e) acc += v[e];
  }
  for (; m < M; ++m) {
    const int64_t i = static_cast<int64_t>(m) * ldx + d;
    acc += BF16 ? bf16_to_f32(static_cast<const bf16_t*>(x)[i]) : static_cast<const float*>(x)[i];
  }
  const float mean = acc / static_cast<float>(M);
  xm[d] = BF16 ? round_bf16(mean) : mean;
}

// Sum over the wave with VALU lane exchanges (DPP inside rows of 16, then
// gfx950's permlane16 / permlane32 swaps); every lane receives the total.
__device__ __forceinline__ float wave_sum_vx(float x) {
  auto dpp = [](float v, int ctrl) {
    switch (ctrl) {  // the DPP control must be a compile-time constant
      case 0xB1: return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, false));
      case 0x4E: return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, false));
      case 0x141: return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xF, 0xF, false));
      default: return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x140, 0xF, 0xF, false));
    }
  };
  x += dpp(x, 0xB1);   // lane ^ 1
  x += dpp(x, 0x4E);   // lane ^ 2
  x += dpp(x, 0x141);  // half-row mirror
  x += dpp(x, 0x140);  // row mirror
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto c = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(c[0]) + __uint_as_float(c[1]);
}

template <bool BF16>
__device__ __forceinline__ float ldval(const void* p, int64_t i) {
  return BF16 ? bf16_to_f32(static_cast<const bf16_t*>(p)[i]) : static_cast<const float*>(p)[i];
}

// One workgroup of 16 waves: projection, rms_norm, scores and top-k selection.
constexpr int PR_THREADS = 1024;
static_assert(PR_THREADS % 64 == 0 && PR_THREADS / 64 <= 16, "the projection reduces over at most 16 waves");
constexpr int PR_LDS_SCORES = 8192;

// Order-preserving 32-bit key of a float for ranking: NaN -> 0xffffffff (above
// +inf), -0 -> the key of +0, otherwise larger floats get larger keys.
__device__ __forceinline__ uint32_t rank_key(float f) {
  if (f != f) return 0xffffffffu;
  if (f == 0.0f) f = 0.0f;
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// One 1024-thread workgroup.  The loads of each phase are issued together and
// as 16-byte vectors (the address unit's cost is per load instruction, so 2-byte
// loads made the projection ~8x slower):
//   * the block keys of block tid (index_dim 16, at most PR_THREADS blocks) are
//     loaded first, beside the projection's loads;
//   * projection: thread t takes the 8 consecutive columns 8 t .. 8 t + 7 (then
//     + 8 PR_THREADS, ...) of x_mean and of every row of Wq, per-row partial sums
//     are reduced over the wave and then over the waves in order;
//   * rank: the scores' order-preserving keys go to LDS once; each remote
//     candidate is ranked by TPC adjacent lanes counting over contiguous quarters
//     of the candidates (4 keys per LDS read), the partial counts summed by lane
//     shuffles.
template <bool BF16>
__device__ __forceinline__ void load8(const void* p, int64_t i, float (&v)[8]) {  // 8 values at element i (16-byte aligned for bf16)
  if (BF16) {
    const u32x4_t w = *reinterpret_cast<const u32x4_t*>(static_cast<const bf16_t*>(p) + i);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[2 * e] = lo_bf16(w[e]);
      v[2 * e + 1] = hi_bf16(w[e]);
    }
  } else {
    const float4 a = *reinterpret_cast<const float4*>(static_cast<const float*>(p) + i);
    const float4 b = *reinterpret_cast<const float4*>(static_cast<const float*>(p) + i + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  }
}

template <bool BF16>
__global__ __launch_bounds__(PR_THREADS) void pooled_route(const float* __restrict__ xm, int D,
                                                           const void* __restrict__ wq, int index_dim,
                                                           const void* __restrict__ keys, int n_blocks,
                                                           int base_blocks, int remote_blocks, float score_scale,
                                                           int32_t* __restrict__ active,
                                                           float* __restrict__ scores_out,
                                                           float* __restrict__ scratch) {
  constexpr int NW = PR_THREADS / 64;
  __shared__ float q[MAX_INDEX_DIM];
  __shared__ float qpart[NW][16];
  __shared__ __attribute__((aligned(16))) uint32_t kk[PR_LDS_SCORES];  // rank keys of the scores
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // the module's shape: 16-D index, every block's keys in one thread, 16-byte rows of Wq
  const bool fast = index_dim == 16 && n_blocks <= PR_THREADS && D % 8 == 0 &&
                    (reinterpret_cast<uintptr_t>(wq) | reinterpret_cast<uintptr_t>(keys) |
                     reinterpret_cast<uintptr_t>(xm)) % 16 == 0;

  float kv[16];
  if (fast && tid < n_blocks) {
    float a[8], b[8];
    load8<BF16>(keys, static_cast<int64_t>(tid) * 16, a);
    load8<BF16>(keys, static_cast<int64_t>(tid) * 16 + 8, b);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      kv[j] = a[j];
      kv[8 + j] = b[j];
    }
  }
  if (fast) {
    // q_j = x_mean . Wq[j]: this thread's 8 columns of x_mean and of every row, loads first
    float acc[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[j] = 0.f;
    for (int d0 = 8 * tid; d0 < D; d0 += 8 * PR_THREADS) {
      float xv[8], wv[16][8];
      load8<false>(xm, d0, xv);
#pragma unroll
      for (int j = 0; j < 16; ++j) load8<BF16>(wq, static_cast<int64_t>(j) * D + d0, wv[j]);
#pragma unroll
      for (int c = 0; c < 8; ++c)
#pragma unroll
        for (int j = 0; j < 16; ++j) acc[j] = fmaf(xv[c], wv[j][c], acc[j]);
    }
    if (64 * wave < (D + 7) / 8) {  // waves holding columns (uniform)
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const float t = wave_sum_vx(acc[j]);
        if (lane == 0) qpart[wave][j] = t;
      }
    } else if (lane < 16) {
      qpart[wave][lane] = 0.f;
    }
    __syncthreads();
    if (tid < 16) {
      float t = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) t += qpart[w][tid];
      q[tid] = BF16 ? round_bf16(t) : t;
    }
  } else {
    // other shapes: wave w handles rows j = w, w + 16, ...
    for (int j = wave; j < index_dim; j += NW) {
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
  }
  __syncthreads();
  if (tid == 0) {
    float ss = 0.f;
    if (index_dim == 16) {
      float qv[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) qv[j] = q[j];
#pragma unroll
      for (int j = 0; j < 16; ++j) ss += qv[j] * qv[j];
      const float r = 1.0f / sqrtf(ss / 16.f + 1.1920928955078125e-07f);
#pragma unroll
      for (int j = 0; j < 16; ++j) q[j] = BF16 ? round_bf16(qv[j] * r) : qv[j] * r;
    } else {
      for (int j = 0; j < index_dim; ++j) ss += q[j] * q[j];
      const float r = 1.0f / sqrtf(ss / static_cast<float>(index_dim) + 1.1920928955078125e-07f);
      for (int j = 0; j < index_dim; ++j) q[j] = BF16 ? round_bf16(q[j] * r) : q[j] * r;
    }
  }
  __syncthreads();
  // scores
  auto finish_score = [&](int b, float acc) -> float {
    if (score_scale != 1.0f) {
      if (BF16) acc = round_bf16(acc);
      acc = acc * score_scale;
    }
    const float s = BF16 ? round_bf16(acc) : acc;
    if (scores_out) scores_out[b] = s;
    return s;
  };
  if (fast) {
    if (tid < n_blocks) {
      float acc = 0.f;
#pragma unroll
      for (int j = 0; j < 16; ++j) acc = fmaf(q[j], kv[j], acc);
      kk[tid] = rank_key(finish_score(tid, acc));
    }
  } else {
    for (int b = tid; b < n_blocks; b += PR_THREADS) {
      float acc = 0.f;
      for (int j = 0; j < index_dim; ++j)
        acc = fmaf(q[j], ldval<BF16>(keys, static_cast<int64_t>(b) * index_dim + j), acc);
      const uint32_t k = rank_key(finish_score(b, acc));
      if (n_blocks <= PR_LDS_SCORES) kk[b] = k;
      else reinterpret_cast<uint32_t*>(scratch)[b] = k;
    }
  }
  __syncthreads();
  // Rank among remote candidates: larger score first, ties broken by lower index.
  // The order-preserving integer keys put NaN above +inf (torch.topk ranks NaN
  // largest) and -0 equal to +0, so the ranks are a permutation and every
  // output slot is written.
  const int n_cand = n_blocks - base_blocks;
  int tpc = 1;  // lanes per candidate: a power of two <= 64 with tpc * n_cand <= PR_THREADS
  while (tpc < 64 && 2 * tpc * n_cand <= PR_THREADS) tpc *= 2;
  const int sub = tid & (tpc - 1);
  // contiguous candidates each lane of a group counts over, a multiple of 4
  const int span = ((n_cand + tpc - 1) / tpc + 3) & ~3;
  auto rank_all = [&](const uint32_t* key, bool vec) {
    // the tpc lanes of a candidate are adjacent and share its loop trips, so the
    // shuffles below stay inside the group
    for (int c0 = tid / tpc; c0 < n_cand; c0 += PR_THREADS / tpc) {
      const int b = base_blocks + c0;
      const uint32_t s = key[b];
      const int o0 = base_blocks + sub * span;
      const int o1 = o0 + span < n_blocks ? o0 + span : n_blocks;
      int rank = 0;
      int o = o0;
      if (vec) {
        for (; o + 4 <= o1; o += 4) {
          const u32x4_t t = *reinterpret_cast<const u32x4_t*>(key + o);
#pragma unroll
          for (int e = 0; e < 4; ++e) rank += (t[e] > s) || (t[e] == s && o + e < b);
        }
      }
      for (; o < o1; ++o) {
        const uint32_t t = key[o];
        rank += (t > s) || (t == s && o < b);
      }
      for (int m = 1; m < tpc; m <<= 1) rank += __shfl_xor(rank, m, 64);
      if (sub == 0 && rank < remote_blocks) active[base_blocks + rank] = b;
    }
  };
  if (n_blocks <= PR_LDS_SCORES) rank_all(kk, base_blocks % 4 == 0);  // uniform
  else rank_all(reinterpret_cast<const uint32_t*>(scratch), false);
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
  const bool direct = M <= MEAN_DIRECT_ROWS;
  const dim3 gd((unsigned)((D + 63) / 64));
  if (dtype == FSI_DTYPE_BF16) {
    if (direct) {
      token_mean_direct<true><<<gd, 64, 0, st>>>(x, ldx, (int)M, (int)D, xm);
    } else {
      token_partial<true><<<gp, 256, 0, st>>>(x, ldx, (int)M, (int)D, rows, part);
      token_mean<true><<<g1, 256, 0, st>>>(part, n_chunks, (int)M, (int)D, xm);
    }
    FSI_HIP_LAUNCH_CHECK("mlp_router mean");
    pooled_route<true><<<1, PR_THREADS, 0, st>>>(xm, (int)D, q_proj_w, (int)index_dim, block_keys, (int)n_blocks,
                                          (int)base_blocks, (int)remote_blocks, score_scale, out_active, out_scores,
                                          scratch);
  } else {
    if (direct) {
      token_mean_direct<false><<<gd, 64, 0, st>>>(x, ldx, (int)M, (int)D, xm);
    } else {
      token_partial<false><<<gp, 256, 0, st>>>(x, ldx, (int)M, (int)D, rows, part);
      token_mean<false><<<g1, 256, 0, st>>>(part, n_chunks, (int)M, (int)D, xm);
    }
    FSI_HIP_LAUNCH_CHECK("mlp_router mean");
    pooled_route<false><<<1, PR_THREADS, 0, st>>>(xm, (int)D, q_proj_w, (int)index_dim, block_keys, (int)n_blocks,
                                           (int)base_blocks, (int)remote_blocks, score_scale, out_active, out_scores,
                                           scratch);
  }
  FSI_HIP_LAUNCH_CHECK("mlp_router route");
  return FSI_OK;
}

}  // extern "C"
