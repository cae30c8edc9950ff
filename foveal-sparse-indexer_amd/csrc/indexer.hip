// 16-D indexer representations on MI355X (gfx950): the non-GEMM parts of
// FovealIndexer (foveal_indexer/core.py:214-312).  The D -> 16 projections are
// plain library GEMMs; everything after them runs here, with the reference's
// rounding points for bf16 tensors:
//   * rms_norm over the 16 components: fp32, x * (1 / sqrt(mean(x^2) + FLT_EPSILON)),
//     rounded once (F.rms_norm, core.py:222,241);
//   * block pooling: mean over the block's tokens accumulated in fp32 in token
//     order, divided by the block size, rounded (core.py:245-246); pooled keys
//     are then L2-normalised in fp32 and rounded again (core.py:249);
//   * cosine block scores: both sides L2-normalised in fp32 and rounded to the
//     tensor dtype, dot products accumulated in fp32 and rounded, then divided
//     by sqrt(index_dim) and rounded (core.py:263-265);
//   * additive-stream context: masked softmax in fp32 (causal: p < q), the
//     probabilities rounded to the values' dtype, contracted with the pooled
//     values in fp32 and rounded (core.py:288-310).
#include "fsi_common.h"

using namespace fsi;

namespace {

constexpr int IX_D = 16;
constexpr float FLT_EPS = 1.1920928955078125e-07f;

template <bool BF16>
__device__ __forceinline__ float ld(const void* p, int64_t i) {
  return BF16 ? bf16_to_f32(static_cast<const bf16_t*>(p)[i]) : static_cast<const float*>(p)[i];
}
template <bool BF16>
__device__ __forceinline__ void st(void* p, int64_t i, float v) {
  if (BF16) static_cast<bf16_t*>(p)[i] = f32_to_bf16(v);
  else static_cast<float*>(p)[i] = v;
}
template <bool BF16>
__device__ __forceinline__ float rnd(float v) {
  return BF16 ? round_bf16(v) : v;
}

__device__ __forceinline__ void rms_norm16(float (&v)[IX_D]) {
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < IX_D; ++c) ss = fmaf(v[c], v[c], ss);
  const float r = 1.0f / sqrtf(ss / static_cast<float>(IX_D) + FLT_EPS);
#pragma unroll
  for (int c = 0; c < IX_D; ++c) v[c] *= r;
}

__device__ __forceinline__ void l2_normalize16(float (&v)[IX_D]) {
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < IX_D; ++c) ss = fmaf(v[c], v[c], ss);
  const float n = fmaxf(sqrtf(ss), 1e-12f);
#pragma unroll
  for (int c = 0; c < IX_D; ++c) v[c] = v[c] / n;
}

// One thread per row of 16.
template <bool BF16>
__global__ __launch_bounds__(256) void rms_norm_rows_kernel(const void* __restrict__ x, int64_t M,
                                                           void* __restrict__ out) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (r >= M) return;
  float v[IX_D];
#pragma unroll
  for (int c = 0; c < IX_D; ++c) v[c] = ld<BF16>(x, r * IX_D + c);
  rms_norm16(v);
#pragma unroll
  for (int c = 0; c < IX_D; ++c) st<BF16>(out, r * IX_D + c, v[c]);
}

// One thread per (batch, block): pooled normalised key and mean value.
//   RMS: rms-normalise (and round) every token's key first (compute_kv_blocks_16d);
//        off for FovealKVCache pages, whose keys arrive normalised (attention.py:305).
//   KF32: write the normalised key in fp32 without rounding (FovealKVCache.kp_cache
//        is fp32, attention.py:52,89-90); otherwise round to the input dtype.
// Outputs are written at row stride out_stride (elements) per pooled row.
template <bool BF16, bool RMS, bool KF32>
__global__ __launch_bounds__(256) void pool_kv_kernel(const void* __restrict__ k_lin, const void* __restrict__ v_lin,
                                                     int64_t n_pool, int block, int64_t in_group_stride,
                                                     int64_t groups_per_batch, int64_t out_batch_stride,
                                                     void* __restrict__ k_out, void* __restrict__ v_out) {
  const int64_t pb = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;  // flat (batch, block)
  if (pb >= n_pool) return;
  const int64_t bb = pb / groups_per_batch, gi = pb % groups_per_batch;
  const int64_t t0 = (bb * groups_per_batch + gi) * in_group_stride;  // element offset of the first token
  const int64_t o = bb * out_batch_stride + gi * IX_D;
  float ks[IX_D], vs[IX_D];
#pragma unroll
  for (int c = 0; c < IX_D; ++c) ks[c] = vs[c] = 0.f;
  for (int t = 0; t < block; ++t) {
    float kv[IX_D];
#pragma unroll
    for (int c = 0; c < IX_D; ++c) kv[c] = ld<BF16>(k_lin, t0 + t * IX_D + c);
    if (RMS) {
      rms_norm16(kv);
#pragma unroll
      for (int c = 0; c < IX_D; ++c) kv[c] = rnd<BF16>(kv[c]);
    }
#pragma unroll
    for (int c = 0; c < IX_D; ++c) {
      ks[c] += kv[c];
      vs[c] += ld<BF16>(v_lin, t0 + t * IX_D + c);
    }
  }
  const float n = static_cast<float>(block);
#pragma unroll
  for (int c = 0; c < IX_D; ++c) {
    ks[c] = rnd<BF16>(ks[c] / n);
    st<BF16>(v_out, o + c, vs[c] / n);
  }
  l2_normalize16(ks);
#pragma unroll
  for (int c = 0; c < IX_D; ++c) {
    if (KF32) static_cast<float*>(k_out)[o + c] = ks[c];
    else st<BF16>(k_out, o + c, ks[c]);
  }
}

// Block scores: workgroup = (batch, 32-query tile, 256-key tile); each thread
// owns one key (normalised in registers) and walks the tile's 32 queries from
// LDS, so every store instruction writes 256 consecutive scores.
constexpr int BS_Q = 32;
constexpr int BS_K = 256;

template <bool BF16>
__global__ __launch_bounds__(BS_K) void block_scores_kernel(const void* __restrict__ q, const void* __restrict__ k,
                                                           int Q, int N, float sqrt_d, void* __restrict__ out) {
  __shared__ float qs[BS_Q][IX_D];
  const int b = blockIdx.z;
  const int q0 = blockIdx.y * BS_Q;
  const int j = blockIdx.x * BS_K + threadIdx.x;
  if (threadIdx.x < BS_Q) {
    float v[IX_D];
    const int qi = q0 + threadIdx.x;
#pragma unroll
    for (int c = 0; c < IX_D; ++c) v[c] = qi < Q ? ld<BF16>(q, (static_cast<int64_t>(b) * Q + qi) * IX_D + c) : 0.f;
    l2_normalize16(v);
#pragma unroll
    for (int c = 0; c < IX_D; ++c) qs[threadIdx.x][c] = rnd<BF16>(v[c]);
  }
  float kv[IX_D];
#pragma unroll
  for (int c = 0; c < IX_D; ++c) kv[c] = j < N ? ld<BF16>(k, (static_cast<int64_t>(b) * N + j) * IX_D + c) : 0.f;
  l2_normalize16(kv);
#pragma unroll
  for (int c = 0; c < IX_D; ++c) kv[c] = rnd<BF16>(kv[c]);
  __syncthreads();
  if (j >= N) return;
  const int qn = Q - q0 < BS_Q ? Q - q0 : BS_Q;
  for (int r = 0; r < qn; ++r) {
    float acc = 0.f;
#pragma unroll
    for (int c = 0; c < IX_D; ++c) acc = fmaf(qs[r][c], kv[c], acc);
    st<BF16>(out, (static_cast<int64_t>(b) * Q + q0 + r) * N + j, rnd<BF16>(acc) / sqrt_d);
  }
}

// Additive-stream context: one workgroup per (batch, query block) row.
constexpr int AC_THREADS = 256;

template <bool BF16>
__global__ __launch_bounds__(AC_THREADS) void additive_context_kernel(const void* __restrict__ scores,
                                                                     const void* __restrict__ v, int Q, int N,
                                                                     int causal, void* __restrict__ ctx) {
  __shared__ float red[AC_THREADS / 64][IX_D];
  const int qb = blockIdx.x, b = blockIdx.y;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(b) * Q + qb;
  const int n_valid = causal ? (qb < N ? qb : N) : N;
  float mx = -INFINITY;
  for (int j = threadIdx.x; j < n_valid; j += AC_THREADS) mx = fmaxf(mx, ld<BF16>(scores, row * N + j));
  mx = wave_max(mx);
  if (lane == 0) red[wave][0] = mx;
  __syncthreads();
  mx = red[0][0];
#pragma unroll
  for (int w = 1; w < AC_THREADS / 64; ++w) mx = fmaxf(mx, red[w][0]);
  __syncthreads();
  if (!isfinite(mx)) mx = 0.0f;
  float z = 0.f;
  for (int j = threadIdx.x; j < n_valid; j += AC_THREADS) z += expf(ld<BF16>(scores, row * N + j) - mx);
  z = wave_sum(z);
  if (lane == 0) red[wave][0] = z;
  __syncthreads();
  z = red[0][0];
#pragma unroll
  for (int w = 1; w < AC_THREADS / 64; ++w) z += red[w][0];
  __syncthreads();
  z = fmaxf(z, 1e-20f);
  float part[IX_D];
#pragma unroll
  for (int c = 0; c < IX_D; ++c) part[c] = 0.f;
  for (int j = threadIdx.x; j < n_valid; j += AC_THREADS) {
    const float p = rnd<BF16>(expf(ld<BF16>(scores, row * N + j) - mx) / z);
#pragma unroll
    for (int c = 0; c < IX_D; ++c) part[c] = fmaf(p, ld<BF16>(v, (static_cast<int64_t>(b) * N + j) * IX_D + c), part[c]);
  }
#pragma unroll
  for (int c = 0; c < IX_D; ++c) {
    const float t = wave_sum(part[c]);
    if (lane == 0) red[wave][c] = t;
  }
  __syncthreads();
  if (threadIdx.x < IX_D) {
    float t = 0.f;
#pragma unroll
    for (int w = 0; w < AC_THREADS / 64; ++w) t += red[w][threadIdx.x];
    st<BF16>(ctx, row * IX_D + threadIdx.x, t);
  }
}

}  // namespace

extern "C" {

FSI_API int fsi_index_rms_norm(const void* x, int dtype, int64_t M, int64_t index_dim, void* out, void* stream) {
  using namespace fsi_host;
  FSI_CHECK_ARG(dtype == FSI_DTYPE_F32 || dtype == FSI_DTYPE_BF16, FSI_ERR_DTYPE, "index_rms_norm: dtype %d", dtype);
  FSI_CHECK_ARG(index_dim == IX_D, FSI_ERR_SHAPE, "index_rms_norm: index_dim %lld != %d", (long long)index_dim, IX_D);
  FSI_CHECK_ARG(M >= 0, FSI_ERR_SHAPE, "index_rms_norm: negative size");
  if (M == 0) return FSI_OK;
  FSI_CHECK_ARG(x && out, FSI_ERR_INVALID_ARG, "index_rms_norm: null pointer");
  FSI_CHECK_ARG((M + 255) / 256 <= 0x7fffffff, FSI_ERR_SHAPE, "index_rms_norm: too many rows");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const unsigned grid = static_cast<unsigned>((M + 255) / 256);
  if (dtype == FSI_DTYPE_BF16) rms_norm_rows_kernel<true><<<grid, 256, 0, st>>>(x, M, out);
  else rms_norm_rows_kernel<false><<<grid, 256, 0, st>>>(x, M, out);
  FSI_HIP_LAUNCH_CHECK("index_rms_norm");
  return FSI_OK;
}

FSI_API int fsi_index_pool_kv(const void* k_lin, const void* v_lin, int dtype, int64_t B, int64_t N,
                              int64_t index_dim, int64_t block_size, void* k_blocks, void* v_blocks, void* stream) {
  using namespace fsi_host;
  FSI_CHECK_ARG(dtype == FSI_DTYPE_F32 || dtype == FSI_DTYPE_BF16, FSI_ERR_DTYPE, "index_pool_kv: dtype %d", dtype);
  FSI_CHECK_ARG(index_dim == IX_D, FSI_ERR_SHAPE, "index_pool_kv: index_dim %lld != %d", (long long)index_dim, IX_D);
  FSI_CHECK_ARG(B >= 0 && N >= 0 && block_size > 0 && block_size <= 0x7fffffff, FSI_ERR_SHAPE,
                "index_pool_kv: bad sizes");
  FSI_CHECK_ARG(N % block_size == 0, FSI_ERR_SHAPE, "index_pool_kv: length %lld not divisible by block_size %lld",
                (long long)N, (long long)block_size);
  const int64_t nb = N / block_size;
  const int64_t n_pool = B * nb;
  if (n_pool == 0) return FSI_OK;
  FSI_CHECK_ARG(k_lin && v_lin && k_blocks && v_blocks, FSI_ERR_INVALID_ARG, "index_pool_kv: null pointer");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const unsigned grid = static_cast<unsigned>((n_pool + 255) / 256);
  const int64_t gs = block_size * IX_D;
  if (dtype == FSI_DTYPE_BF16)
    pool_kv_kernel<true, true, false><<<grid, 256, 0, st>>>(k_lin, v_lin, n_pool, (int)block_size, gs, nb, nb * IX_D,
                                                            k_blocks, v_blocks);
  else
    pool_kv_kernel<false, true, false><<<grid, 256, 0, st>>>(k_lin, v_lin, n_pool, (int)block_size, gs, nb, nb * IX_D,
                                                             k_blocks, v_blocks);
  FSI_HIP_LAUNCH_CHECK("index_pool_kv");
  return FSI_OK;
}

FSI_API int fsi_kv_page_pool(const void* partial_k, const void* partial_v, int dtype, int64_t B, int64_t page_size,
                             int64_t index_dim, float* kp_out, void* vp_out, int64_t out_batch_stride,
                             void* stream) {
  using namespace fsi_host;
  FSI_CHECK_ARG(dtype == FSI_DTYPE_F32 || dtype == FSI_DTYPE_BF16, FSI_ERR_DTYPE, "kv_page_pool: dtype %d", dtype);
  FSI_CHECK_ARG(index_dim == IX_D, FSI_ERR_SHAPE, "kv_page_pool: index_dim %lld != %d", (long long)index_dim, IX_D);
  FSI_CHECK_ARG(B >= 0 && page_size > 0 && page_size <= 0x7fffffff && out_batch_stride >= IX_D, FSI_ERR_SHAPE,
                "kv_page_pool: bad sizes");
  if (B == 0) return FSI_OK;
  FSI_CHECK_ARG(partial_k && partial_v && kp_out && vp_out, FSI_ERR_INVALID_ARG, "kv_page_pool: null pointer");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const unsigned grid = static_cast<unsigned>((B + 255) / 256);
  const int64_t gs = page_size * IX_D;
  if (dtype == FSI_DTYPE_BF16)
    pool_kv_kernel<true, false, true><<<grid, 256, 0, st>>>(partial_k, partial_v, B, (int)page_size, gs, 1,
                                                            out_batch_stride, kp_out, vp_out);
  else
    pool_kv_kernel<false, false, true><<<grid, 256, 0, st>>>(partial_k, partial_v, B, (int)page_size, gs, 1,
                                                             out_batch_stride, kp_out, vp_out);
  FSI_HIP_LAUNCH_CHECK("kv_page_pool");
  return FSI_OK;
}

FSI_API int fsi_block_scores(const void* q, const void* k, int dtype, int64_t B, int64_t Q, int64_t N,
                             int64_t index_dim, void* out, void* stream) {
  using namespace fsi_host;
  FSI_CHECK_ARG(dtype == FSI_DTYPE_F32 || dtype == FSI_DTYPE_BF16, FSI_ERR_DTYPE, "block_scores: dtype %d", dtype);
  FSI_CHECK_ARG(index_dim == IX_D, FSI_ERR_SHAPE, "block_scores: index_dim %lld != %d", (long long)index_dim, IX_D);
  FSI_CHECK_ARG(B >= 0 && Q >= 0 && N >= 0, FSI_ERR_SHAPE, "block_scores: negative size");
  if (B == 0 || Q == 0 || N == 0) return FSI_OK;
  FSI_CHECK_ARG(B <= 65535 && (Q + BS_Q - 1) / BS_Q <= 65535 && N <= (int64_t)0x7fffffff, FSI_ERR_SHAPE,
                "block_scores: grid too large");
  FSI_CHECK_ARG(q && k && out, FSI_ERR_INVALID_ARG, "block_scores: null pointer");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>((N + BS_K - 1) / BS_K), static_cast<unsigned>((Q + BS_Q - 1) / BS_Q),
                  static_cast<unsigned>(B));
  const float sqrt_d = static_cast<float>(sqrt(static_cast<double>(index_dim)));
  if (dtype == FSI_DTYPE_BF16) block_scores_kernel<true><<<grid, BS_K, 0, st>>>(q, k, (int)Q, (int)N, sqrt_d, out);
  else block_scores_kernel<false><<<grid, BS_K, 0, st>>>(q, k, (int)Q, (int)N, sqrt_d, out);
  FSI_HIP_LAUNCH_CHECK("block_scores");
  return FSI_OK;
}

FSI_API int fsi_additive_context(const void* scores, const void* v_blocks, int dtype, int64_t B, int64_t Q,
                                 int64_t N, int64_t index_dim, int causal, void* context, void* stream) {
  using namespace fsi_host;
  FSI_CHECK_ARG(dtype == FSI_DTYPE_F32 || dtype == FSI_DTYPE_BF16, FSI_ERR_DTYPE, "additive_context: dtype %d",
                dtype);
  FSI_CHECK_ARG(index_dim == IX_D, FSI_ERR_SHAPE, "additive_context: index_dim %lld != %d", (long long)index_dim,
                IX_D);
  FSI_CHECK_ARG(B >= 0 && Q >= 0 && N >= 0, FSI_ERR_SHAPE, "additive_context: negative size");
  if (B == 0 || Q == 0) return FSI_OK;
  FSI_CHECK_ARG(B <= 65535 && Q <= (int64_t)0x7fffffff && N <= (int64_t)0x7fffffff, FSI_ERR_SHAPE,
                "additive_context: grid too large");
  FSI_CHECK_ARG(scores && v_blocks && context, FSI_ERR_INVALID_ARG, "additive_context: null pointer");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>(Q), static_cast<unsigned>(B));
  if (dtype == FSI_DTYPE_BF16)
    additive_context_kernel<true><<<grid, AC_THREADS, 0, st>>>(scores, v_blocks, (int)Q, (int)N, causal, context);
  else
    additive_context_kernel<false><<<grid, AC_THREADS, 0, st>>>(scores, v_blocks, (int)Q, (int)N, causal, context);
  FSI_HIP_LAUNCH_CHECK("additive_context");
  return FSI_OK;
}

}  // extern "C"
