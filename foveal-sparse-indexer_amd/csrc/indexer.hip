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


// ---------------------------------------------------------------------------
// Backward passes (the autograd of core.py:214-310).  Gradients are computed in
// fp32 from the saved forward inputs, with the forward's intermediate values
// recomputed, and rounded to the tensor dtype at the points where the
// reference's autograd graph holds a tensor of that dtype.
// ---------------------------------------------------------------------------

// dx of y = x * r, r = 1 / sqrt(mean(x^2) + eps):  r * (dy - y * mean(dy * y)).
__device__ __forceinline__ void rms_norm16_bwd(const float (&x)[IX_D], const float (&dy)[IX_D], float (&dx)[IX_D]) {
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < IX_D; ++c) ss = fmaf(x[c], x[c], ss);
  const float r = 1.0f / sqrtf(ss / static_cast<float>(IX_D) + FLT_EPS);
  float dot = 0.f;
#pragma unroll
  for (int c = 0; c < IX_D; ++c) dot = fmaf(dy[c], x[c] * r, dot);
  const float m = dot / static_cast<float>(IX_D);
#pragma unroll
  for (int c = 0; c < IX_D; ++c) dx[c] = r * (dy[c] - x[c] * r * m);
}

// dx of y = x / max(|x|, 1e-12) (F.normalize): (dy - y (y . dy)) / |x| above the
// clamp, dy / 1e-12 below it (the clamp passes no gradient to the norm).
__device__ __forceinline__ void l2_normalize16_bwd(const float (&x)[IX_D], const float (&dy)[IX_D],
                                                   float (&dx)[IX_D]) {
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < IX_D; ++c) ss = fmaf(x[c], x[c], ss);
  const float n = sqrtf(ss);
  if (n >= 1e-12f) {
    float dot = 0.f;
#pragma unroll
    for (int c = 0; c < IX_D; ++c) dot = fmaf(x[c] / n, dy[c], dot);
#pragma unroll
    for (int c = 0; c < IX_D; ++c) dx[c] = (dy[c] - (x[c] / n) * dot) / n;
  } else {
#pragma unroll
    for (int c = 0; c < IX_D; ++c) dx[c] = dy[c] / 1e-12f;
  }
}

template <bool BF16>
__global__ __launch_bounds__(256) void rms_norm_rows_bwd_kernel(const void* __restrict__ x, const void* __restrict__ dy,
                                                               int64_t M, void* __restrict__ dx) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (r >= M) return;
  float xv[IX_D], g[IX_D], out[IX_D];
#pragma unroll
  for (int c = 0; c < IX_D; ++c) {
    xv[c] = ld<BF16>(x, r * IX_D + c);
    g[c] = ld<BF16>(dy, r * IX_D + c);
  }
  rms_norm16_bwd(xv, g, out);
#pragma unroll
  for (int c = 0; c < IX_D; ++c) st<BF16>(dx, r * IX_D + c, out[c]);
}

// Pooling backward: one wave per (batch, block), lanes over the block's tokens.
// Recomputes the pooled key mean, takes the normalisation's gradient, spreads
// it over the tokens (mean) and through each token's rms_norm; the value
// gradient is dv_blocks / block for every token of the block.
constexpr int PB_WAVES = 4;

template <bool BF16>
__global__ __launch_bounds__(64 * PB_WAVES) void pool_kv_bwd_kernel(const void* __restrict__ k_lin,
                                                                   const void* __restrict__ dk_blocks,
                                                                   const void* __restrict__ dv_blocks, int64_t n_pool,
                                                                   int block, void* __restrict__ dk_lin,
                                                                   void* __restrict__ dv_lin) {
  const int64_t pb = static_cast<int64_t>(blockIdx.x) * PB_WAVES + (threadIdx.x >> 6);
  if (pb >= n_pool) return;  // whole waves exit together; no barrier below
  const int lane = threadIdx.x & 63;
  const int64_t t0 = pb * block;  // first token row
  float ks[IX_D];
#pragma unroll
  for (int c = 0; c < IX_D; ++c) ks[c] = 0.f;
  for (int t = lane; t < block; t += 64) {
    float kv[IX_D];
#pragma unroll
    for (int c = 0; c < IX_D; ++c) kv[c] = ld<BF16>(k_lin, (t0 + t) * IX_D + c);
    rms_norm16(kv);
#pragma unroll
    for (int c = 0; c < IX_D; ++c) ks[c] += rnd<BF16>(kv[c]);
  }
  const float n = static_cast<float>(block);
  float km[IX_D], g[IX_D], gm[IX_D], gv[IX_D];
#pragma unroll
  for (int c = 0; c < IX_D; ++c) {
    km[c] = rnd<BF16>(wave_sum(ks[c]) / n);
    g[c] = ld<BF16>(dk_blocks, pb * IX_D + c);
    gv[c] = rnd<BF16>(ld<BF16>(dv_blocks, pb * IX_D + c) / n);
  }
  l2_normalize16_bwd(km, g, gm);
#pragma unroll
  for (int c = 0; c < IX_D; ++c) gm[c] = rnd<BF16>(rnd<BF16>(gm[c]) / n);  // normalize grad, then mean grad
  for (int t = lane; t < block; t += 64) {
    float kv[IX_D], out[IX_D];
#pragma unroll
    for (int c = 0; c < IX_D; ++c) kv[c] = ld<BF16>(k_lin, (t0 + t) * IX_D + c);
    rms_norm16_bwd(kv, gm, out);
#pragma unroll
    for (int c = 0; c < IX_D; ++c) {
      st<BF16>(dk_lin, (t0 + t) * IX_D + c, out[c]);
      st<BF16>(dv_lin, (t0 + t) * IX_D + c, gv[c]);
    }
  }
}

// Block-score backward.  With qn, kn the normalised (rounded) operands and
// g = dscores / sqrt(d):  dqn = g kn,  dkn = g^T qn  (rounded, as the bmm's
// gradients), then each through the normalisation.  One 64-lane workgroup per
// (batch, 64-row tile); the other side is staged through LDS 64 rows at a time.
constexpr int SB_T = 64;

template <bool BF16>
__global__ __launch_bounds__(SB_T) void block_scores_dq_kernel(const void* __restrict__ q, const void* __restrict__ k,
                                                              const void* __restrict__ ds, int Q, int N, float sqrt_d,
                                                              void* __restrict__ dq) {
  __shared__ float kn[SB_T][IX_D];
  __shared__ float tile[SB_T][SB_T + 1];
  const int b = blockIdx.y, q0 = blockIdx.x * SB_T, lane = threadIdx.x;
  const int nq = Q - q0 < SB_T ? Q - q0 : SB_T;
  float acc[IX_D];
#pragma unroll
  for (int c = 0; c < IX_D; ++c) acc[c] = 0.f;
  for (int n0 = 0; n0 < N; n0 += SB_T) {
    const int j = n0 + lane;
    float kv[IX_D];
#pragma unroll
    for (int c = 0; c < IX_D; ++c) kv[c] = j < N ? ld<BF16>(k, (static_cast<int64_t>(b) * N + j) * IX_D + c) : 0.f;
    l2_normalize16(kv);
#pragma unroll
    for (int c = 0; c < IX_D; ++c) kn[lane][c] = rnd<BF16>(kv[c]);
    for (int r = 0; r < nq; ++r)
      tile[r][lane] = j < N ? ld<BF16>(ds, (static_cast<int64_t>(b) * Q + q0 + r) * N + j) / sqrt_d : 0.f;
    __syncthreads();
    if (lane < nq) {
      for (int jj = 0; jj < SB_T; ++jj) {
        const float gg = tile[lane][jj];
#pragma unroll
        for (int c = 0; c < IX_D; ++c) acc[c] = fmaf(gg, kn[jj][c], acc[c]);
      }
    }
    __syncthreads();
  }
  if (lane >= nq) return;
  const int64_t row = static_cast<int64_t>(b) * Q + q0 + lane;
  float qv[IX_D], out[IX_D];
#pragma unroll
  for (int c = 0; c < IX_D; ++c) {
    qv[c] = ld<BF16>(q, row * IX_D + c);
    acc[c] = rnd<BF16>(acc[c]);
  }
  l2_normalize16_bwd(qv, acc, out);
#pragma unroll
  for (int c = 0; c < IX_D; ++c) st<BF16>(dq, row * IX_D + c, out[c]);
}

template <bool BF16>
__global__ __launch_bounds__(SB_T) void block_scores_dk_kernel(const void* __restrict__ q, const void* __restrict__ k,
                                                              const void* __restrict__ ds, int Q, int N, float sqrt_d,
                                                              void* __restrict__ dk) {
  __shared__ float qn[SB_T][IX_D];
  const int b = blockIdx.y, lane = threadIdx.x;
  const int j = blockIdx.x * SB_T + lane;
  float acc[IX_D];
#pragma unroll
  for (int c = 0; c < IX_D; ++c) acc[c] = 0.f;
  for (int q0 = 0; q0 < Q; q0 += SB_T) {
    const int qi = q0 + lane;
    float qv[IX_D];
#pragma unroll
    for (int c = 0; c < IX_D; ++c) qv[c] = qi < Q ? ld<BF16>(q, (static_cast<int64_t>(b) * Q + qi) * IX_D + c) : 0.f;
    l2_normalize16(qv);
#pragma unroll
    for (int c = 0; c < IX_D; ++c) qn[lane][c] = rnd<BF16>(qv[c]);
    __syncthreads();
    const int nq = Q - q0 < SB_T ? Q - q0 : SB_T;
    if (j < N) {
      for (int r = 0; r < nq; ++r) {
        const float gg = ld<BF16>(ds, (static_cast<int64_t>(b) * Q + q0 + r) * N + j) / sqrt_d;
#pragma unroll
        for (int c = 0; c < IX_D; ++c) acc[c] = fmaf(gg, qn[r][c], acc[c]);
      }
    }
    __syncthreads();
  }
  if (j >= N) return;
  const int64_t row = static_cast<int64_t>(b) * N + j;
  float kv[IX_D], out[IX_D];
#pragma unroll
  for (int c = 0; c < IX_D; ++c) {
    kv[c] = ld<BF16>(k, row * IX_D + c);
    acc[c] = rnd<BF16>(acc[c]);
  }
  l2_normalize16_bwd(kv, acc, out);
#pragma unroll
  for (int c = 0; c < IX_D; ++c) st<BF16>(dk, row * IX_D + c, out[c]);
}

// Additive-context backward, rows: per (batch, query block) row, with p the
// fp32 masked softmax and dp_j = dctx . v_j (rounded, the bmm's gradient):
// dscores_j = p_j (dp_j - sum_k p_k dp_k) on valid keys, 0 elsewhere.  Also
// stores the row's softmax max and normaliser for the value gradient.
template <bool BF16>
__global__ __launch_bounds__(AC_THREADS) void additive_context_bwd_rows_kernel(
    const void* __restrict__ scores, const void* __restrict__ v, const void* __restrict__ dctx, int Q, int N,
    int causal, void* __restrict__ dscores, float2* __restrict__ stats) {
  __shared__ float red[AC_THREADS / 64];
  const int qb = blockIdx.x, b = blockIdx.y;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(b) * Q + qb;
  const int n_valid = causal ? (qb < N ? qb : N) : N;
  auto reduce = [&](float x, bool is_max) {
    x = is_max ? wave_max(x) : wave_sum(x);
    if (lane == 0) red[wave] = x;
    __syncthreads();
    float r = red[0];
#pragma unroll
    for (int w = 1; w < AC_THREADS / 64; ++w) r = is_max ? fmaxf(r, red[w]) : r + red[w];
    __syncthreads();
    return r;
  };
  float g[IX_D];
#pragma unroll
  for (int c = 0; c < IX_D; ++c) g[c] = ld<BF16>(dctx, row * IX_D + c);
  auto dp_of = [&](int j) {
    float a = 0.f;
#pragma unroll
    for (int c = 0; c < IX_D; ++c) a = fmaf(g[c], ld<BF16>(v, (static_cast<int64_t>(b) * N + j) * IX_D + c), a);
    return rnd<BF16>(a);
  };
  float mx = -INFINITY;
  for (int j = threadIdx.x; j < n_valid; j += AC_THREADS) mx = fmaxf(mx, ld<BF16>(scores, row * N + j));
  mx = reduce(mx, true);
  if (!isfinite(mx)) mx = 0.0f;
  float z = 0.f;
  for (int j = threadIdx.x; j < n_valid; j += AC_THREADS) z += expf(ld<BF16>(scores, row * N + j) - mx);
  z = fmaxf(reduce(z, false), 1e-20f);
  float dot = 0.f;
  for (int j = threadIdx.x; j < n_valid; j += AC_THREADS)
    dot = fmaf(expf(ld<BF16>(scores, row * N + j) - mx) / z, dp_of(j), dot);
  dot = reduce(dot, false);
  for (int j = threadIdx.x; j < N; j += AC_THREADS) {
    const float out = j < n_valid ? expf(ld<BF16>(scores, row * N + j) - mx) / z * (dp_of(j) - dot) : 0.0f;
    st<BF16>(dscores, row * N + j, out);
  }
  if (threadIdx.x == 0) stats[row] = make_float2(mx, z);
}

// Additive-context backward, values: dv_j = sum_q p_qj dctx_q with the rounded
// probabilities of the forward.  One 64-lane workgroup per (batch, 64-key tile);
// the query rows' dctx and softmax statistics are staged through LDS.
template <bool BF16>
__global__ __launch_bounds__(SB_T) void additive_context_dv_kernel(const void* __restrict__ scores,
                                                                  const void* __restrict__ dctx,
                                                                  const float2* __restrict__ stats, int Q, int N,
                                                                  int causal, void* __restrict__ dv) {
  __shared__ float gs[SB_T][IX_D];
  __shared__ float2 ms[SB_T];
  const int b = blockIdx.y, lane = threadIdx.x;
  const int j0 = blockIdx.x * SB_T, j = j0 + lane;
  float acc[IX_D];
#pragma unroll
  for (int c = 0; c < IX_D; ++c) acc[c] = 0.f;
  const int q_first = causal ? (j0 + 1) / SB_T * SB_T : 0;  // rows q <= j see no key j when causal
  for (int q0 = q_first; q0 < Q; q0 += SB_T) {
    const int qi = q0 + lane;
    if (qi < Q) {
      const int64_t row = static_cast<int64_t>(b) * Q + qi;
#pragma unroll
      for (int c = 0; c < IX_D; ++c) gs[lane][c] = ld<BF16>(dctx, row * IX_D + c);
      ms[lane] = stats[row];
    }
    __syncthreads();
    const int nq = Q - q0 < SB_T ? Q - q0 : SB_T;
    if (j < N) {
      for (int r = 0; r < nq; ++r) {
        if (causal && j >= q0 + r) continue;
        const float2 st2 = ms[r];
        const float p = rnd<BF16>(expf(ld<BF16>(scores, (static_cast<int64_t>(b) * Q + q0 + r) * N + j) - st2.x) /
                                  st2.y);
#pragma unroll
        for (int c = 0; c < IX_D; ++c) acc[c] = fmaf(p, gs[r][c], acc[c]);
      }
    }
    __syncthreads();
  }
  if (j >= N) return;
#pragma unroll
  for (int c = 0; c < IX_D; ++c) st<BF16>(dv, (static_cast<int64_t>(b) * N + j) * IX_D + c, acc[c]);
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

FSI_API int fsi_index_rms_norm_bwd(const void* x, const void* dy, int dtype, int64_t M, int64_t index_dim, void* dx,
                                   void* stream) {
  using namespace fsi_host;
  FSI_CHECK_ARG(dtype == FSI_DTYPE_F32 || dtype == FSI_DTYPE_BF16, FSI_ERR_DTYPE, "index_rms_norm_bwd: dtype %d", dtype);
  FSI_CHECK_ARG(index_dim == IX_D, FSI_ERR_SHAPE, "index_rms_norm_bwd: index_dim %lld != %d", (long long)index_dim,
                IX_D);
  FSI_CHECK_ARG(M >= 0, FSI_ERR_SHAPE, "index_rms_norm_bwd: negative size");
  if (M == 0) return FSI_OK;
  FSI_CHECK_ARG(x && dy && dx, FSI_ERR_INVALID_ARG, "index_rms_norm_bwd: null pointer");
  FSI_CHECK_ARG((M + 255) / 256 <= 0x7fffffff, FSI_ERR_SHAPE, "index_rms_norm_bwd: too many rows");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const unsigned grid = static_cast<unsigned>((M + 255) / 256);
  if (dtype == FSI_DTYPE_BF16) rms_norm_rows_bwd_kernel<true><<<grid, 256, 0, st>>>(x, dy, M, dx);
  else rms_norm_rows_bwd_kernel<false><<<grid, 256, 0, st>>>(x, dy, M, dx);
  FSI_HIP_LAUNCH_CHECK("index_rms_norm_bwd");
  return FSI_OK;
}

FSI_API int fsi_index_pool_kv_bwd(const void* k_lin, const void* dk_blocks, const void* dv_blocks, int dtype, int64_t B,
                                  int64_t N, int64_t index_dim, int64_t block_size, void* dk_lin, void* dv_lin,
                                  void* stream) {
  using namespace fsi_host;
  FSI_CHECK_ARG(dtype == FSI_DTYPE_F32 || dtype == FSI_DTYPE_BF16, FSI_ERR_DTYPE, "index_pool_kv_bwd: dtype %d", dtype);
  FSI_CHECK_ARG(index_dim == IX_D, FSI_ERR_SHAPE, "index_pool_kv_bwd: index_dim %lld != %d", (long long)index_dim,
                IX_D);
  FSI_CHECK_ARG(B >= 0 && N >= 0 && block_size > 0 && block_size <= 0x7fffffff, FSI_ERR_SHAPE,
                "index_pool_kv_bwd: bad sizes");
  FSI_CHECK_ARG(N % block_size == 0, FSI_ERR_SHAPE,
                "index_pool_kv_bwd: length %lld not divisible by block_size %lld", (long long)N,
                (long long)block_size);
  const int64_t n_pool = B * (N / block_size);
  if (n_pool == 0) return FSI_OK;
  FSI_CHECK_ARG(k_lin && dk_blocks && dv_blocks && dk_lin && dv_lin, FSI_ERR_INVALID_ARG,
                "index_pool_kv_bwd: null pointer");
  FSI_CHECK_ARG((n_pool + PB_WAVES - 1) / PB_WAVES <= 0x7fffffff, FSI_ERR_SHAPE, "index_pool_kv_bwd: too many blocks");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const unsigned grid = static_cast<unsigned>((n_pool + PB_WAVES - 1) / PB_WAVES);
  if (dtype == FSI_DTYPE_BF16)
    pool_kv_bwd_kernel<true><<<grid, 64 * PB_WAVES, 0, st>>>(k_lin, dk_blocks, dv_blocks, n_pool, (int)block_size,
                                                             dk_lin, dv_lin);
  else
    pool_kv_bwd_kernel<false><<<grid, 64 * PB_WAVES, 0, st>>>(k_lin, dk_blocks, dv_blocks, n_pool, (int)block_size,
                                                              dk_lin, dv_lin);
  FSI_HIP_LAUNCH_CHECK("index_pool_kv_bwd");
  return FSI_OK;
}

FSI_API int fsi_block_scores_bwd(const void* q, const void* k, const void* dscores, int dtype, int64_t B, int64_t Q,
                                 int64_t N, int64_t index_dim, void* dq, void* dk, void* stream) {
  using namespace fsi_host;
  FSI_CHECK_ARG(dtype == FSI_DTYPE_F32 || dtype == FSI_DTYPE_BF16, FSI_ERR_DTYPE, "block_scores_bwd: dtype %d", dtype);
  FSI_CHECK_ARG(index_dim == IX_D, FSI_ERR_SHAPE, "block_scores_bwd: index_dim %lld != %d", (long long)index_dim, IX_D);
  FSI_CHECK_ARG(B >= 0 && Q >= 0 && N >= 0, FSI_ERR_SHAPE, "block_scores_bwd: negative size");
  if (B == 0 || (Q == 0 && N == 0)) return FSI_OK;
  FSI_CHECK_ARG(B <= 65535 && Q <= (int64_t)0x7fffffff && N <= (int64_t)0x7fffffff, FSI_ERR_SHAPE,
                "block_scores_bwd: grid too large");
  FSI_CHECK_ARG(q && k && dscores && dq && dk, FSI_ERR_INVALID_ARG, "block_scores_bwd: null pointer");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const float sqrt_d = static_cast<float>(sqrt(static_cast<double>(index_dim)));
  // Q == 0 or N == 0: the kernels still run on the other side and write zero gradients.
  if (Q > 0) {
    const dim3 gq(static_cast<unsigned>((Q + SB_T - 1) / SB_T), static_cast<unsigned>(B));
    if (dtype == FSI_DTYPE_BF16)
      block_scores_dq_kernel<true><<<gq, SB_T, 0, st>>>(q, k, dscores, (int)Q, (int)N, sqrt_d, dq);
    else
      block_scores_dq_kernel<false><<<gq, SB_T, 0, st>>>(q, k, dscores, (int)Q, (int)N, sqrt_d, dq);
    FSI_HIP_LAUNCH_CHECK("block_scores_bwd (dq)");
  }
  if (N > 0) {
    const dim3 gk(static_cast<unsigned>((N + SB_T - 1) / SB_T), static_cast<unsigned>(B));
    if (dtype == FSI_DTYPE_BF16)
      block_scores_dk_kernel<true><<<gk, SB_T, 0, st>>>(q, k, dscores, (int)Q, (int)N, sqrt_d, dk);
    else
      block_scores_dk_kernel<false><<<gk, SB_T, 0, st>>>(q, k, dscores, (int)Q, (int)N, sqrt_d, dk);
    FSI_HIP_LAUNCH_CHECK("block_scores_bwd (dk)");
  }
  return FSI_OK;
}

FSI_API size_t fsi_additive_context_bwd_workspace_size(int64_t B, int64_t Q) {
  return B > 0 && Q > 0 ? static_cast<size_t>(B * Q) * sizeof(float2) : 0;
}

FSI_API int fsi_additive_context_bwd(const void* scores, const void* v_blocks, const void* dcontext, int dtype,
                                     int64_t B, int64_t Q, int64_t N, int64_t index_dim, int causal, void* dscores,
                                     void* dv_blocks, void* workspace, size_t workspace_bytes, void* stream) {
  using namespace fsi_host;
  FSI_CHECK_ARG(dtype == FSI_DTYPE_F32 || dtype == FSI_DTYPE_BF16, FSI_ERR_DTYPE, "additive_context_bwd: dtype %d",
                dtype);
  FSI_CHECK_ARG(index_dim == IX_D, FSI_ERR_SHAPE, "additive_context_bwd: index_dim %lld != %d", (long long)index_dim,
                IX_D);
  FSI_CHECK_ARG(B >= 0 && Q >= 0 && N >= 0, FSI_ERR_SHAPE, "additive_context_bwd: negative size");
  if (B == 0 || (Q == 0 && N == 0)) return FSI_OK;
  FSI_CHECK_ARG(B <= 65535 && Q <= (int64_t)0x7fffffff && N <= (int64_t)0x7fffffff, FSI_ERR_SHAPE,
                "additive_context_bwd: grid too large");
  FSI_CHECK_ARG(scores && v_blocks && dcontext && dscores && dv_blocks, FSI_ERR_INVALID_ARG,
                "additive_context_bwd: null pointer");
  const size_t need = fsi_additive_context_bwd_workspace_size(B, Q);
  FSI_CHECK_ARG(workspace_bytes >= need && (need == 0 || workspace), FSI_ERR_WORKSPACE,
                "additive_context_bwd: workspace %zu < %zu bytes", workspace_bytes, need);
  FSI_CHECK_ARG(reinterpret_cast<uintptr_t>(workspace) % alignof(float2) == 0, FSI_ERR_ALIGN,
                "additive_context_bwd: workspace not 8-byte aligned");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  float2* stats = static_cast<float2*>(workspace);
  if (Q > 0) {
    const dim3 gr(static_cast<unsigned>(Q), static_cast<unsigned>(B));
    if (dtype == FSI_DTYPE_BF16)
      additive_context_bwd_rows_kernel<true><<<gr, AC_THREADS, 0, st>>>(scores, v_blocks, dcontext, (int)Q, (int)N,
                                                                        causal, dscores, stats);
    else
      additive_context_bwd_rows_kernel<false><<<gr, AC_THREADS, 0, st>>>(scores, v_blocks, dcontext, (int)Q, (int)N,
                                                                         causal, dscores, stats);
    FSI_HIP_LAUNCH_CHECK("additive_context_bwd (rows)");
  }
  if (N > 0) {
    const dim3 gv(static_cast<unsigned>((N + SB_T - 1) / SB_T), static_cast<unsigned>(B));
    if (dtype == FSI_DTYPE_BF16)
      additive_context_dv_kernel<true><<<gv, SB_T, 0, st>>>(scores, dcontext, stats, (int)Q, (int)N, causal,
                                                            dv_blocks);
    else
      additive_context_dv_kernel<false><<<gv, SB_T, 0, st>>>(scores, dcontext, stats, (int)Q, (int)N, causal,
                                                             dv_blocks);
    FSI_HIP_LAUNCH_CHECK("additive_context_bwd (values)");
  }
  return FSI_OK;
}

}  // extern "C"
