// Backward of the block-sparse prefill attention (fsi_sparse_attn) on MI355X
// (gfx950), without materialising any (T, T) tensor.
//
//   out[t] = sum_s w(t, s) exp(scale q_t . k_s - m_t) v_s / l_t,
//   l_t = sum_s w(t, s) exp(scale q_t . k_s - m_t)
//
// with the key weights of the forward: FSI_SATTN_LOCAL_REMOTE (attention.py:
// 148-218) w = 1 where t - W < s <= t or the page of s is listed for the query
// block of t (a union), FSI_SATTN_BLOCK_LIST (triton_ops.py:26-93) w = the
// number of times the block of s is listed for the block of t.  Gradients, with
// P_ts = w exp(scale q_t . k_s - m_t) / l_t and D_t = dout_t . out_t:
//   dV_s = sum_t P_ts dout_t,      dP_ts = dout_t . v_s,
//   dS_ts = P_ts (dP_ts - D_t),    dQ_t = scale sum_s dS_ts k_s,
//   dK_s = scale sum_t dS_ts q_t   (GQA: summed over the group's query heads).
//
// Three kernels, fp32 arithmetic on LDS tiles of 64 queries x 64 keys:
//   1. sab_map_kernel: for every (query block, key block) pair of the pattern's
//      block size, its weight class: mode LOCAL_REMOTE 1 = the window reaches
//      it, 2 = listed (every key counts); mode BLOCK_LIST the listing count.
//      Tiles whose pairs are all 0 are skipped below.
//   2. sab_q_kernel: per (sequence, query head, 64-query tile), two passes over
//      the key tiles: the row maxima and sums, then dQ; writes m, l and D per
//      query row.
//   3. sab_kv_kernel: per (sequence, KV head, 64-key tile), every query tile and
//      query head of the group: dV and dK accumulated in registers, no atomics.
#include "fsi_common.h"

namespace {

using namespace fsi;

constexpr int AB_T = 64;        // queries / keys per tile
constexpr int AB_THREADS = 256;

template <typename T>
__device__ __forceinline__ float ldv(const T* p, int64_t i);
template <>
__device__ __forceinline__ float ldv<float>(const float* p, int64_t i) { return p[i]; }
template <>
__device__ __forceinline__ float ldv<bf16_t>(const bf16_t* p, int64_t i) { return bf16_to_f32(p[i]); }

struct AbParams {
  const void* q;
  int64_t qs_b, qs_h, qs_t;
  const void* k;
  int64_t ks_b, ks_h, ks_t;
  const void* v;
  int64_t vs_b, vs_h, vs_t;
  const void* o;
  int64_t os_b, os_h, os_t;
  const void* dout;
  int64_t ds_b, ds_h, ds_t;
  int B, Hq, Hkv, T, hd, block, mode, window;
  const int32_t* lists;
  int64_t ls_b, ls_q;
  int cap;
  const int32_t* counts;
  int64_t cs_b, cs_q;
  float scale;
  int nb;             // blocks of the pattern: ceil(T / block)
  int32_t* map;       // (B, nb, nb) weight classes
  float* stat_m;      // (B, Hq, T)
  float* stat_l;
  float* stat_d;
  float* dq;          // (B, Hq, T, hd) fp32, contiguous
  float* dk;          // (B, Hkv, T, hd) fp32
  float* dv;
  int* err;
};

// 1. Weight classes of query block qb against every key block.
__global__ __launch_bounds__(AB_THREADS) void sab_map_kernel(AbParams P) {
  const int qb = blockIdx.x, b = blockIdx.y;
  int32_t* row = P.map + (static_cast<int64_t>(b) * P.nb + qb) * P.nb;
  const int t_lo = qb * P.block, t_hi = min(P.T, t_lo + P.block) - 1;
  for (int kb = threadIdx.x; kb < P.nb; kb += AB_THREADS) {
    int w = 0;
    if (P.mode == FSI_SATTN_LOCAL_REMOTE) {
      const int s_lo = kb * P.block, s_hi = min(P.T, s_lo + P.block) - 1;
      // some s <= t and s > t - W with t, s in the two blocks
      if (s_lo <= t_hi && s_hi > t_lo - P.window) w = 1;
    }
    row[kb] = w;
  }
  __syncthreads();
  int cnt = P.counts[b * P.cs_b + qb * P.cs_q];
  cnt = cnt < 0 ? 0 : (cnt > P.cap ? P.cap : cnt);
  const int32_t* list = P.lists ? P.lists + b * P.ls_b + qb * P.ls_q : nullptr;
  bool bad = false;
  for (int j = threadIdx.x; j < cnt; j += AB_THREADS) {
    const int pg = list[j];
    if (pg < 0 || pg >= P.nb) {
      bad = true;
      continue;
    }
    if (P.mode == FSI_SATTN_LOCAL_REMOTE) atomicOr(row + pg, 2);
    else atomicAdd(row + pg, 1);
  }
  if (bad) set_error(P.err, FSI_ERR_INDEX_RANGE);
}

// Weight of key s for query t (both < T) given the class of their blocks.
__device__ __forceinline__ float sab_weight(const AbParams& P, int cls, int t, int s) {
  if (P.mode == FSI_SATTN_LOCAL_REMOTE) return ((cls & 2) || (s <= t && s > t - P.window)) ? 1.f : 0.f;
  return static_cast<float>(cls);
}

// Whether the tile of queries [t0, t0 + 64) and keys [s0, s0 + 64) has a
// non-zero block class (every thread gets the answer).
__device__ __forceinline__ bool sab_tile_live(const AbParams& P, const int32_t* map_b, int t0, int s0) {
  const int qb0 = t0 / P.block, qb1 = (min(P.T, t0 + AB_T) - 1) / P.block;
  const int kb0 = s0 / P.block, kb1 = (min(P.T, s0 + AB_T) - 1) / P.block;
  const int nq = qb1 - qb0 + 1, nk = kb1 - kb0 + 1;
  int live = 0;
  for (int i = threadIdx.x; i < nq * nk; i += AB_THREADS)
    live |= map_b[static_cast<int64_t>(qb0 + i / nk) * P.nb + kb0 + i % nk] != 0;
  return __syncthreads_or(live) != 0;
}

// 64 rows of a (T, hd) matrix at row stride rs into an LDS tile of HD (>= hd)
// columns and row stride HD + 1 floats (rows past T and columns past hd read
// as 0).
template <typename T, int HD>
__device__ __forceinline__ void sab_load_tile(const T* base, int64_t rs, int r0, int nrows, int hd, float* tile) {
  for (int i = threadIdx.x; i < AB_T * HD; i += AB_THREADS) {
    const int r = i / HD, d = i % HD;
    tile[r * (HD + 1) + d] =
        r0 + r < nrows && d < hd ? ldv<T>(base, static_cast<int64_t>(r0 + r) * rs + d) : 0.f;
  }
}

// S[r][c] for this thread's 4 x 4 block (rows 4 ti.., cols 4 tj..): scale x
// row r of A . row c of B over HD dims.
template <int HD>
__device__ __forceinline__ void sab_dot4x4(const float* A, const float* Bm, int ti, int tj, float (&s)[4][4]) {
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int c = 0; c < 4; ++c) s[a][c] = 0.f;
  for (int d = 0; d < HD; ++d) {
    float x[4], y[4];
#pragma unroll
    for (int a = 0; a < 4; ++a) x[a] = A[(4 * ti + a) * (HD + 1) + d];
#pragma unroll
    for (int c = 0; c < 4; ++c) y[c] = Bm[(4 * tj + c) * (HD + 1) + d];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int c = 0; c < 4; ++c) s[a][c] = fmaf(x[a], y[c], s[a][c]);
  }
}

// 2. dQ and the row statistics for one (b, h, 64-query tile).
template <typename T, int HD>
__global__ __launch_bounds__(AB_THREADS) void sab_q_kernel(AbParams P) {
  constexpr int R = HD + 1;
  constexpr int DPT = HD / 16;  // dims per thread of dQ
  __shared__ float Qs[AB_T * R], Os[AB_T * R], Ks[AB_T * R], Vs[AB_T * R];
  __shared__ float Ss[AB_T * (AB_T + 1)];
  __shared__ float row_m[AB_T], row_l[AB_T], row_d[AB_T];
  const int t0 = blockIdx.x * AB_T;
  const int b = blockIdx.y / P.Hq, h = blockIdx.y % P.Hq;
  const int g = h / (P.Hq / P.Hkv);
  const int tid = threadIdx.x, ti = tid >> 4, tj = tid & 15;
  const T* q = static_cast<const T*>(P.q) + b * P.qs_b + h * P.qs_h;
  const T* o = static_cast<const T*>(P.o) + b * P.os_b + h * P.os_h;
  const T* dout = static_cast<const T*>(P.dout) + b * P.ds_b + h * P.ds_h;
  const T* k = static_cast<const T*>(P.k) + b * P.ks_b + g * P.ks_h;
  const T* v = static_cast<const T*>(P.v) + b * P.vs_b + g * P.vs_h;
  const int32_t* map_b = P.map + static_cast<int64_t>(b) * P.nb * P.nb;

  sab_load_tile<T, HD>(q, P.qs_t, t0, P.T, P.hd, Qs);
  sab_load_tile<T, HD>(o, P.os_t, t0, P.T, P.hd, Os);
  sab_load_tile<T, HD>(dout, P.ds_t, t0, P.T, P.hd, Ks);  // dout staged in Ks for D
  __syncthreads();
  if (tid < AB_T) {
    float d = 0.f;
    for (int c = 0; c < HD; ++c) d = fmaf(Ks[tid * R + c], Os[tid * R + c], d);
    row_d[tid] = d;
    row_m[tid] = -INFINITY;
    row_l[tid] = 0.f;
  }
  __syncthreads();
  // dout stays in Os from here on (O was only needed for D)
  for (int i = tid; i < AB_T * R; i += AB_THREADS) Os[i] = Ks[i];

  // pass 1: row maxima and sums over every live key tile
  for (int s0 = 0; s0 < P.T; s0 += AB_T) {
    if (!sab_tile_live(P, map_b, t0, s0)) continue;
    sab_load_tile<T, HD>(k, P.ks_t, s0, P.T, P.hd, Ks);
    __syncthreads();
    float s[4][4];
    sab_dot4x4<HD>(Qs, Ks, ti, tj, s);
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      const int t = t0 + 4 * ti + a;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int sk = s0 + 4 * tj + c;
        float w = 0.f;
        if (t < P.T && sk < P.T) w = sab_weight(P, map_b[static_cast<int64_t>(t / P.block) * P.nb + sk / P.block], t, sk);
        // the weight folded into the logit: exp(x - m) = w exp(scale q.k - m); m
        // only stabilises, and every use below takes P with this same m and l
        Ss[(4 * ti + a) * (AB_T + 1) + 4 * tj + c] = w > 0.f ? s[a][c] * P.scale + logf(w) : -INFINITY;
      }
    }
    __syncthreads();
    if (tid < AB_T) {  // one thread per row: the online maximum and sum
      float m = row_m[tid], l = row_l[tid];
      float cm = -INFINITY;
      for (int c = 0; c < AB_T; ++c) cm = fmaxf(cm, Ss[tid * (AB_T + 1) + c]);
      if (cm > -INFINITY) {
        const float mn = fmaxf(m, cm);
        float add = 0.f;
        for (int c = 0; c < AB_T; ++c) {
          const float x = Ss[tid * (AB_T + 1) + c];
          if (x > -INFINITY) add += expf(x - mn);
        }
        l = (m > -INFINITY ? l * expf(m - mn) : 0.f) + add;
        row_m[tid] = mn;
        row_l[tid] = l;
      }
    }
    __syncthreads();
  }

  // pass 2: dQ = scale sum_s dS k_s
  float acc[4][DPT];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int e = 0; e < DPT; ++e) acc[a][e] = 0.f;
  for (int s0 = 0; s0 < P.T; s0 += AB_T) {
    if (!sab_tile_live(P, map_b, t0, s0)) continue;
    sab_load_tile<T, HD>(k, P.ks_t, s0, P.T, P.hd, Ks);
    sab_load_tile<T, HD>(v, P.vs_t, s0, P.T, P.hd, Vs);
    __syncthreads();
    float s[4][4], dp[4][4];
    sab_dot4x4<HD>(Qs, Ks, ti, tj, s);
    sab_dot4x4<HD>(Os, Vs, ti, tj, dp);  // dout . v
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      const int r = 4 * ti + a, t = t0 + r;
      const float m = row_m[r], l = row_l[r], dd = row_d[r];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int sk = s0 + 4 * tj + c;
        float ds = 0.f;
        if (t < P.T && sk < P.T && l > 0.f) {
          const float w = sab_weight(P, map_b[static_cast<int64_t>(t / P.block) * P.nb + sk / P.block], t, sk);
          if (w > 0.f) {
            const float p = w * expf(s[a][c] * P.scale - m) / l;
            ds = p * (dp[a][c] - dd);
          }
        }
        Ss[r * (AB_T + 1) + 4 * tj + c] = ds;
      }
    }
    __syncthreads();
    // acc[a][e] += sum_c dS[4 ti + a][c] k[c][tj + 16 e]
    for (int c = 0; c < AB_T; ++c) {
      float kk[DPT];
#pragma unroll
      for (int e = 0; e < DPT; ++e) kk[e] = Ks[c * R + tj + 16 * e];
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const float x = Ss[(4 * ti + a) * (AB_T + 1) + c];
#pragma unroll
        for (int e = 0; e < DPT; ++e) acc[a][e] = fmaf(x, kk[e], acc[a][e]);
      }
    }
    __syncthreads();
  }
  const int64_t rowbase = (static_cast<int64_t>(b) * P.Hq + h) * P.T;
#pragma unroll
  for (int a = 0; a < 4; ++a) {
    const int t = t0 + 4 * ti + a;
    if (t >= P.T) continue;
#pragma unroll
    for (int e = 0; e < DPT; ++e)
      if (tj + 16 * e < P.hd) P.dq[(rowbase + t) * P.hd + tj + 16 * e] = acc[a][e] * P.scale;
  }
  if (tid < AB_T && t0 + tid < P.T) {
    P.stat_m[rowbase + t0 + tid] = row_m[tid];
    P.stat_l[rowbase + t0 + tid] = row_l[tid];
    P.stat_d[rowbase + t0 + tid] = row_d[tid];
  }
}

// 3. dK and dV for one (b, g, 64-key tile) over every query tile and query
//    head of the group.
template <typename T, int HD>
__global__ __launch_bounds__(AB_THREADS) void sab_kv_kernel(AbParams P) {
  constexpr int R = HD + 1;
  constexpr int DPT = HD / 16;
  __shared__ float Ks[AB_T * R], Vs[AB_T * R], Qs[AB_T * R], Ds[AB_T * R];
  __shared__ float Ps[AB_T * (AB_T + 1)];
  __shared__ float row_m[AB_T], row_l[AB_T], row_d[AB_T];
  const int s0 = blockIdx.x * AB_T;
  const int b = blockIdx.y / P.Hkv, g = blockIdx.y % P.Hkv;
  const int G = P.Hq / P.Hkv;
  const int tid = threadIdx.x, ti = tid >> 4, tj = tid & 15;
  const T* k = static_cast<const T*>(P.k) + b * P.ks_b + g * P.ks_h;
  const T* v = static_cast<const T*>(P.v) + b * P.vs_b + g * P.vs_h;
  const int32_t* map_b = P.map + static_cast<int64_t>(b) * P.nb * P.nb;
  sab_load_tile<T, HD>(k, P.ks_t, s0, P.T, P.hd, Ks);
  sab_load_tile<T, HD>(v, P.vs_t, s0, P.T, P.hd, Vs);
  // this thread: keys 4 ti + a, dims tj + 16 e
  float dk[4][DPT], dv[4][DPT];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int e = 0; e < DPT; ++e) dk[a][e] = dv[a][e] = 0.f;
  for (int t0 = 0; t0 < P.T; t0 += AB_T) {
    if (!sab_tile_live(P, map_b, t0, s0)) continue;
    for (int hh = 0; hh < G; ++hh) {
      const int h = g * G + hh;
      const T* q = static_cast<const T*>(P.q) + b * P.qs_b + h * P.qs_h;
      const T* dout = static_cast<const T*>(P.dout) + b * P.ds_b + h * P.ds_h;
      const int64_t rowbase = (static_cast<int64_t>(b) * P.Hq + h) * P.T;
      sab_load_tile<T, HD>(q, P.qs_t, t0, P.T, P.hd, Qs);
      sab_load_tile<T, HD>(dout, P.ds_t, t0, P.T, P.hd, Ds);
      if (tid < AB_T) {
        const int t = t0 + tid;
        row_m[tid] = t < P.T ? P.stat_m[rowbase + t] : -INFINITY;
        row_l[tid] = t < P.T ? P.stat_l[rowbase + t] : 0.f;
        row_d[tid] = t < P.T ? P.stat_d[rowbase + t] : 0.f;
      }
      __syncthreads();
      // this thread's scores: queries 4 ti + a, keys 4 tj + c
      float s[4][4], dp[4][4];
      sab_dot4x4<HD>(Qs, Ks, ti, tj, s);
      sab_dot4x4<HD>(Ds, Vs, ti, tj, dp);
      float ds[4][4];
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const int r = 4 * ti + a, t = t0 + r;
        const float m = row_m[r], l = row_l[r], dd = row_d[r];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const int sk = s0 + 4 * tj + c;
          float p = 0.f;
          if (t < P.T && sk < P.T && l > 0.f) {
            const float w =
                sab_weight(P, map_b[static_cast<int64_t>(t / P.block) * P.nb + sk / P.block], t, sk);
            if (w > 0.f) p = w * expf(s[a][c] * P.scale - m) / l;
          }
          Ps[r * (AB_T + 1) + 4 * tj + c] = p;
          ds[a][c] = p * (dp[a][c] - dd);
        }
      }
      __syncthreads();
      // dV[key][dim] += sum_r P[r][key] dout[r][dim]
      for (int r = 0; r < AB_T; ++r) {
        float x[DPT];
#pragma unroll
        for (int e = 0; e < DPT; ++e) x[e] = Ds[r * R + tj + 16 * e];
#pragma unroll
        for (int a = 0; a < 4; ++a) {
          const float p = Ps[r * (AB_T + 1) + 4 * ti + a];
#pragma unroll
          for (int e = 0; e < DPT; ++e) dv[a][e] = fmaf(p, x[e], dv[a][e]);
        }
      }
      __syncthreads();
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int c = 0; c < 4; ++c) Ps[(4 * ti + a) * (AB_T + 1) + 4 * tj + c] = ds[a][c];
      __syncthreads();
      // dK[key][dim] += sum_r dS[r][key] q[r][dim]
      for (int r = 0; r < AB_T; ++r) {
        float x[DPT];
#pragma unroll
        for (int e = 0; e < DPT; ++e) x[e] = Qs[r * R + tj + 16 * e];
#pragma unroll
        for (int a = 0; a < 4; ++a) {
          const float d = Ps[r * (AB_T + 1) + 4 * ti + a];
#pragma unroll
          for (int e = 0; e < DPT; ++e) dk[a][e] = fmaf(d, x[e], dk[a][e]);
        }
      }
      __syncthreads();
    }
  }
  const int64_t kbase = (static_cast<int64_t>(b) * P.Hkv + g) * P.T;
#pragma unroll
  for (int a = 0; a < 4; ++a) {
    const int s = s0 + 4 * ti + a;
    if (s >= P.T) continue;
#pragma unroll
    for (int e = 0; e < DPT; ++e) {
      if (tj + 16 * e >= P.hd) continue;
      P.dk[(kbase + s) * P.hd + tj + 16 * e] = dk[a][e] * P.scale;
      P.dv[(kbase + s) * P.hd + tj + 16 * e] = dv[a][e];
    }
  }
}

// Workspace: the counter area (left untouched), the block map, then m, l, D.
size_t sab_map_bytes(int64_t B, int64_t T, int64_t block) {
  const int64_t nb = (T + block - 1) / block;
  return fsi_host::align_up(sizeof(int32_t) * static_cast<size_t>(B * nb * nb), 256);
}

}  // namespace

extern "C" {

FSI_API size_t fsi_sparse_attn_bwd_workspace_size(int64_t B, int64_t Hq, int64_t T, int64_t block) {
  if (B <= 0 || Hq <= 0 || T <= 0 || block <= 0) return 0;
  return FSI_WORKSPACE_COUNTER_BYTES + sab_map_bytes(B, T, block) +
         3 * fsi_host::align_up(sizeof(float) * static_cast<size_t>(B * Hq * T), 256);
}

FSI_API int fsi_sparse_attn_bwd(const void* q, int64_t qs_b, int64_t qs_h, int64_t qs_t, const void* k, int64_t ks_b,
                                int64_t ks_h, int64_t ks_t, const void* v, int64_t vs_b, int64_t vs_h, int64_t vs_t,
                                const void* out, int64_t os_b, int64_t os_h, int64_t os_t, const void* dout,
                                int64_t ds_b, int64_t ds_h, int64_t ds_t, int64_t B, int64_t Hq, int64_t Hkv,
                                int64_t T, int64_t head_dim, int64_t block, int mode, int64_t window,
                                const int32_t* lists, int64_t ls_b, int64_t ls_q, int64_t capacity,
                                const int32_t* counts, int64_t cs_b, int64_t cs_q, float scale, int dtype, float* dq,
                                float* dk, float* dv, void* workspace, size_t workspace_bytes, int* err,
                                void* stream) {
  using namespace fsi_host;
  FSI_CHECK_ARG(dtype == FSI_DTYPE_F32 || dtype == FSI_DTYPE_BF16, FSI_ERR_DTYPE, "sparse_attn_bwd: dtype %d", dtype);
  FSI_CHECK_ARG(mode == FSI_SATTN_LOCAL_REMOTE || mode == FSI_SATTN_BLOCK_LIST, FSI_ERR_INVALID_ARG,
                "sparse_attn_bwd: mode %d", mode);
  FSI_CHECK_ARG(head_dim >= 1 && head_dim <= 128, FSI_ERR_SHAPE, "sparse_attn_bwd: head_dim %lld (1..128)",
                (long long)head_dim);
  FSI_CHECK_ARG(B > 0 && T > 0 && Hkv > 0 && Hq > 0 && Hq % Hkv == 0 && block > 0, FSI_ERR_SHAPE,
                "sparse_attn_bwd: B=%lld T=%lld Hq=%lld Hkv=%lld block=%lld", (long long)B, (long long)T,
                (long long)Hq, (long long)Hkv, (long long)block);
  FSI_CHECK_ARG(T <= (int64_t(1) << 30) && B * Hq <= 65535 && (T + AB_T - 1) / AB_T <= 0x7fffffff, FSI_ERR_SHAPE,
                "sparse_attn_bwd: sizes beyond range");
  const int64_t nb = (T + block - 1) / block;
  FSI_CHECK_ARG(nb <= 65535 && B * nb * nb <= (int64_t(1) << 31), FSI_ERR_SHAPE,
                "sparse_attn_bwd: %lld blocks per sequence beyond the block map", (long long)nb);
  FSI_CHECK_ARG(capacity >= 0 && capacity <= 4096, FSI_ERR_CAPACITY, "sparse_attn_bwd: capacity %lld",
                (long long)capacity);
  FSI_CHECK_ARG(mode != FSI_SATTN_LOCAL_REMOTE || window > 0, FSI_ERR_SHAPE, "sparse_attn_bwd: window %lld",
                (long long)window);
  FSI_CHECK_ARG(q && k && v && out && dout && counts && (lists || capacity == 0) && dq && dk && dv, FSI_ERR_INVALID_ARG,
                "sparse_attn_bwd: null pointer");
  const size_t need = fsi_sparse_attn_bwd_workspace_size(B, Hq, T, block);
  FSI_CHECK_ARG(workspace && workspace_bytes >= need && reinterpret_cast<uintptr_t>(workspace) % 16 == 0,
                FSI_ERR_WORKSPACE, "sparse_attn_bwd: workspace %zu < %zu (or misaligned)", workspace_bytes, need);
  AbParams P{};
  P.q = q;
  P.qs_b = qs_b;
  P.qs_h = qs_h;
  P.qs_t = qs_t;
  P.k = k;
  P.ks_b = ks_b;
  P.ks_h = ks_h;
  P.ks_t = ks_t;
  P.v = v;
  P.vs_b = vs_b;
  P.vs_h = vs_h;
  P.vs_t = vs_t;
  P.o = out;
  P.os_b = os_b;
  P.os_h = os_h;
  P.os_t = os_t;
  P.dout = dout;
  P.ds_b = ds_b;
  P.ds_h = ds_h;
  P.ds_t = ds_t;
  P.B = (int)B;
  P.Hq = (int)Hq;
  P.Hkv = (int)Hkv;
  P.T = (int)T;
  P.hd = (int)head_dim;
  P.block = (int)block;
  P.mode = mode;
  P.window = (int)(window < 0x7fffffff ? window : 0x7fffffff);
  P.lists = lists;
  P.ls_b = ls_b;
  P.ls_q = ls_q;
  P.cap = (int)capacity;
  P.counts = counts;
  P.cs_b = cs_b;
  P.cs_q = cs_q;
  P.scale = scale;
  P.nb = (int)nb;
  char* ws = static_cast<char*>(workspace) + FSI_WORKSPACE_COUNTER_BYTES;
  P.map = reinterpret_cast<int32_t*>(ws);
  const size_t st_bytes = align_up(sizeof(float) * static_cast<size_t>(B * Hq * T), 256);
  P.stat_m = reinterpret_cast<float*>(ws + sab_map_bytes(B, T, block));
  P.stat_l = reinterpret_cast<float*>(ws + sab_map_bytes(B, T, block) + st_bytes);
  P.stat_d = reinterpret_cast<float*>(ws + sab_map_bytes(B, T, block) + 2 * st_bytes);
  P.dq = dq;
  P.dk = dk;
  P.dv = dv;
  P.err = err;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  sab_map_kernel<<<dim3(static_cast<unsigned>(nb), static_cast<unsigned>(B)), AB_THREADS, 0, st>>>(P);
  const unsigned ntiles = static_cast<unsigned>((T + AB_T - 1) / AB_T);
  const dim3 gq(ntiles, static_cast<unsigned>(B * Hq)), gkv(ntiles, static_cast<unsigned>(B * Hkv));
  auto run = [&](auto hd_tag) {
    constexpr int HD = decltype(hd_tag)::value;
    if (dtype == FSI_DTYPE_F32) {
      sab_q_kernel<float, HD><<<gq, AB_THREADS, 0, st>>>(P);
      sab_kv_kernel<float, HD><<<gkv, AB_THREADS, 0, st>>>(P);
    } else {
      sab_q_kernel<bf16_t, HD><<<gq, AB_THREADS, 0, st>>>(P);
      sab_kv_kernel<bf16_t, HD><<<gkv, AB_THREADS, 0, st>>>(P);
    }
  };
  if (head_dim <= 16) run(std::integral_constant<int, 16>{});
  else if (head_dim <= 32) run(std::integral_constant<int, 32>{});
  else if (head_dim <= 64) run(std::integral_constant<int, 64>{});
  else run(std::integral_constant<int, 128>{});
  FSI_HIP_LAUNCH_CHECK("sparse_attn_bwd");
  return FSI_OK;
}

}  // extern "C"
