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
// Three kernels on tiles of 64 queries x 64 keys (bf16 inputs with head_dim 32 / 64 / 128:
// the sab_*_bf kernels below, every product on bf16 MFMA; otherwise fp32 arithmetic on
// v_mfma_f32_16x16x4_f32):
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
  bool vec4;          // head_dim one of the tile widths (16 / 32 / 64 / 128), rows 4-element aligned
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

// Class of the block pair (query t, key s), both < T.
__device__ __forceinline__ int sab_class(const AbParams& P, const int32_t* map_b, int t, int s) {
  return map_b[static_cast<int64_t>(t / P.block) * P.nb + s / P.block];
}

// Weight of key s for query t (both < T) given the class of their blocks.
__device__ __forceinline__ float sab_weight(const AbParams& P, int cls, int t, int s) {
  if (P.mode == FSI_SATTN_LOCAL_REMOTE) return ((cls & 2) || (s <= t && s > t - P.window)) ? 1.f : 0.f;
  return static_cast<float>(cls);
}

// Class of the tile of queries [t0, t0 + 64) and keys [s0, s0 + 64), the
// same for every thread: the block class (> 0) when the tile lies in one block
// pair, 0 when every block pair it touches has class 0 (nothing to do), -1
// when it spans several block pairs and some is non-zero (classes then looked
// up per element).
__device__ __forceinline__ int sab_tile_class(const AbParams& P, const int32_t* map_b, int t0, int s0) {
  const int qb0 = t0 / P.block, qb1 = (min(P.T, t0 + AB_T) - 1) / P.block;
  const int kb0 = s0 / P.block, kb1 = (min(P.T, s0 + AB_T) - 1) / P.block;
  const int nq = qb1 - qb0 + 1, nk = kb1 - kb0 + 1;
  if (nq == 1 && nk == 1) return map_b[static_cast<int64_t>(qb0) * P.nb + kb0];
  int live = 0;
  for (int i = threadIdx.x; i < nq * nk; i += AB_THREADS)
    live |= map_b[static_cast<int64_t>(qb0 + i / nk) * P.nb + kb0 + i % nk] != 0;
  return __syncthreads_or(live) != 0 ? -1 : 0;
}

// Weight of key s for query t (both < T) in a tile of class tcls (as returned by
// sab_tile_class, non-zero); the block map is read only for a mixed tile.
__device__ __forceinline__ float sab_tile_weight(const AbParams& P, const int32_t* map_b, int tcls, int t, int s) {
  if (tcls < 0) return sab_weight(P, sab_class(P, map_b, t, s), t, s);
  return sab_weight(P, tcls, t, s);
}

// Logits of keys s0 + 16 t + 4 kg + e against query tq (S^T accumulators st),
// with the weight folded in (exp(x - m) = w exp(scale q.k - m)); -inf where the
// weight is 0 or the query / key is past T.  A tile of one block pair takes its
// weight from the class (one log per tile); a local tile of the local/remote
// pattern tests the window per element.
__device__ __forceinline__ void sab_logits(const AbParams& P, const int32_t* map_b, int tq, int kg, int s0, int tcls,
                                           f32x4_t (&st)[4]) {
  if (tcls > 0 && (P.mode == FSI_SATTN_BLOCK_LIST || (tcls & 2))) {
    // one weight for the whole tile: keys below lim are valid
    const float lw = P.mode == FSI_SATTN_BLOCK_LIST ? __logf(static_cast<float>(tcls)) : 0.f;
    const int lim = tq < P.T ? P.T : 0;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int sk = s0 + 16 * t + 4 * kg + e;
        st[t][e] = sk < lim ? st[t][e] * P.scale + lw : -INFINITY;
      }
  } else if (tcls > 0) {
    // local/remote tile reached by the window only: tq - W < sk <= tq (< T)
    const int hi = tq < P.T ? tq : -1, lo = tq - P.window;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int sk = s0 + 16 * t + 4 * kg + e;
        st[t][e] = sk <= hi && sk > lo ? st[t][e] * P.scale : -INFINITY;
      }
  } else {
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int sk = s0 + 16 * t + 4 * kg + e;
        float x = -INFINITY;
        if (tq < P.T && sk < P.T) {
          const float w = sab_tile_weight(P, map_b, tcls, tq, sk);
          if (w > 0.f) x = st[t][e] * P.scale + __logf(w);
        }
        st[t][e] = x;
      }
  }
}

// 64 rows of a (T, hd) matrix at row stride rs into an LDS tile of row stride
// HD + 4 floats (rows past T and columns past hd read as 0).  The 4-float pad
// puts the 8 rows a 128-bit read serves at once on distinct bank groups, and
// the 16 rows of a column read on two halves of the banks.
// vec: head_dim == HD and every row starts 4-element aligned (host-checked), so
// a thread moves 4 consecutive elements at once.
template <typename T>
__device__ __forceinline__ f32x4_t ld4(const T* p);
template <>
__device__ __forceinline__ f32x4_t ld4<float>(const float* p) { return *reinterpret_cast<const f32x4_t*>(p); }
template <>
__device__ __forceinline__ f32x4_t ld4<bf16_t>(const bf16_t* p) {
  const uint2 w = *reinterpret_cast<const uint2*>(p);
  return f32x4_t{__uint_as_float(w.x << 16), __uint_as_float(w.x & 0xffff0000u), __uint_as_float(w.y << 16),
                 __uint_as_float(w.y & 0xffff0000u)};
}
template <typename T, int HD>
__device__ __forceinline__ void sab_load_tile(const T* base, int64_t rs, int r0, int nrows, int hd, float* tile,
                                              bool vec) {
  if (vec) {
    for (int i = threadIdx.x; i < AB_T * HD / 4; i += AB_THREADS) {
      const int r = i / (HD / 4), d = 4 * (i % (HD / 4));
      f32x4_t x = f32x4_t{0.f, 0.f, 0.f, 0.f};
      if (r0 + r < nrows) x = ld4<T>(base + static_cast<int64_t>(r0 + r) * rs + d);
      *reinterpret_cast<f32x4_t*>(&tile[r * (HD + 4) + d]) = x;
    }
    return;
  }
  for (int i = threadIdx.x; i < AB_T * HD; i += AB_THREADS) {
    const int r = i / HD, d = i % HD;
    tile[r * (HD + 4) + d] =
        r0 + r < nrows && d < hd ? ldv<T>(base, static_cast<int64_t>(r0 + r) * rs + d) : 0.f;
  }
}

// Row `row` (< T) of a (T, hd) matrix as this lane's MFMA k-operand: dims
// 16 dg + 4 kg .. +4 of every 16-dim group (0 past hd).
template <typename T, int HD>
__device__ __forceinline__ void sab_row_frag(const T* base, int64_t rs, int row, int hd, int kg,
                                             f32x4_t (&f)[HD / 16]) {
#pragma unroll
  for (int dg = 0; dg < HD / 16; ++dg)
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int d = 16 * dg + 4 * kg + kk;
      f[dg][kk] = d < hd ? ldv<T>(base, static_cast<int64_t>(row) * rs + d) : 0.f;
    }
}

__device__ __forceinline__ f32x4_t ab_mfma(float a, float b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Two floats holding bf16 values as one packed bf16 pair (their upper halves).
__device__ __forceinline__ uint32_t ab_pk(float x, float y) {
  return __builtin_amdgcn_perm(__float_as_uint(y), __float_as_uint(x), 0x07060302u);
}
// 8 consecutive floats of an LDS row (bf16 values) as a bf16 MFMA operand.
__device__ __forceinline__ u32x4_t ab_pack8(const float* p) {
  const f32x4_t a = *reinterpret_cast<const f32x4_t*>(p);
  const f32x4_t b = *reinterpret_cast<const f32x4_t*>(p + 4);
  return u32x4_t{ab_pk(a[0], a[1]), ab_pk(a[2], a[3]), ab_pk(b[0], b[1]), ab_pk(b[2], b[3])};
}
// Row `row` of a bf16 (T, hd) matrix as this lane's bf16 MFMA operand: dims
// 32 ks + 8 kg .. +8 of every 32-dim step (0 past hd).
template <typename T, int HD>
__device__ __forceinline__ void sab_row_frag_bf(const T* base, int64_t rs, int row, int hd, int kg,
                                                u32x4_t (&f)[HD / 32]) {
#pragma unroll
  for (int ks = 0; ks < HD / 32; ++ks) {
    float x[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int d = 32 * ks + 8 * kg + j;
      x[j] = d < hd ? ldv<T>(base, static_cast<int64_t>(row) * rs + d) : 0.f;
    }
    f[ks] = u32x4_t{ab_pk(x[0], x[1]), ab_pk(x[2], x[3]), ab_pk(x[4], x[5]), ab_pk(x[6], x[7])};
  }
}

// 2. dQ and the row statistics for one (b, h, 64-query tile).  Wave w owns
//    queries t0 + 16 w .. +16 and keeps their Q and dout rows as the B operand
//    of S^T = K Q^T and dP^T = V dout^T (v_mfma_f32_16x16x4_f32, k-step kk taking
//    dims 4 (lane / 16) + kk of each 16-dim group); lane (r, kg) then holds keys
//    16 t + 4 kg + e of query r, so dS^T's element kk is the B operand of
//    dQ^T = K^T dS^T for the keys 16 t + 4 kg + kk (K^T read by column from LDS).
template <typename T, int HD>
__global__ __launch_bounds__(AB_THREADS) void sab_q_kernel(AbParams P) {
  constexpr int DG = HD / 16, R = HD + 4;
  __shared__ float Ks[AB_T * R], Vs[AB_T * R];
  // heads fastest and the latest query tiles first: under a causal pattern they
  // reach the most key tiles, so the longest blocks start first
  const int t0 = ((P.T + AB_T - 1) / AB_T - 1 - static_cast<int>(blockIdx.x / P.Hq)) * AB_T;
  const int b = blockIdx.y, h = blockIdx.x % P.Hq;
  const int g = h / (P.Hq / P.Hkv);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, kg = lane >> 4;
  const int tq = t0 + 16 * wave + r;             // this lane's query
  const int tql = tq < P.T ? tq : P.T - 1;       // rows past T read row T - 1, never stored
  const T* q = static_cast<const T*>(P.q) + b * P.qs_b + h * P.qs_h;
  const T* o = static_cast<const T*>(P.o) + b * P.os_b + h * P.os_h;
  const T* dout = static_cast<const T*>(P.dout) + b * P.ds_b + h * P.ds_h;
  const T* k = static_cast<const T*>(P.k) + b * P.ks_b + g * P.ks_h;
  const T* v = static_cast<const T*>(P.v) + b * P.vs_b + g * P.vs_h;
  const int32_t* map_b = P.map + static_cast<int64_t>(b) * P.nb * P.nb;

  // bf16 inputs: S^T and dP^T on v_mfma_f32_16x16x32_bf16 (products of bf16 values
  // are exact in fp32, so this loses nothing against the fp32 form)
  constexpr bool BFR = sizeof(T) == 2 && HD >= 32;
  constexpr int KS32 = HD >= 32 ? HD / 32 : 1;
  f32x4_t qf[DG], df[DG];
  sab_row_frag<T, HD>(q, P.qs_t, tql, P.hd, kg, qf);
  sab_row_frag<T, HD>(dout, P.ds_t, tql, P.hd, kg, df);
  u32x4_t qb[KS32], db[KS32];
  if constexpr (BFR) {
    sab_row_frag_bf<T, HD>(q, P.qs_t, tql, P.hd, kg, qb);
    sab_row_frag_bf<T, HD>(dout, P.ds_t, tql, P.hd, kg, db);
  }
  float dd;  // D = dout . out of query r
  {
    f32x4_t of[DG];
    sab_row_frag<T, HD>(o, P.os_t, tql, P.hd, kg, of);
    float part = 0.f;
#pragma unroll
    for (int dg = 0; dg < DG; ++dg)
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) part = fmaf(df[dg][kk], of[dg][kk], part);
    dd = sum_rows4(part);
  }

  auto logits = [&](int s0, int tcls, f32x4_t (&st)[4]) { sab_logits(P, map_b, tq, kg, s0, tcls, st); };
  // S^T tiles of the 64 keys in Ks against this wave's queries
  auto scores = [&](f32x4_t (&st)[4], const float* Xs, const f32x4_t (&bf)[DG], const u32x4_t (&bb)[KS32]) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      st[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      if constexpr (BFR) {
#pragma unroll
        for (int ks = 0; ks < KS32; ++ks)
          st[t] = mfma16x16x32(ab_pack8(&Xs[(16 * t + r) * R + 32 * ks + 8 * kg]), bb[ks], st[t]);
      } else {
#pragma unroll
        for (int dg = 0; dg < DG; ++dg) {
          const f32x4_t a = *reinterpret_cast<const f32x4_t*>(&Xs[(16 * t + r) * R + 16 * dg + 4 * kg]);
#pragma unroll
          for (int kk = 0; kk < 4; ++kk) st[t] = ab_mfma(a[kk], bf[dg][kk], st[t]);
        }
      }
    }
  };

  // pass 1: row maximum and sum over every live key tile (the sum kept per lane
  // and reduced over the lane group at the end)
  float m = -INFINITY, lpart = 0.f;
  for (int s0 = 0; s0 < P.T; s0 += AB_T) {
    const int tcls = sab_tile_class(P, map_b, t0, s0);
    if (tcls == 0) continue;
    sab_load_tile<T, HD>(k, P.ks_t, s0, P.T, P.hd, Ks, P.vec4);
    __syncthreads();
    f32x4_t st[4];
    scores(st, Ks, qf, qb);
    logits(s0, tcls, st);
    float cm = -INFINITY;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int e = 0; e < 4; ++e) cm = fmaxf(cm, st[t][e]);
    cm = max_rows4(cm);
    if (cm > -INFINITY) {
      const float mn = fmaxf(m, cm);
      float add = 0.f;
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e) add += __expf(st[t][e] - mn);
      lpart = (m > -INFINITY ? lpart * __expf(m - mn) : 0.f) + add;
      m = mn;
    }
    __syncthreads();
  }
  const float l = sum_rows4(lpart);
  const float il = l > 0.f ? 1.f / l : 0.f;

  // pass 2: dQ^T[dim][query] = scale sum_key K[key][dim] dS[query][key]
  f32x4_t dqa[DG];
#pragma unroll
  for (int dt = 0; dt < DG; ++dt) dqa[dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < P.T; s0 += AB_T) {
    const int tcls = sab_tile_class(P, map_b, t0, s0);
    if (tcls == 0) continue;
    sab_load_tile<T, HD>(k, P.ks_t, s0, P.T, P.hd, Ks, P.vec4);
    sab_load_tile<T, HD>(v, P.vs_t, s0, P.T, P.hd, Vs, P.vec4);
    __syncthreads();
    f32x4_t st[4], dp[4];
    scores(st, Ks, qf, qb);
    scores(dp, Vs, df, db);  // dP^T = V dout^T
    logits(s0, tcls, st);
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float p = l > 0.f ? __expf(st[t][e] - m) * il : 0.f;  // exp(-inf) = 0 where w = 0
        st[t][e] = p * (dp[t][e] - dd);                            // dS^T
      }
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const float* krow = &Ks[(16 * t + 4 * kg + kk) * R + r];
#pragma unroll
        for (int dt = 0; dt < DG; ++dt) dqa[dt] = ab_mfma(krow[16 * dt], st[t][kk], dqa[dt]);
      }
    __syncthreads();
  }
  // lane (r, kg) holds dQ[query r][dims 16 dt + 4 kg + e]
  const int64_t rowbase = (static_cast<int64_t>(b) * P.Hq + h) * P.T;
  if (tq < P.T) {
#pragma unroll
    for (int dt = 0; dt < DG; ++dt)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int d = 16 * dt + 4 * kg + e;
        if (d < P.hd) P.dq[(rowbase + tq) * P.hd + d] = dqa[dt][e] * P.scale;
      }
    if (kg == 0) {
      P.stat_m[rowbase + tq] = m;
      P.stat_l[rowbase + tq] = l;
      P.stat_d[rowbase + tq] = dd;
    }
  }
}

// 3. dK and dV for one (b, g, 64-key tile) over every query tile and query
//    head of the group.  Wave w owns keys s0 + 16 w .. +16 and keeps their K and
//    V rows as the B operand of S = Q K^T and dP = dout V^T; lane (r, kg) then
//    holds queries 16 qt + 4 kg + e of key r, so the elements of P and dS are the
//    B operands of dV^T = dout^T P and dK^T = Q^T dS (dout^T, Q^T read by column
//    from LDS).  Accumulated in registers, no atomics.
template <typename T, int HD>
__global__ __launch_bounds__(AB_THREADS) void sab_kv_kernel(AbParams P) {
  constexpr int DG = HD / 16, R = HD + 4;
  __shared__ float Qs[AB_T * R], Ds[AB_T * R];
  __shared__ float row_m[AB_T], row_il[AB_T], row_d[AB_T];
  // heads fastest and the earliest key tiles first: under a causal pattern the
  // most query tiles reach them, so the longest blocks start first
  const int s0 = static_cast<int>(blockIdx.x / P.Hkv) * AB_T;
  const int b = blockIdx.y, g = blockIdx.x % P.Hkv;
  const int G = P.Hq / P.Hkv;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, kg = lane >> 4;
  const int sk = s0 + 16 * wave + r;       // this lane's key
  const int skl = sk < P.T ? sk : P.T - 1;
  const T* k = static_cast<const T*>(P.k) + b * P.ks_b + g * P.ks_h;
  const T* v = static_cast<const T*>(P.v) + b * P.vs_b + g * P.vs_h;
  const int32_t* map_b = P.map + static_cast<int64_t>(b) * P.nb * P.nb;
  constexpr bool BFR = sizeof(T) == 2 && HD >= 32;  // S and dP on bf16 MFMA (exact products)
  constexpr int KS32 = HD >= 32 ? HD / 32 : 1;
  f32x4_t kf[BFR ? 1 : DG], vf[BFR ? 1 : DG];
  u32x4_t kb[KS32], vb[KS32];
  if constexpr (BFR) {
    sab_row_frag_bf<T, HD>(k, P.ks_t, skl, P.hd, kg, kb);
    sab_row_frag_bf<T, HD>(v, P.vs_t, skl, P.hd, kg, vb);
  } else {
    sab_row_frag<T, HD>(k, P.ks_t, skl, P.hd, kg, kf);
    sab_row_frag<T, HD>(v, P.vs_t, skl, P.hd, kg, vf);
  }
  f32x4_t dka[DG], dva[DG];
#pragma unroll
  for (int dt = 0; dt < DG; ++dt) dka[dt] = dva[dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  for (int t0 = 0; t0 < P.T; t0 += AB_T) {
    const int tcls = sab_tile_class(P, map_b, t0, s0);
    if (tcls == 0) continue;
    // weight of the whole tile when it lies in one block pair and needs no window test
    const float wall = tcls > 0 && (P.mode == FSI_SATTN_BLOCK_LIST || (tcls & 2))
                           ? (P.mode == FSI_SATTN_BLOCK_LIST ? static_cast<float>(tcls) : 1.f)
                           : 0.f;
    for (int hh = 0; hh < G; ++hh) {
      const int h = g * G + hh;
      const T* q = static_cast<const T*>(P.q) + b * P.qs_b + h * P.qs_h;
      const T* dout = static_cast<const T*>(P.dout) + b * P.ds_b + h * P.ds_h;
      const int64_t rowbase = (static_cast<int64_t>(b) * P.Hq + h) * P.T;
      sab_load_tile<T, HD>(q, P.qs_t, t0, P.T, P.hd, Qs, P.vec4);
      sab_load_tile<T, HD>(dout, P.ds_t, t0, P.T, P.hd, Ds, P.vec4);
      if (tid < AB_T) {
        const int t = t0 + tid;
        const float lq = t < P.T ? P.stat_l[rowbase + t] : 0.f;
        row_m[tid] = t < P.T ? P.stat_m[rowbase + t] : -INFINITY;
        row_il[tid] = lq > 0.f ? 1.f / lq : 0.f;
        row_d[tid] = t < P.T ? P.stat_d[rowbase + t] : 0.f;
      }
      __syncthreads();
#pragma unroll 1
      for (int qt = 0; qt < 4; ++qt) {  // not unrolled: K, V, dK and dV already hold 128 registers
        f32x4_t s = f32x4_t{0.f, 0.f, 0.f, 0.f}, dp = s;
        if constexpr (BFR) {
#pragma unroll
          for (int ks = 0; ks < KS32; ++ks) {
            s = mfma16x16x32(ab_pack8(&Qs[(16 * qt + r) * R + 32 * ks + 8 * kg]), kb[ks], s);
            dp = mfma16x16x32(ab_pack8(&Ds[(16 * qt + r) * R + 32 * ks + 8 * kg]), vb[ks], dp);
          }
        } else {
#pragma unroll
          for (int dg = 0; dg < DG; ++dg) {
            const f32x4_t a = *reinterpret_cast<const f32x4_t*>(&Qs[(16 * qt + r) * R + 16 * dg + 4 * kg]);
            const f32x4_t c = *reinterpret_cast<const f32x4_t*>(&Ds[(16 * qt + r) * R + 16 * dg + 4 * kg]);
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) {
              s = ab_mfma(a[kk], kf[dg][kk], s);
              dp = ab_mfma(c[kk], vf[dg][kk], dp);
            }
          }
        }
        // s[e], dp[e]: query 16 qt + 4 kg + e, key r
        f32x4_t pp, ds;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int rq = 16 * qt + 4 * kg + e, t = t0 + rq;
          float p = 0.f;
          const float il = row_il[rq];
          if (t < P.T && sk < P.T && il > 0.f) {
            const float w = wall > 0.f ? wall : sab_tile_weight(P, map_b, tcls, t, sk);
            if (w > 0.f) p = w * __expf(s[e] * P.scale - row_m[rq]) * il;
          }
          pp[e] = p;
          ds[e] = p * (dp[e] - row_d[rq]);
        }
        // dV^T[dim][key] += dout[query][dim] P[query][key], dK^T += Q[query][dim] dS[query][key]
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          const float* drow = &Ds[(16 * qt + 4 * kg + kk) * R + r];
          const float* qrow = &Qs[(16 * qt + 4 * kg + kk) * R + r];
#pragma unroll
          for (int dt = 0; dt < DG; ++dt) {
            dva[dt] = ab_mfma(drow[16 * dt], pp[kk], dva[dt]);
            dka[dt] = ab_mfma(qrow[16 * dt], ds[kk], dka[dt]);
          }
        }
      }
      __syncthreads();
    }
  }
  // lane (r, kg) holds dK, dV [key r][dims 16 dt + 4 kg + e]
  const int64_t kbase = (static_cast<int64_t>(b) * P.Hkv + g) * P.T;
  if (sk < P.T) {
#pragma unroll
    for (int dt = 0; dt < DG; ++dt)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int d = 16 * dt + 4 * kg + e;
        if (d >= P.hd) continue;
        P.dk[(kbase + sk) * P.hd + d] = dka[dt][e] * P.scale;
        P.dv[(kbase + sk) * P.hd + d] = dva[dt][e];
      }
  }
}

// ---------------------------------------------------------------------------
// bf16 inputs with head_dim 32 / 64 / 128 and 4-element-aligned rows: every
// product on v_mfma_f32_16x16x32_bf16.  Tiles sit in LDS as bf16, row-major at
// stride HD + 8 (the 8 rows a 128-bit read serves at once start on distinct
// bank quads) and, where a product contracts over the tile's rows, transposed
// as well at stride 64 + 4 (the 16 rows of a 64-bit read on distinct bank
// pairs).  P and dS enter their products as a pair of bf16 operands hi + lo
// (hi = the value rounded to bf16, lo = the remainder rounded): the pair holds
// the value to ~2^-17 relative, the other operand is an exact bf16 input and
// the MFMA accumulates in fp32.
//
// A lane's k slots 8 kg + e of a 32-row product: rows 4 kg + e (e < 4) and
// 16 + 4 kg + e - 4 (e >= 4) of the 32, i.e. the rows its two 16 x 16
// accumulators of P / dS hold, so those enter the MFMA where they are; the
// transposed tile is read at the same rows.
// ---------------------------------------------------------------------------
constexpr int BF_TS = AB_T + 4;  // transposed-tile row stride (bf16 elements)

// Rows [r0, r0 + 64) of a (T, HD) bf16 matrix move in two halves, so the next
// tile's loads can be in flight while the current tile is used: bf_load reads
// them into registers (thread = 4-row group x 4-dim group, one 8-byte load per
// row; rows past T read as 0), bf_store writes them to the row-major tile rt
// and, when TR, to the transposed tile tt after a 4 x 4 transpose in registers.
// Transposed rows d hold their 4-column groups in the order g ^ ((d >> 4) & 3):
// the 16 rows 4 apart that one store instruction writes then land on distinct
// banks, and the 16 consecutive rows of an operand read (one swizzle value)
// stay on distinct bank pairs.
template <int HD>
constexpr int bf_rounds() { return HD >= 64 ? HD / 64 : 1; }

// Rows past T re-read row T - 1: every product that uses them is multiplied by
// a zero P / dS or masked, so they only need to be finite.
template <int HD>
__device__ __forceinline__ void bf_load(const bf16_t* base, int64_t rs, int r0, int T, uint2 (&x)[bf_rounds<HD>()][4]) {
  constexpr int DGN = HD / 4, QG = AB_THREADS / DGN;
  const int dg = threadIdx.x % DGN;
  const int qg0 = QG * bf_rounds<HD>() > AB_T / 4 ? (threadIdx.x / DGN) % (AB_T / 4) : threadIdx.x / DGN;
  if (r0 + AB_T <= T) {
    // every row inside: a scalar row base and 32-bit lane offsets (row strides
    // below 2^24 elements, host-checked), one add per load
    const char* rb = reinterpret_cast<const char*>(base + static_cast<int64_t>(r0) * rs);
    const uint32_t rsb = static_cast<uint32_t>(rs) * 2u;
    const uint32_t lo = static_cast<uint32_t>(4 * qg0) * rsb + 8u * static_cast<uint32_t>(dg);
#pragma unroll
    for (int rr = 0; rr < bf_rounds<HD>(); ++rr)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        x[rr][j] = *reinterpret_cast<const uint2*>(rb + (lo + static_cast<uint32_t>(4 * rr * QG + j) * rsb));
    return;
  }
#pragma unroll
  for (int rr = 0; rr < bf_rounds<HD>(); ++rr)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int r = r0 + 4 * (qg0 + rr * QG) + j;
      x[rr][j] = *reinterpret_cast<const uint2*>(base + static_cast<int64_t>(r < T ? r : T - 1) * rs + 4 * dg);
    }
}

template <int HD, bool TR>
__device__ __forceinline__ void bf_store(const uint2 (&x)[bf_rounds<HD>()][4], bf16_t* rt, bf16_t* tt) {
  constexpr int DGN = HD / 4, QG = AB_THREADS / DGN;
  const int dg = threadIdx.x % DGN, qg0 = threadIdx.x / DGN;
#pragma unroll
  for (int rr = 0; rr < bf_rounds<HD>(); ++rr) {
    const int qg = qg0 + rr * QG;
    if (QG * bf_rounds<HD>() > AB_T / 4 && qg >= AB_T / 4) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) *reinterpret_cast<uint2*>(&rt[(4 * qg + j) * (HD + 8) + 4 * dg]) = x[rr][j];
    if constexpr (TR) {
      constexpr uint32_t LO = 0x05040100u, HI = 0x07060302u;  // low / high bf16 of each source
      const uint2* y = x[rr];
      bf16_t* t = &tt[4 * dg * BF_TS + 4 * (qg ^ ((dg >> 2) & 3))];
      *reinterpret_cast<uint2*>(t) =
          make_uint2(__builtin_amdgcn_perm(y[1].x, y[0].x, LO), __builtin_amdgcn_perm(y[3].x, y[2].x, LO));
      *reinterpret_cast<uint2*>(t + BF_TS) =
          make_uint2(__builtin_amdgcn_perm(y[1].x, y[0].x, HI), __builtin_amdgcn_perm(y[3].x, y[2].x, HI));
      *reinterpret_cast<uint2*>(t + 2 * BF_TS) =
          make_uint2(__builtin_amdgcn_perm(y[1].y, y[0].y, LO), __builtin_amdgcn_perm(y[3].y, y[2].y, LO));
      *reinterpret_cast<uint2*>(t + 3 * BF_TS) =
          make_uint2(__builtin_amdgcn_perm(y[1].y, y[0].y, HI), __builtin_amdgcn_perm(y[3].y, y[2].y, HI));
    }
  }
}

// Class of the tile pair (queries [t0, t0 + 64), keys [s0, s0 + 64)) computed by
// one thread (sab_tile_class without the workgroup reduction).
__device__ __forceinline__ int sab_pair_class(const AbParams& P, const int32_t* map_b, int t0, int s0) {
  const int qb0 = t0 / P.block, qb1 = (min(P.T, t0 + AB_T) - 1) / P.block;
  const int kb0 = s0 / P.block, kb1 = (min(P.T, s0 + AB_T) - 1) / P.block;
  if (qb0 == qb1 && kb0 == kb1) return map_b[static_cast<int64_t>(qb0) * P.nb + kb0];
  int live = 0;
  for (int qb = qb0; qb <= qb1; ++qb)
    for (int kb = kb0; kb <= kb1; ++kb) live |= map_b[static_cast<int64_t>(qb) * P.nb + kb] != 0;
  return live ? -1 : 0;
}

// sab_logits in log2 units for the bf16 kernels: x2 = scale log2(e) q.k + log2(w)
// (sl2 = scale log2(e)), -inf where the weight is 0 or the query / key is past
// T.  Tiles of one weight with every query and key inside T take one fma per score.
__device__ __forceinline__ void sab_logits2(const AbParams& P, const int32_t* map_b, int tq, int kg, int t0, int s0,
                                            int tcls, float sl2, f32x4_t (&st)[4]) {
  if (tcls > 0 && (P.mode == FSI_SATTN_BLOCK_LIST || (tcls & 2))) {
    const float lw2 = P.mode == FSI_SATTN_BLOCK_LIST ? __log2f(static_cast<float>(tcls)) : 0.f;
    if (t0 + AB_T <= P.T && s0 + AB_T <= P.T) {
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e) st[t][e] = fmaf(st[t][e], sl2, lw2);
    } else {
      const int lim = tq < P.T ? P.T : 0;
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          st[t][e] = s0 + 16 * t + 4 * kg + e < lim ? fmaf(st[t][e], sl2, lw2) : -INFINITY;
    }
  } else if (tcls > 0) {
    const int hi = tq < P.T ? tq : -1, lo = tq - P.window;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int sk = s0 + 16 * t + 4 * kg + e;
        st[t][e] = sk <= hi && sk > lo ? st[t][e] * sl2 : -INFINITY;
      }
  } else {
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int sk = s0 + 16 * t + 4 * kg + e;
        float x = -INFINITY;
        if (tq < P.T && sk < P.T) {
          const float w = sab_tile_weight(P, map_b, tcls, tq, sk);
          if (w > 0.f) x = fmaf(st[t][e], sl2, __log2f(w));
        }
        st[t][e] = x;
      }
  }
}

// The live tiles among [c0, c0 + 256) of one tile row (ROW: the query tile t0 is
// fixed, key tiles vary) or column (the key tile is fixed), ascending, with their
// classes, compacted into idx / cls; returns their number (every thread).
template <bool ROW>
__device__ __forceinline__ int sab_live_chunk(const AbParams& P, const int32_t* map_b, int fixed0, int c0, int ntiles,
                                              int* idx, int* cls, int* wcount) {
  const int i = c0 + static_cast<int>(threadIdx.x), lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int c = 0;
  if (i < ntiles) c = ROW ? sab_pair_class(P, map_b, fixed0, i * AB_T) : sab_pair_class(P, map_b, i * AB_T, fixed0);
  const uint64_t bal = __ballot(c != 0);
  if (lane == 0) wcount[wave] = __popcll(bal);
  __syncthreads();
  int base = 0, total = 0;
#pragma unroll
  for (int w = 0; w < AB_THREADS / 64; ++w) {
    base += w < wave ? wcount[w] : 0;
    total += wcount[w];
  }
  if (c != 0) {
    const int pos = base + __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(bal >> 32),
                                                     __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(bal), 0));
    idx[pos] = i;
    cls[pos] = c;
  }
  __syncthreads();
  return total;
}

// Row `row` of a row-major tile as the lane's operand of a 32-dim step ks.
template <int HD>
__device__ __forceinline__ u32x4_t bf_row(const bf16_t* rt, int row, int ks, int kg) {
  return *reinterpret_cast<const u32x4_t*>(&rt[row * (HD + 8) + 32 * ks + 8 * kg]);
}
// Row `row` of a transposed tile at the lane's k slots of the 32 columns
// [32 j, 32 j + 32): column groups 8 j + kg and 8 j + 4 + kg, stored swizzled.
__device__ __forceinline__ u32x4_t bf_trow(const bf16_t* tt, int row, int j, int kg) {
  const int sw = kg ^ ((row >> 4) & 3);
  const uint2 a = *reinterpret_cast<const uint2*>(&tt[row * BF_TS + 32 * j + 4 * sw]);
  const uint2 b = *reinterpret_cast<const uint2*>(&tt[row * BF_TS + 32 * j + 16 + 4 * sw]);
  return u32x4_t{a.x, a.y, b.x, b.y};
}

__device__ __forceinline__ uint32_t bf_cvt2(float a, float b) {
  typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2_t;
  const bf16x2_t v = {static_cast<__bf16>(a), static_cast<__bf16>(b)};
  return __builtin_bit_cast(uint32_t, v);
}
// The lane's 8 k-slot values (4 of accumulator a, then 4 of b) as hi + lo bf16 operands.
__device__ __forceinline__ void bf_split8(const f32x4_t& a, const f32x4_t& b, u32x4_t& hi, u32x4_t& lo) {
  float x[8] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const uint32_t h = bf_cvt2(x[2 * w], x[2 * w + 1]);
    hi[w] = h;
    lo[w] = bf_cvt2(x[2 * w] - __uint_as_float(h << 16), x[2 * w + 1] - __uint_as_float(h & 0xffff0000u));
  }
}

// dQ and the row statistics (as sab_q_kernel) with K, V as bf16 tiles, K also
// transposed for dQ^T = K^T dS^T.
template <int HD>
__global__ __launch_bounds__(AB_THREADS, 2) void sab_q_bf_kernel(AbParams P) {
  constexpr int DG = HD / 16, KS32 = HD / 32, RS = HD + 8;
  __shared__ __attribute__((aligned(16))) bf16_t Kr[AB_T * RS], Vr[AB_T * RS], Kt[HD * BF_TS];
  __shared__ int lt_idx[AB_THREADS], lt_cls[AB_THREADS], wcount[AB_THREADS / 64];
  const int ntiles = (P.T + AB_T - 1) / AB_T;
  const int t0 = (ntiles - 1 - static_cast<int>(blockIdx.x / P.Hq)) * AB_T;
  const int b = blockIdx.y, h = blockIdx.x % P.Hq;
  const int g = h / (P.Hq / P.Hkv);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, kg = lane >> 4;
  const int tq = t0 + 16 * wave + r;
  const int tql = tq < P.T ? tq : P.T - 1;
  const bf16_t* q = static_cast<const bf16_t*>(P.q) + b * P.qs_b + h * P.qs_h;
  const bf16_t* o = static_cast<const bf16_t*>(P.o) + b * P.os_b + h * P.os_h;
  const bf16_t* dout = static_cast<const bf16_t*>(P.dout) + b * P.ds_b + h * P.ds_h;
  const bf16_t* k = static_cast<const bf16_t*>(P.k) + b * P.ks_b + g * P.ks_h;
  const bf16_t* v = static_cast<const bf16_t*>(P.v) + b * P.vs_b + g * P.vs_h;
  const int32_t* map_b = P.map + static_cast<int64_t>(b) * P.nb * P.nb;

  u32x4_t qb[KS32], db[KS32];
  sab_row_frag_bf<bf16_t, HD>(q, P.qs_t, tql, P.hd, kg, qb);
  sab_row_frag_bf<bf16_t, HD>(dout, P.ds_t, tql, P.hd, kg, db);
  float dd;  // D = dout . out of query r
  {
    f32x4_t of[DG], df[DG];
    sab_row_frag<bf16_t, HD>(o, P.os_t, tql, P.hd, kg, of);
    sab_row_frag<bf16_t, HD>(dout, P.ds_t, tql, P.hd, kg, df);
    float part = 0.f;
#pragma unroll
    for (int d = 0; d < DG; ++d)
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) part = fmaf(df[d][kk], of[d][kk], part);
    dd = sum_rows4(part);
  }
  auto scores = [&](f32x4_t (&st)[4], const bf16_t* Xr, const u32x4_t (&bb)[KS32]) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      st[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS32; ++ks) st[t] = mfma16x16x32(bf_row<HD>(Xr, 16 * t + r, ks, kg), bb[ks], st[t]);
    }
  };

  // pass 1: row maximum and sum (log2 units) over the live key tiles (listed 256
  // at a time; the next tile's K rows load while this one's scores run)
  const float sl2 = P.scale * 1.4426950408889634f;
  float m = -INFINITY, lpart = 0.f;
  uint2 xk[bf_rounds<HD>()][4], xv[bf_rounds<HD>()][4];
  for (int c0 = 0; c0 < ntiles; c0 += AB_THREADS) {
   const int n = sab_live_chunk<true>(P, map_b, t0, c0, ntiles, lt_idx, lt_cls, wcount);
   if (n > 0) bf_load<HD>(k, P.ks_t, lt_idx[0] * AB_T, P.T, xk);
   for (int li = 0; li < n; ++li) {
    const int s0 = __builtin_amdgcn_readfirstlane(lt_idx[li]) * AB_T;
    const int tcls = __builtin_amdgcn_readfirstlane(lt_cls[li]);
    bf_store<HD, false>(xk, Kr, nullptr);
    __syncthreads();
    if (li + 1 < n) bf_load<HD>(k, P.ks_t, lt_idx[li + 1] * AB_T, P.T, xk);
    f32x4_t st[4];
    scores(st, Kr, qb);
    sab_logits2(P, map_b, tq, kg, t0, s0, tcls, sl2, st);
    float cm = -INFINITY;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int e = 0; e < 4; ++e) cm = fmaxf(cm, st[t][e]);
    cm = max_rows4(cm);
    if (cm > -INFINITY) {
      const float mn = fmaxf(m, cm);
      float add = 0.f;
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e) add += __builtin_amdgcn_exp2f(st[t][e] - mn);
      lpart = (m > -INFINITY ? lpart * __builtin_amdgcn_exp2f(m - mn) : 0.f) + add;
      m = mn;
    }
    __syncthreads();
   }
  }
  const float l = sum_rows4(lpart);
  // log2 of the row's softmax denominator: P = exp2(x2 - lse2); +inf for a row
  // with no key (every P 0, no NaN)
  const float lse2 = l > 0.f ? m + __log2f(l) : INFINITY;

  // pass 2: dQ^T[dim][query] = sum_key K^T[dim][key] dS^T[key][query]
  f32x4_t dqa[DG];
#pragma unroll
  for (int dt = 0; dt < DG; ++dt) dqa[dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  for (int c0 = 0; c0 < ntiles; c0 += AB_THREADS) {
   const int n = sab_live_chunk<true>(P, map_b, t0, c0, ntiles, lt_idx, lt_cls, wcount);
   if (n > 0) {
     bf_load<HD>(k, P.ks_t, lt_idx[0] * AB_T, P.T, xk);
     bf_load<HD>(v, P.vs_t, lt_idx[0] * AB_T, P.T, xv);
   }
   for (int li = 0; li < n; ++li) {
    const int s0 = __builtin_amdgcn_readfirstlane(lt_idx[li]) * AB_T;
    const int tcls = __builtin_amdgcn_readfirstlane(lt_cls[li]);
    bf_store<HD, true>(xk, Kr, Kt);
    bf_store<HD, false>(xv, Vr, nullptr);
    __syncthreads();
    if (li + 1 < n) {
      bf_load<HD>(k, P.ks_t, lt_idx[li + 1] * AB_T, P.T, xk);
      bf_load<HD>(v, P.vs_t, lt_idx[li + 1] * AB_T, P.T, xv);
    }
    f32x4_t st[4], dp[4];
    scores(st, Kr, qb);
    scores(dp, Vr, db);  // dP^T = V dout^T
    sab_logits2(P, map_b, tq, kg, t0, s0, tcls, sl2, st);
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float p = __builtin_amdgcn_exp2f(st[t][e] - lse2);
        st[t][e] = p * (dp[t][e] - dd);  // dS^T
      }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      u32x4_t hi, lo;
      bf_split8(st[2 * j], st[2 * j + 1], hi, lo);
#pragma unroll
      for (int dt = 0; dt < DG; ++dt) {
        const u32x4_t a = bf_trow(Kt, 16 * dt + r, j, kg);
        dqa[dt] = mfma16x16x32(a, hi, dqa[dt]);
        dqa[dt] = mfma16x16x32(a, lo, dqa[dt]);
      }
    }
    __syncthreads();
   }
  }
  const int64_t rowbase = (static_cast<int64_t>(b) * P.Hq + h) * P.T;
  if (tq < P.T) {
#pragma unroll
    for (int dt = 0; dt < DG; ++dt)
#pragma unroll
      for (int e = 0; e < 4; ++e) P.dq[(rowbase + tq) * P.hd + 16 * dt + 4 * kg + e] = dqa[dt][e] * P.scale;
    if (kg == 0) {
      P.stat_m[rowbase + tq] = lse2;  // the bf16 kernels keep log2 units
      P.stat_l[rowbase + tq] = l;
      P.stat_d[rowbase + tq] = dd;
    }
  }
}

// dK and dV (as sab_kv_kernel) with Q and dout as bf16 tiles, both also
// transposed for dK^T = Q^T dS and dV^T = dout^T P.
template <int HD>
__global__ __launch_bounds__(AB_THREADS, 2) void sab_kv_bf_kernel(AbParams P) {
  constexpr int DG = HD / 16, KS32 = HD / 32, RS = HD + 8;
  __shared__ __attribute__((aligned(16))) bf16_t Qr[AB_T * RS], Dr[AB_T * RS], Qt[HD * BF_TS], Dt[HD * BF_TS];
  __shared__ float row_lse[AB_T], row_d[AB_T];  // log2 softmax denominators (+inf past T), D
  __shared__ int lt_idx[AB_THREADS], lt_cls[AB_THREADS], wcount[AB_THREADS / 64];
  const int ntiles = (P.T + AB_T - 1) / AB_T;
  const int s0 = static_cast<int>(blockIdx.x / P.Hkv) * AB_T;
  const float sl2 = P.scale * 1.4426950408889634f;
  const int b = blockIdx.y, g = blockIdx.x % P.Hkv;
  const int G = P.Hq / P.Hkv;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, kg = lane >> 4;
  const int sk = s0 + 16 * wave + r;
  const int skl = sk < P.T ? sk : P.T - 1;
  const bf16_t* k = static_cast<const bf16_t*>(P.k) + b * P.ks_b + g * P.ks_h;
  const bf16_t* v = static_cast<const bf16_t*>(P.v) + b * P.vs_b + g * P.vs_h;
  const int32_t* map_b = P.map + static_cast<int64_t>(b) * P.nb * P.nb;
  u32x4_t kb[KS32], vb[KS32];
  sab_row_frag_bf<bf16_t, HD>(k, P.ks_t, skl, P.hd, kg, kb);
  sab_row_frag_bf<bf16_t, HD>(v, P.vs_t, skl, P.hd, kg, vb);
  f32x4_t dka[DG], dva[DG];
#pragma unroll
  for (int dt = 0; dt < DG; ++dt) dka[dt] = dva[dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // (live query tile, query head of the group) pairs, the tiles listed 256 at a
  // time; the next pair's Q and dout rows and row statistics load while this
  // pair's products run
  uint2 xq[bf_rounds<HD>()][4], xd[bf_rounds<HD>()][4];
  float nlse = INFINITY, nd = 0.f;
  auto load_pair = [&](int li, int hh) {
    const int t0 = __builtin_amdgcn_readfirstlane(lt_idx[li]) * AB_T, h = g * G + hh;
    bf_load<HD>(static_cast<const bf16_t*>(P.q) + b * P.qs_b + h * P.qs_h, P.qs_t, t0, P.T, xq);
    bf_load<HD>(static_cast<const bf16_t*>(P.dout) + b * P.ds_b + h * P.ds_h, P.ds_t, t0, P.T, xd);
    const int64_t rowbase = (static_cast<int64_t>(b) * P.Hq + h) * P.T;
    const int t = t0 + tid;
    if (tid < AB_T && t < P.T) {
      nlse = P.stat_m[rowbase + t];
      nd = P.stat_d[rowbase + t];
    } else {
      nlse = INFINITY;
      nd = 0.f;
    }
  };
  for (int c0 = 0; c0 < ntiles; c0 += AB_THREADS) {
   const int n = sab_live_chunk<false>(P, map_b, s0, c0, ntiles, lt_idx, lt_cls, wcount);
   if (n > 0) load_pair(0, 0);
   for (int it = 0; it < n * G; ++it) {
    const int li = it / G;
    const int t0 = __builtin_amdgcn_readfirstlane(lt_idx[li]) * AB_T;
    const int tcls = __builtin_amdgcn_readfirstlane(lt_cls[li]);
    // one weight for the whole tile (all: log2 weight lw2; inner: every query and
    // key inside T), the window only (win), or per element
    const bool all = tcls > 0 && (P.mode == FSI_SATTN_BLOCK_LIST || (tcls & 2));
    const bool win = tcls > 0 && !all;
    const bool inner = t0 + AB_T <= P.T && s0 + AB_T <= P.T;
    const float lw2 = all && P.mode == FSI_SATTN_BLOCK_LIST ? __log2f(static_cast<float>(tcls)) : 0.f;
    {
      bf_store<HD, true>(xq, Qr, Qt);
      bf_store<HD, true>(xd, Dr, Dt);
      if (tid < AB_T) {
        row_lse[tid] = nlse;
        row_d[tid] = nd;
      }
      __syncthreads();
      if (it + 1 < n * G) load_pair((it + 1) / G, (it + 1) % G);
      // two 16-query sub-tiles at a time (not unrolled: the operand reads of all
      // four would be hoisted past the register budget)
#pragma unroll 1
      for (int j = 0; j < 2; ++j) {
        f32x4_t pp[2], ds[2];  // P, dS [query 32 j + 16 i + 4 kg + e][key r]
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const int qt = 2 * j + i;
          f32x4_t s = f32x4_t{0.f, 0.f, 0.f, 0.f}, dp = s;
#pragma unroll
          for (int ks = 0; ks < KS32; ++ks) {
            s = mfma16x16x32(bf_row<HD>(Qr, 16 * qt + r, ks, kg), kb[ks], s);
            dp = mfma16x16x32(bf_row<HD>(Dr, 16 * qt + r, ks, kg), vb[ks], dp);
          }
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int rq = 16 * qt + 4 * kg + e, t = t0 + rq;
            const float lse = row_lse[rq];  // +inf past T: P = 0
            float p;
            if (all) {
              p = __builtin_amdgcn_exp2f(fmaf(s[e], sl2, lw2 - lse));
              if (!inner) p = sk < P.T ? p : 0.f;
            } else if (win) {
              const float x = __builtin_amdgcn_exp2f(fmaf(s[e], sl2, -lse));
              p = sk <= t && sk > t - P.window ? x : 0.f;
            } else {
              p = 0.f;
              if (t < P.T && sk < P.T) {
                const float w = sab_tile_weight(P, map_b, tcls, t, sk);
                if (w > 0.f) p = __builtin_amdgcn_exp2f(fmaf(s[e], sl2, __log2f(w) - lse));
              }
            }
            pp[i][e] = p;
            ds[i][e] = p * (dp[e] - row_d[rq]);
          }
        }
        // dV^T[dim][key] += dout^T[dim][query] P[query][key], dK^T += Q^T dS
        u32x4_t ph, pl, dh, dl;
        bf_split8(pp[0], pp[1], ph, pl);
        bf_split8(ds[0], ds[1], dh, dl);
#pragma unroll
        for (int dt = 0; dt < DG; ++dt) {
          const u32x4_t ad = bf_trow(Dt, 16 * dt + r, j, kg);
          const u32x4_t aq = bf_trow(Qt, 16 * dt + r, j, kg);
          dva[dt] = mfma16x16x32(ad, ph, dva[dt]);
          dva[dt] = mfma16x16x32(ad, pl, dva[dt]);
          dka[dt] = mfma16x16x32(aq, dh, dka[dt]);
          dka[dt] = mfma16x16x32(aq, dl, dka[dt]);
        }
      }
      __syncthreads();
    }
   }
  }
  const int64_t kbase = (static_cast<int64_t>(b) * P.Hkv + g) * P.T;
  if (sk < P.T) {
#pragma unroll
    for (int dt = 0; dt < DG; ++dt)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int d = 16 * dt + 4 * kg + e;
        P.dk[(kbase + sk) * P.hd + d] = dka[dt][e] * P.scale;
        P.dv[(kbase + sk) * P.hd + d] = dva[dt][e];
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
  FSI_CHECK_ARG(T <= (int64_t(1) << 30) && B <= 65535 && (T + AB_T - 1) / AB_T * Hq <= 0x7fffffff, FSI_ERR_SHAPE,
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
  {
    const int64_t esz = dtype == FSI_DTYPE_F32 ? 4 : 2;
    auto al = [&](const void* p, int64_t sb, int64_t sh, int64_t st) {
      return reinterpret_cast<uintptr_t>(p) % (4 * esz) == 0 && sb % 4 == 0 && sh % 4 == 0 && st % 4 == 0;
    };
    P.vec4 = (head_dim == 16 || head_dim == 32 || head_dim == 64 || head_dim == 128) && al(q, qs_b, qs_h, qs_t) && al(k, ks_b, ks_h, ks_t) && al(v, vs_b, vs_h, vs_t) &&
             al(dout, ds_b, ds_h, ds_t);
  }
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
  const dim3 gq(ntiles * static_cast<unsigned>(Hq), static_cast<unsigned>(B)),
      gkv(ntiles * static_cast<unsigned>(Hkv), static_cast<unsigned>(B));
  auto run = [&](auto hd_tag) {
    constexpr int HD = decltype(hd_tag)::value;
    if (dtype == FSI_DTYPE_F32) {
      sab_q_kernel<float, HD><<<gq, AB_THREADS, 0, st>>>(P);
      sab_kv_kernel<float, HD><<<gkv, AB_THREADS, 0, st>>>(P);
    } else {
      if constexpr (HD >= 32) {
        // the bf16 kernels address a tile's rows with 32-bit offsets: row strides below 2^24
        const bool short_rows = qs_t < (int64_t(1) << 24) && ks_t < (int64_t(1) << 24) &&
                                vs_t < (int64_t(1) << 24) && ds_t < (int64_t(1) << 24);
        if (head_dim == HD && P.vec4 && short_rows) {
          sab_q_bf_kernel<HD><<<gq, AB_THREADS, 0, st>>>(P);
          sab_kv_bf_kernel<HD><<<gkv, AB_THREADS, 0, st>>>(P);
          return;
        }
      }
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
