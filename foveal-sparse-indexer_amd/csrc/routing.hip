// 16-D indexer routing on MI355X (gfx950): adaptive top-p / K_min / K_max
// block selection, fused cosine scoring + selection, and decode-step page
// routing with the additive 16-D stream.
//
// Semantics follow foveal_indexer/core.py:36-160 (masked_softmax,
// select_blocks), core.py:263-265 (cosine / sqrt(d) scoring, computed here in
// fp32 end to end) and foveal_indexer/attention.py:313-337,369-377 (decode_step
// page routing and additive stream).
//
// One wavefront owns one row.  Element j of a row lives in lane j % 64,
// register slot j / 64.  Per row:
//   1. fp32 softmax over the valid entries (max, exp, sum; masked entries 0);
//   2. every candidate gets an order-preserving 32-bit key (prob bits + 1;
//      0 = not a candidate; probabilities are >= 0 so their bit patterns sort
//      like the values);
//   3. the R-th largest key T is found exactly by bisection over key values;
//      keys > T are taken and the rest of the R come from keys == T in
//      ascending index order;
//   4. the R winners are sorted by (prob desc, index asc) with a bitonic network
//      across lanes and register slots;
//   5. their running mass is accumulated sequentially in fp64 and rounded to
//      fp32 per element (ATen's CPU cumsum of fp32 accumulates in double), and
//      the reference's count rule is applied.
// torch.sort leaves the order of equal probabilities unspecified; lower index
// first is used here.  That, and ulp-level exp/sum differences, are the only
// ways a selection can differ from the CPU reference (near-ties).
#include <atomic>

#include "decode_attn_body.h"
#include "fsi_common.h"

using namespace fsi;

namespace {

constexpr int R_MAX = FSI_ROUTE_MAX_RANKED;

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

__device__ __forceinline__ int lanes_below(uint64_t mask) {
  return static_cast<int>(__builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mask >> 32),
                                                    __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask), 0u)));
}

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int m) {
  const uint32_t lo = __shfl_xor(static_cast<uint32_t>(v), m, 64);
  const uint32_t hi = __shfl_xor(static_cast<uint32_t>(v >> 32), m, 64);
  return (static_cast<uint64_t>(hi) << 32) | lo;
}

// Composite sort key: larger probability first, then lower index.
__device__ __forceinline__ uint64_t comp_key(uint32_t key, uint32_t idx) {
  return (static_cast<uint64_t>(key) << 32) | (0xffffffffu - idx);
}
__device__ __forceinline__ int32_t comp_index(uint64_t c) {
  return static_cast<int32_t>(0xffffffffu - static_cast<uint32_t>(c));
}
__device__ __forceinline__ float comp_prob(uint64_t c) {
  return __uint_as_float(static_cast<uint32_t>(c >> 32) - 1u);
}

// Bitonic sort (descending) of 64 * E composite keys; element k lives in lane
// k % 64, slot k / 64.
template <int E>
__device__ __forceinline__ void bitonic_desc(uint64_t (&v)[E]) {
  constexpr int n = 64 * E;
  const int lane = lane_id();
#pragma unroll
  for (int s = 2; s <= n; s <<= 1) {
#pragma unroll
    for (int j = s >> 1; j > 0; j >>= 1) {
      uint64_t nv[E];
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const int k = e * 64 + lane;
        const int p = k ^ j;
        const uint64_t other = j < 64 ? shfl_xor_u64(v[e], j) : v[(e * 64 ^ j) >> 6];
        const bool want_max = (k < p) == ((k & s) == 0);
        const uint64_t mx = v[e] > other ? v[e] : other;
        const uint64_t mn = v[e] > other ? other : v[e];
        nv[e] = want_max ? mx : mn;
      }
#pragma unroll
      for (int e = 0; e < E; ++e) v[e] = nv[e];
    }
  }
}

// Sum of an int over the wave with VALU operations only: DPP steps inside each
// row of 16 lanes (quad xor 1, quad xor 2, half-row mirror, row mirror), then
// gfx950's permlane16 / permlane32 swaps across the four rows.  Every lane
// receives the total.
__device__ __forceinline__ int wave_sum_dpp(int x) {
  x += __builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, false);
  x += __builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, false);
  x += __builtin_amdgcn_mov_dpp(x, 0x141, 0xF, 0xF, false);
  x += __builtin_amdgcn_mov_dpp(x, 0x140, 0xF, 0xF, false);
  const auto a = __builtin_amdgcn_permlane16_swap(static_cast<uint32_t>(x), static_cast<uint32_t>(x), false, false);
  x = static_cast<int>(a[0]) + static_cast<int>(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(static_cast<uint32_t>(x), static_cast<uint32_t>(x), false, false);
  return static_cast<int>(b[0]) + static_cast<int>(b[1]);
}

// Number of keys >= t in the row: a per-lane compare-and-add over the register
// slots, then one wave sum.  (A ballot + scalar popcount per slot chains every
// compare to a scalar instruction; this form measured 1.2x faster at 32 slots
// and 1.8x at 64 on gfx950.)
template <int PL>
__device__ __forceinline__ int count_ge(const uint32_t (&key)[PL], uint32_t t) {
  int c = 0;
#pragma unroll
  for (int i = 0; i < PL; ++i) c += key[i] >= t ? 1 : 0;
  return __builtin_amdgcn_readfirstlane(wave_sum_dpp(c));
}

// Threshold of the R largest keys of the wave (R > 0; keys 0 are never counted):
// T = the R-th largest key (or 1 when fewer than R keys are non-zero) and
// clo = the number of keys >= T, found by bisection on scalars.
template <int PL>
__device__ __forceinline__ void top_threshold(const uint32_t (&key)[PL], int R, uint32_t& T, int& clo) {
  uint32_t mx = 0;
#pragma unroll
  for (int i = 0; i < PL; ++i) mx = key[i] > mx ? key[i] : mx;
  uint32_t mn = mx;  // smallest lane maximum: every lane holds a key >= it, so >= 64 keys do
  for (int off = 32; off > 0; off >>= 1) {
    const uint32_t o = __shfl_xor(mx, off, 64), p = __shfl_xor(mn, off, 64);
    mx = o > mx ? o : mx;
    mn = p < mn ? p : mn;
  }
  mx = __builtin_amdgcn_readfirstlane(mx);  // uniform: the bisection runs on scalars
  mn = __builtin_amdgcn_readfirstlane(mn);
  // Invariant: count_ge(lo) >= R > count_ge(hi) (or lo = 1 with fewer keys).  For
  // R <= 64 the search starts at the smallest lane maximum.
  uint32_t lo = R <= 64 && mn > 0 ? mn : 1, hi = mx + 1;
  clo = count_ge<PL>(key, lo);
  while (clo != R && hi - lo > 1) {
    const uint32_t mid = lo + (hi - lo) / 2;
    const int c = count_ge<PL>(key, mid);
    if (c >= R) {
      lo = mid;
      clo = c;
    } else {
      hi = mid;
    }
  }
  T = lo;
}

// The R largest keys by (key desc, slot asc), compacted in slot order (slot i of
// lane l is element 64 i + l) into lds_k[0..n) with index idx(i) in lds_i;
// returns n = min(R, #non-zero keys).  When clo == R every key >= T is taken;
// otherwise the keys > T, then keys == T in slot order.
template <int PL, class IdxFn>
__device__ __forceinline__ int take_top(const uint32_t (&key)[PL], int R, uint32_t T, int clo, uint32_t* lds_k,
                                        uint32_t* lds_i, IdxFn idx) {
  const uint32_t strict = clo == R ? T : T + 1;
  int base = 0;
#pragma unroll
  for (int i = 0; i < PL; ++i) {
    const bool take = key[i] >= strict;
    const uint64_t b = __ballot(take);
    if (take) {
      const int pos = base + lanes_below(b);
      lds_k[pos] = key[i];
      lds_i[pos] = idx(i);
    }
    base += __popcll(b);
  }
  if (base < R) {
#pragma unroll
    for (int i = 0; i < PL; ++i) {
      const bool eq = key[i] == T;
      const uint64_t b = __ballot(eq);
      const int pos = base + lanes_below(b);
      if (eq && pos < R) {
        lds_k[pos] = key[i];
        lds_i[pos] = idx(i);
      }
      base += __popcll(b);
    }
  }
  return base < R ? base : R;
}

// Composite keys of lds_k / lds_i[0..R), sorted descending into out[] (element k
// at lane k % 64, slot k / 64); entries k >= R hold 0.
template <int E>
__device__ __forceinline__ void sort_taken(int R, uint64_t (&out)[E], const uint32_t* lds_k, const uint32_t* lds_i) {
  const int lane = lane_id();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int k = e * 64 + lane;
    out[e] = k < R ? comp_key(lds_k[k], lds_i[k]) : 0;
  }
  bitonic_desc<E>(out);
}

// The R largest keys (0 < R <= min(64 E, #candidates)), sorted descending into
// out[] (element k at lane k % 64, slot k / 64); entries k >= R hold 0.
// lds_k / lds_i: this wave's 64 E words each.
template <int PL, int E>
__device__ void rank_top(const uint32_t (&key)[PL], int R, uint64_t (&out)[E], uint32_t* lds_k, uint32_t* lds_i) {
  const int lane = lane_id();
#pragma unroll
  for (int e = 0; e < E; ++e) out[e] = 0;
  if (R <= 0) return;
  uint32_t T;
  int clo;
  top_threshold<PL>(key, R, T, clo);
  take_top<PL>(key, R, T, clo, lds_k, lds_i, [&](int i) { return static_cast<uint32_t>(i * 64 + lane); });
  sort_taken<E>(R, out, lds_k, lds_i);
}

// Running mass of the sorted probabilities for k < n; 0 elsewhere.
//   fp32 rows: cum[k] = fp32(sum_{i<=k} p_i accumulated in fp64) (ATen CPU
//              cumsum of float accumulates in double);
//   bf16 rows: cum[k] = bf16(sum_{i<=k} p_i accumulated in fp32) (its
//              accumulator for bfloat16 is float).
template <int E, bool RB>
__device__ __forceinline__ void running_mass(const uint64_t (&sorted)[E], int n, float (&cum)[E]) {
  const int lane = lane_id();
  double acc = 0.0;
  float accf = 0.f;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const float p = comp_prob(sorted[e]);
    cum[e] = 0.f;
    const int m = n - e * 64 < 64 ? n - e * 64 : 64;
    for (int l = 0; l < m; ++l) {
      const float pl = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p), l));
      float c;
      if (RB) {
        accf += pl;
        c = round_bf16(accf);
      } else {
        acc += static_cast<double>(pl);
        c = static_cast<float>(acc);
      }
      if (lane == l) cum[e] = c;
    }
  }
}

// First k < n with cum[k] >= target, or n if there is none.
template <int E>
__device__ __forceinline__ int first_reaching(const float (&cum)[E], int n, float target) {
  const int lane = lane_id();
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const uint64_t b = __ballot(e * 64 + lane < n && cum[e] >= target);
    if (b) return e * 64 + __ffsll(static_cast<long long>(b)) - 1;
  }
  return n;
}

// Value of a per-lane register array at element k (uniform k).
template <int E>
__device__ __forceinline__ float element_at(const float (&v)[E], int k) {
  float r = 0.f;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const float x = __shfl(v[e], k & 63, 64);
    if ((k >> 6) == e) r = x;
  }
  return r;
}

// Row masks of select_blocks (core.py:79-99): 0 = not complete, 1 = local, 2 = remote.
__device__ __forceinline__ int mask_kind(int p, int qb, int causal, int lw) {
  if (causal) {
    if (p >= qb) return 0;
    if (lw > 0) return p >= (qb - lw > 0 ? qb - lw : 0) ? 1 : 2;
    return 2;
  }
  if (lw > 0) return p < lw ? 1 : 2;
  return 2;
}

struct SelectParams {
  int causal, local_window, capacity;
  float top_p;
  int k_min, k_max;
  const float* top_p_rows;  // optional per-row values (B * Qb)
  const int32_t* k_min_rows;
  const int32_t* k_max_rows;
};

// select_blocks for one row whose scores (upcast to fp32) are s[] (slot
// layout).  RB: the scores tensor is bf16, so masked_softmax returns bf16
// probabilities and local mass, cumulative mass and target are bf16 values
// (core.py:43,103,111 evaluated in bfloat16).  Writes indices[capacity], count
// and (optionally) mass = local mass + cum[count-1].
template <int PL, int E, bool RB>
__device__ void select_row(float (&s)[PL], int N, int qb, int64_t row, const SelectParams& sp,
                           int32_t* __restrict__ out_idx, int32_t* __restrict__ out_cnt,
                           float* __restrict__ out_mass, uint32_t* lds_k, uint32_t* lds_i) {
  const int lane = lane_id();
  const float top_p = sp.top_p_rows ? sp.top_p_rows[row] : sp.top_p;
  const int k_min = sp.k_min_rows ? sp.k_min_rows[row] : sp.k_min;
  const int k_max = sp.k_max_rows ? sp.k_max_rows[row] : sp.k_max;

  // masked_softmax over complete entries (core.py:36-43).  A non-causal row with
  // no local window over N >= 64 PL keys has every slot complete and remote: it
  // takes passes without per-slot masks (kept live across the three passes, 64
  // lane masks overflow the scalar registers).
  float lmass = 0.f;
  int avail = 0;
  uint32_t key[PL];
  if (!sp.causal && sp.local_window == 0 && N >= 64 * PL) {  // uniform
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < PL; ++i) mx = fmaxf(mx, s[i]);
    mx = wave_max(mx);
    if (!isfinite(mx)) mx = 0.0f;
    float z = 0.f;
#pragma unroll
    for (int i = 0; i < PL; ++i) {
      s[i] = expf(s[i] - mx);
      z += s[i];
    }
    z = fmaxf(wave_sum(z), 1e-20f);
#pragma unroll
    for (int i = 0; i < PL; ++i) {
      float p = s[i] / z;
      if (RB) p = round_bf16(p);
      key[i] = __float_as_uint(p) + 1u;
    }
    avail = 64 * PL;
  } else {
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < PL; ++i) {
      const int j = i * 64 + lane;
      if (j < N && mask_kind(j, qb, sp.causal, sp.local_window)) mx = fmaxf(mx, s[i]);
    }
    mx = wave_max(mx);
    if (!isfinite(mx)) mx = 0.0f;
    float z = 0.f;
#pragma unroll
    for (int i = 0; i < PL; ++i) {
      const int j = i * 64 + lane;
      s[i] = j < N && mask_kind(j, qb, sp.causal, sp.local_window) ? expf(s[i] - mx) : 0.0f;
      z += s[i];
    }
    z = fmaxf(wave_sum(z), 1e-20f);
#pragma unroll
    for (int i = 0; i < PL; ++i) {
      const int j = i * 64 + lane;
      const int kind = j < N ? mask_kind(j, qb, sp.causal, sp.local_window) : 0;
      float p = s[i] / z;
      if (RB) p = round_bf16(p);
      if (kind == 1) lmass += p;
      key[i] = kind == 2 ? __float_as_uint(p) + 1u : 0u;
      avail += kind == 2;
    }
    lmass = wave_sum(lmass);
    if (RB) lmass = round_bf16(lmass);
    avail = wave_sum_i(avail);
  }

  int R = k_max > sp.capacity ? k_max : sp.capacity;
  R = R < avail ? R : avail;
  R = R < 64 * E ? R : 64 * E;  // the host guarantees this does not truncate
  uint64_t sorted[E];
  rank_top<PL, E>(key, R, sorted, lds_k, lds_i);

  // counts (core.py:107-119)
  const float target = RB ? fmaxf(round_bf16(round_bf16(top_p) - lmass), 0.0f) : fmaxf(top_p - lmass, 0.0f);
  int nr = k_max < avail ? k_max : avail;  // cum is only consulted below this rank
  nr = nr < 0 ? 0 : nr;
  nr = nr < R ? nr : R;
  float cum[E];
  running_mass<E, RB>(sorted, nr, cum);
  int count;
  if (avail <= 0) {
    count = 0;
  } else {
    // needed = #(cum < target) + (target > 0); any value past nr caps to min(avail, K_max)
    const int first = first_reaching<E>(cum, nr, target);
    int needed = first >= nr ? 0x7fffffff : first + (target > 0.0f ? 1 : 0);
    needed = needed > k_min ? needed : k_min;
    count = needed < avail ? needed : avail;
  }
  count = count < k_max ? count : k_max;

  // indices: ranked candidates, then the other entries in index order, then
  // zero padding past N (sorted_idx[..., :capacity] padded, core.py:121-123).
  int32_t* idx = out_idx + row * sp.capacity;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int k = e * 64 + lane;
    if (k < R && k < sp.capacity) idx[k] = comp_index(sorted[e]);
  }
  if (sp.capacity > R) {
    // R == avail here: the non-remote entries (ranked -1) follow, lowest index first
    int base = R;
#pragma unroll
    for (int i = 0; i < PL; ++i) {
      const int j = i * 64 + lane;
      const bool other = j < N && mask_kind(j, qb, sp.causal, sp.local_window) != 2;
      const uint64_t b = __ballot(other);
      const int pos = base + lanes_below(b);
      if (other && pos < sp.capacity) idx[pos] = j;
      base += __popcll(b);
    }
    for (int k = N + lane; k < sp.capacity; k += 64) idx[k] = 0;
  }
  const float ck = count > 0 ? element_at<E>(cum, count - 1) : 0.f;
  if (lane == 0) {
    out_cnt[row] = count;
    if (out_mass) out_mass[row] = count > 0 ? (RB ? round_bf16(lmass + ck) : lmass + ck) : lmass;
  }
}

// ---------------------------------------------------------------------------
// select_blocks on materialised scores (B, Qb, Nb): one wave per row.
// ---------------------------------------------------------------------------
constexpr int RS_WAVES = 4;

template <int PL, int E, bool BF16>
__global__ __launch_bounds__(64 * RS_WAVES) void route_scores_kernel(const void* __restrict__ scores,
                                                                     int64_t n_rows, int Qb, int N,
                                                                     SelectParams sp,
                                                                     int32_t* __restrict__ out_idx,
                                                                     int32_t* __restrict__ out_cnt,
                                                                     float* __restrict__ out_mass) {
  __shared__ uint32_t lk[RS_WAVES][64 * E], li[RS_WAVES][64 * E];
  const int wave = threadIdx.x >> 6, lane = lane_id();
  const int64_t row = static_cast<int64_t>(blockIdx.x) * RS_WAVES + wave;
  if (row >= n_rows) return;  // whole wave leaves; no workgroup barrier follows
  float s[PL];
#pragma unroll
  for (int i = 0; i < PL; ++i) {
    const int j = i * 64 + lane;
    if (BF16) s[i] = j < N ? bf16_to_f32(static_cast<const bf16_t*>(scores)[row * N + j]) : 0.f;
    else s[i] = j < N ? static_cast<const float*>(scores)[row * N + j] : 0.f;
  }
  select_row<PL, E, BF16>(s, N, static_cast<int>(row % Qb), row, sp, out_idx, out_cnt, out_mass, lk[wave],
                          li[wave]);
}

// ---------------------------------------------------------------------------
// Fused fp32 cosine scoring + select_blocks (the indexer routing workload).
// One query row per wave, SR_WAVES rows per workgroup.  Keys are staged through
// LDS in chunks of SR_CHUNK: the workgroup L2-normalises the chunk into
// component-major float4 planes, then every wave scores its row against the
// chunk, each lane taking the keys of its own register slots.  The query is
// normalised once and held in scalar registers.
// q: (B, Q, 16), k: (N, 16) per batch entry at b * k_batch_stride elements.
// ---------------------------------------------------------------------------
constexpr int SR_WAVES = 8;
constexpr int SR_CHUNK = 1024;
constexpr int SR_D = 16;

template <int PL, int E, bool BF16>
__global__ __launch_bounds__(64 * SR_WAVES) void score_route_kernel(const void* __restrict__ q,
                                                                    const void* __restrict__ k, int Q, int N,
                                                                    int64_t k_batch_stride, float sqrt_d,
                                                                    SelectParams sp,
                                                                    int32_t* __restrict__ out_idx,
                                                                    int32_t* __restrict__ out_cnt,
                                                                    float* __restrict__ out_mass) {
  __shared__ float4 kn[SR_D / 4][SR_CHUNK];
  __shared__ float qn[SR_WAVES][SR_D];
  __shared__ uint32_t lk[SR_WAVES][64 * E], li[SR_WAVES][64 * E];
  const int wave = threadIdx.x >> 6, lane = lane_id();
  const int b = blockIdx.y;
  const int row_q = blockIdx.x * SR_WAVES + wave;

  // query: x / max(||x||, 1e-12) in fp32 (F.normalize)
  if (lane == 0) {
    float v[SR_D];
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < SR_D; ++c) {
      float x = 0.f;
      if (row_q < Q) {
        const int64_t off = (static_cast<int64_t>(b) * Q + row_q) * SR_D + c;
        x = BF16 ? bf16_to_f32(static_cast<const bf16_t*>(q)[off]) : static_cast<const float*>(q)[off];
      }
      v[c] = x;
      ss = fmaf(x, x, ss);
    }
    const float nrm = fmaxf(sqrtf(ss), 1e-12f);
#pragma unroll
    for (int c = 0; c < SR_D; ++c) qn[wave][c] = v[c] / nrm;
  }
  __syncthreads();
  float qa[SR_D];
#pragma unroll
  for (int c = 0; c < SR_D; ++c) qa[c] = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(qn[wave][c])));

  float sa[PL];
#pragma unroll
  for (int i = 0; i < PL; ++i) sa[i] = 0.f;
  const char* kb = static_cast<const char*>(k) + static_cast<int64_t>(b) * k_batch_stride * (BF16 ? 2 : 4);
  constexpr int SLOTS_PER_CHUNK = SR_CHUNK / 64;
#pragma unroll
  for (int ch = 0; ch < (PL + SLOTS_PER_CHUNK - 1) / SLOTS_PER_CHUNK; ++ch) {
    if (ch * SR_CHUNK >= N) break;  // uniform
    __syncthreads();                // previous chunk fully consumed
    for (int t = threadIdx.x; t < SR_CHUNK; t += 64 * SR_WAVES) {
      const int j = ch * SR_CHUNK + t;
      float v[SR_D];
      float ss = 0.f;
      if (j < N) {
        if (BF16) {
          const u32x4_t* src = reinterpret_cast<const u32x4_t*>(reinterpret_cast<const bf16_t*>(kb) +
                                                                 static_cast<int64_t>(j) * SR_D);
          const u32x4_t a = src[0], c2 = src[1];
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            v[2 * w] = lo_bf16(a[w]);
            v[2 * w + 1] = hi_bf16(a[w]);
            v[8 + 2 * w] = lo_bf16(c2[w]);
            v[8 + 2 * w + 1] = hi_bf16(c2[w]);
          }
        } else {
          const float4* src = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(kb) +
                                                              static_cast<int64_t>(j) * SR_D);
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            const float4 f = src[w];
            v[4 * w] = f.x;
            v[4 * w + 1] = f.y;
            v[4 * w + 2] = f.z;
            v[4 * w + 3] = f.w;
          }
        }
#pragma unroll
        for (int c = 0; c < SR_D; ++c) ss = fmaf(v[c], v[c], ss);
      } else {
#pragma unroll
        for (int c = 0; c < SR_D; ++c) v[c] = 0.f;
      }
      const float nrm = fmaxf(sqrtf(ss), 1e-12f);
#pragma unroll
      for (int w = 0; w < 4; ++w)
        kn[w][t] = make_float4(v[4 * w] / nrm, v[4 * w + 1] / nrm, v[4 * w + 2] / nrm, v[4 * w + 3] / nrm);
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < SLOTS_PER_CHUNK; ++i) {
      const int slot = ch * SLOTS_PER_CHUNK + i;
      if (slot < PL) {
        float acc = 0.f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const float4 f = kn[w][i * 64 + lane];
          acc = fmaf(qa[4 * w], f.x, acc);
          acc = fmaf(qa[4 * w + 1], f.y, acc);
          acc = fmaf(qa[4 * w + 2], f.z, acc);
          acc = fmaf(qa[4 * w + 3], f.w, acc);
        }
        sa[slot] = acc;
      }
    }
  }
  // / sqrt(d): a multiply by the exact reciprocal when sqrt(d) is a power of two
  // (the same rounding as the division), the division otherwise
  if ((__float_as_uint(sqrt_d) & 0x007fffffu) == 0u) {  // uniform
    const float inv = 1.f / sqrt_d;
#pragma unroll
    for (int i = 0; i < PL; ++i) sa[i] *= inv;
  } else {
#pragma unroll
    for (int i = 0; i < PL; ++i) sa[i] /= sqrt_d;
  }
  if (row_q < Q)
    select_row<PL, E, false>(sa, N, row_q, static_cast<int64_t>(b) * Q + row_q, sp, out_idx, out_cnt, out_mass, lk[wave],
                      li[wave]);
}

// ---------------------------------------------------------------------------
// decode_step page routing (attention.py:313-337) and additive-stream context
// (attention.py:369-376), one 4-wave workgroup per sequence.
//   qi: (B, d) 16-D query (dtype), kp: (B, P, d) fp32 page keys,
//   vp: (B, P, d) page values (dtype); pages [0, completed) are complete.
// Every thread scores pages t, t + 1024, ... into LDS; the context is the
// softmax over all completed pages (probabilities cast to vp's dtype)
// contracted with vp; routing runs when completed > flp > 0 (flp = first local
// page) over pages [0, flp): count = max(K_min, min(#(cum < top_p) + 1,
// min(K_max, flp))), at most flp.  The top candidates are selected in two
// stages (every wave over its slice, then wave 0 over their candidates) and
// sorted by wave 0.
// ---------------------------------------------------------------------------
constexpr int DR_THREADS = 256;
constexpr int DR_WAVES = DR_THREADS / 64;

// Barrier among the DR_THREADS threads that route: the workgroup barrier when
// the workgroup is exactly those threads (decode_route_kernel), an LDS counter
// among waves [0, DR_WAVES) when other waves of the workgroup run other work
// (decode_step_fused_kernel).
struct DrWgBarrier {
  __device__ __forceinline__ void operator()() const { __syncthreads(); }
};
struct DrSubBarrier {
  int* ctr;    // LDS, zero before the first use
  int target;  // arrivals this wave has waited for so far
  int* err;
  __device__ __forceinline__ void operator()() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    if (lane_id() == 0) __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    target += DR_WAVES;
    // bounded: every routing wave arrives; the bound only guarantees an exit
    for (int spins = 0; __hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < target; ++spins) {
      if (spins >= (1 << 22)) {
        if (err) set_error(err, FSI_ERR_HIP);
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  }
};

template <class Bar>
__device__ __forceinline__ float dr_block_max(float v, float* red, Bar& bar) {
  const int wave = threadIdx.x >> 6, lane = lane_id();
  v = wave_max(v);
  bar();
  if (lane == 0) red[wave] = v;
  bar();
  float r = red[0];
#pragma unroll
  for (int w = 1; w < DR_WAVES; ++w) r = fmaxf(r, red[w]);
  return r;
}

template <class Bar>
__device__ __forceinline__ float dr_block_sum(float v, float* red, Bar& bar) {
  const int wave = threadIdx.x >> 6, lane = lane_id();
  v = wave_sum(v);
  bar();
  if (lane == 0) red[wave] = v;
  bar();
  float r = red[0];
#pragma unroll
  for (int w = 1; w < DR_WAVES; ++w) r += red[w];
  return r;
}

// Wave sums of 16 per-lane values, scattered over the lanes: lane l returns the
// sum over the wave of v[which], and the four lanes of each quad share one
// `which`.  Cross-lane steps are VALU permutes (permlane32 / permlane16 swaps,
// then DPP row mirrors and quad permutes), each halving the values a lane
// carries: 17 exchanges in all instead of 16 butterfly sums of 6 LDS permutes.
// The channel each lane ends up with is found by passing labels through the
// same swaps.
__device__ __forceinline__ float dpp_f(float x, int ctrl) {
  switch (ctrl) {  // the DPP control must be a compile-time constant
    case 0x140: return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x140, 0xF, 0xF, false));
    case 0x141: return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x141, 0xF, 0xF, false));
    case 0xB1: return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0xB1, 0xF, 0xF, false));
    default: return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x4E, 0xF, 0xF, false));
  }
}
__device__ __forceinline__ float dr_wave_sum16_scatter(const float (&v)[16], int& which) {
  const int lane = lane_id();
  // lanes l and l ^ 32: value c stays in one half, c + 8 in the other
  float a[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[c]), __float_as_uint(v[c + 8]), false, false);
    a[c] = __uint_as_float(s[0]) + __uint_as_float(s[1]);
  }
  const int l32 = static_cast<int>(__builtin_amdgcn_permlane32_swap(0u, 8u, false, false)[0]);
  // lanes l and l ^ 16: c and c + 4
  float b[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(a[c]), __float_as_uint(a[c + 4]), false, false);
    b[c] = __uint_as_float(s[0]) + __uint_as_float(s[1]);
  }
  const int l16 = static_cast<int>(__builtin_amdgcn_permlane16_swap(0u, 4u, false, false)[0]);
  // row mirror (i <-> 15 - i): lanes with bit 3 set keep c + 2
  const bool up8 = (lane & 8) != 0;
  float d[2];
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const float keep = up8 ? b[c + 2] : b[c];
    const float give = up8 ? b[c] : b[c + 2];
    d[c] = keep + dpp_f(give, 0x140);
  }
  // half-row mirror (i <-> 7 - i): lanes with bit 2 set keep c + 1
  const bool up4 = (lane & 4) != 0;
  float e = (up4 ? d[1] : d[0]) + dpp_f(up4 ? d[0] : d[1], 0x141);
  // the four lanes of a quad hold parts of the same value
  e += dpp_f(e, 0xB1);
  e += dpp_f(e, 0x4E);
  which = l32 + l16 + (up8 ? 2 : 0) + (up4 ? 1 : 0);
  return e;
}

struct RouteArgs {
  const void* qi;
  const float* kp;
  const void* vp;
  const int32_t* pos_rows;
  int32_t* out_pages;
  int32_t* out_cnt;
  void* out_ctx;
  int B, P, pos, page, window, completed, k_min, k_max, cap;
  float top_p, sqrt_d;
};

// Loads of decode_route_block for sequence b, issued together so the routing
// pays one memory latency: the 16-D query and, for pages t + DR_THREADS i of
// thread t, the page keys and (for the context) the page values.
template <int PL>
struct RouteRegs {
  static constexpr int NPT = (64 * PL + DR_THREADS - 1) / DR_THREADS;
  float qv[SR_D];
  float4 kreg[NPT][4];
  u32x4_t vreg[NPT][2];
};

template <int PL, bool BF16>
__device__ __forceinline__ void decode_route_loads(const RouteArgs& A, int b, RouteRegs<PL>& rr) {
  constexpr int NPT = RouteRegs<PL>::NPT;
#pragma unroll
  for (int c = 0; c < SR_D; ++c) {
    const int64_t off = static_cast<int64_t>(b) * SR_D + c;
    rr.qv[c] = BF16 ? bf16_to_f32(static_cast<const bf16_t*>(A.qi)[off]) : static_cast<const float*>(A.qi)[off];
  }
#pragma unroll
  for (int i = 0; i < NPT; ++i) {
    const int j = threadIdx.x + DR_THREADS * i;
    const int jj = j < A.completed ? j : 0;
    const float4* kr = reinterpret_cast<const float4*>(A.kp + (static_cast<int64_t>(b) * A.P + jj) * SR_D);
#pragma unroll
    for (int w = 0; w < 4; ++w) rr.kreg[i][w] = kr[w];
    if (BF16 && A.out_ctx) {
      const u32x4_t* vr = reinterpret_cast<const u32x4_t*>(static_cast<const bf16_t*>(A.vp) +
                                                           (static_cast<int64_t>(b) * A.P + jj) * SR_D);
      rr.vreg[i][0] = vr[0];
      rr.vreg[i][1] = vr[1];
    }
  }
}

// Routing of sequence b by one DR_THREADS workgroup from the loads in rr.
// write_out: write the pages and counts (and, when A.out_ctx is set, the
// context); pg_lds / cnt_lds (optional): wave 0 also leaves the page list
// (64 E entries, -1 past the count) and the count in LDS.
template <int PL, int E, bool BF16, class Bar>
__device__ __forceinline__ void decode_route_compute(const RouteArgs& A, int b, RouteRegs<PL>& rr, bool write_out,
                                                     int32_t* pg_lds, int* cnt_lds, Bar& bar) {
  const float* __restrict__ kp = A.kp;
  const void* __restrict__ vp = A.vp;
  const int32_t* __restrict__ pos_rows = A.pos_rows;
  int32_t* __restrict__ out_pages = A.out_pages;
  int32_t* __restrict__ out_cnt = A.out_cnt;
  void* __restrict__ out_ctx = A.out_ctx;
  const int P = A.P, pos = A.pos, page = A.page, window = A.window, completed = A.completed;
  const int k_min = A.k_min, k_max = A.k_max, cap = A.cap;
  const float top_p = A.top_p, sqrt_d = A.sqrt_d;
  __shared__ float sc[64 * PL];
  __shared__ float red[DR_WAVES];
  __shared__ float ctx_part[DR_WAVES][SR_D];
  __shared__ uint32_t lk[64 * E], li[64 * E];
  const int lane = lane_id(), wave = threadIdx.x >> 6;
  const int mypos = pos_rows ? pos_rows[b] : pos;
  const int local_start = mypos + 1 - window > 0 ? mypos + 1 - window : 0;
  const int flp = local_start / page;
  (void)kp;
  (void)vp;
  (void)P;

  float qv[SR_D];
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < SR_D; ++c) {
    qv[c] = rr.qv[c];
    ss = fmaf(qv[c], qv[c], ss);
  }
  const float nrm = fmaxf(sqrtf(ss), 1e-12f);
#pragma unroll
  for (int c = 0; c < SR_D; ++c) qv[c] = qv[c] / nrm;

  constexpr int NPT = RouteRegs<PL>::NPT;
#pragma unroll
  for (int i = 0; i < NPT; ++i) {
    const int j = threadIdx.x + DR_THREADS * i;
    if (j >= completed) continue;
    float acc = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float4 f = rr.kreg[i][w];
      acc = fmaf(qv[4 * w], f.x, acc);
      acc = fmaf(qv[4 * w + 1], f.y, acc);
      acc = fmaf(qv[4 * w + 2], f.z, acc);
      acc = fmaf(qv[4 * w + 3], f.w, acc);
    }
    sc[j] = acc / sqrt_d;
  }
  bar();

  if (out_ctx && write_out) {  // uniform across the workgroup
    float ctx = 0.f;
    if (completed > 0) {
      float mx = -INFINITY;
      for (int j = threadIdx.x; j < completed; j += DR_THREADS) mx = fmaxf(mx, sc[j]);
      mx = dr_block_max(mx, red, bar);
      float z = 0.f;
      for (int j = threadIdx.x; j < completed; j += DR_THREADS) z += expf(sc[j] - mx);
      z = dr_block_sum(z, red, bar);
      float part[SR_D];
#pragma unroll
      for (int c = 0; c < SR_D; ++c) part[c] = 0.f;
#pragma unroll
      for (int i = 0; i < NPT; ++i) {
        const int j = threadIdx.x + DR_THREADS * i;
        if (j >= completed) continue;
        float pj = expf(sc[j] - mx) / z;
        if (BF16) {
          pj = round_bf16(pj);
          const u32x4_t a = rr.vreg[i][0], c2 = rr.vreg[i][1];
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            part[2 * w] = fmaf(pj, lo_bf16(a[w]), part[2 * w]);
            part[2 * w + 1] = fmaf(pj, hi_bf16(a[w]), part[2 * w + 1]);
            part[8 + 2 * w] = fmaf(pj, lo_bf16(c2[w]), part[8 + 2 * w]);
            part[9 + 2 * w] = fmaf(pj, hi_bf16(c2[w]), part[9 + 2 * w]);
          }
        } else {
          const int64_t off = (static_cast<int64_t>(b) * P + j) * SR_D;
          const float4* vr = reinterpret_cast<const float4*>(static_cast<const float*>(vp) + off);
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            const float4 f = vr[w];
            part[4 * w] = fmaf(pj, f.x, part[4 * w]);
            part[4 * w + 1] = fmaf(pj, f.y, part[4 * w + 1]);
            part[4 * w + 2] = fmaf(pj, f.z, part[4 * w + 2]);
            part[4 * w + 3] = fmaf(pj, f.w, part[4 * w + 3]);
          }
        }
      }
      int which;
      const float t = dr_wave_sum16_scatter(part, which);
      if ((lane & 3) == 0) ctx_part[wave][which] = t;
      bar();
      if (threadIdx.x < SR_D) {
#pragma unroll
        for (int w = 0; w < DR_WAVES; ++w) ctx += ctx_part[w][threadIdx.x];
      }
    }
    if (threadIdx.x < SR_D) {
      const int64_t off = static_cast<int64_t>(b) * SR_D + threadIdx.x;
      if (BF16) static_cast<bf16_t*>(out_ctx)[off] = f32_to_bf16(ctx);
      else static_cast<float*>(out_ctx)[off] = ctx;
    }
  }

  const bool route = completed > flp && flp > 0;
  float z = 1.f, mx = 0.f;
  if (route) {  // uniform
    float m = -INFINITY;
    for (int j = threadIdx.x; j < flp; j += DR_THREADS) m = fmaxf(m, sc[j]);
    mx = dr_block_max(m, red, bar);
    float zz = 0.f;
    for (int j = threadIdx.x; j < flp; j += DR_THREADS) zz += expf(sc[j] - mx);
    z = dr_block_sum(zz, red, bar);
  }
  int count = 0;
  uint64_t sorted[E];
#pragma unroll
  for (int e = 0; e < E; ++e) sorted[e] = 0;
  const int kcap = k_max < flp ? k_max : flp;  // k_max = min(K_max, first_local_page)
  int R = kcap > k_min ? kcap : k_min;
  R = R < flp ? R : flp;
  R = R < cap ? R : cap;
  // Selection in two stages when the pages fill every wave: wave w takes the R
  // best of its own slice [64 PW w, 64 PW (w + 1)) (key desc, index asc), then
  // wave 0 takes the R best of those <= DR_WAVES R candidates, kept in index
  // order so ties resolve as over the whole row.  (The R best of the row are
  // among the candidates: a page with R pages of its slice ahead of it has R
  // pages of the row ahead of it.)  Each stage is a scalar bisection without
  // workgroup barriers; one barrier separates them.
  constexpr int PW = PL / DR_WAVES;  // slots per lane of one wave's slice
  constexpr int RS = 64 * E;         // candidate slots per wave
  __shared__ uint32_t cand_k[PW >= 1 ? DR_WAVES * RS : 1], cand_i[PW >= 1 ? DR_WAVES * RS : 1];
  __shared__ int n_cand[DR_WAVES];
  if constexpr (PW >= 1) {
    if (route && R > 0) {  // uniform
      uint32_t key[PW];
#pragma unroll
      for (int i = 0; i < PW; ++i) {
        const int j = 64 * (PW * wave + i) + lane;
        key[i] = j < flp ? __float_as_uint(expf(sc[j] - mx) / z) + 1u : 0u;
      }
      uint32_t T;
      int clo;
      top_threshold<PW>(key, R, T, clo);
      const int n = take_top<PW>(key, R, T, clo, cand_k + wave * RS, cand_i + wave * RS,
                                 [&](int i) { return static_cast<uint32_t>(64 * (PW * wave + i) + lane); });
      if (lane == 0) n_cand[wave] = n;
    }
    bar();
  }
  if (wave != 0) return;  // no workgroup barrier follows
  if (route && R > 0) {
    if constexpr (PW >= 1) {
      constexpr int PC = DR_WAVES * RS / 64;  // candidate slots per lane
      uint32_t key[PC];
#pragma unroll
      for (int i = 0; i < PC; ++i) {
        const int f = 64 * i + lane;  // candidate f = slot f % RS of wave f / RS: index order
        key[i] = f % RS < n_cand[f / RS] ? cand_k[f] : 0u;
      }
      uint32_t T;
      int clo;
      top_threshold<PC>(key, R, T, clo);
      take_top<PC>(key, R, T, clo, lk, li, [&](int i) { return cand_i[64 * i + lane]; });
      sort_taken<E>(R, sorted, lk, li);
    } else {
      uint32_t key[PL];
#pragma unroll
      for (int i = 0; i < PL; ++i) {
        const int j = 64 * i + lane;
        key[i] = j < flp ? __float_as_uint(expf(sc[j] - mx) / z) + 1u : 0u;
      }
      rank_top<PL, E>(key, R, sorted, lk, li);
    }
    float cum[E];
    running_mass<E, false>(sorted, R, cum);
    const int first = first_reaching<E>(cum, R, top_p);
    const int needed = first >= R ? 0x7fffffff : first + 1;  // #(cum < top_p) + 1
    count = needed < kcap ? needed : kcap;
    count = count > k_min ? count : k_min;
    count = count < flp ? count : flp;  // sorted_idx[b, :needed] has flp entries
    count = count < cap ? count : cap;
  }
  if (pg_lds) {
#pragma unroll
    for (int e = 0; e < E; ++e) pg_lds[e * 64 + lane] = e * 64 + lane < count ? comp_index(sorted[e]) : -1;
    if (lane == 0) *cnt_lds = count;
  }
  if (!write_out) return;
  int32_t* pages = out_pages + static_cast<int64_t>(b) * cap;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int k = e * 64 + lane;
    if (k < cap) pages[k] = k < count ? comp_index(sorted[e]) : -1;
  }
  for (int k = 64 * E + lane; k < cap; k += 64) pages[k] = -1;
  if (lane == 0) out_cnt[b] = count;
}

template <int PL, int E, bool BF16>
__device__ __forceinline__ void decode_route_block(const RouteArgs& A, int b) {
  RouteRegs<PL> rr;
  decode_route_loads<PL, BF16>(A, b, rr);
  DrWgBarrier bar;
  decode_route_compute<PL, E, BF16>(A, b, rr, true, nullptr, nullptr, bar);
}

template <int PL, int E, bool BF16>
__global__ __launch_bounds__(DR_THREADS) void decode_route_kernel(RouteArgs A) {
  decode_route_block<PL, E, BF16>(A, blockIdx.x);
}

// ---------------------------------------------------------------------------
// Rows longer than one wave holds (more than 64 x 64 entries, up to
// LARGE_MAX): one LW-wave workgroup per row.  Wave w holds the contiguous slice
// [64 PLW w, 64 PLW (w + 1)) of the row (element j in lane j % 64, slot
// (j / 64) % PLW).  The softmax maximum and sum, the local mass and the
// candidate count are combined across the waves through LDS (waves summed in
// wave order).  Each wave ranks the R best of its slice (threshold bisection,
// ties in index order) into its candidate list; wave 0 then ranks the R best of
// the LW lists, read wave-major with each list in slice order, which keeps
// equal keys in index order: the R best of the row are among the candidates,
// since an entry with R entries of its slice ahead of it has R entries of the
// row ahead of it.
// ---------------------------------------------------------------------------
constexpr int LW = 16;
constexpr int LW_THREADS = 64 * LW;
constexpr int LARGE_MAX = 64 * 64 * LW;

template <int E>
struct LargeLds {
  float redf[LW];
  int redi[LW];
  int other[LW];
  int n_cand[LW];
  uint32_t cand_k[LW * 64 * E], cand_i[LW * 64 * E];
  uint32_t lk[64 * E], li[64 * E];
};

// Workgroup maximum / sum (waves added in wave order) / integer sum; every
// thread of the LW waves must call them, and every thread gets the result.
__device__ __forceinline__ float lw_max(float v, float* red) {
  v = wave_max(v);
  __syncthreads();
  if (lane_id() == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int w = 1; w < LW; ++w) r = fmaxf(r, red[w]);
  return r;
}
__device__ __forceinline__ float lw_sum(float v, float* red) {
  v = wave_sum(v);
  __syncthreads();
  if (lane_id() == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int w = 1; w < LW; ++w) r += red[w];
  return r;
}
__device__ __forceinline__ int lw_sum_i(int v, int* red) {
  v = wave_sum_i(v);
  __syncthreads();
  if (lane_id() == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  int r = 0;
#pragma unroll
  for (int w = 0; w < LW; ++w) r += red[w];
  return r;
}

// Stage 1 (every wave, over its slice) and stage 2 (wave 0, over the
// candidates) of the R-best ranking; wave 0 returns the R best sorted
// descending in sorted[] (the other waves' sorted[] stay 0).  Ends with every
// wave past the barrier between the stages.
template <int PLW, int E, class IdxFn>
__device__ __forceinline__ void lw_rank_top(const uint32_t (&key)[PLW], int R, uint64_t (&sorted)[E], LargeLds<E>& L,
                                            IdxFn idx) {
  const int lane = lane_id(), wave = threadIdx.x >> 6;
  constexpr int RS = 64 * E;
#pragma unroll
  for (int e = 0; e < E; ++e) sorted[e] = 0;
  if (R > 0) {  // uniform across the workgroup
    uint32_t T;
    int clo;
    top_threshold<PLW>(key, R, T, clo);
    const int n = take_top<PLW>(key, R, T, clo, L.cand_k + wave * RS, L.cand_i + wave * RS, idx);
    if (lane == 0) L.n_cand[wave] = n;
  }
  __syncthreads();
  if (wave != 0 || R <= 0) return;
  constexpr int PC = LW * E;  // candidate slots per lane
  uint32_t ck[PC];
#pragma unroll
  for (int i = 0; i < PC; ++i) {
    const int f = 64 * i + lane;  // candidate f: slot f % RS of wave f / RS
    ck[i] = f % RS < L.n_cand[f / RS] ? L.cand_k[f] : 0u;
  }
  uint32_t T;
  int clo;
  top_threshold<PC>(ck, R, T, clo);
  take_top<PC>(ck, R, T, clo, L.lk, L.li, [&](int i) { return L.cand_i[64 * i + lane]; });
  sort_taken<E>(R, sorted, L.lk, L.li);
}

// select_row for a row held by the LW waves of the workgroup (s: this wave's
// slice, upcast to fp32).  Same outputs and rules as select_row.
template <int PLW, int E, bool RB>
__device__ void select_row_large(float (&s)[PLW], int N, int qb, int64_t row, const SelectParams& sp,
                                 int32_t* __restrict__ out_idx, int32_t* __restrict__ out_cnt,
                                 float* __restrict__ out_mass, LargeLds<E>& L) {
  const int lane = lane_id(), wave = threadIdx.x >> 6;
  const float top_p = sp.top_p_rows ? sp.top_p_rows[row] : sp.top_p;
  const int k_min = sp.k_min_rows ? sp.k_min_rows[row] : sp.k_min;
  const int k_max = sp.k_max_rows ? sp.k_max_rows[row] : sp.k_max;
  auto elem = [&](int i) { return (wave * PLW + i) * 64 + lane; };

  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < PLW; ++i) {
    const int j = elem(i);
    if (j < N && mask_kind(j, qb, sp.causal, sp.local_window)) mx = fmaxf(mx, s[i]);
  }
  mx = lw_max(mx, L.redf);
  if (!isfinite(mx)) mx = 0.0f;
  float z = 0.f;
#pragma unroll
  for (int i = 0; i < PLW; ++i) {
    const int j = elem(i);
    s[i] = j < N && mask_kind(j, qb, sp.causal, sp.local_window) ? expf(s[i] - mx) : 0.0f;
    z += s[i];
  }
  z = fmaxf(lw_sum(z, L.redf), 1e-20f);
  float lm = 0.f;
  int av = 0, ot = 0;
  uint32_t key[PLW];
#pragma unroll
  for (int i = 0; i < PLW; ++i) {
    const int j = elem(i);
    const int kind = j < N ? mask_kind(j, qb, sp.causal, sp.local_window) : 0;
    float p = s[i] / z;
    if (RB) p = round_bf16(p);
    if (kind == 1) lm += p;
    key[i] = kind == 2 ? __float_as_uint(p) + 1u : 0u;
    av += kind == 2;
    ot += j < N && kind != 2;
  }
  float lmass = lw_sum(lm, L.redf);
  if (RB) lmass = round_bf16(lmass);
  ot = wave_sum_i(ot);
  if (lane == 0) L.other[wave] = ot;
  const int avail = lw_sum_i(av, L.redi);  // its barriers also publish L.other

  int R = k_max > sp.capacity ? k_max : sp.capacity;
  R = R < avail ? R : avail;
  R = R < 64 * E ? R : 64 * E;  // the host guarantees this does not truncate
  int32_t* idx = out_idx + row * sp.capacity;
  if (sp.capacity > R) {
    // R == avail here: the non-remote entries (ranked -1) follow in index order
    int base = R;
    for (int w = 0; w < wave; ++w) base += L.other[w];
#pragma unroll
    for (int i = 0; i < PLW; ++i) {
      const int j = elem(i);
      const bool other = j < N && mask_kind(j, qb, sp.causal, sp.local_window) != 2;
      const uint64_t b = __ballot(other);
      const int pos = base + lanes_below(b);
      if (other && pos < sp.capacity) idx[pos] = j;
      base += __popcll(b);
    }
  }
  uint64_t sorted[E];
  lw_rank_top<PLW, E>(key, R, sorted, L, [&](int i) { return static_cast<uint32_t>(elem(i)); });
  if (wave != 0) return;

  const float target = RB ? fmaxf(round_bf16(round_bf16(top_p) - lmass), 0.0f) : fmaxf(top_p - lmass, 0.0f);
  int nr = k_max < avail ? k_max : avail;
  nr = nr < 0 ? 0 : nr;
  nr = nr < R ? nr : R;
  float cum[E];
  running_mass<E, RB>(sorted, nr, cum);
  int count;
  if (avail <= 0) {
    count = 0;
  } else {
    const int first = first_reaching<E>(cum, nr, target);
    int needed = first >= nr ? 0x7fffffff : first + (target > 0.0f ? 1 : 0);
    needed = needed > k_min ? needed : k_min;
    count = needed < avail ? needed : avail;
  }
  count = count < k_max ? count : k_max;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int k = e * 64 + lane;
    if (k < R && k < sp.capacity) idx[k] = comp_index(sorted[e]);
  }
  const float ck = count > 0 ? element_at<E>(cum, count - 1) : 0.f;
  if (lane == 0) {
    out_cnt[row] = count;
    if (out_mass) out_mass[row] = count > 0 ? (RB ? round_bf16(lmass + ck) : lmass + ck) : lmass;
  }
}

// select_blocks on materialised scores, one workgroup per row of N > 64 x 64.
template <int PLW, int E, bool BF16>
__global__ __launch_bounds__(LW_THREADS) void route_scores_large_kernel(const void* __restrict__ scores, int Qb,
                                                                        int N, SelectParams sp,
                                                                        int32_t* __restrict__ out_idx,
                                                                        int32_t* __restrict__ out_cnt,
                                                                        float* __restrict__ out_mass) {
  __shared__ LargeLds<E> L;
  const int64_t row = blockIdx.x;
  const int lane = lane_id(), wave = threadIdx.x >> 6;
  float s[PLW];
#pragma unroll
  for (int i = 0; i < PLW; ++i) {
    const int j = (wave * PLW + i) * 64 + lane;
    if (BF16) s[i] = j < N ? bf16_to_f32(static_cast<const bf16_t*>(scores)[row * N + j]) : 0.f;
    else s[i] = j < N ? static_cast<const float*>(scores)[row * N + j] : 0.f;
  }
  select_row_large<PLW, E, BF16>(s, N, static_cast<int>(row % Qb), row, sp, out_idx, out_cnt, out_mass, L);
}

// fp32 cosine / sqrt(d) score of query qa (normalised) against key j, with the
// arithmetic of score_route_kernel (key L2-normalised in fp32, products summed
// in component order).
template <bool BF16>
__device__ __forceinline__ float cosine_score(const char* kb, int j, const float (&qa)[SR_D], float sqrt_d) {
  float v[SR_D];
  if (BF16) {
    const u32x4_t* src = reinterpret_cast<const u32x4_t*>(reinterpret_cast<const bf16_t*>(kb) +
                                                           static_cast<int64_t>(j) * SR_D);
    const u32x4_t a = src[0], c2 = src[1];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      v[2 * w] = lo_bf16(a[w]);
      v[2 * w + 1] = hi_bf16(a[w]);
      v[8 + 2 * w] = lo_bf16(c2[w]);
      v[8 + 2 * w + 1] = hi_bf16(c2[w]);
    }
  } else {
    const float4* src = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(kb) +
                                                        static_cast<int64_t>(j) * SR_D);
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float4 f = src[w];
      v[4 * w] = f.x;
      v[4 * w + 1] = f.y;
      v[4 * w + 2] = f.z;
      v[4 * w + 3] = f.w;
    }
  }
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < SR_D; ++c) ss = fmaf(v[c], v[c], ss);
  const float nrm = fmaxf(sqrtf(ss), 1e-12f);
  float acc = 0.f;
#pragma unroll
  for (int c = 0; c < SR_D; ++c) acc = fmaf(qa[c], v[c] / nrm, acc);
  return acc / sqrt_d;
}

// Fused cosine scoring + select_blocks for rows of N > 64 x 64 keys: one
// workgroup per query row (grid (Q, B)).
template <int PLW, int E, bool BF16>
__global__ __launch_bounds__(LW_THREADS) void score_route_large_kernel(const void* __restrict__ q,
                                                                       const void* __restrict__ k, int Q, int N,
                                                                       int64_t k_batch_stride, float sqrt_d,
                                                                       SelectParams sp,
                                                                       int32_t* __restrict__ out_idx,
                                                                       int32_t* __restrict__ out_cnt,
                                                                       float* __restrict__ out_mass) {
  __shared__ LargeLds<E> L;
  __shared__ float qn[SR_D];
  const int lane = lane_id(), wave = threadIdx.x >> 6;
  const int row_q = blockIdx.x, b = blockIdx.y;
  if (threadIdx.x == 0) {
    float v[SR_D];
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < SR_D; ++c) {
      const int64_t off = (static_cast<int64_t>(b) * Q + row_q) * SR_D + c;
      v[c] = BF16 ? bf16_to_f32(static_cast<const bf16_t*>(q)[off]) : static_cast<const float*>(q)[off];
      ss = fmaf(v[c], v[c], ss);
    }
    const float nrm = fmaxf(sqrtf(ss), 1e-12f);
#pragma unroll
    for (int c = 0; c < SR_D; ++c) qn[c] = v[c] / nrm;
  }
  __syncthreads();
  float qa[SR_D];
#pragma unroll
  for (int c = 0; c < SR_D; ++c) qa[c] = qn[c];
  const char* kb = static_cast<const char*>(k) + static_cast<int64_t>(b) * k_batch_stride * (BF16 ? 2 : 4);
  float s[PLW];
#pragma unroll
  for (int i = 0; i < PLW; ++i) {
    const int j = (wave * PLW + i) * 64 + lane;
    s[i] = j < N ? cosine_score<BF16>(kb, j, qa, sqrt_d) : 0.f;
  }
  select_row_large<PLW, E, false>(s, N, row_q, static_cast<int64_t>(b) * Q + row_q, sp, out_idx, out_cnt, out_mass,
                                  L);
}

// decode_route_block for more than 64 x 64 completed pages: one LW-wave
// workgroup per sequence, the page scores in registers.
template <int PLW, int E, bool BF16>
__global__ __launch_bounds__(LW_THREADS) void decode_route_large_kernel(RouteArgs A) {
  __shared__ LargeLds<E> L;
  __shared__ float ctx_part[LW][SR_D];
  const int b = blockIdx.x;
  const int lane = lane_id(), wave = threadIdx.x >> 6;
  const int P = A.P, page = A.page, window = A.window, completed = A.completed;
  const int k_min = A.k_min, k_max = A.k_max, cap = A.cap;
  const int mypos = A.pos_rows ? A.pos_rows[b] : A.pos;
  const int local_start = mypos + 1 - window > 0 ? mypos + 1 - window : 0;
  const int flp = local_start / page;
  auto elem = [&](int i) { return (wave * PLW + i) * 64 + lane; };

  float qv[SR_D];
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < SR_D; ++c) {
    const int64_t off = static_cast<int64_t>(b) * SR_D + c;
    qv[c] = BF16 ? bf16_to_f32(static_cast<const bf16_t*>(A.qi)[off]) : static_cast<const float*>(A.qi)[off];
    ss = fmaf(qv[c], qv[c], ss);
  }
  const float nrm = fmaxf(sqrtf(ss), 1e-12f);
#pragma unroll
  for (int c = 0; c < SR_D; ++c) qv[c] = qv[c] / nrm;
  float sc[PLW];
#pragma unroll
  for (int i = 0; i < PLW; ++i) {
    const int j = elem(i);
    float acc = 0.f;
    if (j < completed) {
      const float4* kr = reinterpret_cast<const float4*>(A.kp + (static_cast<int64_t>(b) * P + j) * SR_D);
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float4 f = kr[w];
        acc = fmaf(qv[4 * w], f.x, acc);
        acc = fmaf(qv[4 * w + 1], f.y, acc);
        acc = fmaf(qv[4 * w + 2], f.z, acc);
        acc = fmaf(qv[4 * w + 3], f.w, acc);
      }
    }
    sc[i] = acc / A.sqrt_d;
  }

  if (A.out_ctx) {  // uniform: softmax over every completed page, contracted with vp
    float ctx = 0.f;
    if (completed > 0) {
      float m = -INFINITY;
#pragma unroll
      for (int i = 0; i < PLW; ++i)
        if (elem(i) < completed) m = fmaxf(m, sc[i]);
      const float cmx = lw_max(m, L.redf);
      float zz = 0.f;
#pragma unroll
      for (int i = 0; i < PLW; ++i)
        if (elem(i) < completed) zz += expf(sc[i] - cmx);
      const float cz = lw_sum(zz, L.redf);
      float part[SR_D];
#pragma unroll
      for (int c = 0; c < SR_D; ++c) part[c] = 0.f;
#pragma unroll
      for (int i = 0; i < PLW; ++i) {
        const int j = elem(i);
        if (j >= completed) continue;
        float pj = expf(sc[i] - cmx) / cz;
        const int64_t off = (static_cast<int64_t>(b) * P + j) * SR_D;
        if (BF16) {
          pj = round_bf16(pj);
          const u32x4_t* vr = reinterpret_cast<const u32x4_t*>(static_cast<const bf16_t*>(A.vp) + off);
          const u32x4_t a = vr[0], c2 = vr[1];
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            part[2 * w] = fmaf(pj, lo_bf16(a[w]), part[2 * w]);
            part[2 * w + 1] = fmaf(pj, hi_bf16(a[w]), part[2 * w + 1]);
            part[8 + 2 * w] = fmaf(pj, lo_bf16(c2[w]), part[8 + 2 * w]);
            part[9 + 2 * w] = fmaf(pj, hi_bf16(c2[w]), part[9 + 2 * w]);
          }
        } else {
          const float4* vr = reinterpret_cast<const float4*>(static_cast<const float*>(A.vp) + off);
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            const float4 f = vr[w];
            part[4 * w] = fmaf(pj, f.x, part[4 * w]);
            part[4 * w + 1] = fmaf(pj, f.y, part[4 * w + 1]);
            part[4 * w + 2] = fmaf(pj, f.z, part[4 * w + 2]);
            part[4 * w + 3] = fmaf(pj, f.w, part[4 * w + 3]);
          }
        }
      }
      int which;
      const float t = dr_wave_sum16_scatter(part, which);
      if ((lane & 3) == 0) ctx_part[wave][which] = t;
      __syncthreads();
      if (threadIdx.x < SR_D) {
#pragma unroll
        for (int w = 0; w < LW; ++w) ctx += ctx_part[w][threadIdx.x];
      }
    }
    if (threadIdx.x < SR_D) {
      const int64_t off = static_cast<int64_t>(b) * SR_D + threadIdx.x;
      if (BF16) static_cast<bf16_t*>(A.out_ctx)[off] = f32_to_bf16(ctx);
      else static_cast<float*>(A.out_ctx)[off] = ctx;
    }
  }

  const bool route = completed > flp && flp > 0;  // uniform
  const int kcap = k_max < flp ? k_max : flp;     // k_max = min(K_max, first_local_page)
  int R = kcap > k_min ? kcap : k_min;
  R = R < flp ? R : flp;
  R = R < cap ? R : cap;
  if (!route) R = 0;
  uint32_t key[PLW];
#pragma unroll
  for (int i = 0; i < PLW; ++i) key[i] = 0u;
  if (R > 0) {
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < PLW; ++i)
      if (elem(i) < flp) m = fmaxf(m, sc[i]);
    const float mx = lw_max(m, L.redf);
    float zz = 0.f;
#pragma unroll
    for (int i = 0; i < PLW; ++i)
      if (elem(i) < flp) zz += expf(sc[i] - mx);
    const float z = lw_sum(zz, L.redf);
#pragma unroll
    for (int i = 0; i < PLW; ++i)
      if (elem(i) < flp) key[i] = __float_as_uint(expf(sc[i] - mx) / z) + 1u;
  }
  uint64_t sorted[E];
  lw_rank_top<PLW, E>(key, R, sorted, L, [&](int i) { return static_cast<uint32_t>(elem(i)); });
  if (wave != 0) return;
  int count = 0;
  if (R > 0) {
    float cum[E];
    running_mass<E, false>(sorted, R, cum);
    const int first = first_reaching<E>(cum, R, A.top_p);
    const int needed = first >= R ? 0x7fffffff : first + 1;  // #(cum < top_p) + 1
    count = needed < kcap ? needed : kcap;
    count = count > k_min ? count : k_min;
    count = count < flp ? count : flp;
    count = count < cap ? count : cap;
  }
  int32_t* pages = A.out_pages + static_cast<int64_t>(b) * cap;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int k = e * 64 + lane;
    if (k < cap) pages[k] = k < count ? comp_index(sorted[e]) : -1;
  }
  for (int k = 64 * E + lane; k < cap; k += 64) pages[k] = -1;
  if (lane == 0) A.out_cnt[b] = count;
}

// Slots per lane of one wave's slice for a large row of n entries.
int pick_plw(int64_t n) {
  const int64_t per_wave = (n + LW - 1) / LW;
  const int plw = static_cast<int>((per_wave + 63) / 64);
  if (plw <= 8) return 8;
  if (plw <= 16) return 16;
  if (plw <= 32) return 32;
  return 64;
}

#define FSI_DISPATCH_PLW(PLV, ...) \
  switch (PLV) {                   \
    case 8: {                      \
      constexpr int PLW = 8;       \
      __VA_ARGS__;                 \
    } break;                       \
    case 16: {                     \
      constexpr int PLW = 16;      \
      __VA_ARGS__;                 \
    } break;                       \
    case 32: {                     \
      constexpr int PLW = 32;      \
      __VA_ARGS__;                 \
    } break;                       \
    default: {                     \
      constexpr int PLW = 64;      \
      __VA_ARGS__;                 \
    } break;                       \
  }

// ---------------------------------------------------------------------------
// masked_softmax (core.py:36-43): fp32 softmax over mask, masked entries 0,
// all-masked rows 0, result in the scores' dtype.  One workgroup per row;
// three passes over the row (max, sum, write), the later two from L2.
// mask: uint8 with element strides (msb, msq, msn) over (B, Q, N).
// ---------------------------------------------------------------------------
constexpr int MS_THREADS = 256;

__device__ __forceinline__ float block_reduce(float v, float* red, bool is_max) {
  const int wave = threadIdx.x >> 6, lane = lane_id();
  v = is_max ? wave_max(v) : wave_sum(v);
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int w = 1; w < MS_THREADS / 64; ++w) r = is_max ? fmaxf(r, red[w]) : r + red[w];
  __syncthreads();
  return r;
}

template <bool BF16>
__global__ __launch_bounds__(MS_THREADS) void masked_softmax_kernel(const void* __restrict__ scores, int Q, int N,
                                                                    const uint8_t* __restrict__ mask, int64_t msb,
                                                                    int64_t msq, int64_t msn, void* __restrict__ out) {
  __shared__ float red[MS_THREADS / 64];
  const int q = blockIdx.x, b = blockIdx.y;
  const int64_t row = static_cast<int64_t>(b) * Q + q;
  const uint8_t* mrow = mask + b * msb + q * msq;
  auto load = [&](int j) -> float {
    return BF16 ? bf16_to_f32(static_cast<const bf16_t*>(scores)[row * N + j])
                : static_cast<const float*>(scores)[row * N + j];
  };
  float mx = -INFINITY;
  for (int j = threadIdx.x; j < N; j += MS_THREADS)
    if (mrow[j * msn]) mx = fmaxf(mx, load(j));
  mx = block_reduce(mx, red, true);
  if (!isfinite(mx)) mx = 0.0f;
  float z = 0.f;
  for (int j = threadIdx.x; j < N; j += MS_THREADS)
    if (mrow[j * msn]) z += expf(load(j) - mx);
  z = fmaxf(block_reduce(z, red, false), 1e-20f);
  for (int j = threadIdx.x; j < N; j += MS_THREADS) {
    const float p = mrow[j * msn] ? expf(load(j) - mx) / z : 0.0f;
    if (BF16) static_cast<bf16_t*>(out)[row * N + j] = f32_to_bf16(p);
    else static_cast<float*>(out)[row * N + j] = p;
  }
}

// Backward of masked_softmax (autograd of core.py:36-43): with p the fp32
// softmax over the mask, dscores = p * (dp - sum_k p_k dp_k) on masked-in
// entries and 0 elsewhere (all-masked rows: 0).  p is recomputed from the scores
// in fp32, as the reference's autograd keeps fp32 intermediates; dscores is
// rounded once to the scores' dtype.
template <bool BF16>
__global__ __launch_bounds__(MS_THREADS) void masked_softmax_bwd_kernel(
    const void* __restrict__ scores, const void* __restrict__ dprobs, int Q, int N, const uint8_t* __restrict__ mask,
    int64_t msb, int64_t msq, int64_t msn, void* __restrict__ dscores) {
  __shared__ float red[MS_THREADS / 64];
  const int q = blockIdx.x, b = blockIdx.y;
  const int64_t row = static_cast<int64_t>(b) * Q + q;
  const uint8_t* mrow = mask + b * msb + q * msq;
  auto load = [&](const void* p, int j) -> float {
    return BF16 ? bf16_to_f32(static_cast<const bf16_t*>(p)[row * N + j]) : static_cast<const float*>(p)[row * N + j];
  };
  float mx = -INFINITY;
  for (int j = threadIdx.x; j < N; j += MS_THREADS)
    if (mrow[j * msn]) mx = fmaxf(mx, load(scores, j));
  mx = block_reduce(mx, red, true);
  if (!isfinite(mx)) mx = 0.0f;
  float z = 0.f;
  for (int j = threadIdx.x; j < N; j += MS_THREADS)
    if (mrow[j * msn]) z += expf(load(scores, j) - mx);
  z = fmaxf(block_reduce(z, red, false), 1e-20f);
  float dot = 0.f;
  for (int j = threadIdx.x; j < N; j += MS_THREADS)
    if (mrow[j * msn]) dot = fmaf(expf(load(scores, j) - mx) / z, load(dprobs, j), dot);
  dot = block_reduce(dot, red, false);
  for (int j = threadIdx.x; j < N; j += MS_THREADS) {
    const float g = mrow[j * msn] ? expf(load(scores, j) - mx) / z * (load(dprobs, j) - dot) : 0.0f;
    if (BF16) static_cast<bf16_t*>(dscores)[row * N + j] = f32_to_bf16(g);
    else static_cast<float*>(dscores)[row * N + j] = g;
  }
}

int pick_pl(int64_t n) {
  const int pl = static_cast<int>((n + 63) / 64);
  if (pl <= 4) return 4;
  if (pl <= 16) return 16;
  if (pl <= 32) return 32;
  return 64;
}

int pick_e(int64_t r) { return r <= 64 ? 1 : 4; }

#define FSI_DISPATCH_PL(PLV, ...) \
  switch (PLV) {                  \
    case 4: {                     \
      constexpr int PL = 4;       \
      __VA_ARGS__;                \
    } break;                      \
    case 16: {                    \
      constexpr int PL = 16;      \
      __VA_ARGS__;                \
    } break;                      \
    case 32: {                    \
      constexpr int PL = 32;      \
      __VA_ARGS__;                \
    } break;                      \
    default: {                    \
      constexpr int PL = 64;      \
      __VA_ARGS__;                \
    } break;                      \
  }

#define FSI_DISPATCH_E(EV, ...) \
  if ((EV) == 1) {              \
    constexpr int E = 1;        \
    __VA_ARGS__;                \
  } else {                      \
    constexpr int E = 4;        \
    __VA_ARGS__;                \
  }

int decode_route_check(const void* qi, const float* kp, const void* vp, int dtype, int64_t B, int64_t P,
                       int64_t index_dim, int64_t pos, int64_t page_size, int64_t window, int64_t completed_pages,
                       int capacity, const int32_t* out_pages, const int32_t* out_counts, const void* out_context) {
  using namespace fsi_host;
  FSI_CHECK_ARG(dtype == FSI_DTYPE_F32 || dtype == FSI_DTYPE_BF16, FSI_ERR_DTYPE, "decode_route: dtype %d", dtype);
  FSI_CHECK_ARG(index_dim == SR_D, FSI_ERR_SHAPE, "decode_route: index_dim %lld != %d", (long long)index_dim, SR_D);
  FSI_CHECK_ARG(B >= 0 && P >= 0 && page_size > 0 && window >= 0 && pos >= 0 && completed_pages >= 0 &&
                    completed_pages <= P && pos < (int64_t)0x7fffffff,
                FSI_ERR_SHAPE, "decode_route: inconsistent sizes");
  FSI_CHECK_ARG(completed_pages <= FSI_ROUTE_MAX_BLOCKS, FSI_ERR_CAPACITY, "decode_route: %lld pages > %d",
                (long long)completed_pages, FSI_ROUTE_MAX_BLOCKS);
  FSI_CHECK_ARG(capacity >= 0 && capacity <= R_MAX, FSI_ERR_CAPACITY, "decode_route: capacity %d > %d", capacity,
                R_MAX);
  if (B == 0) return FSI_OK;
  FSI_CHECK_ARG(B <= (int64_t)0x7fffffff, FSI_ERR_SHAPE, "decode_route: batch too large");
  FSI_CHECK_ARG(qi && kp && out_pages && out_counts && (vp || !out_context), FSI_ERR_INVALID_ARG,
                "decode_route: null pointer");
  FSI_CHECK_ARG(reinterpret_cast<uintptr_t>(kp) % 16 == 0 &&
                    (!out_context || reinterpret_cast<uintptr_t>(vp) % 16 == 0),
                FSI_ERR_ALIGN, "decode_route: page keys/values must be 16-byte aligned");
  return FSI_OK;
}


// Ranked slots a routing call needs: min(max(K_max, K_min), capacity).
int64_t want_of(int k_min, int k_max, int capacity) {
  const int64_t want = k_max > k_min ? k_max : k_min;
  return want < capacity ? want : capacity;
}

// Workgroups of `kernel` one CU holds at once (DR_THREADS threads, no dynamic LDS).
template <class K>
int resident_per_cu(K kernel) {
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, DR_THREADS, 0) != hipSuccess || n <= 0) n = 1;
  return n;
}

// Compute units of the current device (queried once per device).
int compute_units() {
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n > 0) return n;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
  cached[dev].store(n, std::memory_order_relaxed);
  return n;
}

RouteArgs route_args(const void* qi, const float* kp, const void* vp, int64_t B, int64_t P, const int32_t* pos_rows,
                     int64_t pos, int64_t page_size, int64_t window, int64_t completed_pages, float top_p, int k_min,
                     int k_max, int capacity, int32_t* out_pages, int32_t* out_counts, void* out_context) {
  const int win = static_cast<int>(window < 0x7fffffff ? window : 0x7fffffff);
  const float sqrt_d = static_cast<float>(sqrt(static_cast<double>(SR_D)));
  return RouteArgs{qi, kp, vp, pos_rows, out_pages, out_counts, out_context, (int)B, (int)P, (int)pos,
                   (int)page_size, win, (int)completed_pages, k_min, k_max, capacity, top_p, sqrt_d};
}

// Fused decode step, launch 1: workgroups [0, B) route sequence b (bf16 index
// query and page values) while the others run the local-window attention
// partials, DS_WAVES independent waves each; the routing workgroups come first
// in dispatch order.
constexpr int DS_WAVES = DR_THREADS / 64;

template <int PL, int E, int HD>
__global__ __launch_bounds__(DR_THREADS) void decode_step_kernel(RouteArgs A, DecodeParams L) {
  if (static_cast<int>(blockIdx.x) < A.B) {
    decode_route_block<PL, E, true>(A, blockIdx.x);
    return;
  }
  decode_partial_wave<HD>(L, (static_cast<int>(blockIdx.x) - A.B) * DS_WAVES + (threadIdx.x >> 6));
}


// ---------------------------------------------------------------------------
// One-launch decode step: one FS_WAVES-wave workgroup per (sequence b, KV head
// g), nothing exchanged between workgroups, no workgroup barrier between the
// routing and the attention:
//   waves [0, DR_WAVES) route sequence b (decode_route_loads /
//     decode_route_compute, the code of decode_route_kernel with an LDS
//     counter for its barriers: the same pages, counts and context); wave 0
//     then looks up the selected pages' physical offsets, leaves them in LDS
//     and releases a flag;
//   waves [DR_WAVES, FS_WAVES) meanwhile stream the local-window chunks
//     (wave w takes chunks w - DR_WAVES + FS_STREAM i), so HBM stays busy
//     while the routing runs;
//   every wave then streams a static, contiguous range of the selected pages'
//   chunks (after acquiring the flag), continuing its online softmax, the
//   routing waves taking more of them to make up for their late start, and
//   writes partial slot w; after one barrier the waves merge the group's query
//   heads over the FS_SLOTS slots.
// Every KV head of a sequence routes it again (the workgroups of one sequence
// run on one XCD, so the page keys come from that XCD's L2); KV head 0 writes
// the pages, counts and context.
// ---------------------------------------------------------------------------
constexpr int FS_WAVES = 8;
constexpr int FS_THREADS = 64 * FS_WAVES;
constexpr int FS_STREAM = FS_WAVES - DR_WAVES;  // waves streaming the window while the others route
constexpr int FS_MAX_PAGES = 64 * 32;           // routing loads held in registers (PL <= 32)
// The routing's length in chunk times of a streaming wave (about 13 us against
// ~5 us per chunk at the C4 shape): the routing waves take that many fewer
// selected-page chunks.
#ifndef FSI_FS_ROUTE_CHUNKS
#define FSI_FS_ROUTE_CHUNKS 2
#endif
constexpr int FS_ROUTE_CHUNKS = FSI_FS_ROUTE_CHUNKS;
static_assert(FS_SLOTS == FS_WAVES, "one partial slot per wave of the one-launch step");

template <int PL, int E, int HD>
__global__ __launch_bounds__(FS_THREADS) void decode_step_fused_kernel(RouteArgs A, DecodeParams L, bf16_t* out) {
  constexpr int DT = HD / 16;
  __shared__ int32_t pg_lds[64 * E];
  __shared__ int64_t rem_off[64 * E];  // element offset of selected page r's (page, g) block, -1 if invalid
  __shared__ int cnt_lds, flag, bar_ctr;
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int b = static_cast<int>(blockIdx.x) % A.B, g = static_cast<int>(blockIdx.x) / A.B;
  if (threadIdx.x == 0) {
    flag = 0;
    bar_ctr = 0;
    cnt_lds = 0;
  }
  __syncthreads();

  const int pos = L.pos_rows ? L.pos_rows[b] : L.pos;
  const int ls = pos + 1 - L.window > 0 ? pos + 1 - L.window : 0;
  const int c_lo = ls / CHUNK, c_hi = pos / CHUNK;
  const int nl = c_hi - c_lo + 1;

  // this wave's local-window chunks (streaming waves only): lane i holds chunk sw + FS_STREAM i
  const int sw = wave - DR_WAVES;
  const int n_loc = sw >= 0 && sw < nl ? (nl - sw + FS_STREAM - 1) / FS_STREAM : 0;  // <= 64 (host-checked)
  int tl_loc = 0, th_loc = CHUNK;
  int64_t cb_loc = 0;
  if (lane < n_loc)
    cb_loc = decode_chunk_addr<HD>(L, b, g, sw + FS_STREAM * lane, nl, c_lo, ls, pos, pg_lds, tl_loc, th_loc);

  if (wave < DR_WAVES) {
    RouteArgs Ab = A;
    if (g != 0) Ab.out_ctx = nullptr;  // the context is written once per sequence
    RouteRegs<PL> rr;
    decode_route_loads<PL, true>(Ab, b, rr);
    DrSubBarrier bar{&bar_ctr, 0, L.err};
    decode_route_compute<PL, E, true>(Ab, b, rr, g == 0, pg_lds, &cnt_lds, bar);
    if (wave == 0) {
      // physical offsets of the selected pages for KV head g, then the release
      int cnt = cnt_lds;
      cnt = cnt < 0 ? 0 : (cnt > L.cap ? L.cap : cnt);
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const int r = 64 * e + lane;
        if (r < cnt) {
          const int lp = pg_lds[r];
          int64_t phys = -1;
          if (lp >= 0 && lp < L.max_pages) phys = L.page_table[static_cast<int64_t>(b) * L.max_pages + lp];
          if (phys < 0 || phys >= L.n_phys) {
            if (L.err) set_error(L.err, FSI_ERR_INDEX_RANGE);
            rem_off[r] = -1;
          } else {
            rem_off[r] = ((phys * L.Hkv + g) * PAGE) * HD;
          }
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
      if (lane == 0) __hip_atomic_store(&flag, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
  }

  u32x4_t qb[HD / 32];
  decode_load_q<HD>(L, b, g, qb);
  f32x4_t acc[DT];
#pragma unroll
  for (int i = 0; i < DT; ++i) acc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;

  // Chunk sequence of this wave: its local chunks, then a contiguous range of the
  // selected pages' chunks.  The ranges are static (the same inputs give the same
  // chunks in the same order to every wave, so the output is reproducible bit for
  // bit) and balance the routing waves' late start: with n = nl + n_sel chunks and
  // the routing worth FS_ROUTE_CHUNKS chunk times, each wave should finish after
  // T = (n + DR_WAVES FS_ROUTE_CHUNKS) / FS_WAVES chunk times, so a streaming wave
  // takes T - nl / FS_STREAM selected chunks and the routing waves share the rest.
  int taken_loc = 0, n_sel = -1, r_lo = 0, r_hi = 0, r_next = 0;
  auto next_chunk = [&](int64_t& info, int& lo, int& hi) -> bool {  // uniform
    if (taken_loc < n_loc) {
      const uint32_t l32 = __builtin_amdgcn_readlane(static_cast<uint32_t>(cb_loc), taken_loc);
      const uint32_t h32 = __builtin_amdgcn_readlane(static_cast<uint32_t>(cb_loc >> 32), taken_loc);
      info = static_cast<int64_t>((static_cast<uint64_t>(h32) << 32) | l32);
      lo = __builtin_amdgcn_readlane(tl_loc, taken_loc);
      hi = __builtin_amdgcn_readlane(th_loc, taken_loc);
      ++taken_loc;
      return true;
    }
    if (n_sel < 0) {
      n_sel = 0;
      for (int spins = 0;; ++spins) {  // bounded: wave 0 always releases; the bound only guarantees an exit
        if (__hip_atomic_load(&flag, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) != 0) {
          int cnt = cnt_lds;
          n_sel = 2 * (cnt < 0 ? 0 : (cnt > L.cap ? L.cap : cnt));
          break;
        }
        if (spins >= (1 << 22)) {
          if (L.err) set_error(L.err, FSI_ERR_HIP);
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
      // chunks per streaming wave (x 8 to keep fractions): T - nl / FS_STREAM, at least 0
      const int t8 = (8 * (nl + n_sel) + 8 * DR_WAVES * FS_ROUTE_CHUNKS) / FS_WAVES;
      int per_s = (t8 - 8 * nl / FS_STREAM + 4) / 8;
      per_s = per_s < 0 ? 0 : (FS_STREAM * per_s > n_sel ? n_sel / FS_STREAM : per_s);
      const int for_route = n_sel - FS_STREAM * per_s;  // the routing waves' chunks [0, for_route)
      const int per_r = (for_route + DR_WAVES - 1) / DR_WAVES;
      if (wave < DR_WAVES) {
        r_lo = wave * per_r < for_route ? wave * per_r : for_route;
        r_hi = r_lo + per_r < for_route ? r_lo + per_r : for_route;
      } else {
        r_lo = for_route + sw * per_s;
        r_hi = r_lo + per_s;
      }
      r_next = r_lo;
    }
    if (r_next >= r_hi) return false;
    const int r = r_next++;
    const int64_t off = rem_off[r >> 1];
    info = off < 0 ? 0 : off + (r & 1);
    lo = 0;
    hi = off < 0 ? 0 : CHUNK;  // an invalid page is read from offset 0 and masked out
    return true;
  };

  u32x4_t kcur[DT], vcur[DT], knxt[DT], vnxt[DT];
  int64_t info;
  int lo_c, hi_c;
  bool have = next_chunk(info, lo_c, hi_c);
  if (have) decode_load_chunk<HD>(L, info, kcur, vcur);
  while (have) {
    int lo_n = 0, hi_n = 0;
    const bool more = next_chunk(info, lo_n, hi_n);
    if (more) decode_load_chunk<HD>(L, info, knxt, vnxt);
    decode_chunk_math<HD>(L, kcur, vcur, qb, lo_c, hi_c, m_run, l_run, acc);
    if (!more) break;
#pragma unroll
    for (int d = 0; d < DT; ++d) kcur[d] = knxt[d];
#pragma unroll
    for (int d = 0; d < DT; ++d) vcur[d] = vnxt[d];
    lo_c = lo_n;
    hi_c = hi_n;
  }
  decode_store_partial<HD>(L, b, g, wave, m_run, l_run, acc);
  __syncthreads();
  for (int h = wave; h < L.G; h += FS_WAVES)
    decode_merge_wave<HD>(L.m_part, L.l_part, L.o_part, L.Hq, L.Hkv, L.G, L.S, out, b * L.Hq + g * L.G + h);
}

}  // namespace

extern "C" {

FSI_API int fsi_route_from_scores(const void* scores, int dtype, int64_t B, int64_t Qb, int64_t Nb, int causal,
                                  int local_window_blocks, float top_p, int k_min, int k_max, int capacity,
                                  const float* top_p_rows, const int32_t* k_min_rows, const int32_t* k_max_rows,
                                  int k_max_bound, int32_t* out_indices, int32_t* out_counts, float* out_mass,
                                  void* stream) {
  using namespace fsi_host;
  FSI_CHECK_ARG(dtype == FSI_DTYPE_F32 || dtype == FSI_DTYPE_BF16, FSI_ERR_DTYPE, "route_from_scores: dtype %d",
                dtype);
  FSI_CHECK_ARG(B >= 0 && Qb >= 0 && Nb >= 0 && capacity >= 0 && local_window_blocks >= 0, FSI_ERR_SHAPE,
                "route_from_scores: negative size");
  FSI_CHECK_ARG(Nb <= FSI_ROUTE_MAX_BLOCKS, FSI_ERR_CAPACITY, "route_from_scores: %lld blocks per row > %d",
                (long long)Nb, FSI_ROUTE_MAX_BLOCKS);
  const int kmax_all = k_max_rows ? k_max_bound : k_max;
  int64_t want = kmax_all > capacity ? kmax_all : capacity;
  want = want < Nb ? want : Nb;
  FSI_CHECK_ARG(want <= R_MAX, FSI_ERR_CAPACITY,
                "route_from_scores: min(max(K_max, capacity), blocks) = %lld > %d ranked candidates", (long long)want,
                R_MAX);
  const int64_t rows = B * Qb;
  if (rows == 0) return FSI_OK;
  FSI_CHECK_ARG(rows <= (int64_t)0x7fffffff * RS_WAVES, FSI_ERR_SHAPE, "route_from_scores: too many rows");
  FSI_CHECK_ARG(scores && out_indices && out_counts, FSI_ERR_INVALID_ARG, "route_from_scores: null pointer");
  SelectParams sp{causal, local_window_blocks, capacity, top_p, k_min, k_max, top_p_rows, k_min_rows, k_max_rows};
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (Nb > 64 * 64) {  // one workgroup per row
    FSI_CHECK_ARG(rows <= (int64_t)0x7fffffff, FSI_ERR_SHAPE, "route_from_scores: too many rows");
    FSI_DISPATCH_PLW(pick_plw(Nb), FSI_DISPATCH_E(pick_e(want), {
      if (dtype == FSI_DTYPE_BF16)
        route_scores_large_kernel<PLW, E, true><<<(unsigned)rows, LW_THREADS, 0, st>>>(
            scores, (int)Qb, (int)Nb, sp, out_indices, out_counts, out_mass);
      else
        route_scores_large_kernel<PLW, E, false><<<(unsigned)rows, LW_THREADS, 0, st>>>(
            scores, (int)Qb, (int)Nb, sp, out_indices, out_counts, out_mass);
    }))
    FSI_HIP_LAUNCH_CHECK("route_from_scores");
    return FSI_OK;
  }
  const dim3 grid(static_cast<unsigned>((rows + RS_WAVES - 1) / RS_WAVES));
  FSI_DISPATCH_PL(pick_pl(Nb), FSI_DISPATCH_E(pick_e(want), {
    if (dtype == FSI_DTYPE_BF16)
      route_scores_kernel<PL, E, true><<<grid, 64 * RS_WAVES, 0, st>>>(scores, rows, (int)Qb, (int)Nb, sp,
                                                                      out_indices, out_counts, out_mass);
    else
      route_scores_kernel<PL, E, false><<<grid, 64 * RS_WAVES, 0, st>>>(scores, rows, (int)Qb, (int)Nb, sp,
                                                                       out_indices, out_counts, out_mass);
  }))
  FSI_HIP_LAUNCH_CHECK("route_from_scores");
  return FSI_OK;
}

FSI_API int fsi_score_and_route(const void* q, const void* k, int dtype, int64_t B, int64_t Q,
                                int64_t N, int64_t index_dim, int64_t k_batch_stride, int causal,
                                int local_window_blocks, float top_p, int k_min, int k_max, int capacity,
                                int32_t* out_indices, int32_t* out_counts, float* out_mass, void* stream) {
  using namespace fsi_host;
  FSI_CHECK_ARG(dtype == FSI_DTYPE_F32 || dtype == FSI_DTYPE_BF16, FSI_ERR_DTYPE, "score_and_route: dtype %d", dtype);
  FSI_CHECK_ARG(index_dim == SR_D, FSI_ERR_SHAPE, "score_and_route: index_dim %lld != %d", (long long)index_dim,
                SR_D);
  FSI_CHECK_ARG(B >= 0 && Q >= 0 && N >= 0 && capacity >= 0 && local_window_blocks >= 0 && k_batch_stride >= 0,
                FSI_ERR_SHAPE, "score_and_route: negative size");
  FSI_CHECK_ARG(N <= FSI_SCORE_ROUTE_MAX_KEYS, FSI_ERR_CAPACITY, "score_and_route: %lld keys > %d", (long long)N,
                FSI_SCORE_ROUTE_MAX_KEYS);
  int64_t want = k_max > capacity ? k_max : capacity;
  want = want < N ? want : N;
  FSI_CHECK_ARG(want <= R_MAX, FSI_ERR_CAPACITY, "score_and_route: min(max(K_max, capacity), keys) = %lld > %d",
                (long long)want, R_MAX);
  if (B == 0 || Q == 0) return FSI_OK;
  FSI_CHECK_ARG(B <= 65535 && Q <= (int64_t)0x7fffffff, FSI_ERR_SHAPE, "score_and_route: grid too large");
  FSI_CHECK_ARG(q && k && out_indices && out_counts, FSI_ERR_INVALID_ARG, "score_and_route: null pointer");
  FSI_CHECK_ARG(reinterpret_cast<uintptr_t>(k) % 16 == 0 &&
                    (k_batch_stride * (dtype == FSI_DTYPE_BF16 ? 2 : 4)) % 16 == 0,
                FSI_ERR_ALIGN, "score_and_route: keys must be 16-byte aligned");
  SelectParams sp{causal, local_window_blocks, capacity, top_p, k_min, k_max, nullptr, nullptr, nullptr};
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const float sqrt_d = static_cast<float>(sqrt(static_cast<double>(index_dim)));
  if (N > 64 * 64) {  // one workgroup per query row
    const dim3 lgrid(static_cast<unsigned>(Q), static_cast<unsigned>(B));
    FSI_DISPATCH_PLW(pick_plw(N), FSI_DISPATCH_E(pick_e(want), {
      if (dtype == FSI_DTYPE_BF16)
        score_route_large_kernel<PLW, E, true><<<lgrid, LW_THREADS, 0, st>>>(
            q, k, (int)Q, (int)N, k_batch_stride, sqrt_d, sp, out_indices, out_counts, out_mass);
      else
        score_route_large_kernel<PLW, E, false><<<lgrid, LW_THREADS, 0, st>>>(
            q, k, (int)Q, (int)N, k_batch_stride, sqrt_d, sp, out_indices, out_counts, out_mass);
    }))
    FSI_HIP_LAUNCH_CHECK("score_and_route");
    return FSI_OK;
  }
  const dim3 grid(static_cast<unsigned>((Q + SR_WAVES - 1) / SR_WAVES), static_cast<unsigned>(B));
  int pl = pick_pl(N);
  pl = pl < 16 ? 16 : pl;
  FSI_DISPATCH_PL(pl, FSI_DISPATCH_E(pick_e(want), {
    if constexpr (PL >= 16) {
      if (dtype == FSI_DTYPE_BF16)
        score_route_kernel<PL, E, true><<<grid, 64 * SR_WAVES, 0, st>>>(q, k, (int)Q, (int)N, k_batch_stride, sqrt_d,
                                                                       sp, out_indices, out_counts, out_mass);
      else
        score_route_kernel<PL, E, false><<<grid, 64 * SR_WAVES, 0, st>>>(q, k, (int)Q, (int)N, k_batch_stride,
                                                                        sqrt_d, sp, out_indices, out_counts, out_mass);
    }
  }))
  FSI_HIP_LAUNCH_CHECK("score_and_route");
  return FSI_OK;
}

FSI_API int fsi_decode_route(const void* qi, const float* kp, const void* vp, int dtype, int64_t B, int64_t P,
                             int64_t index_dim, const int32_t* pos_rows, int64_t pos, int64_t page_size,
                             int64_t window, int64_t completed_pages, float top_p, int k_min, int k_max,
                             int capacity, int32_t* out_pages, int32_t* out_counts, void* out_context,
                             void* stream) {
  const int c = decode_route_check(qi, kp, vp, dtype, B, P, index_dim, pos, page_size, window, completed_pages,
                                   capacity, out_pages, out_counts, out_context);
  if (c != FSI_OK || B == 0) return c;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const RouteArgs A = route_args(qi, kp, vp, B, P, pos_rows, pos, page_size, window, completed_pages, top_p, k_min,
                                 k_max, capacity, out_pages, out_counts, out_context);
  int64_t want = k_max > k_min ? k_max : k_min;
  want = want < capacity ? want : capacity;
  if (completed_pages > 64 * 64) {  // one 16-wave workgroup per sequence
    FSI_DISPATCH_PLW(pick_plw(completed_pages), FSI_DISPATCH_E(pick_e(want), {
      if (dtype == FSI_DTYPE_BF16)
        decode_route_large_kernel<PLW, E, true><<<(unsigned)B, LW_THREADS, 0, st>>>(A);
      else
        decode_route_large_kernel<PLW, E, false><<<(unsigned)B, LW_THREADS, 0, st>>>(A);
    }))
    FSI_HIP_LAUNCH_CHECK("decode_route");
    return FSI_OK;
  }
  FSI_DISPATCH_PL(pick_pl(completed_pages), FSI_DISPATCH_E(pick_e(want), {
    if (dtype == FSI_DTYPE_BF16)
      decode_route_kernel<PL, E, true><<<(unsigned)B, DR_THREADS, 0, st>>>(A);
    else
      decode_route_kernel<PL, E, false><<<(unsigned)B, DR_THREADS, 0, st>>>(A);
  }))
  FSI_HIP_LAUNCH_CHECK("decode_route");
  return FSI_OK;
}

FSI_API int fsi_decode_step_attn(const void* qi, const float* kp, const void* vp, int64_t P, int64_t completed_pages,
                                 float top_p, int k_min, int k_max, int capacity, int32_t* out_pages,
                                 int32_t* out_counts, void* out_context, const void* q, const void* k_pool,
                                 const void* v_pool, const int32_t* page_table, int64_t max_pages,
                                 int64_t n_phys_pages, const int32_t* pos_rows, int64_t pos, int64_t window,
                                 int64_t B, int64_t Hq, int64_t Hkv, int64_t head_dim, float scale, int batch0,
                                 void* out, void* workspace, size_t workspace_bytes, int* err, void* stream) {
  int c = decode_route_check(qi, kp, vp, FSI_DTYPE_BF16, B, P, SR_D, pos, PAGE, window, completed_pages, capacity,
                             out_pages, out_counts, out_context);
  if (c != FSI_OK) return c;
  c = decode_attn_check(q, k_pool, v_pool, page_table, max_pages, n_phys_pages, pos_rows, pos, window, out_pages,
                        out_counts, capacity, B, Hq, Hkv, head_dim, out);
  if (c != FSI_OK || B == 0) return c;
  const size_t need = FSI_WORKSPACE_COUNTER_BYTES +
                      decode_attn_partials_bytes(B, Hq, Hkv, head_dim, window, capacity, max_pages) + 256;
  FSI_CHECK_ARG(workspace && workspace_bytes >= need, FSI_ERR_WORKSPACE,
                "decode_step_attn: workspace %zu < %zu bytes", workspace_bytes, need);
  FSI_CHECK_ARG(reinterpret_cast<uintptr_t>(workspace) % 16 == 0, FSI_ERR_ALIGN,
                "decode_step_attn: workspace must be 16-byte aligned");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace) + FSI_WORKSPACE_COUNTER_BYTES;
  const RouteArgs A = route_args(qi, kp, vp, B, P, pos_rows, pos, PAGE, window, completed_pages, top_p, k_min, k_max,
                                 capacity, out_pages, out_counts, out_context);
  if (completed_pages > 64 * 64) {
    // more pages than the routing workgroups of the fused launch hold: the
    // large-row routing kernel, then the selected pages and the window in one
    // partial launch and the merge (same workspace layout)
    FSI_DISPATCH_PLW(pick_plw(completed_pages), FSI_DISPATCH_E(pick_e(want_of(k_min, k_max, capacity)), {
      decode_route_large_kernel<PLW, E, true><<<(unsigned)B, LW_THREADS, 0, st>>>(A);
    }))
    FSI_HIP_LAUNCH_CHECK("decode_step_attn route");
    const DecodeParams D = decode_params(q, k_pool, v_pool, page_table, max_pages, n_phys_pages, pos_rows, pos, window,
                                         out_pages, out_counts, batch0 ? 0 : capacity, capacity, B, Hq, Hkv, scale, ws,
                                         err, DA_ALL);
    return decode_partial_merge_launch(D, head_dim, out, st);
  }
  // one launch when every (sequence, KV head) pair gets a workgroup of its own on the chip
  if (!batch0 && completed_pages <= FS_MAX_PAGES && B * Hkv >= FS_MIN_PAIRS && B * Hkv >= compute_units() &&
      local_chunks_of(window, max_pages) <= FS_STREAM * static_cast<int64_t>(MAX_CHUNKS_PER_WAVE)) {
    DecodeParams L = decode_params(q, k_pool, v_pool, page_table, max_pages, n_phys_pages, pos_rows, pos, window,
                                   nullptr, nullptr, capacity, capacity, B, Hq, Hkv, scale, ws, err, DA_LOCAL);
    const int64_t parts = B * Hkv * FS_SLOTS;  // fits: the workspace holds at least FS_SLOTS slots per pair
    L.m_part = reinterpret_cast<float*>(ws);
    L.l_part = L.m_part + parts * 16;
    L.o_part = L.l_part + parts * 16;
    L.S = FS_SLOTS;
    L.S_sub = FS_SLOTS;
    L.s_off = 0;
    const unsigned grid = static_cast<unsigned>(B * Hkv);
    bf16_t* o = static_cast<bf16_t*>(out);
    FSI_DISPATCH_PL(pick_pl(completed_pages), FSI_DISPATCH_E(pick_e(want_of(k_min, k_max, capacity)), {
      if constexpr (PL <= 32) {
        if (head_dim == 128) decode_step_fused_kernel<PL, E, 128><<<grid, FS_THREADS, 0, st>>>(A, L, o);
        else decode_step_fused_kernel<PL, E, 64><<<grid, FS_THREADS, 0, st>>>(A, L, o);
      }
    }))
    FSI_HIP_LAUNCH_CHECK("decode_step_attn one launch");
    return FSI_OK;
  }
  // launch 1: routing workgroups [0, B) beside the local-window partials (which read no routing result),
  // with as many local waves as fit beside the routing workgroups in one round of resident workgroups,
  // so that no second round trails the first
  int per_cu = 1;
  FSI_DISPATCH_PL(pick_pl(completed_pages), FSI_DISPATCH_E(pick_e(want_of(k_min, k_max, capacity)), {
    per_cu = head_dim == 128 ? resident_per_cu(decode_step_kernel<PL, E, 128>)
                             : resident_per_cu(decode_step_kernel<PL, E, 64>);
  }))
  const int64_t slots = static_cast<int64_t>(compute_units()) * per_cu;
  const int s_fit = slots > B ? static_cast<int>((slots - B) * DS_WAVES / (B * Hkv)) : 1;
  const int s_local = s_fit > 0 ? s_fit : 1;
  const DecodeParams L = decode_params(q, k_pool, v_pool, page_table, max_pages, n_phys_pages, pos_rows, pos, window,
                                       nullptr, nullptr, capacity, capacity, B, Hq, Hkv, scale, ws, err, DA_LOCAL,
                                       s_local);
  const int64_t local_waves = B * Hkv * L.S_sub;
  const unsigned grid = static_cast<unsigned>(B + (local_waves + DS_WAVES - 1) / DS_WAVES);
  FSI_DISPATCH_PL(pick_pl(completed_pages), FSI_DISPATCH_E(pick_e(want_of(k_min, k_max, capacity)), {
    if (head_dim == 128) decode_step_kernel<PL, E, 128><<<grid, DR_THREADS, 0, st>>>(A, L);
    else decode_step_kernel<PL, E, 64><<<grid, DR_THREADS, 0, st>>>(A, L);
  }))
  FSI_HIP_LAUNCH_CHECK("decode_step_attn route + local");
  // launch 2: the remote pages' partials and the merge of both (one fused launch
  // when a workgroup holds a pair's remote waves)
  const DecodeParams R = decode_params(q, k_pool, v_pool, page_table, max_pages, n_phys_pages, pos_rows, pos, window,
                                       out_pages, out_counts, batch0 ? 0 : capacity, capacity, B, Hq, Hkv, scale, ws,
                                       err, DA_REMOTE, s_local);
  return decode_partial_merge_launch(R, head_dim, out, st);
}



FSI_API int fsi_masked_softmax(const void* scores, int dtype, int64_t B, int64_t Q, int64_t N, const uint8_t* mask,
                               int64_t mask_stride_b, int64_t mask_stride_q, int64_t mask_stride_n, void* out,
                               void* stream) {
  using namespace fsi_host;
  FSI_CHECK_ARG(dtype == FSI_DTYPE_F32 || dtype == FSI_DTYPE_BF16, FSI_ERR_DTYPE, "masked_softmax: dtype %d", dtype);
  FSI_CHECK_ARG(B >= 0 && Q >= 0 && N >= 0, FSI_ERR_SHAPE, "masked_softmax: negative size");
  if (B == 0 || Q == 0 || N == 0) return FSI_OK;
  FSI_CHECK_ARG(B <= 65535 && Q <= (int64_t)0x7fffffff && N <= (int64_t)0x7fffffff, FSI_ERR_SHAPE,
                "masked_softmax: grid too large");
  FSI_CHECK_ARG(scores && mask && out, FSI_ERR_INVALID_ARG, "masked_softmax: null pointer");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>(Q), static_cast<unsigned>(B));
  if (dtype == FSI_DTYPE_BF16)
    masked_softmax_kernel<true><<<grid, MS_THREADS, 0, st>>>(scores, (int)Q, (int)N, mask, mask_stride_b,
                                                             mask_stride_q, mask_stride_n, out);
  else
    masked_softmax_kernel<false><<<grid, MS_THREADS, 0, st>>>(scores, (int)Q, (int)N, mask, mask_stride_b,
                                                              mask_stride_q, mask_stride_n, out);
  FSI_HIP_LAUNCH_CHECK("masked_softmax");
  return FSI_OK;
}

FSI_API int fsi_masked_softmax_bwd(const void* scores, const void* dprobs, int dtype, int64_t B, int64_t Q, int64_t N,
                                   const uint8_t* mask, int64_t mask_stride_b, int64_t mask_stride_q,
                                   int64_t mask_stride_n, void* dscores, void* stream) {
  using namespace fsi_host;
  FSI_CHECK_ARG(dtype == FSI_DTYPE_F32 || dtype == FSI_DTYPE_BF16, FSI_ERR_DTYPE, "masked_softmax_bwd: dtype %d",
                dtype);
  FSI_CHECK_ARG(B >= 0 && Q >= 0 && N >= 0, FSI_ERR_SHAPE, "masked_softmax_bwd: negative size");
  if (B == 0 || Q == 0 || N == 0) return FSI_OK;
  FSI_CHECK_ARG(B <= 65535 && Q <= (int64_t)0x7fffffff && N <= (int64_t)0x7fffffff, FSI_ERR_SHAPE,
                "masked_softmax_bwd: grid too large");
  FSI_CHECK_ARG(scores && dprobs && mask && dscores, FSI_ERR_INVALID_ARG, "masked_softmax_bwd: null pointer");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>(Q), static_cast<unsigned>(B));
  if (dtype == FSI_DTYPE_BF16)
    masked_softmax_bwd_kernel<true><<<grid, MS_THREADS, 0, st>>>(scores, dprobs, (int)Q, (int)N, mask, mask_stride_b,
                                                                 mask_stride_q, mask_stride_n, dscores);
  else
    masked_softmax_bwd_kernel<false><<<grid, MS_THREADS, 0, st>>>(scores, dprobs, (int)Q, (int)N, mask, mask_stride_b,
                                                                  mask_stride_q, mask_stride_n, dscores);
  FSI_HIP_LAUNCH_CHECK("masked_softmax_bwd");
  return FSI_OK;
}

}  // extern "C"
