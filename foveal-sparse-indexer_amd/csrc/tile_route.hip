// 2-D tile routing of BlockwiseMatMul2D (foveal_indexer/block_matmul.py:355-377).
//
// Per token row r over T tiles:
//   p      = softmax(scores[r])                         (fp32; rounded to bf16 for bf16 rows)
//   order  = tiles by p descending (equal p: lower tile id first)
//   cum_k  = sum of the first k+1 sorted p              (fp64 sum, compared after rounding to
//                                                        the row dtype, as ATen's CPU cumsum)
//   needed = min(#(cum < top_p) + 1, T)                 (no K_min, no K_max)
//   mask[group(r)][order[:needed]] = 1, plus tiles [0, base_tiles) of every group.
//
// No sort: cum is nondecreasing, so the selected set is every tile above the
// value v at which the running mass first reaches top_p, plus part of v's tie
// group.  v is the largest probability whose "mass at or above" reaches top_p;
// one wave per row finds it by bisection over the order-preserving bit pattern
// of p (31 rounds of a masked fp64 wave sum, the row held in registers), then
// takes just enough of the tie group, in tile order, to cross top_p.  The
// count is unbounded (up to T), which a rank-and-sort select would not handle.
// Rows of one group write 1 into the same mask bytes; every writer stores the
// same value.
#include "fsi_common.h"

namespace {

using namespace fsi;

constexpr int TR_WAVES = 4;
constexpr int TR_MAX_VPL = 64;  // values per lane: T <= 4096

__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = min(v, static_cast<uint32_t>(__shfl_xor(static_cast<int>(v), off, 64)));
  return v;
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = max(v, static_cast<uint32_t>(__shfl_xor(static_cast<int>(v), off, 64)));
  return v;
}

// fp32 or bf16 rounding of a running mass, as the row's cumsum stores it.
template <bool BF16>
__device__ __forceinline__ float store_round(double m) {
  const float f = static_cast<float>(m);
  return BF16 ? round_bf16(f) : f;
}

__global__ __launch_bounds__(256) void tile_mask_init_kernel(uint8_t* __restrict__ mask, int64_t groups,
                                                             int64_t n_tiles, int64_t base_tiles) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i < groups * n_tiles) mask[i] = (i % n_tiles) < base_tiles ? 1 : 0;
}

template <int VPL, bool BF16>
__global__ __launch_bounds__(64 * TR_WAVES) void tile_route_kernel(
    const void* __restrict__ scores, int64_t ld, int64_t rows, int T, int64_t rows_per_group, float top_p,
    uint8_t* __restrict__ mask, int32_t* __restrict__ needed_out, void* __restrict__ probs_out) {
  const int lane = threadIdx.x & 63;
  const int64_t r = static_cast<int64_t>(blockIdx.x) * TR_WAVES + (threadIdx.x >> 6);
  if (r >= rows) return;
  const int64_t base = r * ld;

  // 1. softmax in fp32 (tile i = 64 j + lane)
  float p[VPL];
  float m = -INFINITY;
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int i = 64 * j + lane;
    float s = -INFINITY;
    if (i < T)
      s = BF16 ? bf16_to_f32(static_cast<const bf16_t*>(scores)[base + i])
               : static_cast<const float*>(scores)[base + i];
    p[j] = s;
    m = fmaxf(m, s);
  }
  m = wave_max(m);
  float z = 0.f;
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int i = 64 * j + lane;
    p[j] = i < T ? expf(p[j] - m) : 0.f;
    z += p[j];
  }
  z = wave_sum(z);
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int i = 64 * j + lane;
    float q = p[j] / z;
    if (BF16) q = round_bf16(q);
    p[j] = i < T ? q : 0.f;
    if (probs_out && i < T) {
      if (BF16)
        static_cast<bf16_t*>(probs_out)[r * static_cast<int64_t>(T) + i] = f32_to_bf16(q);
      else
        static_cast<float*>(probs_out)[r * static_cast<int64_t>(T) + i] = q;
    }
  }
  // top_p as the row dtype compares it (a bf16 tensor compares against a bf16 scalar)
  const float tp = BF16 ? round_bf16(top_p) : top_p;

  // 2. total mass; if it never reaches top_p every tile is needed
  double tot = 0.0;
#pragma unroll
  for (int j = 0; j < VPL; ++j) tot += static_cast<double>(p[j]);
  tot = wave_sum_f64(tot);
  const int64_t g = r / rows_per_group;
  uint8_t* mrow = mask + g * static_cast<int64_t>(T);
  if (!(store_round<BF16>(tot) >= tp)) {
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      const int i = 64 * j + lane;
      if (i < T) mrow[i] = 1;
    }
    if (needed_out && lane == 0) needed_out[r] = T;
    return;
  }

  // 3. bisection: largest key K with mass(p >= K) >= top_p (p >= 0: bit patterns
  //    order like the values; padding lanes hold 0 and add nothing)
  uint32_t kmax = 0u;
#pragma unroll
  for (int j = 0; j < VPL; ++j) kmax = max(kmax, __float_as_uint(p[j]));
  kmax = wave_max_u32(kmax);
  // Invariant: mass(p >= lo) reaches tp, mass(p >= hi) does not (nothing lies above
  // the largest p).  With tp <= 0 every key qualifies and the top tile alone is needed.
  uint32_t lo = tp > 0.f ? 0u : kmax, hi = kmax + 1u;
  while (hi - lo > 1u) {
    const uint32_t mid = lo + ((hi - lo) >> 1);
    double acc = 0.0;
#pragma unroll
    for (int j = 0; j < VPL; ++j)
      if (__float_as_uint(p[j]) >= mid) acc += static_cast<double>(p[j]);
    acc = wave_sum_f64(acc);
    if (store_round<BF16>(acc) >= tp)
      lo = mid;
    else
      hi = mid;
  }
  // v = the smallest probability at or above lo: the value where the mass crosses
  uint32_t vk = 0xffffffffu;
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int i = 64 * j + lane;
    const uint32_t k = __float_as_uint(p[j]);
    if (i < T && k >= lo) vk = min(vk, k);
  }
  vk = wave_min_u32(vk);
  const float v = __uint_as_float(vk);
  double above = 0.0;
  int n_above = 0, n_tie = 0;
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int i = 64 * j + lane;
    const uint32_t k = __float_as_uint(p[j]);
    if (i < T && k > vk) {
      above += static_cast<double>(p[j]);
      ++n_above;
    }
    n_tie += (i < T && k == vk);
  }
  above = wave_sum_f64(above);
  n_above = wave_sum_i(n_above);
  n_tie = wave_sum_i(n_tie);
  // tie members taken in tile order until the running mass reaches top_p
  int take = n_tie;
  {
    double run = above;
    for (int t = 1; t <= n_tie; ++t) {
      run += static_cast<double>(v);
      if (store_round<BF16>(run) >= tp) {
        take = t;
        break;
      }
    }
  }
  // 4. mark the selected tiles
  int tie_before = 0;  // tie members with a lower tile id in earlier strips
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int i = 64 * j + lane;
    const uint32_t k = __float_as_uint(p[j]);
    const bool tie = i < T && k == vk;
    const uint64_t bal = __ballot(tie);
    const int rank = tie_before + __popcll(bal & ((uint64_t(1) << lane) - 1));
    if (i < T && (k > vk || (tie && rank < take))) mrow[i] = 1;
    tie_before += __popcll(bal);
  }
  if (needed_out && lane == 0) needed_out[r] = n_above + take;
}

template <bool BF16>
int launch_rows(int vpl, dim3 grid, hipStream_t st, const void* scores, int64_t ld, int64_t rows, int T,
                int64_t rpg, float top_p, uint8_t* mask, int32_t* needed, void* probs) {
#define FSI_TR_CASE(V)                                                                                        \
  case V:                                                                                                     \
    tile_route_kernel<V, BF16><<<grid, 64 * TR_WAVES, 0, st>>>(scores, ld, rows, T, rpg, top_p, mask, needed, \
                                                               probs);                                        \
    break;
  switch (vpl) {
    FSI_TR_CASE(1)
    FSI_TR_CASE(2)
    FSI_TR_CASE(4)
    FSI_TR_CASE(8)
    FSI_TR_CASE(16)
    FSI_TR_CASE(32)
    FSI_TR_CASE(64)
    default: return FSI_ERR_SHAPE;
  }
#undef FSI_TR_CASE
  return FSI_OK;
}

}  // namespace

extern "C" {

FSI_API int fsi_tile_route(const void* scores, int dtype, int64_t rows, int64_t n_tiles, int64_t ld_scores,
                           int64_t rows_per_group, int64_t base_tiles, float top_p, uint8_t* out_mask,
                           int32_t* out_needed, void* out_probs, void* stream) {
  FSI_CHECK_ARG(dtype == FSI_DTYPE_F32 || dtype == FSI_DTYPE_BF16, FSI_ERR_DTYPE, "tile_route: dtype %d", dtype);
  FSI_CHECK_ARG(out_mask && (rows == 0 || scores), FSI_ERR_INVALID_ARG, "tile_route: null pointer");
  FSI_CHECK_ARG(rows >= 0 && n_tiles > 0 && ld_scores >= n_tiles && rows_per_group > 0 && base_tiles >= 0,
                FSI_ERR_SHAPE, "tile_route: rows=%lld tiles=%lld ld=%lld rows_per_group=%lld base=%lld",
                (long long)rows, (long long)n_tiles, (long long)ld_scores, (long long)rows_per_group,
                (long long)base_tiles);
  FSI_CHECK_ARG(n_tiles <= 64 * TR_MAX_VPL, FSI_ERR_CAPACITY, "tile_route: %lld tiles > %d", (long long)n_tiles,
                64 * TR_MAX_VPL);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int64_t groups = rows == 0 ? 1 : (rows + rows_per_group - 1) / rows_per_group;
  const int64_t cells = groups * n_tiles;
  tile_mask_init_kernel<<<dim3(static_cast<unsigned>((cells + 255) / 256)), 256, 0, st>>>(out_mask, groups, n_tiles,
                                                                                         base_tiles);
  FSI_HIP_LAUNCH_CHECK("tile_route init");
  if (rows == 0) return FSI_OK;
  int vpl = 1;
  while (64 * vpl < n_tiles) vpl <<= 1;
  const dim3 grid(static_cast<unsigned>((rows + TR_WAVES - 1) / TR_WAVES));
  const int s = dtype == FSI_DTYPE_BF16
                    ? launch_rows<true>(vpl, grid, st, scores, ld_scores, rows, (int)n_tiles, rows_per_group, top_p,
                                        out_mask, out_needed, out_probs)
                    : launch_rows<false>(vpl, grid, st, scores, ld_scores, rows, (int)n_tiles, rows_per_group, top_p,
                                         out_mask, out_needed, out_probs);
  if (s != FSI_OK) return s;
  FSI_HIP_LAUNCH_CHECK("tile_route rows");
  return FSI_OK;
}

}  // extern "C"
