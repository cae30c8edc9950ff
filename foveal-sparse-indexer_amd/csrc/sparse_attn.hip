// Block-sparse prefill attention on MI355X (gfx950).
//
//   FSI_SATTN_LOCAL_REMOTE (FovealSparseAttention.forward with _build_sparse_mask,
//     foveal_indexer/attention.py:148-269): query q of query block qb attends the
//     keys k with k <= q and k > q - window, plus every key of the remote pages
//     listed for (b, qb) (a boolean union: keys in both count once);
//   FSI_SATTN_BLOCK_LIST (triton_foveal_sparse_attention,
//     foveal_indexer/triton_ops.py:26-93,256-313): query block qb attends every key
//     of each listed key block (a block listed twice is summed twice, as the
//     Triton kernel does).
//
// Work: one wave per (sequence, query head, 16 queries).  A workgroup holds up
// to four query heads of one KV head (a GQA group) at the same 16 queries, so
// their K and V reads hit the CU's L1.  The wave walks a list of 32-key chunks
// (local window chunks, then the chunks of the listed pages) with an online
// softmax:
//   S^T[t][q] = sum_d K[t][d] Q[q][d]       (A = K tile straight from k,
//                                            B = Q^T kept in registers)
//   O^T[d][q] += sum_t V^T[d][t] P^T[t][q]   (A = V^T tile, B = P^T taken from
//                                            S^T's accumulators, as a bf16 hi + lo
//                                            pair so P keeps ~16 bits)
// V^T comes from a workspace copy of v, dim-major per 32-token chunk with the
// chunk's tokens in the MFMA k order of P^T, written by a first kernel.  The
// 64-query kernel (sparse_attn_lds_kernel) takes that copy in fp16, scaled per
// (sequence, KV head) by a power of two that puts the largest finite |v| in
// [2^14, 2^15), and P in fp16 (P <= 2^8 under its lazy running max, rounded
// toward zero, the softmax denominators summed from the same fp16 values): one
// v_mfma_f32_16x16x32_f16 per P V tile, where bf16 P needs the hi + lo pair to
// stay inside the bf16 output tolerance.
#include <algorithm>
#include <type_traits>

#include "fsi_common.h"

using namespace fsi;

namespace fsi_attn_generic {  // csrc/attn_generic.hip
int sparse_attn(const void* q, int64_t qs_b, int64_t qs_h, int64_t qs_t, const void* k, int64_t ks_b, int64_t ks_h,
                int64_t ks_t, const void* v, int64_t vs_b, int64_t vs_h, int64_t vs_t, int64_t B, int64_t Hq,
                int64_t Hkv, int64_t T, int64_t head_dim, int64_t block, int mode, int64_t window,
                const int32_t* lists, int64_t ls_b, int64_t ls_q, int64_t capacity, const int32_t* counts,
                int64_t cs_b, int64_t cs_q, float scale, int dtype, void* out, int64_t os_b, int64_t os_h,
                int64_t os_t, int* err, void* stream);
}  // namespace fsi_attn_generic

namespace fsi_attn_f32 {  // csrc/sparse_attn_f32.hip: 1 when the shape does not fit its kernel
int sparse_attn(const float* q, int64_t qs_b, int64_t qs_h, int64_t qs_t, const float* k, int64_t ks_b, int64_t ks_h,
                int64_t ks_t, const float* v, int64_t vs_b, int64_t vs_h, int64_t vs_t, int64_t B, int64_t Hq,
                int64_t Hkv, int64_t T, int64_t head_dim, int64_t block, int mode, int64_t window,
                const int32_t* lists, int64_t ls_b, int64_t ls_q, int64_t capacity, const int32_t* counts,
                int64_t cs_b, int64_t cs_q, float scale, float* out, int64_t os_b, int64_t os_h, int64_t os_t,
                float* vt, int* err, hipStream_t st);
}  // namespace fsi_attn_f32

namespace {

constexpr int SA_WAVES = 4;   // query heads per workgroup
constexpr int SA_CHUNK = 32;  // keys per chunk
constexpr float SA_LOG2E = 1.4426950408889634f;

// storage position (MFMA k index) of token tau within a 32-token chunk: lane
// group g of the P^T operand holds tokens 4 g .. 4 g + 3 and 16 + 4 g .. 16 + 4 g + 3
__host__ __device__ __forceinline__ int sa_slot(int tau) { return 8 * ((tau & 15) >> 2) + 4 * (tau >> 4) + (tau & 3); }

// ---------------------------------------------------------------------------
// V^T copy: vt[((b Hkv + g) n32 + c) HD 32 + d 32 + sa_slot(tau)] = v[b][g][32 c + tau][d],
// zero past T.  One thread per (b, g, token, 8 dims).
// ---------------------------------------------------------------------------
template <int HD>
__global__ __launch_bounds__(256) void sa_vt_kernel(const bf16_t* __restrict__ v, int64_t vs_b, int64_t vs_g,
                                                    int64_t vs_t, int B, int Hkv, int T, int n32,
                                                    bf16_t* __restrict__ vt) {
  constexpr int PIECES = HD / 8;
  const int64_t total = static_cast<int64_t>(B) * Hkv * n32 * SA_CHUNK * PIECES;
  for (int64_t gid = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; gid < total;
       gid += static_cast<int64_t>(gridDim.x) * 256) {
    const int piece = static_cast<int>(gid % PIECES);
    int64_t r = gid / PIECES;
    const int t = static_cast<int>(r % (static_cast<int64_t>(n32) * SA_CHUNK));
    r /= static_cast<int64_t>(n32) * SA_CHUNK;
    const int g = static_cast<int>(r % Hkv);
    const int b = static_cast<int>(r / Hkv);
    u32x4_t val = u32x4_t{0u, 0u, 0u, 0u};
    if (t < T) val = *reinterpret_cast<const u32x4_t*>(v + b * vs_b + g * vs_g + t * vs_t + 8 * piece);
    const int c = t / SA_CHUNK, tau = t % SA_CHUNK;
    bf16_t* o = vt + ((static_cast<int64_t>(b) * Hkv + g) * n32 + c) * HD * SA_CHUNK + sa_slot(tau);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t w = val[e >> 1];
      o[(8 * piece + e) * SA_CHUNK] = static_cast<bf16_t>((e & 1) ? (w >> 16) : (w & 0xffffu));
    }
  }
}

// ---------------------------------------------------------------------------
// fp16 V^T for sparse_attn_lds_kernel, in two kernels:
//   sa_vmax_kernel: one wave per (b, g, 32-token chunk) writes the chunk's
//     largest finite |v| as a bf16 magnitude pattern (0 .. 0x7f7f) to cmax;
//   sa_vt16_kernel: workgroup (x, bg) reduces head bg's chunk maxima to the
//     head exponent e (largest finite |v| 2^-e in [2^14, 2^15)), stores it in
//     head_e, and writes chunks [x SA_VT_CHUNKS, ..) of the head as fp16 v 2^-e
//     in the layout of sa_vt_kernel: the chunks' token rows are staged in LDS
//     with 16-byte loads and every thread writes 16 bytes of one output row.
// Values below the largest by more than 2^28 become fp16 subnormals (absolute
// error <= 2^-25 of the largest); infinities and NaNs stay what they are.
// ---------------------------------------------------------------------------
constexpr int SA_VT_CHUNKS = 4;  // chunks per sa_vt16_kernel workgroup

template <int HD>
__global__ __launch_bounds__(256) void sa_vmax_kernel(const bf16_t* __restrict__ v, int64_t vs_b, int64_t vs_g,
                                                      int64_t vs_t, int B, int Hkv, int T, int n32,
                                                      uint32_t* __restrict__ cmax) {
  constexpr int PIECES = HD / 8;
  constexpr int PER = SA_CHUNK * PIECES / 64;  // 16-byte pieces per lane
  const int lane = threadIdx.x & 63;
  const int64_t id = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (id >= static_cast<int64_t>(B) * Hkv * n32) return;
  const int c = static_cast<int>(id % n32);
  const int64_t bg = id / n32;
  const int b = static_cast<int>(bg / Hkv), g = static_cast<int>(bg % Hkv);
  uint32_t m = 0;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int idx = i * 64 + lane;
    const int t = c * SA_CHUNK + idx / PIECES, piece = idx % PIECES;
    if (t < T) {
      const u32x4_t w = *reinterpret_cast<const u32x4_t*>(v + b * vs_b + g * vs_g + t * vs_t + 8 * piece);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t lo = w[j] & 0x7fffu, hi = (w[j] >> 16) & 0x7fffu;
        m = lo < 0x7f80u && lo > m ? lo : m;  // infinities and NaNs (>= 0x7f80) are left out
        m = hi < 0x7f80u && hi > m ? hi : m;
      }
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const uint32_t o = __shfl_xor(m, off, 64);
    m = o > m ? o : m;
  }
  if (lane == 0) cmax[id] = m;
}

// Exponent e with the bf16 magnitude pattern mag 2^-e in [2^14, 2^15); 0 for an
// all-zero head, at least -100 (2^100 is the largest scale applied).
__device__ __forceinline__ int sa_head_exponent(uint32_t mag) {
  if (mag == 0) return 0;
  const int E = static_cast<int>(mag >> 7);  // biased exponent; E == 0: subnormal, below 2^-126
  const int e = (E == 0 ? -127 : E - 127) - 14;
  return e < -100 ? -100 : e;
}

template <int HD>
__global__ __launch_bounds__(256) void sa_vt16_kernel(const bf16_t* __restrict__ v, int64_t vs_b, int64_t vs_g,
                                                      int64_t vs_t, int Hkv, int T, int n32,
                                                      const uint32_t* __restrict__ cmax, int32_t* __restrict__ head_e,
                                                      uint16_t* __restrict__ vt) {
  constexpr int PIECES = HD / 8;                        // 16-byte pieces of a token row
  constexpr int ROW = HD * 2 + 16;                      // LDS row of a token (padded: conflict-free column reads)
  constexpr int IN = SA_VT_CHUNKS * SA_CHUNK * PIECES;  // input pieces of the workgroup
  constexpr int OUT = SA_VT_CHUNKS * HD * 4;            // output pieces: (chunk, dim, 8-slot group)
  static_assert(IN % 256 == 0 && OUT % 256 == 0, "pieces must split over the threads");
  __shared__ __attribute__((aligned(16))) char tile[SA_VT_CHUNKS * SA_CHUNK * ROW];
  __shared__ uint32_t red[4];
  const int bg = blockIdx.y;
  const int b = bg / Hkv, g = bg % Hkv;
  const int c0 = blockIdx.x * SA_VT_CHUNKS;

  // the workgroup's tokens, row-major as in v (one latency for all of them)
  u32x4_t val[IN / 256];
#pragma unroll
  for (int i = 0; i < IN / 256; ++i) {
    const int q = threadIdx.x + 256 * i;
    const int t = c0 * SA_CHUNK + q / PIECES, piece = q % PIECES;
    val[i] = u32x4_t{0u, 0u, 0u, 0u};
    if (t < T) val[i] = *reinterpret_cast<const u32x4_t*>(v + b * vs_b + g * vs_g + t * vs_t + 8 * piece);
  }
  uint32_t m = 0;
  for (int c = threadIdx.x; c < n32; c += 256) {
    const uint32_t x = cmax[static_cast<int64_t>(bg) * n32 + c];
    m = x > m ? x : m;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const uint32_t o = __shfl_xor(m, off, 64);
    m = o > m ? o : m;
  }
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
#pragma unroll
  for (int i = 0; i < IN / 256; ++i) {
    const int q = threadIdx.x + 256 * i;
    *reinterpret_cast<u32x4_t*>(tile + (q / PIECES) * ROW + (q % PIECES) * 16) = val[i];
  }
  __syncthreads();
  m = red[0];
#pragma unroll
  for (int w = 1; w < 4; ++w) m = red[w] > m ? red[w] : m;
  const int e = sa_head_exponent(m);
  if (blockIdx.x == 0 && threadIdx.x == 0) head_e[bg] = e;
  const float sc = __builtin_ldexpf(1.f, -e);  // exact power of two

  // output piece (chunk cc, dim d, slots 8 k .. 8 k + 7): slot 8 k + j holds token
  // 16 (j >> 2) + 4 k + (j & 3) (the inverse of sa_slot)
#pragma unroll
  for (int i = 0; i < OUT / 256; ++i) {
    const int q = threadIdx.x + 256 * i;
    const int cc = q / (HD * 4), r = q % (HD * 4);
    const int d = r >> 2, k = r & 3;
    const int c = c0 + cc;
    if (c >= n32) continue;
    uint32_t w[4];
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      uint16_t h2[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int j = 2 * jj + u;
        const int tau = 16 * (j >> 2) + 4 * k + (j & 3);
        const uint16_t bits = *reinterpret_cast<const uint16_t*>(tile + (cc * SA_CHUNK + tau) * ROW + 2 * d);
        const float f = __uint_as_float(static_cast<uint32_t>(bits) << 16);
        h2[u] = __builtin_bit_cast(uint16_t, static_cast<_Float16>(f * sc));
      }
      w[jj] = static_cast<uint32_t>(h2[0]) | (static_cast<uint32_t>(h2[1]) << 16);
    }
    *reinterpret_cast<u32x4_t*>(vt + ((static_cast<int64_t>(bg) * n32 + c) * HD + d) * SA_CHUNK + 8 * k) =
        u32x4_t{w[0], w[1], w[2], w[3]};
  }
}

struct SAParams {
  const bf16_t* q;
  int64_t qs_b, qs_h, qs_t;
  const bf16_t* k;
  int64_t ks_b, ks_h, ks_t;
  const bf16_t* vt;  // workspace copy of v (fp16, scaled by 2^-head_e, for sparse_attn_lds_kernel)
  const int32_t* head_e;  // (B, Hkv) exponents of the fp16 copy
  int B, Hq, Hkv, G, T, n32, block, mode, window;
  const int32_t* lists;  // (B, Qb, cap) page / block ids, strides ls_b, ls_q
  int64_t ls_b, ls_q;
  const int32_t* counts;  // (B, Qb), strides cs_b, cs_q
  int64_t cs_b, cs_q;
  int cap, n_blocks;  // list capacity; key blocks in [0, n_blocks)
  float scale_log2;
  bf16_t* out;
  int64_t os_b, os_h, os_t;
  int* err;
};

// chunk descriptor: absolute chunk index << 16 | local << 12 | hi << 6 | lo, with
// [lo, hi) the chunk's keys taken (a chunk whose range is empty is skipped)
__device__ __forceinline__ int64_t sa_desc(int64_t c, int lo, int hi, int local) {
  return (c << 16) | (static_cast<int64_t>(local) << 12) | (static_cast<int64_t>(hi) << 6) | lo;
}

template <int HD>
__global__ __launch_bounds__(64 * SA_WAVES) void sparse_attn_kernel(SAParams P) {
  constexpr int KS = (HD + 31) / 32;  // k-steps of S^T (head_dim 16 pads dims 16..31 with 0)
  constexpr int DT = HD / 16;         // dim tiles of O^T
  constexpr int KL = 2 * KS;          // K loads per chunk
  constexpr bool NARROW = HD < 32;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int q0 = blockIdx.x * 16;
  const int per_g = (P.G + SA_WAVES - 1) / SA_WAVES;
  int y = blockIdx.y;
  const int hsub = y % per_g;
  y /= per_g;
  const int g = y % P.Hkv;
  const int b = y / P.Hkv;
  const int hg = hsub * SA_WAVES + wave;
  if (hg >= P.G) return;  // whole wave; no barriers in this kernel
  const int h = g * P.G + hg;
  const int r = lane & 15, grp = lane >> 4;
  const bool dims_live = !NARROW || grp < 2;  // this lane's 8 dims of each k-step exist
  const int qb = q0 / P.block;
  const int myq = q0 + r;  // this lane's query column

  // ---- chunk list: local window chunks, then the chunks of the listed blocks ----
  int cnt = P.counts[b * P.cs_b + qb * P.cs_q];
  cnt = cnt < 0 ? 0 : (cnt > P.cap ? P.cap : cnt);
  int n_local = 0, c_lo = 0;
  if (P.mode == FSI_SATTN_LOCAL_REMOTE) {
    const int klo = q0 - P.window + 1 > 0 ? q0 - P.window + 1 : 0;
    const int khi = q0 + 15 < P.T - 1 ? q0 + 15 : P.T - 1;
    c_lo = klo / SA_CHUNK;
    n_local = khi / SA_CHUNK - c_lo + 1;
  }
  const int per_block = (P.block + SA_CHUNK - 1) / SA_CHUNK + 1;  // chunk slots per listed block
  const int n_chunks = n_local + cnt * per_block;

  const int32_t* list = P.lists + b * P.ls_b + qb * P.ls_q;

  // Q^T operand: lane supplies Q[q0 + r][32 ks + 8 grp .. +8] (rows past T read row T - 1)
  u32x4_t qop[KS];
  {
    const int qq = myq < P.T ? myq : P.T - 1;
    const bf16_t* qp = P.q + b * P.qs_b + h * P.qs_h + static_cast<int64_t>(qq) * P.qs_t + 8 * grp;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      qop[ks] = dims_live ? *reinterpret_cast<const u32x4_t*>(qp + 32 * ks) : u32x4_t{0u, 0u, 0u, 0u};
  }
  const bf16_t* kbase = P.k + b * P.ks_b + g * P.ks_h + 8 * grp;
  const bf16_t* vtbase = P.vt + (static_cast<int64_t>(b) * P.Hkv + g) * P.n32 * HD * SA_CHUNK + 8 * grp;

  f32x4_t acc[DT];
#pragma unroll
  for (int i = 0; i < DT; ++i) acc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;

  for (int pass0 = 0; pass0 < n_chunks; pass0 += 64) {
    // lane i describes chunk pass0 + i
    int64_t desc = 0;  // empty range: skipped
    {
      const int i = pass0 + lane;
      if (i < n_local) {
        desc = sa_desc(c_lo + i, 0, SA_CHUNK, 1);
      } else if (i < n_chunks) {
        const int slot = (i - n_local) / per_block, part = (i - n_local) % per_block;
        const int blk = list[slot];
        bool ok = blk >= 0 && blk < P.n_blocks;
        if (!ok && P.err) set_error(P.err, FSI_ERR_INDEX_RANGE);
        if (ok && P.mode == FSI_SATTN_LOCAL_REMOTE) {
          // the mask is a union: a page listed twice counts once
          for (int s2 = 0; s2 < slot; ++s2) ok = ok && list[s2] != blk;
        }
        if (ok) {
          const int k0 = blk * P.block;
          const int k1 = k0 + P.block < P.T ? k0 + P.block : P.T;
          const int c = k0 / SA_CHUNK + part;
          const int lo = k0 - c * SA_CHUNK > 0 ? k0 - c * SA_CHUNK : 0;
          const int hi = k1 - c * SA_CHUNK < SA_CHUNK ? k1 - c * SA_CHUNK : SA_CHUNK;
          if (hi > lo) desc = sa_desc(c, lo, hi, 0);
        }
      }
    }
    const int n_here = n_chunks - pass0 < 64 ? n_chunks - pass0 : 64;

    u32x4_t kc[KL], vc[DT];
    auto load_chunk = [&](int64_t d, u32x4_t (&kr)[KL], u32x4_t (&vr)[DT]) {
      const int64_t c = d >> 16;
#pragma unroll
      for (int tile = 0; tile < 2; ++tile) {
        int key = static_cast<int>(c * SA_CHUNK) + 16 * tile + r;
        key = key < P.T ? key : P.T - 1;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
          kr[tile * KS + ks] = dims_live ? *reinterpret_cast<const u32x4_t*>(kbase + static_cast<int64_t>(key) * P.ks_t +
                                                                                32 * ks)
                                         : u32x4_t{0u, 0u, 0u, 0u};
      }
      const bf16_t* vp = vtbase + c * HD * SA_CHUNK;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) vr[dt] = *reinterpret_cast<const u32x4_t*>(vp + (16 * dt + r) * SA_CHUNK);
    };

    for (int i = 0; i < n_here; ++i) {
      const uint32_t dlo = __builtin_amdgcn_readlane(static_cast<uint32_t>(desc), i);
      const uint32_t dhi = __builtin_amdgcn_readlane(static_cast<uint32_t>(desc >> 32), i);
      const int64_t d = static_cast<int64_t>((static_cast<uint64_t>(dhi) << 32) | dlo);
      const int lo = static_cast<int>(d & 63), hi = static_cast<int>((d >> 6) & 63);
      if (hi <= lo) continue;  // uniform
      const bool local = ((d >> 12) & 1) != 0;
      const int kc0 = static_cast<int>((d >> 16) * SA_CHUNK);
      load_chunk(d, kc, vc);

      f32x4_t st[2];
#pragma unroll
      for (int tile = 0; tile < 2; ++tile) {
        st[tile] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) st[tile] = mfma16x16x32(kc[tile * KS + ks], qop[ks], st[tile]);
      }
      // lane holds keys kc0 + 16 tile + 4 grp + j for query myq
      float sv[8];
      float mx = -INFINITY;
#pragma unroll
      for (int tile = 0; tile < 2; ++tile)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int tau = 16 * tile + 4 * grp + j;
          const int key = kc0 + tau;
          bool ok = tau >= lo && tau < hi && key < P.T;
          if (P.mode == FSI_SATTN_LOCAL_REMOTE) {
            const bool in_win = key <= myq && key > myq - P.window;
            ok = ok && (local ? in_win : !in_win);
          }
          const float v = ok ? st[tile][j] * P.scale_log2 : -INFINITY;
          sv[tile * 4 + j] = v;
          mx = fmaxf(mx, v);
        }
      mx = max_rows4(mx);
      const float m_new = fmaxf(m_run, mx);
      float alpha = 1.f, psum = 0.f;
      uint32_t pk_hi[4], pk_lo[4];
      if (m_new == -INFINITY) {  // nothing valid yet for this query
#pragma unroll
        for (int w = 0; w < 4; ++w) pk_hi[w] = pk_lo[w] = 0u;
      } else {
        alpha = exp2f(m_run - m_new);
        float phi[8], plo[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float pe = exp2f(sv[e] - m_new);
          psum += pe;
          phi[e] = round_bf16(pe);
          plo[e] = pe - phi[e];
        }
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          pk_hi[w] = pack_bf16x2(phi[2 * w], phi[2 * w + 1]);
          pk_lo[w] = pack_bf16x2(plo[2 * w], plo[2 * w + 1]);
        }
      }
      psum = sum_rows4(psum);
      l_run = l_run * alpha + psum;
      m_run = m_new;
      const u32x4_t pbh = u32x4_t{pk_hi[0], pk_hi[1], pk_hi[2], pk_hi[3]};
      const u32x4_t pbl = u32x4_t{pk_lo[0], pk_lo[1], pk_lo[2], pk_lo[3]};
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[dt][j] *= alpha;
        acc[dt] = mfma16x16x32(vc[dt], pbh, acc[dt]);
        acc[dt] = mfma16x16x32(vc[dt], pbl, acc[dt]);
      }
    }
  }

  // lane holds O^T[16 dt + 4 grp + j][query r]
  if (myq < P.T) {
    const float inv = l_run > 0.f ? 1.f / l_run : 0.f;
    bf16_t* o = P.out + b * P.os_b + h * P.os_h + static_cast<int64_t>(myq) * P.os_t + 4 * grp;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const u32x2_t w = u32x2_t{pack_bf16x2(acc[dt][0] * inv, acc[dt][1] * inv),
                                pack_bf16x2(acc[dt][2] * inv, acc[dt][3] * inv)};
      *reinterpret_cast<u32x2_t*>(o + 16 * dt) = w;
    }
  }
}


// ---------------------------------------------------------------------------
// LDS variant for query blocks of a multiple of 64 (FovealSparseAttention's
// pages; power-of-two block, at most 64 listed pages, positive scale).  A
// workgroup is the GQA group's query heads (up to 4) at 64 queries: 8 waves,
// each one head x SAL_QT query tiles (32 queries at SAL_QT = 2, two waves per
// SIMD; 4 tiles at one wave per SIMD measured 2.53 vs 1.63 ms at 16K tokens).
// Every 32-key chunk (K rows and the V^T copy) is moved once per workgroup
// into a ring of LDS stages with direct-to-LDS loads, SAL_AHEAD chunks ahead,
// and read from there by all 8 waves: a chunk serves 4 heads x 64 queries.  The
// 16-byte pieces of each LDS row are XOR-swizzled so the 16 rows of a fragment
// read fall on 16 different bank groups.  Q^T operands stay in registers.  The
// block's remote pages are checked, de-duplicated and compacted once; chunks
// are described by wave-uniform scalar code.  Per chunk the S^T tiles of all
// query tiles are formed first, then their softmax, then the P V products, so
// consecutive MFMAs are independent.  The softmax skips the per-key mask for
// chunks every query sees, moves its running max only by jumps above 2^8
// (rescaling the accumulators rarely), and packs P in fp16 for one f16 MFMA
// per P V tile against the fp16 V^T copy (sa_vt16_kernel); the softmax
// denominators are one more MFMA per query tile.  Query blocks run from the last
// (most keys) to the first.
// ---------------------------------------------------------------------------
// Two fp32 values to a packed bf16 pair (round to nearest even) with gfx950's
// v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t cvt_pk_bf16(float a, float b) {
  typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2_t;
  const bf16x2_t v = {static_cast<__bf16>(a), static_cast<__bf16>(b)};
  return __builtin_bit_cast(uint32_t, v);
}

// v_mfma_f32_16x16x32_f16 with the operand layout of mfma16x16x32.
__device__ __forceinline__ f32x4_t mfma16x16x32_f16(const u32x4_t& a, const u32x4_t& b, f32x4_t c) {
  typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c, 0,
                                                0, 0);
}

#ifndef FSI_SAL_QT
#define FSI_SAL_QT 2
#endif
// With one pair per barrier (FSI_SAL_GROUP=1), 64-key pairs loaded ahead of the one
// computed: 1 (a 2-pair ring, 64 KiB) measured 0.9 % faster than 2 at 16K tokens in
// alternating runs on one box, 3 within noise
#ifndef FSI_SAL_AHEAD
#define FSI_SAL_AHEAD 1
#endif
constexpr int SAL_QT = FSI_SAL_QT;           // query tiles per wave
constexpr int SAL_HALVES = 4 / SAL_QT;       // waves per query head (64 queries split)
constexpr int SAL_WAVES = 4 * SAL_HALVES;    // 4 query heads per workgroup
constexpr int SAL_MAX_CAP = 64;              // listed pages per query block
// Pairs computed per workgroup barrier: G > 1 loads the next G pairs while the
// current G are computed (one barrier and one wait per group, a ring of 2 G pairs).
// G = 2 (a 128 KiB ring) measured 0.820-0.823 against 0.824-0.827 ms for one pair per
// barrier and one pair ahead, in four alternating pairs of 100-step runs.
#ifndef FSI_SAL_GROUP
#define FSI_SAL_GROUP 2
#endif
constexpr int SAL_GROUP = FSI_SAL_GROUP;
constexpr int SAL_AHEAD = SAL_GROUP > 1 ? SAL_GROUP : FSI_SAL_AHEAD;  // 64-key stages in flight ahead
constexpr int SAL_RING = SAL_GROUP > 1 ? 2 * SAL_GROUP : SAL_AHEAD + 1;  // 64-key pairs held by the LDS ring
constexpr int SAL_SLOTS = 2 * SAL_RING;       // 32-key chunk slots of the LDS ring
typedef __attribute__((address_space(3))) void sal_lds_t;
typedef __attribute__((address_space(1))) void sal_glb_t;

template <int N>
__device__ __forceinline__ void sal_wait_vmcnt() {
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}
__device__ __forceinline__ void sal_barrier() { asm volatile("s_barrier" ::: "memory"); }
// Keeps the compiler's scheduler from moving instructions across this point: the
// fragment reads issued before it stay ahead of the MFMAs / softmax after it.
#ifndef FSI_SAL_PF
#define FSI_SAL_PF 1
#endif
__device__ __forceinline__ void sal_order() {
#if FSI_SAL_PF
  __builtin_amdgcn_sched_barrier(0);
#endif
}

// Largest of 16 scores (finite or -inf) in 8 v_max3_f32 (max3_raw: no operand quieting).
__device__ __forceinline__ float sal_max16(const float* v) {
  const float a = max3_raw(v[0], v[1], v[2]), b = max3_raw(v[3], v[4], v[5]), c = max3_raw(v[6], v[7], v[8]);
  const float d = max3_raw(v[9], v[10], v[11]), e = max3_raw(v[12], v[13], v[14]);
  const float f = max3_raw(a, b, c), g = max3_raw(d, e, v[15]);
  return max3_raw(f, g, g);
}

template <int HD>
__global__ __launch_bounds__(64 * SAL_WAVES) void sparse_attn_lds_kernel(SAParams P) {
  constexpr int KS = HD / 32;
  constexpr int DT = HD / 16;
  constexpr int KROW = HD * 2;                  // bytes of one key row
  constexpr int KBYTES = SA_CHUNK * KROW;       // K rows of a chunk
  constexpr int VBYTES = HD * SA_CHUNK * 2;     // V^T of a chunk: HD rows of 64 B
  constexpr int SLOT = KBYTES + VBYTES;         // one 32-key chunk in LDS
  constexpr int LOADS = SLOT / 1024;            // 1 KiB direct loads per chunk
  constexpr int LPW = LOADS / SAL_WAVES;        // per wave
  static_assert(LPW >= 1 && LOADS % SAL_WAVES == 0, "chunk loads must split over the waves");
  static_assert(KBYTES % (1024 * LPW) == 0, "a wave's loads of a chunk are all K or all V^T");
  constexpr int KPR = KROW / 16;                // 16-byte pieces per key row
  // One LDS array holds the chunk ring and the block list.  Separate __shared__
  // arrays would get alias scopes, and the compiler would then make every ring
  // read wait for all direct loads in flight (vmcnt(0)), including the chunks
  // issued ahead; with one array the explicit waits below order the ring.
  __shared__ __attribute__((aligned(1024))) char smem[SAL_SLOTS * SLOT + SAL_MAX_CAP * 4];
  char (*ring)[SLOT] = reinterpret_cast<char (*)[SLOT]>(smem);
  int* wl = reinterpret_cast<int*>(smem + SAL_SLOTS * SLOT);

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int qblk0 = (gridDim.x - 1 - blockIdx.x) * 64;  // the workgroup's 64 queries
  const int half = wave / 4;                               // this wave's part of them
  const int q0 = qblk0 + half * 16 * SAL_QT;
  const int per_g = (P.G + 3) / 4;
  int y = blockIdx.y;
  const int hsub = y % per_g;
  y /= per_g;
  const int g = y % P.Hkv;
  const int b = y / P.Hkv;
  const int hg = hsub * 4 + (wave & 3);
  const bool head_live = hg < P.G;  // idle waves still load and meet the barriers
  const int h = g * P.G + (head_live ? hg : 0);
  const int r = lane & 15, grp = lane >> 4;
  const int qb = qblk0 / P.block;
  const float vscale = __builtin_ldexpf(1.f, P.head_e[b * P.Hkv + g]);  // undoes the fp16 copy's 2^-e
  const float sl2 = P.scale_log2, inv_sl2 = 1.f / P.scale_log2;

  // ---- listed pages: validity, first-listing de-duplication, compaction ----
  int cnt = P.counts[b * P.cs_b + qb * P.cs_q];
  cnt = cnt < 0 ? 0 : (cnt > P.cap ? P.cap : cnt);
  const int32_t* list = P.lists + b * P.ls_b + qb * P.ls_q;
  const int myblk = lane < cnt ? list[lane] : -1;
  bool okl = lane < cnt && myblk >= 0 && myblk < P.n_blocks;
  if (wave == 0 && lane < cnt && !okl && P.err) set_error(P.err, FSI_ERR_INDEX_RANGE);
  if (P.mode == FSI_SATTN_LOCAL_REMOTE) {
    // the mask is a union: a page listed twice counts once
    for (int s2 = 0; s2 < SAL_MAX_CAP; ++s2) {
      if (s2 >= cnt) break;  // uniform
      const int other = __builtin_amdgcn_readlane(myblk, s2);
      okl = okl && !(s2 < lane && other == myblk);
    }
  }
  const uint64_t vmask = __ballot(okl);
  if (wave == 0 && okl) wl[__popcll(vmask & ((uint64_t(1) << lane) - 1))] = myblk;
  const int n_remote = __popcll(vmask);

  // local window chunks [c_lo, c_hi], walked in 64-key pairs from the even chunk c_lo2
  int n_lp = 0, c_lo = 0, c_hi = -1, c_lo2 = 0;
  if (P.mode == FSI_SATTN_LOCAL_REMOTE) {
    const int klo = qblk0 - P.window + 1 > 0 ? qblk0 - P.window + 1 : 0;
    const int khi = qblk0 + 63 < P.T - 1 ? qblk0 + 63 : P.T - 1;
    c_lo = klo / SA_CHUNK;
    c_hi = khi / SA_CHUNK;
    c_lo2 = c_lo & ~1;
    n_lp = (c_hi - c_lo2) / 2 + 1;
  }
  const int pp_block = P.block / (2 * SA_CHUNK);  // 64-key pairs per page, a power of two (host-checked)
  const int pp_shift = __builtin_ctz(pp_block);
  const int n_pairs = n_lp + n_remote * pp_block;
  __syncthreads();  // wl is written
  // Each wave keeps, per listed page (lane i: entry i), the page's first chunk and
  // its number of keys inside the sequence, and reads them with v_readlane: an LDS
  // read inside the loop would make the compiler wait for every direct-to-LDS
  // chunk load in flight before the loop's LDS reads.
  const int blk_j = lane < n_remote ? wl[lane] : 0;
  const int pg_c0 = blk_j * (P.block / SA_CHUNK);
  const int pg_len = P.T - blk_j * P.block < P.block ? P.T - blk_j * P.block : P.block;

  // pair p: chunks c0 and c0 + 1, of which keys [0, hi0) and [0, hi1) are taken
  // (local pairs take whole chunks; keys past the sequence are masked)
  auto describe = [&](int p, int& c0, int& hi0, int& hi1, bool& local) {
    if (p < n_lp) {
      c0 = c_lo2 + 2 * p;
      hi0 = c0 >= c_lo ? SA_CHUNK : 0;
      hi1 = c0 + 1 <= c_hi ? SA_CHUNK : 0;
      local = true;
    } else {
      const int j = p - n_lp;
      const int pg = j >> pp_shift, sub = j & (pp_block - 1);
      c0 = __builtin_amdgcn_readlane(pg_c0, pg) + 2 * sub;
      const int len = __builtin_amdgcn_readlane(pg_len, pg) - 2 * SA_CHUNK * sub;
      hi0 = len <= 0 ? 0 : (len > SA_CHUNK ? SA_CHUNK : len);
      hi1 = len <= SA_CHUNK ? 0 : (len > 2 * SA_CHUNK ? SA_CHUNK : len - SA_CHUNK);
      local = false;
    }
  };

  // ---- direct loads of chunk c into ring slot sl: this wave's LPW KiB of it ----
  const char* kbase = reinterpret_cast<const char*>(P.k + b * P.ks_b + g * P.ks_h);
  const char* vtbase =
      reinterpret_cast<const char*>(P.vt + (static_cast<int64_t>(b) * P.Hkv + g) * P.n32 * HD * SA_CHUNK);
  // Per-lane byte offsets, fixed for the whole kernel: load i of this wave is K
  // row krow[i] / 16-byte piece, or V^T row / piece of the chunk.  Whether a load
  // is K or V^T depends on the wave only, so the base pointer is scalar.
  const bool wave_k = wave * LPW * 1024 < KBYTES;
  uint32_t loff[LPW];
  int krow[LPW];
#pragma unroll
  for (int i = 0; i < LPW; ++i) {
    const int off = (wave * LPW + i) * 1024 + lane * 16;  // byte offset in the slot
    if (wave_k) {
      const int row = off / KROW, slot = (off % KROW) / 16;  // key row, 16-byte slot
      krow[i] = row;
      loff[i] = static_cast<uint32_t>(row * P.ks_t * 2 + 16 * (slot ^ (row & (KPR - 1) & 15)));
    } else {
      const int vo = off - KBYTES;
      const int row = vo / 64, slot = (vo % 64) / 16;  // V^T row (dim), 16-byte slot
      krow[i] = 0;
      loff[i] = static_cast<uint32_t>(row * SA_CHUNK * 2 + 16 * (slot ^ ((row >> 1) & 3)));
    }
  }
  auto issue = [&](int c, int sl) {
    c = c < P.n32 - 1 ? c : P.n32 - 1;  // an empty chunk past the sequence loads the last one
    const char* base = wave_k ? kbase + static_cast<int64_t>(c) * SA_CHUNK * P.ks_t * 2
                              : vtbase + static_cast<int64_t>(c) * HD * SA_CHUNK * 2;
    sal_lds_t* dst = (sal_lds_t*)(&ring[sl][wave * LPW * 1024]);
    if (!wave_k || (c + 1) * SA_CHUNK <= P.T) {
#pragma unroll
      for (int i = 0; i < LPW; ++i)
        __builtin_amdgcn_global_load_lds((sal_glb_t*)(base + loff[i]), (sal_lds_t*)((char __attribute__((address_space(3)))*)dst + i * 1024), 16, 0, 0);
    } else {  // the sequence's last chunk: rows past T read row T - 1
#pragma unroll
      for (int i = 0; i < LPW; ++i) {
        const int row = c * SA_CHUNK + krow[i] < P.T ? krow[i] : P.T - 1 - c * SA_CHUNK;
        const char* src = base + loff[i] + static_cast<int64_t>(row - krow[i]) * P.ks_t * 2;
        __builtin_amdgcn_global_load_lds((sal_glb_t*)src, (sal_lds_t*)((char __attribute__((address_space(3)))*)dst + i * 1024), 16, 0, 0);
      }
    }
  };

  // Q^T operands in registers for the whole kernel: lane (r, grp) holds
  // Q[query 16 qt + r][32 ks + 8 grp .. +8]
  u32x4_t qreg[SAL_QT][KS];
#pragma unroll
  for (int qt = 0; qt < SAL_QT; ++qt) {
    const int myq = q0 + 16 * qt + r;
    const int qq = myq < P.T ? myq : P.T - 1;
    const bf16_t* qp = P.q + b * P.qs_b + h * P.qs_h + static_cast<int64_t>(qq) * P.qs_t + 8 * grp;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qreg[qt][ks] = *reinterpret_cast<const u32x4_t*>(qp + 32 * ks);
  }
  f32x4_t acc[SAL_QT][DT];
  // Softmax denominators come out of one more MFMA per query tile, against an
  // all-ones fp16 A operand: every row of lsum[qt] is the sum of the same fp16 P
  // the P V product uses, so the rounding of P (toward zero) leaves no bias.
  // The running max (log2 units) starts at a finite -1e30: the first valid score
  // passes its threshold, and masked scores (-inf) give p = 0 without a special case.
  float m_run[SAL_QT], m_thr[SAL_QT];  // m_thr: raw score whose log2-scaled value is m_run + 8
  f32x4_t lsum[SAL_QT];
  const u32x4_t ones = u32x4_t{0x3C003C00u, 0x3C003C00u, 0x3C003C00u, 0x3C003C00u};
#pragma unroll
  for (int qt = 0; qt < SAL_QT; ++qt) {
    m_run[qt] = -1e30f;
    m_thr[qt] = (-1e30f + 8.f) * inv_sl2;
    lsum[qt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < DT; ++i) acc[qt][i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }

  // the Q loads above are this wave's only other vector loads: let them land
  // before the ring's vmcnt accounting starts
  sal_wait_vmcnt<0>();
  for (int p = 0; p < SAL_AHEAD; ++p) {
    if (p >= n_pairs) break;
    int c0, hi0, hi1;
    bool lc;
    describe(p, c0, hi0, hi1, lc);
    issue(c0, 2 * p);
    issue(c0 + 1, 2 * p + 1);
  }

  // Scores of pair p (its slots sl, sl + 1) into st.
  f32x4_t st[2][SAL_QT][2];
  auto scores = [&](int sl) {
    // K fragments of both chunks, all read before the first MFMA (the LDS latency
    // is paid once per pair): lane (r, grp) reads key 16 tile + r, dims 32 ks + 8 grp .. +8
    u32x4_t kf[2][2 * KS];
#pragma unroll
    for (int hc = 0; hc < 2; ++hc)
#pragma unroll
      for (int tile = 0; tile < 2; ++tile)
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const int row = 16 * tile + r;
          kf[hc][tile * KS + ks] = *reinterpret_cast<const u32x4_t*>(
              ring[sl + hc] + row * KROW + 16 * ((4 * ks + grp) ^ (row & (KPR - 1) & 15)));
        }
    sal_order();
    // query tile by query tile, so the softmax of the first can start while the
    // MFMAs of the second run
#pragma unroll
    for (int qt = 0; qt < SAL_QT; ++qt) {
#pragma unroll
      for (int hc = 0; hc < 2; ++hc) st[hc][qt][0] = st[hc][qt][1] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int hc = 0; hc < 2; ++hc)
#pragma unroll
          for (int tile = 0; tile < 2; ++tile)
            st[hc][qt][tile] = mfma16x16x32(kf[hc][tile * KS + ks], qreg[qt][ks], st[hc][qt][tile]);
    }
  };

  // Softmax of the scores in st and the P V products of the pair in slots sl,
  // sl + 1 (chunks c0, c0 + 1 with keys [0, hi0), [0, hi1) taken).
  auto finish = [&](int sl, int c0, int hi0, int hi1, bool local) {
    const int kc0 = c0 * SA_CHUNK;
    // V^T fragments of both chunks, read ahead of the softmax so their LDS latency
    // hides under it: lane (r, grp) reads dim 16 dt + r, slots 8 grp .. +8
    u32x4_t vf[2][DT];
#pragma unroll
    for (int hc = 0; hc < 2; ++hc)
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const int row = 16 * dt + r;
        vf[hc][dt] = *reinterpret_cast<const u32x4_t*>(ring[sl + hc] + KBYTES + row * 64 + 16 * (grp ^ ((row >> 1) & 3)));
      }
    sal_order();
    // Pairs whose keys every query of the wave sees (inside all windows, or a page
    // wholly before them) skip the per-key mask.
    const bool full = hi0 == SA_CHUNK && hi1 == SA_CHUNK;
    const bool nomask =
        full && (local ? (kc0 + 2 * SA_CHUNK - 1 <= q0 && kc0 > q0 + 16 * SAL_QT - 1 - P.window &&
                          kc0 + 2 * SA_CHUNK <= P.T)
                       : (P.mode != FSI_SATTN_LOCAL_REMOTE || kc0 + 2 * SA_CHUNK - 1 <= q0 - P.window));
    float alpha[SAL_QT];
    u32x4_t pb[2][SAL_QT];
#pragma unroll
    for (int qt = 0; qt < SAL_QT; ++qt) {
      const int myq = q0 + 16 * qt + r;
      float sv[16];  // raw scores of chunk hc, key tile t, row j at 8 hc + 4 t + j; -inf where masked
#pragma unroll
      for (int hc = 0; hc < 2; ++hc)
#pragma unroll
        for (int tile = 0; tile < 2; ++tile)
#pragma unroll
          for (int j = 0; j < 4; ++j) sv[8 * hc + 4 * tile + j] = st[hc][qt][tile][j];
      if (!nomask) {
        // Branch-free: a score is kept when its sign word is negative (a taken key
        // inside T, and inside / outside the window for a local / listed pair).
        // wlo >= -1 keeps every difference inside int range.
        // (the lane's key offset passes through an empty asm so the compiler forms
        // these values here instead of holding them in registers across the loop)
        int lk = 4 * grp;
        asm volatile("" : "+v"(lk));
        const int wlo = myq - (P.window < myq + 1 ? P.window : myq + 1);  // window: wlo < key <= myq
        const int wmode = P.mode == FSI_SATTN_LOCAL_REMOTE ? (local ? 1 : 2) : 0;
#pragma unroll
        for (int hc = 0; hc < 2; ++hc)
#pragma unroll
          for (int tile = 0; tile < 2; ++tile)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const int tau = 16 * tile + lk + j;
              const int key = kc0 + SA_CHUNK * hc + tau;
              int keep = (tau - (hc ? hi1 : hi0)) & (key - P.T);
              const int inw = (key - myq - 1) & (wlo - key);
              keep &= wmode == 0 ? -1 : (wmode == 1 ? inw : ~inw);
              sv[8 * hc + 4 * tile + j] = keep < 0 ? sv[8 * hc + 4 * tile + j] : -INFINITY;
            }
      }
      // The running max (log2 units) moves only when a score exceeds it by more
      // than 8: P then stays below 2^8 and the accumulators are rescaled rarely.
      // Most pairs only need to know that no score of the wave passes that
      // threshold (a max3 tree and one compare); the row maxima are formed only
      // when one does.
      float mx = sal_max16(sv);
      alpha[qt] = 1.f;
#ifdef FSI_SAL_ALWAYSMAX
      if (true) {
#else
      if (__ballot(mx > m_thr[qt]) != 0) {  // uniform
#endif
        mx = max_rows4(mx);
        const float m_cand = mx * sl2;
        const bool bump = m_cand > m_run[qt] + 8.f;
        const float m_new = bump ? m_cand : m_run[qt];
        alpha[qt] = bump ? __builtin_amdgcn_exp2f(m_run[qt] - m_new) : 1.f;
        m_run[qt] = m_new;
        // scores above this move the max; scale_log2 > 0 on this kernel's path
        m_thr[qt] = (m_new + 8.f) * inv_sl2;
      }
      uint32_t pk[8];
#pragma unroll
      for (int w = 0; w < 8; ++w) {
        // P in fp16, one v_cvt_pkrtz_f16_f32 per pair (P <= 2^8)
        const float p0 = __builtin_amdgcn_exp2f(fmaf(sv[2 * w], sl2, -m_run[qt]));
        const float p1 = __builtin_amdgcn_exp2f(fmaf(sv[2 * w + 1], sl2, -m_run[qt]));
        pk[w] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(p0, p1));
      }
      pb[0][qt] = u32x4_t{pk[0], pk[1], pk[2], pk[3]};
      pb[1][qt] = u32x4_t{pk[4], pk[5], pk[6], pk[7]};
    }
    // rescale (skipped while no query's running max moved), then P V per chunk
#pragma unroll
    for (int qt = 0; qt < SAL_QT; ++qt) {
      if (__ballot(alpha[qt] != 1.f) != 0) {
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[qt][dt][j] *= alpha[qt];
#pragma unroll
        for (int j = 0; j < 4; ++j) lsum[qt][j] *= alpha[qt];
      }
    }
#pragma unroll
    for (int hc = 0; hc < 2; ++hc) {
      if ((hc ? hi1 : hi0) == 0) continue;  // uniform: an empty chunk (its slot holds other keys)
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int qt = 0; qt < SAL_QT; ++qt) acc[qt][dt] = mfma16x16x32_f16(vf[hc][dt], pb[hc][qt], acc[qt][dt]);
#pragma unroll
      for (int qt = 0; qt < SAL_QT; ++qt) lsum[qt] = mfma16x16x32_f16(ones, pb[hc][qt], lsum[qt]);
    }
  };

#if FSI_SAL_GROUP > 1
  for (int p0 = 0; p0 < n_pairs; p0 += SAL_GROUP) {
    sal_wait_vmcnt<0>();  // this group's pairs landed (nothing else is in flight)
    sal_barrier();
#pragma unroll
    for (int j = 0; j < SAL_GROUP; ++j) {  // the next group into the previous group's slots
      const int pn = p0 + SAL_GROUP + j;
      if (pn < n_pairs) {
        const int sn = 2 * (pn % SAL_RING);
        int n0, nh0, nh1;
        bool nl;
        describe(pn, n0, nh0, nh1, nl);
        issue(n0, sn);
        issue(n0 + 1, sn + 1);
      }
    }
    for (int j = 0; j < SAL_GROUP; ++j) {
      const int p = p0 + j;
      if (p >= n_pairs) break;
      int c0, hi0, hi1;
      bool local;
      describe(p, c0, hi0, hi1, local);
      if ((hi0 | hi1) == 0 || !head_live) continue;  // uniform: an empty pair or an idle wave
      const int sl = 2 * (p % SAL_RING);
      scores(sl);
      finish(sl, c0, hi0, hi1, local);
    }
  }
#else
  for (int p = 0; p < n_pairs; ++p) {
    // pair p landed: at most the loads of pairs p + 1 .. p + AHEAD - 1 remain
    const int later = (p + SAL_AHEAD - 1 < n_pairs - 1 ? p + SAL_AHEAD - 1 : n_pairs - 1) - p;
    if constexpr (SAL_AHEAD >= 3) {
      if (later >= 2) sal_wait_vmcnt<4 * LPW>();
      else if (later == 1) sal_wait_vmcnt<2 * LPW>();
      else sal_wait_vmcnt<0>();
    } else {
      if (later >= 1) sal_wait_vmcnt<2 * LPW>();
      else sal_wait_vmcnt<0>();
    }
    sal_barrier();
    if (p + SAL_AHEAD < n_pairs) {  // into the slots of pair p - 1, which every wave has finished
      const int pn = p + SAL_AHEAD;
      const int sn = 2 * (pn % SAL_RING);
      int n0, nh0, nh1;
      bool nl;
      describe(pn, n0, nh0, nh1, nl);
      issue(n0, sn);
      issue(n0 + 1, sn + 1);
    }
    int c0, hi0, hi1;
    bool local;
    describe(p, c0, hi0, hi1, local);
    if ((hi0 | hi1) == 0 || !head_live) continue;  // uniform: an empty pair or an idle wave
    const int sl = 2 * (p % SAL_RING);
    scores(sl);
    finish(sl, c0, hi0, hi1, local);
  }
#endif

  if (!head_live) return;
#pragma unroll
  for (int qt = 0; qt < SAL_QT; ++qt) {
    const int myq = q0 + 16 * qt + r;
    if (myq < P.T) {
      const float inv = lsum[qt][0] > 0.f ? 1.f / lsum[qt][0] : 0.f;
      bf16_t* o = P.out + b * P.os_b + h * P.os_h + static_cast<int64_t>(myq) * P.os_t + 4 * grp;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const u32x2_t w = u32x2_t{pack_bf16x2(acc[qt][dt][0] * inv * vscale, acc[qt][dt][1] * inv * vscale),
                                  pack_bf16x2(acc[qt][dt][2] * inv * vscale, acc[qt][dt][3] * inv * vscale)};
        *reinterpret_cast<u32x2_t*>(o + 16 * dt) = w;
      }
    }
  }
}

}  // namespace

extern "C" {

FSI_API size_t fsi_sparse_attn_workspace_size(int64_t B, int64_t Hkv, int64_t T, int64_t head_dim) {
  if (B <= 0 || Hkv <= 0 || T <= 0 || head_dim <= 0) return FSI_WORKSPACE_COUNTER_BYTES;
  const int64_t n32 = (T + SA_CHUNK - 1) / SA_CHUNK;
  // V^T copy (fp16 / bf16, or fp32 for the fp32 kernel: 4 bytes an element are
  // reserved either way), the per-chunk maxima and the per-head exponents
  return FSI_WORKSPACE_COUNTER_BYTES +
         fsi_host::align_up(sizeof(float) * static_cast<size_t>(B * Hkv * n32 * SA_CHUNK * head_dim), 256) +
         fsi_host::align_up(sizeof(uint32_t) * static_cast<size_t>(B * Hkv * n32), 256) +
         fsi_host::align_up(sizeof(int32_t) * static_cast<size_t>(B * Hkv), 256);
}

FSI_API int fsi_sparse_attn(const void* q, int64_t qs_b, int64_t qs_h, int64_t qs_t, const void* k, int64_t ks_b,
                            int64_t ks_h, int64_t ks_t, const void* v, int64_t vs_b, int64_t vs_h, int64_t vs_t,
                            int64_t B, int64_t Hq, int64_t Hkv, int64_t T, int64_t head_dim, int64_t block, int mode,
                            int64_t window, const int32_t* lists, int64_t ls_b, int64_t ls_q, int64_t capacity,
                            const int32_t* counts, int64_t cs_b, int64_t cs_q, float scale, int dtype, void* out,
                            int64_t os_b, int64_t os_h, int64_t os_t, void* workspace, size_t workspace_bytes,
                            int* err, void* stream) {
  using namespace fsi_host;
  FSI_CHECK_ARG(mode == FSI_SATTN_LOCAL_REMOTE || mode == FSI_SATTN_BLOCK_LIST, FSI_ERR_INVALID_ARG,
                "sparse_attn: mode %d", mode);
  // fp32, blocks that are not multiples of 16, other head dims and unaligned
  // operands run the generic kernel (csrc/attn_generic.hip)
  const bool mfma_path =
      dtype == FSI_DTYPE_BF16 && block > 0 && block % 16 == 0 &&
      (head_dim == 16 || head_dim == 32 || head_dim == 64 || head_dim == 128) && qs_t % 8 == 0 && qs_h % 8 == 0 &&
      qs_b % 8 == 0 && ks_t % 8 == 0 && ks_h % 8 == 0 && ks_b % 8 == 0 && vs_t % 8 == 0 && vs_h % 8 == 0 &&
      vs_b % 8 == 0 && os_t % 4 == 0 && os_h % 4 == 0 && os_b % 4 == 0 &&
      reinterpret_cast<uintptr_t>(q) % 16 == 0 && reinterpret_cast<uintptr_t>(k) % 16 == 0 &&
      reinterpret_cast<uintptr_t>(v) % 16 == 0 && reinterpret_cast<uintptr_t>(out) % 8 == 0;
  if (dtype == FSI_DTYPE_F32 && B > 0 && T > 0 && Hkv > 0 && Hq > 0 && Hq % Hkv == 0 && capacity >= 0 &&
      (mode != FSI_SATTN_LOCAL_REMOTE || window > 0) && q && k && v && out && counts && (lists || capacity == 0) &&
      workspace && workspace_bytes >= fsi_sparse_attn_workspace_size(B, Hkv, T, head_dim)) {
    // fp32 on MFMA when the shape fits the 64-query kernel (csrc/sparse_attn_f32.hip)
    const int rc = fsi_attn_f32::sparse_attn(
        static_cast<const float*>(q), qs_b, qs_h, qs_t, static_cast<const float*>(k), ks_b, ks_h, ks_t,
        static_cast<const float*>(v), vs_b, vs_h, vs_t, B, Hq, Hkv, T, head_dim, block, mode, window, lists, ls_b,
        ls_q, capacity, counts, cs_b, cs_q, scale, static_cast<float*>(out), os_b, os_h, os_t,
        reinterpret_cast<float*>(static_cast<char*>(workspace) + FSI_WORKSPACE_COUNTER_BYTES), err,
        reinterpret_cast<hipStream_t>(stream));
    if (rc != 1) return rc;
  }
  if (!mfma_path) {
    FSI_CHECK_ARG(B > 0 && T > 0 && Hkv > 0 && Hq > 0 && Hq % Hkv == 0, FSI_ERR_SHAPE,
                  "sparse_attn: B=%lld T=%lld Hq=%lld Hkv=%lld", (long long)B, (long long)T, (long long)Hq,
                  (long long)Hkv);
    FSI_CHECK_ARG(capacity >= 0 && capacity <= 4096, FSI_ERR_CAPACITY, "sparse_attn: capacity %lld",
                  (long long)capacity);
    FSI_CHECK_ARG(mode != FSI_SATTN_LOCAL_REMOTE || window > 0, FSI_ERR_SHAPE, "sparse_attn: window %lld",
                  (long long)window);
    FSI_CHECK_ARG(q && k && v && out && counts && (lists || capacity == 0), FSI_ERR_INVALID_ARG,
                  "sparse_attn: null pointer");
    return fsi_attn_generic::sparse_attn(q, qs_b, qs_h, qs_t, k, ks_b, ks_h, ks_t, v, vs_b, vs_h, vs_t, B, Hq, Hkv, T,
                                         head_dim, block, mode, window, lists, ls_b, ls_q, capacity, counts, cs_b,
                                         cs_q, scale, dtype, out, os_b, os_h, os_t, err, stream);
  }
  FSI_CHECK_ARG(head_dim == 16 || head_dim == 32 || head_dim == 64 || head_dim == 128, FSI_ERR_SHAPE,
                "sparse_attn: head_dim %lld (16, 32, 64 or 128)", (long long)head_dim);
  FSI_CHECK_ARG(B > 0 && T > 0 && Hkv > 0 && Hq > 0 && Hq % Hkv == 0, FSI_ERR_SHAPE,
                "sparse_attn: B=%lld T=%lld Hq=%lld Hkv=%lld", (long long)B, (long long)T, (long long)Hq,
                (long long)Hkv);
  FSI_CHECK_ARG(block > 0 && block % 16 == 0, FSI_ERR_SHAPE, "sparse_attn: block %lld must be a multiple of 16",
                (long long)block);
  FSI_CHECK_ARG(capacity >= 0 && capacity <= 4096, FSI_ERR_CAPACITY, "sparse_attn: capacity %lld",
                (long long)capacity);
  FSI_CHECK_ARG(mode != FSI_SATTN_LOCAL_REMOTE || window > 0, FSI_ERR_SHAPE, "sparse_attn: window %lld",
                (long long)window);
  FSI_CHECK_ARG(T <= (int64_t(1) << 30) && B * Hkv * ((Hq / Hkv + SA_WAVES - 1) / SA_WAVES) <= 65535, FSI_ERR_SHAPE,
                "sparse_attn: sizes beyond range");
  FSI_CHECK_ARG(q && k && v && out && counts && (lists || capacity == 0), FSI_ERR_INVALID_ARG,
                "sparse_attn: null pointer");
  FSI_CHECK_ARG(qs_t % 8 == 0 && qs_h % 8 == 0 && qs_b % 8 == 0 && ks_t % 8 == 0 && ks_h % 8 == 0 &&
                    ks_b % 8 == 0 && vs_t % 8 == 0 && vs_h % 8 == 0 && vs_b % 8 == 0 && os_t % 4 == 0 &&
                    os_h % 4 == 0 && os_b % 4 == 0,
                FSI_ERR_ALIGN, "sparse_attn: strides must be multiples of 8 elements (out: 4)");
  FSI_CHECK_ARG(reinterpret_cast<uintptr_t>(q) % 16 == 0 && reinterpret_cast<uintptr_t>(k) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(v) % 16 == 0 && reinterpret_cast<uintptr_t>(out) % 8 == 0,
                FSI_ERR_ALIGN, "sparse_attn: q, k, v 16-byte and out 8-byte aligned");
  FSI_CHECK_ARG(B * Hkv * ((T + SA_CHUNK - 1) / SA_CHUNK) <= (int64_t(1) << 32), FSI_ERR_SHAPE,
                "sparse_attn: B x Hkv x T / 32 = %lld chunks beyond the grid", (long long)(B * Hkv * ((T + 31) / 32)));
  const size_t need = fsi_sparse_attn_workspace_size(B, Hkv, T, head_dim);
  FSI_CHECK_ARG(workspace && workspace_bytes >= need, FSI_ERR_WORKSPACE, "sparse_attn: workspace %zu < %zu",
                workspace_bytes, need);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int n32 = static_cast<int>((T + SA_CHUNK - 1) / SA_CHUNK);
  char* wsp = static_cast<char*>(workspace) + FSI_WORKSPACE_COUNTER_BYTES;
  bf16_t* vt = reinterpret_cast<bf16_t*>(wsp);
  wsp += fsi_host::align_up(sizeof(float) * static_cast<size_t>(B * Hkv * n32 * SA_CHUNK * head_dim), 256);
  uint32_t* cmax = reinterpret_cast<uint32_t*>(wsp);
  wsp += fsi_host::align_up(sizeof(uint32_t) * static_cast<size_t>(B * Hkv * n32), 256);
  int32_t* head_e = reinterpret_cast<int32_t*>(wsp);
  const int64_t vt_items = B * Hkv * static_cast<int64_t>(n32) * SA_CHUNK * (head_dim / 8);
  const unsigned g1 = static_cast<unsigned>(std::min<int64_t>((vt_items + 255) / 256, 1 << 20));

  SAParams P{};
  P.q = static_cast<const bf16_t*>(q);
  P.qs_b = qs_b;
  P.qs_h = qs_h;
  P.qs_t = qs_t;
  P.k = static_cast<const bf16_t*>(k);
  P.ks_b = ks_b;
  P.ks_h = ks_h;
  P.ks_t = ks_t;
  P.vt = vt;
  P.head_e = head_e;
  P.B = static_cast<int>(B);
  P.Hq = static_cast<int>(Hq);
  P.Hkv = static_cast<int>(Hkv);
  P.G = static_cast<int>(Hq / Hkv);
  P.T = static_cast<int>(T);
  P.n32 = n32;
  P.block = static_cast<int>(block);
  P.mode = mode;
  P.window = static_cast<int>(window);
  P.lists = lists;
  P.ls_b = ls_b;
  P.ls_q = ls_q;
  P.counts = counts;
  P.cs_b = cs_b;
  P.cs_q = cs_q;
  P.cap = static_cast<int>(capacity);
  P.n_blocks = static_cast<int>((T + block - 1) / block);
  P.scale_log2 = scale * SA_LOG2E;
  P.out = static_cast<bf16_t*>(out);
  P.os_b = os_b;
  P.os_h = os_h;
  P.os_t = os_t;
  P.err = err;
  const dim3 grid(static_cast<unsigned>((T + 15) / 16),
                  static_cast<unsigned>(B * Hkv * ((P.G + SA_WAVES - 1) / SA_WAVES)));
  // 64 queries per wave when a query block holds whole 64-query tiles and its list fits one wave
  const bool wide = block % 64 == 0 && fsi_host::is_pow2(block) && capacity <= SAL_MAX_CAP && scale > 0.f;
  const dim3 grid_w(static_cast<unsigned>((T + 63) / 64), grid.y);
  const unsigned g_vmax = static_cast<unsigned>((B * Hkv * static_cast<int64_t>(n32) + 3) / 4);
  const dim3 g_vt16(static_cast<unsigned>((n32 + SA_VT_CHUNKS - 1) / SA_VT_CHUNKS), static_cast<unsigned>(B * Hkv));
  auto launch = [&](auto hd_tag) -> int {
    constexpr int HD = decltype(hd_tag)::value;
    const bf16_t* vb = static_cast<const bf16_t*>(v);
    if constexpr (HD >= 64) {
      if (wide) {  // fp16 V^T scaled per head, then the 64-query kernel
        sa_vmax_kernel<HD><<<g_vmax, 256, 0, st>>>(vb, vs_b, vs_h, vs_t, P.B, P.Hkv, P.T, n32, cmax);
        FSI_HIP_LAUNCH_CHECK("sparse_attn v maxima");
        sa_vt16_kernel<HD><<<g_vt16, 256, 0, st>>>(vb, vs_b, vs_h, vs_t, P.Hkv, P.T, n32, cmax, head_e,
                                                   reinterpret_cast<uint16_t*>(vt));
        FSI_HIP_LAUNCH_CHECK("sparse_attn v copy");
        sparse_attn_lds_kernel<HD><<<grid_w, 64 * SAL_WAVES, 0, st>>>(P);
        FSI_HIP_LAUNCH_CHECK("sparse_attn");
        return FSI_OK;
      }
    }
    sa_vt_kernel<HD><<<g1, 256, 0, st>>>(vb, vs_b, vs_h, vs_t, P.B, P.Hkv, P.T, n32, vt);
    FSI_HIP_LAUNCH_CHECK("sparse_attn v copy");
    sparse_attn_kernel<HD><<<grid, 64 * SA_WAVES, 0, st>>>(P);
    FSI_HIP_LAUNCH_CHECK("sparse_attn");
    return FSI_OK;
  };
  switch (head_dim) {
    case 16: return launch(std::integral_constant<int, 16>{});
    case 32: return launch(std::integral_constant<int, 32>{});
    case 64: return launch(std::integral_constant<int, 64>{});
    default: return launch(std::integral_constant<int, 128>{});
  }
}

}  // extern "C"
