// Foveal sparse decode attention on MI355X (gfx950): one query token per
// sequence attends its local window [max(0, pos + 1 - W), pos] plus the remote
// pages chosen by the 16-D indexer (foveal_indexer/attention.py:339-367).
//
// Paged KV pools, one page = 64 tokens of one sequence, all KV heads:
//   K pool: [page][Hkv][HD/32][64][32]  — per 32-dim chunk, token-major
//   V pool: [page][Hkv][2][HD][32]      — per 32-token half, dim-major, the
//                                        half's tokens stored in MFMA k order
// so every wave-wide load below reads 1 KiB of contiguous memory and feeds a
// v_mfma_f32_16x16x32_bf16 operand directly, with no LDS staging.
//
// Work split: the support of a sequence is a list of 32-token chunks (local
// window halves first, then two halves per selected page).  Wave (b, g, s)
// takes a contiguous share of sequence b's chunks for KV head g and keeps an
// online softmax for the GQA group's query heads (up to 16, the MFMA N
// dimension):
//   S^T[t][h] = sum_d K[t][d] Q[h][d]        (A = K tile, B = Q^T)
//   O^T[d][h] += sum_t V^T[d][t] P^T[t][h]   (A = V^T tile, B = P^T from S^T's
//                                             accumulators, no data movement;
//                                             P as a bf16 hi + lo pair, two MFMAs)
// Per-wave partials (max, sum, O) are merged by a second kernel; nothing is
// synchronised across workgroups.
#include <algorithm>
#include <atomic>
#include <mutex>

#include "fsi_common.h"

using namespace fsi;

namespace {

constexpr int PAGE = 64;
constexpr int CHUNK = 32;
constexpr int DA_WAVES = 4;
constexpr int MAX_CHUNKS_PER_WAVE = 64;
constexpr float LOG2E = 1.4426950408889634f;

// storage position (MFMA k index) of token tau within a 32-token half
__host__ __device__ __forceinline__ int v_slot(int tau) { return 8 * ((tau & 15) >> 2) + 4 * (tau >> 4) + (tau & 3); }

// ---------------------------------------------------------------------------
// Writer: scatter n_tok tokens per sequence from (B, Hkv, n_tok, HD) K and V
// (any strides in elements) into the paged pools at positions start .. start+n_tok-1
// (start per sequence or shared).  One thread per (b, g, token, 8 dims).
// ---------------------------------------------------------------------------
template <int HD>
__global__ __launch_bounds__(256) void kv_write_kernel(const bf16_t* __restrict__ k, const bf16_t* __restrict__ v,
                                                      int64_t ks_b, int64_t ks_g, int64_t ks_t, int64_t vs_b,
                                                      int64_t vs_g, int64_t vs_t, int B, int Hkv, int n_tok,
                                                      const int32_t* __restrict__ start_rows, int start,
                                                      const int32_t* __restrict__ page_table, int max_pages,
                                                      int64_t n_phys, bf16_t* __restrict__ k_pool,
                                                      bf16_t* __restrict__ v_pool, int* __restrict__ err) {
  constexpr int PIECES = HD / 8;
  const int64_t total = static_cast<int64_t>(B) * Hkv * n_tok * PIECES;
  for (int64_t gid = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; gid < total;
       gid += static_cast<int64_t>(gridDim.x) * 256) {
  const int piece = static_cast<int>(gid % PIECES);
  int64_t r = gid / PIECES;
  const int t = static_cast<int>(r % n_tok);
  r /= n_tok;
  const int g = static_cast<int>(r % Hkv);
  const int b = static_cast<int>(r / Hkv);
  const int p = (start_rows ? start_rows[b] : start) + t;
  const int lp = p / PAGE, off = p % PAGE;
  if (p < 0 || lp >= max_pages) {
    if (err) set_error(err, FSI_ERR_INDEX_RANGE);
    continue;
  }
  const int64_t phys = page_table[static_cast<int64_t>(b) * max_pages + lp];
  if (phys < 0 || phys >= n_phys) {
    if (err) set_error(err, FSI_ERR_INDEX_RANGE);
    continue;
  }
  const int64_t page_base = (phys * Hkv + g) * PAGE * HD;
  const int d0 = piece * 8;
  // K: chunk d0/32, token off, dims d0%32 .. +8 (16 contiguous bytes)
  const u32x4_t kv = *reinterpret_cast<const u32x4_t*>(k + b * ks_b + g * ks_g + t * ks_t + d0);
  *reinterpret_cast<u32x4_t*>(k_pool + page_base + (d0 / 32) * PAGE * 32 + off * 32 + (d0 % 32)) = kv;
  // V: half off/32, dim rows d0..d0+7, slot v_slot(off%32)
  const u32x4_t vv = *reinterpret_cast<const u32x4_t*>(v + b * vs_b + g * vs_g + t * vs_t + d0);
  bf16_t* vb = v_pool + page_base + (off / CHUNK) * HD * CHUNK + v_slot(off % CHUNK);
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    vb[(d0 + 2 * w) * CHUNK] = static_cast<bf16_t>(vv[w] & 0xffffu);
    vb[(d0 + 2 * w + 1) * CHUNK] = static_cast<bf16_t>(vv[w] >> 16);
  }
  }
}

// Reader for tests and cache export: pooled tokens [0, n_tok) of every
// sequence back to (B, Hkv, n_tok, HD).
template <int HD>
__global__ __launch_bounds__(256) void kv_read_kernel(const bf16_t* __restrict__ k_pool,
                                                     const bf16_t* __restrict__ v_pool, int B, int Hkv, int n_tok,
                                                     const int32_t* __restrict__ page_table, int max_pages,
                                                     int64_t n_phys, bf16_t* __restrict__ k_out,
                                                     bf16_t* __restrict__ v_out) {
  const int64_t total = static_cast<int64_t>(B) * Hkv * n_tok * HD;
  for (int64_t gid = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; gid < total;
       gid += static_cast<int64_t>(gridDim.x) * 256) {
  const int d = static_cast<int>(gid % HD);
  int64_t r = gid / HD;
  const int t = static_cast<int>(r % n_tok);
  r /= n_tok;
  const int g = static_cast<int>(r % Hkv);
  const int b = static_cast<int>(r / Hkv);
  const int lp = t / PAGE, off = t % PAGE;
  const int64_t phys = lp < max_pages ? page_table[static_cast<int64_t>(b) * max_pages + lp] : -1;
  bf16_t kk = 0, vv = 0;
  if (phys >= 0 && phys < n_phys) {
    const int64_t base = (phys * Hkv + g) * PAGE * HD;
    kk = k_pool[base + (d / 32) * PAGE * 32 + off * 32 + (d % 32)];
    vv = v_pool[base + (off / CHUNK) * HD * CHUNK + d * CHUNK + v_slot(off % CHUNK)];
  }
  k_out[gid] = kk;
  v_out[gid] = vv;
  }
}

// ---------------------------------------------------------------------------
// Attention partials.
// ---------------------------------------------------------------------------
struct DecodeParams {
  const bf16_t* q;  // (B, Hq, HD)
  const bf16_t* k_pool;
  const bf16_t* v_pool;
  const int32_t* page_table;  // (B, max_pages)
  const int32_t* pos_rows;    // (B) or null
  const int32_t* remote;      // (B, cap) logical pages in rank order
  const int32_t* counts;      // (B)
  float* m_part;              // (B, Hkv, S, 16)
  float* l_part;              // (B, Hkv, S, 16)
  float* o_part;              // (B, Hkv, S, G, HD)
  int* err;
  int64_t n_phys;
  int B, Hq, Hkv, G, S, max_pages, cap, pos, window;
  float scale_log2;
};

template <int HD>
__global__ __launch_bounds__(64 * DA_WAVES) void decode_attn_partial_kernel(DecodeParams P) {
  constexpr int KS = HD / 32;   // k-steps of the S^T product
  constexpr int DT = HD / 16;   // dim tiles of O^T
  constexpr int KLOADS = 2 * KS;
  const int lane = threadIdx.x & 63;
  const int wave_id = blockIdx.x * DA_WAVES + (threadIdx.x >> 6);
  if (wave_id >= P.B * P.Hkv * P.S) return;  // whole wave; no barriers below
  const int s = wave_id % P.S;
  const int g = (wave_id / P.S) % P.Hkv;
  const int b = wave_id / (P.S * P.Hkv);
  const int h = lane & 15, grp = lane >> 4;

  const int pos = P.pos_rows ? P.pos_rows[b] : P.pos;
  const int ls = pos + 1 - P.window > 0 ? pos + 1 - P.window : 0;
  const int c_lo = ls / CHUNK, c_hi = pos / CHUNK;
  const int nl = c_hi - c_lo + 1;
  int cnt = P.counts ? P.counts[b] : 0;
  cnt = cnt < 0 ? 0 : (cnt > P.cap ? P.cap : cnt);
  const int total = nl + 2 * cnt;
  const int per = (total + P.S - 1) / P.S;
  const int c0 = s * per;
  int c1 = c0 + per < total ? c0 + per : total;
  if (c1 - c0 > MAX_CHUNKS_PER_WAVE) {  // only with per-sequence positions beyond the sizing bound
    if (P.err) set_error(P.err, FSI_ERR_CAPACITY);
    c1 = c0 + MAX_CHUNKS_PER_WAVE;
  }

  // chunk c0 + lane: element offset of its (page, head) block with the half in
  // bit 0 (blocks are PAGE * HD elements, so the bit is free), and the valid
  // token range within the half
  int64_t cbase = 0;
  int tok_lo = 0, tok_hi = CHUNK;  // valid token range [lo, hi) within the half
  {
    const int c = c0 + lane;
    if (c < c1) {
      int lp, half;
      if (c < nl) {
        const int ca = c_lo + c;  // absolute chunk index
        lp = ca >> 1;
        half = ca & 1;
        const int first = ca * CHUNK;
        tok_lo = ls - first > 0 ? ls - first : 0;
        tok_hi = pos + 1 - first < CHUNK ? pos + 1 - first : CHUNK;
      } else {
        const int r = (c - nl) >> 1;
        half = (c - nl) & 1;
        lp = P.remote[static_cast<int64_t>(b) * P.cap + r];
      }
      int64_t phys = -1;
      if (lp >= 0 && lp < P.max_pages) phys = P.page_table[static_cast<int64_t>(b) * P.max_pages + lp];
      if (phys < 0 || phys >= P.n_phys) {
        if (P.err) set_error(P.err, FSI_ERR_INDEX_RANGE);
        phys = 0;
        tok_lo = tok_hi = 0;  // nothing valid: the chunk is read from page 0 and masked out
      }
      cbase = ((phys * P.Hkv + g) * PAGE) * HD + half;
    }
  }

  // Q^T operand: lane supplies Q[h][32 ks + 8 grp .. +8]
  u32x4_t qb[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    if (h < P.G) {
      qb[ks] = *reinterpret_cast<const u32x4_t*>(P.q + (static_cast<int64_t>(b) * P.Hq + g * P.G + h) * HD + 32 * ks +
                                                 8 * grp);
    } else {
      qb[ks] = u32x4_t{0u, 0u, 0u, 0u};
    }
  }

  f32x4_t acc[DT];
#pragma unroll
  for (int i = 0; i < DT; ++i) acc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;

  u32x4_t kcur[KLOADS], vcur[DT], knxt[KLOADS], vnxt[DT];
  auto load_chunk = [&](int c, u32x4_t (&kr)[KLOADS], u32x4_t (&vr)[DT]) {
    const int i = c - c0;
    const uint32_t lo = __builtin_amdgcn_readlane(static_cast<uint32_t>(cbase), i);
    const uint32_t hi = __builtin_amdgcn_readlane(static_cast<uint32_t>(cbase >> 32), i);
    const int64_t info = static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
    const int half = static_cast<int>(info & 1);
    const int64_t head_base = info - half;
    // K [HD/32][64][32]: the half starts at token 32 half of every dim chunk;
    // V [2][HD][32]: the half is the outer index
    const bf16_t* kp = P.k_pool + head_base + half * CHUNK * 32;
    const bf16_t* vp = P.v_pool + head_base + half * CHUNK * HD;
#pragma unroll
    for (int tile = 0; tile < 2; ++tile)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        kr[tile * KS + ks] =
            *reinterpret_cast<const u32x4_t*>(kp + ks * PAGE * 32 + (16 * tile + h) * 32 + 8 * grp);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
      vr[dt] = *reinterpret_cast<const u32x4_t*>(vp + (16 * dt + h) * CHUNK + 8 * grp);
  };

  if (c0 < c1) load_chunk(c0, kcur, vcur);
  for (int c = c0; c < c1; ++c) {
    const int cn = c + 1 < c1 ? c + 1 : c;  // straight-line prefetch (the last one re-reads)
    load_chunk(cn, knxt, vnxt);
    const int i = c - c0;
    const int lo_t = __builtin_amdgcn_readlane(tok_lo, i);
    const int hi_t = __builtin_amdgcn_readlane(tok_hi, i);

    // S^T for the chunk's two 16-token tiles
    f32x4_t st[2];
#pragma unroll
    for (int tile = 0; tile < 2; ++tile) {
      st[tile] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) st[tile] = mfma16x16x32(kcur[tile * KS + ks], qb[ks], st[tile]);
    }
    // lane holds tokens 16 tile + 4 grp + j for head h
    float sv[8];
    float mx = -INFINITY;
#pragma unroll
    for (int tile = 0; tile < 2; ++tile)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int tau = 16 * tile + 4 * grp + j;
        const bool ok = tau >= lo_t && tau < hi_t;
        const float v = ok ? st[tile][j] * P.scale_log2 : -INFINITY;
        sv[tile * 4 + j] = v;
        mx = fmaxf(mx, v);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m_run, mx);
    float alpha, psum = 0.f;
    uint32_t pk_hi[4], pk_lo[4];  // P = hi + lo, both bf16: the PV product keeps ~16 bits of P
    if (m_new == -INFINITY) {
      alpha = 1.f;
#pragma unroll
      for (int w = 0; w < 4; ++w) pk_hi[w] = pk_lo[w] = 0u;
    } else {
      alpha = exp2f(m_run - m_new);
      float hi[8], lo[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float pe = exp2f(sv[e] - m_new);
        psum += pe;
        hi[e] = round_bf16(pe);
        lo[e] = pe - hi[e];
      }
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        pk_hi[w] = pack_bf16x2(hi[2 * w], hi[2 * w + 1]);
        pk_lo[w] = pack_bf16x2(lo[2 * w], lo[2 * w + 1]);
      }
    }
    psum += __shfl_xor(psum, 16, 64);
    psum += __shfl_xor(psum, 32, 64);
    l_run = l_run * alpha + psum;
    m_run = m_new;
    // V^T tile: zero the slots of masked tokens (their memory may hold anything)
    if (lo_t > 0 || hi_t < CHUNK) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const int e0 = 2 * w, e1 = 2 * w + 1;
          const int t0 = e0 < 4 ? 4 * grp + e0 : 16 + 4 * grp + e0 - 4;
          const int t1 = e1 < 4 ? 4 * grp + e1 : 16 + 4 * grp + e1 - 4;
          const uint32_t m0 = (t0 >= lo_t && t0 < hi_t) ? 0x0000ffffu : 0u;
          const uint32_t m1 = (t1 >= lo_t && t1 < hi_t) ? 0xffff0000u : 0u;
          vcur[dt][w] &= (m0 | m1);
        }
    }
    const u32x4_t pbh = u32x4_t{pk_hi[0], pk_hi[1], pk_hi[2], pk_hi[3]};
    const u32x4_t pbl = u32x4_t{pk_lo[0], pk_lo[1], pk_lo[2], pk_lo[3]};
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[dt][j] *= alpha;
      acc[dt] = mfma16x16x32(vcur[dt], pbh, acc[dt]);
      acc[dt] = mfma16x16x32(vcur[dt], pbl, acc[dt]);
    }
#pragma unroll
    for (int t = 0; t < KLOADS; ++t) kcur[t] = knxt[t];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) vcur[dt] = vnxt[dt];
  }

  const int64_t part = (static_cast<int64_t>(b) * P.Hkv + g) * P.S + s;
  if (grp == 0) {
    P.m_part[part * 16 + h] = m_run;
    P.l_part[part * 16 + h] = l_run;
  }
  if (h < P.G) {
    float* o = P.o_part + (part * P.G + h) * HD;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
      *reinterpret_cast<f32x4_t*>(o + 16 * dt + 4 * grp) = acc[dt];
  }
}

// One wave per (sequence, query head): lanes read the split maxima and sums in
// parallel, then every lane merges HD / 64 dimensions over the splits.
constexpr int MG_WAVES = 4;

template <int HD>
__global__ __launch_bounds__(64 * MG_WAVES) void decode_attn_merge_kernel(const float* __restrict__ m_part,
                                                                         const float* __restrict__ l_part,
                                                                         const float* __restrict__ o_part, int B,
                                                                         int Hq, int Hkv, int G, int S,
                                                                         bf16_t* __restrict__ out) {
  constexpr int DPL = HD / 64;  // dimensions per lane
  const int lane = threadIdx.x & 63;
  const int item = blockIdx.x * MG_WAVES + (threadIdx.x >> 6);
  if (item >= B * Hq) return;
  const int b = item / Hq, hq = item % Hq;
  const int g = hq / G, h = hq % G;
  const int64_t part0 = (static_cast<int64_t>(b) * Hkv + g) * S;
  float M = -INFINITY;
  for (int s = lane; s < S; s += 64) M = fmaxf(M, m_part[(part0 + s) * 16 + h]);
  M = wave_max(M);
  float o[DPL];
#pragma unroll
  for (int i = 0; i < DPL; ++i) o[i] = 0.f;
  float L = 0.f;
  if (M != -INFINITY) {
    for (int s0 = 0; s0 < S; s0 += 64) {
      const int s = s0 + lane;
      float w = 0.f, lw = 0.f;
      if (s < S) {
        const float ms = m_part[(part0 + s) * 16 + h];
        w = ms == -INFINITY ? 0.f : exp2f(ms - M);
        lw = l_part[(part0 + s) * 16 + h] * w;
      }
      L += wave_sum(lw);
      const int n = S - s0 < 64 ? S - s0 : 64;
#pragma unroll 4
      for (int k = 0; k < n; ++k) {
        const float wk = __shfl(w, k, 64);
        const float* src = o_part + ((part0 + s0 + k) * G + h) * HD + lane * DPL;
#pragma unroll
        for (int i = 0; i < DPL; ++i) o[i] = fmaf(src[i], wk, o[i]);
      }
    }
  }
  bf16_t* dst = out + (static_cast<int64_t>(b) * Hq + hq) * HD + lane * DPL;
#pragma unroll
  for (int i = 0; i < DPL; ++i) dst[i] = f32_to_bf16(L > 0.f ? o[i] / L : 0.f);
}

int split_count(int64_t B, int64_t Hkv, int64_t max_chunks) {
  // enough waves to cover the chip several times, at most 64 chunks per wave
  int64_t S = (2048 + B * Hkv - 1) / (B * Hkv);
  const int64_t min_s = (max_chunks + MAX_CHUNKS_PER_WAVE - 1) / MAX_CHUNKS_PER_WAVE;
  if (S < min_s) S = min_s;
  if (S > max_chunks) S = max_chunks;
  if (S < 1) S = 1;
  return static_cast<int>(S);
}

// Upper bound on a sequence's chunks: the local window spans at most
// ceil(W / 32) + 1 halves and never more than the page table holds.
int64_t max_chunks_of(int64_t window, int64_t cap, int64_t max_pages) {
  int64_t local = (window + CHUNK - 1) / CHUNK + 1;
  if (local > 2 * max_pages) local = 2 * max_pages;
  return local + 2 * cap;
}

}  // namespace

extern "C" {

FSI_API int fsi_kv_write(const void* k, const void* v, int64_t k_stride_b, int64_t k_stride_h, int64_t k_stride_t,
                         int64_t v_stride_b, int64_t v_stride_h, int64_t v_stride_t, int64_t B, int64_t Hkv,
                         int64_t n_tok, int64_t head_dim, const int32_t* start_rows, int64_t start,
                         const int32_t* page_table, int64_t max_pages, int64_t n_phys_pages, void* k_pool,
                         void* v_pool, int* err, void* stream) {
  using namespace fsi_host;
  FSI_CHECK_ARG(head_dim == 64 || head_dim == 128, FSI_ERR_SHAPE, "kv_write: head_dim %lld not 64 or 128",
                (long long)head_dim);
  FSI_CHECK_ARG(B >= 0 && Hkv > 0 && n_tok >= 0 && max_pages > 0 && n_phys_pages > 0 && start >= 0, FSI_ERR_SHAPE,
                "kv_write: bad sizes");
  FSI_CHECK_ARG(max_pages * PAGE <= 0x7fffffff && B <= 0x7fffffff && n_tok <= 0x7fffffff, FSI_ERR_SHAPE,
                "kv_write: sizes beyond int32");
  if (B == 0 || n_tok == 0) return FSI_OK;
  FSI_CHECK_ARG(k && v && page_table && k_pool && v_pool, FSI_ERR_INVALID_ARG, "kv_write: null pointer");
  FSI_CHECK_ARG(reinterpret_cast<uintptr_t>(k) % 16 == 0 && reinterpret_cast<uintptr_t>(v) % 16 == 0 &&
                    (k_stride_b | k_stride_h | k_stride_t | v_stride_b | v_stride_h | v_stride_t) % 8 == 0,
                FSI_ERR_ALIGN, "kv_write: K/V rows must be 16-byte aligned");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int64_t total = B * Hkv * n_tok * (head_dim / 8);
  const unsigned grid = static_cast<unsigned>(std::min<int64_t>((total + 255) / 256, 1 << 20));
#define KVW(HDV)                                                                                                   \
  kv_write_kernel<HDV><<<grid, 256, 0, st>>>(                                                                      \
      static_cast<const bf16_t*>(k), static_cast<const bf16_t*>(v), k_stride_b, k_stride_h, k_stride_t,             \
      v_stride_b, v_stride_h, v_stride_t, (int)B, (int)Hkv, (int)n_tok, start_rows, (int)start, page_table,         \
      (int)max_pages, n_phys_pages, static_cast<bf16_t*>(k_pool), static_cast<bf16_t*>(v_pool), err)
  if (head_dim == 128) KVW(128);
  else KVW(64);
#undef KVW
  FSI_HIP_LAUNCH_CHECK("kv_write");
  return FSI_OK;
}

FSI_API int fsi_kv_read(const void* k_pool, const void* v_pool, int64_t B, int64_t Hkv, int64_t n_tok,
                        int64_t head_dim, const int32_t* page_table, int64_t max_pages, int64_t n_phys_pages,
                        void* k_out, void* v_out, void* stream) {
  using namespace fsi_host;
  FSI_CHECK_ARG(head_dim == 64 || head_dim == 128, FSI_ERR_SHAPE, "kv_read: head_dim %lld not 64 or 128",
                (long long)head_dim);
  FSI_CHECK_ARG(B >= 0 && Hkv > 0 && n_tok >= 0 && max_pages > 0 && n_phys_pages > 0, FSI_ERR_SHAPE,
                "kv_read: bad sizes");
  if (B == 0 || n_tok == 0) return FSI_OK;
  FSI_CHECK_ARG(k_pool && v_pool && page_table && k_out && v_out, FSI_ERR_INVALID_ARG, "kv_read: null pointer");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int64_t total = B * Hkv * n_tok * head_dim;
  const unsigned grid = static_cast<unsigned>(std::min<int64_t>((total + 255) / 256, 1 << 20));
#define KVR(HDV)                                                                                                  \
  kv_read_kernel<HDV><<<grid, 256, 0, st>>>(static_cast<const bf16_t*>(k_pool), static_cast<const bf16_t*>(v_pool), \
                                            (int)B, (int)Hkv, (int)n_tok, page_table, (int)max_pages,              \
                                            n_phys_pages, static_cast<bf16_t*>(k_out), static_cast<bf16_t*>(v_out))
  if (head_dim == 128) KVR(128);
  else KVR(64);
#undef KVR
  FSI_HIP_LAUNCH_CHECK("kv_read");
  return FSI_OK;
}

}  // extern "C"

namespace {

// Checks shared by fsi_decode_attn and fsi_decode_attn_noalloc that do not
// involve the partials buffer.  Returns FSI_OK or a status with the message set.
int decode_attn_check(const void* q, const void* k_pool, const void* v_pool, const int32_t* page_table,
                      int64_t max_pages, int64_t n_phys_pages, const int32_t* pos_rows, int64_t pos, int64_t window,
                      const int32_t* remote_pages, const int32_t* remote_counts, int64_t capacity, int64_t B,
                      int64_t Hq, int64_t Hkv, int64_t head_dim, void* out) {
  FSI_CHECK_ARG(head_dim == 64 || head_dim == 128, FSI_ERR_SHAPE, "decode_attn: head_dim %lld not 64 or 128",
                (long long)head_dim);
  FSI_CHECK_ARG(B >= 0 && Hkv > 0 && Hq > 0 && Hq % Hkv == 0 && Hq / Hkv <= 16, FSI_ERR_SHAPE,
                "decode_attn: need Hq %% Hkv == 0 and Hq / Hkv <= 16 (Hq %lld, Hkv %lld)", (long long)Hq,
                (long long)Hkv);
  FSI_CHECK_ARG(max_pages > 0 && n_phys_pages > 0 && window >= 0 && pos >= 0 && capacity >= 0, FSI_ERR_SHAPE,
                "decode_attn: bad sizes");
  FSI_CHECK_ARG(max_pages * PAGE <= 0x7fffffff && window <= 0x7fffffff && B <= 65535 * 64, FSI_ERR_SHAPE,
                "decode_attn: sizes beyond int32");
  FSI_CHECK_ARG(pos_rows || pos < max_pages * PAGE, FSI_ERR_INDEX_RANGE,
                "decode_attn: position %lld beyond the page table (%lld pages)", (long long)pos, (long long)max_pages);
  if (B == 0) return FSI_OK;
  FSI_CHECK_ARG(q && k_pool && v_pool && page_table && out, FSI_ERR_INVALID_ARG, "decode_attn: null pointer");
  FSI_CHECK_ARG(capacity == 0 || (remote_pages && remote_counts), FSI_ERR_INVALID_ARG,
                "decode_attn: remote page list or counts missing");
  FSI_CHECK_ARG(reinterpret_cast<uintptr_t>(q) % 16 == 0 && reinterpret_cast<uintptr_t>(k_pool) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(v_pool) % 16 == 0,
                FSI_ERR_ALIGN, "decode_attn: q and pools must be 16-byte aligned");
  return FSI_OK;
}

// Bytes of per-wave partials (max, sum, O) the partial and merge kernels exchange.
size_t decode_attn_partials_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t head_dim, int64_t window,
                                  int64_t capacity, int64_t max_pages) {
  const int64_t S = split_count(B, Hkv, max_chunks_of(window, capacity, max_pages));
  const int64_t parts = B * Hkv * S;
  return static_cast<size_t>(parts) * (2 * 16 + (Hq / Hkv) * head_dim) * sizeof(float);
}

// The partial and merge kernels with the partials at `ws` (16-byte aligned,
// decode_attn_partials_bytes long; every byte read is written first in the
// same call, so it needs no clearing).
int decode_attn_launch(const void* q, const void* k_pool, const void* v_pool, const int32_t* page_table,
                       int64_t max_pages, int64_t n_phys_pages, const int32_t* pos_rows, int64_t pos, int64_t window,
                       const int32_t* remote_pages, const int32_t* remote_counts, int64_t capacity, int64_t B,
                       int64_t Hq, int64_t Hkv, int64_t head_dim, float scale, void* out, char* ws, int* err,
                       void* stream) {
  const int64_t max_chunks = max_chunks_of(window, capacity, max_pages);
  const int S = split_count(B, Hkv, max_chunks);
  const int64_t parts = B * Hkv * S;
  DecodeParams P;
  P.q = static_cast<const bf16_t*>(q);
  P.k_pool = static_cast<const bf16_t*>(k_pool);
  P.v_pool = static_cast<const bf16_t*>(v_pool);
  P.page_table = page_table;
  P.pos_rows = pos_rows;
  P.remote = remote_pages;
  P.counts = capacity > 0 ? remote_counts : nullptr;
  P.m_part = reinterpret_cast<float*>(ws);
  P.l_part = P.m_part + parts * 16;
  P.o_part = P.l_part + parts * 16;
  P.err = err;
  P.n_phys = n_phys_pages;
  P.B = (int)B;
  P.Hq = (int)Hq;
  P.Hkv = (int)Hkv;
  P.G = (int)(Hq / Hkv);
  P.S = S;
  P.max_pages = (int)max_pages;
  P.cap = (int)capacity;
  P.pos = (int)pos;
  P.window = (int)window;
  P.scale_log2 = scale * LOG2E;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const unsigned grid = static_cast<unsigned>((parts + DA_WAVES - 1) / DA_WAVES);
  const unsigned merge_grid = static_cast<unsigned>((B * Hq + MG_WAVES - 1) / MG_WAVES);
  if (head_dim == 128) {
    decode_attn_partial_kernel<128><<<grid, 64 * DA_WAVES, 0, st>>>(P);
    FSI_HIP_LAUNCH_CHECK("decode_attn partial");
    decode_attn_merge_kernel<128><<<merge_grid, 64 * MG_WAVES, 0, st>>>(P.m_part, P.l_part, P.o_part, (int)B,
                                                                        (int)Hq, (int)Hkv, P.G, S,
                                                                        static_cast<bf16_t*>(out));
  } else {
    decode_attn_partial_kernel<64><<<grid, 64 * DA_WAVES, 0, st>>>(P);
    FSI_HIP_LAUNCH_CHECK("decode_attn partial");
    decode_attn_merge_kernel<64><<<merge_grid, 64 * MG_WAVES, 0, st>>>(P.m_part, P.l_part, P.o_part, (int)B,
                                                                       (int)Hq, (int)Hkv, P.G, S,
                                                                       static_cast<bf16_t*>(out));
  }
  FSI_HIP_LAUNCH_CHECK("decode_attn merge");
  return FSI_OK;
}

// Scratch of fsi_decode_attn_noalloc: the per-wave partials live in this
// file-scope device array, one copy per GPU, held until the process ends.  Host
// code never passes the symbol itself to a kernel: the array's device address
// is looked up once per device with hipGetSymbolAddress.
constexpr size_t NOALLOC_SCRATCH_BYTES = FSI_DECODE_ATTN_NOALLOC_MAX_BYTES;
__device__ __align__(256) char scratch[NOALLOC_SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;
std::atomic<char*> g_scratch_ptr[MAX_DEVICES];
std::mutex g_scratch_mu;

// Device address of `scratch` on the current device (looked up on the first call
// there, with that device current), or null with the last-error message set.
char* scratch_on_current_device() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) {
    fsi_host::set_last_error("decode_attn_noalloc: no current HIP device (or index >= %d)", MAX_DEVICES);
    return nullptr;
  }
  char* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (p) return p;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
  if (p) return p;
  void* addr = nullptr;
  const hipError_t e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
  if (e != hipSuccess || addr == nullptr) {
    fsi_host::set_last_error("decode_attn_noalloc: hipGetSymbolAddress(scratch) on device %d: %s", dev,
                             hipGetErrorString(e));
    return nullptr;
  }
  p = static_cast<char*>(addr);
  g_scratch_ptr[dev].store(p, std::memory_order_release);
  return p;
}

}  // namespace

extern "C" {

FSI_API size_t fsi_decode_attn_workspace_size(int64_t B, int64_t Hq, int64_t Hkv, int64_t head_dim, int64_t window,
                                              int64_t capacity, int64_t max_pages) {
  if (B <= 0 || Hkv <= 0 || Hq <= 0 || head_dim <= 0 || max_pages <= 0 || window < 0 || capacity < 0)
    return FSI_WORKSPACE_COUNTER_BYTES;
  return FSI_WORKSPACE_COUNTER_BYTES + decode_attn_partials_bytes(B, Hq, Hkv, head_dim, window, capacity, max_pages) +
         256;
}

FSI_API int fsi_decode_attn(const void* q, const void* k_pool, const void* v_pool, const int32_t* page_table,
                            int64_t max_pages, int64_t n_phys_pages, const int32_t* pos_rows, int64_t pos,
                            int64_t window, const int32_t* remote_pages, const int32_t* remote_counts,
                            int64_t capacity, int64_t B, int64_t Hq, int64_t Hkv, int64_t head_dim, float scale,
                            void* out, void* workspace, size_t workspace_bytes, int* err, void* stream) {
  const int c = decode_attn_check(q, k_pool, v_pool, page_table, max_pages, n_phys_pages, pos_rows, pos, window,
                                  remote_pages, remote_counts, capacity, B, Hq, Hkv, head_dim, out);
  if (c != FSI_OK || B == 0) return c;
  const size_t need = fsi_decode_attn_workspace_size(B, Hq, Hkv, head_dim, window, capacity, max_pages);
  FSI_CHECK_ARG(workspace && workspace_bytes >= need, FSI_ERR_WORKSPACE, "decode_attn: workspace %zu < %zu bytes",
                workspace_bytes, need);
  FSI_CHECK_ARG(reinterpret_cast<uintptr_t>(workspace) % 16 == 0, FSI_ERR_ALIGN,
                "decode_attn: workspace must be 16-byte aligned");
  return decode_attn_launch(q, k_pool, v_pool, page_table, max_pages, n_phys_pages, pos_rows, pos, window,
                            remote_pages, remote_counts, capacity, B, Hq, Hkv, head_dim, scale, out,
                            static_cast<char*>(workspace) + FSI_WORKSPACE_COUNTER_BYTES, err, stream);
}

FSI_API int fsi_decode_attn_noalloc(const void* q, const void* k_pool, const void* v_pool, const int32_t* page_table,
                                    int64_t max_pages, int64_t n_phys_pages, const int32_t* pos_rows, int64_t pos,
                                    int64_t window, const int32_t* remote_pages, const int32_t* remote_counts,
                                    int64_t capacity, int64_t B, int64_t Hq, int64_t Hkv, int64_t head_dim,
                                    float scale, void* out, int* err, void* stream) {
  const int c = decode_attn_check(q, k_pool, v_pool, page_table, max_pages, n_phys_pages, pos_rows, pos, window,
                                  remote_pages, remote_counts, capacity, B, Hq, Hkv, head_dim, out);
  if (c != FSI_OK || B == 0) return c;
  const size_t need = decode_attn_partials_bytes(B, Hq, Hkv, head_dim, window, capacity, max_pages);
  FSI_CHECK_ARG(need <= NOALLOC_SCRATCH_BYTES, FSI_ERR_CAPACITY,
                "decode_attn_noalloc: %zu bytes of partials exceed the %zu-byte device scratch "
                "(use fsi_decode_attn with a workspace)",
                need, NOALLOC_SCRATCH_BYTES);
  char* ws = scratch_on_current_device();
  if (!ws) return FSI_ERR_HIP;
  return decode_attn_launch(q, k_pool, v_pool, page_table, max_pages, n_phys_pages, pos_rows, pos, window,
                            remote_pages, remote_counts, capacity, B, Hq, Hkv, head_dim, scale, out, ws, err, stream);
}

}  // extern "C"
