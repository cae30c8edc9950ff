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
// synchronised across workgroups.  The local-window chunks and the remote-page
// chunks can also run as separate launches (DA_LOCAL, then DA_REMOTE and the
// merge) into disjoint partial slots: the local part reads no routing result,
// so it can run beside the page routing.
//
// This header is shared by decode_attn.hip (fsi_decode_attn and its
// no-allocation form) and routing.hip (the fused decode step); every includer
// gets its own copy (anonymous namespace).
#pragma once

#include <algorithm>

#include "fsi_common.h"

namespace {

using namespace fsi;


constexpr int PAGE = 64;
constexpr int CHUNK = 32;
constexpr int DA_WAVES = 4;
constexpr int MAX_CHUNKS_PER_WAVE = 64;
constexpr float LOG2E = 1.4426950408889634f;

// storage position (MFMA k index) of token tau within a 32-token half
__host__ __device__ __forceinline__ int v_slot(int tau) { return 8 * ((tau & 15) >> 2) + 4 * (tau >> 4) + (tau & 3); }

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
  int remote_stride;  // elements between sequences' rows of remote / counts (cap, or 0: every row reads row 0)
  int mode;           // DA_ALL, DA_LOCAL or DA_REMOTE: which chunks this launch covers
  int s_off;          // first partial slot of this launch
  int S_sub;          // waves (partial slots) per (sequence, KV head) in this launch
  float scale_log2;
};

enum DecodeMode : int { DA_ALL = 0, DA_LOCAL = 1, DA_REMOTE = 2 };

// Pieces of a partial wave, shared by decode_partial_wave and the one-launch
// decode step (routing.hip).
//
// Chunk c of sequence b's list (local-window halves [0, nl), then two halves
// per listed page, the page ids at remote_row): the element offset of its
// (page, KV head g) block with the half in bit 0 (blocks are PAGE * HD
// elements, so the bit is free) and the valid token range [tok_lo, tok_hi)
// within the half.
template <int HD>
__device__ __forceinline__ int64_t decode_chunk_addr(const DecodeParams& P, int b, int g, int c, int nl, int c_lo,
                                                     int ls, int pos, const int32_t* remote_row, int& tok_lo,
                                                     int& tok_hi) {
  int lp, half;
  tok_lo = 0;
  tok_hi = CHUNK;
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
    lp = remote_row[r];
  }
  int64_t phys = -1;
  if (lp >= 0 && lp < P.max_pages) phys = P.page_table[static_cast<int64_t>(b) * P.max_pages + lp];
  if (phys < 0 || phys >= P.n_phys) {
    if (P.err) set_error(P.err, FSI_ERR_INDEX_RANGE);
    phys = 0;
    tok_lo = tok_hi = 0;  // nothing valid: the chunk is read from page 0 and masked out
  }
  return ((phys * P.Hkv + g) * PAGE) * HD + half;
}

// The K and V^T operands of the chunk whose offset (with the half in bit 0) is info.
template <int HD>
__device__ __forceinline__ void decode_load_chunk(const DecodeParams& P, int64_t info, u32x4_t (&kr)[HD / 16],
                                                  u32x4_t (&vr)[HD / 16]) {
  constexpr int KS = HD / 32;
  constexpr int DT = HD / 16;
  const int lane = threadIdx.x & 63;
  const int h = lane & 15, grp = lane >> 4;
  const int half = static_cast<int>(info & 1);
  const int64_t head_base = info - half;
  // K [HD/32][64][32]: the half starts at token 32 half of every dim chunk;
  // V [2][HD][32]: the half is the outer index
  const bf16_t* kp = P.k_pool + head_base + half * CHUNK * 32;
  const bf16_t* vp = P.v_pool + head_base + half * CHUNK * HD;
  // every K / V byte is read once per decode step: non-temporal loads keep the
  // stream from displacing the queries, page tables and partials in L2
#pragma unroll
  for (int tile = 0; tile < 2; ++tile)
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      kr[tile * KS + ks] = __builtin_nontemporal_load(
          reinterpret_cast<const u32x4_t*>(kp + ks * PAGE * 32 + (16 * tile + h) * 32 + 8 * grp));
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
    vr[dt] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(vp + (16 * dt + h) * CHUNK + 8 * grp));
}

// Q^T operand of (sequence b, KV head g): lane supplies Q[h][32 ks + 8 grp .. +8].
template <int HD>
__device__ __forceinline__ void decode_load_q(const DecodeParams& P, int b, int g, u32x4_t (&qb)[HD / 32]) {
  const int lane = threadIdx.x & 63;
  const int h = lane & 15, grp = lane >> 4;
#pragma unroll
  for (int ks = 0; ks < HD / 32; ++ks) {
    if (h < P.G) {
      qb[ks] = *reinterpret_cast<const u32x4_t*>(P.q + (static_cast<int64_t>(b) * P.Hq + g * P.G + h) * HD + 32 * ks +
                                                 8 * grp);
    } else {
      qb[ks] = u32x4_t{0u, 0u, 0u, 0u};
    }
  }
}

// One chunk of the online softmax: S^T, the running max and sum, P as a bf16
// hi + lo pair, O^T += V^T P^T.  Tokens outside [lo_t, hi_t) are masked (their
// V slots zeroed: the memory may hold anything).
template <int HD>
__device__ __forceinline__ void decode_chunk_math(const DecodeParams& P, const u32x4_t (&kcur)[HD / 16],
                                                  u32x4_t (&vcur)[HD / 16], const u32x4_t (&qb)[HD / 32], int lo_t,
                                                  int hi_t, float& m_run, float& l_run, f32x4_t (&acc)[HD / 16]) {
  constexpr int KS = HD / 32;
  constexpr int DT = HD / 16;
  const int lane = threadIdx.x & 63;
  const int grp = lane >> 4;
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
  // V^T tile: zero the slots of masked tokens
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
}

// The wave's (max, sum, O) into partial slot s of (sequence b, KV head g).
template <int HD>
__device__ __forceinline__ void decode_store_partial(const DecodeParams& P, int b, int g, int s, float m_run,
                                                     float l_run, const f32x4_t (&acc)[HD / 16]) {
  const int lane = threadIdx.x & 63;
  const int h = lane & 15, grp = lane >> 4;
  const int64_t part = (static_cast<int64_t>(b) * P.Hkv + g) * P.S + s;
  if (grp == 0) {
    P.m_part[part * 16 + h] = m_run;
    P.l_part[part * 16 + h] = l_run;
  }
  if (h < P.G) {
    float* o = P.o_part + (part * P.G + h) * HD;
#pragma unroll
    for (int dt = 0; dt < HD / 16; ++dt) *reinterpret_cast<f32x4_t*>(o + 16 * dt + 4 * grp) = acc[dt];
  }
}

// One wave's share of the partials: wave_id in [0, B Hkv S_sub).  Whole-wave
// work with no workgroup barriers, so it can run in any workgroup shape.
template <int HD>
__device__ __forceinline__ void decode_partial_wave(const DecodeParams& P, int wave_id) {
  constexpr int DT = HD / 16;
  const int lane = threadIdx.x & 63;
  if (wave_id >= P.B * P.Hkv * P.S_sub) return;
  const int s_loc = wave_id % P.S_sub;
  const int s = P.s_off + s_loc;
  const int g = (wave_id / P.S_sub) % P.Hkv;
  const int b = wave_id / (P.S_sub * P.Hkv);

  const int pos = P.pos_rows ? P.pos_rows[b] : P.pos;
  const int ls = pos + 1 - P.window > 0 ? pos + 1 - P.window : 0;
  const int c_lo = ls / CHUNK, c_hi = pos / CHUNK;
  const int nl = c_hi - c_lo + 1;
  int cnt = P.counts && P.mode != DA_LOCAL ? P.counts[static_cast<int64_t>(b) * (P.remote_stride ? 1 : 0)] : 0;
  cnt = cnt < 0 ? 0 : (cnt > P.cap ? P.cap : cnt);
  // this launch's chunks: [first, first + count) of the sequence's list
  const int first = P.mode == DA_REMOTE ? nl : 0;
  const int count = P.mode == DA_LOCAL ? nl : (P.mode == DA_REMOTE ? 2 * cnt : nl + 2 * cnt);
  const int per = (count + P.S_sub - 1) / P.S_sub;
  const int c0 = first + s_loc * per;
  int c1 = c0 + per < first + count ? c0 + per : first + count;
  if (c1 - c0 > MAX_CHUNKS_PER_WAVE) {  // only with per-sequence positions beyond the sizing bound
    if (P.err) set_error(P.err, FSI_ERR_CAPACITY);
    c1 = c0 + MAX_CHUNKS_PER_WAVE;
  }

  // chunk c0 + lane: offset with the half in bit 0 and valid token range
  int64_t cbase = 0;
  int tok_lo = 0, tok_hi = CHUNK;
  if (c0 + lane < c1)
    cbase = decode_chunk_addr<HD>(P, b, g, c0 + lane, nl, c_lo, ls, pos,
                                  P.remote + static_cast<int64_t>(b) * P.remote_stride, tok_lo, tok_hi);

  u32x4_t qb[HD / 32];
  decode_load_q<HD>(P, b, g, qb);
  f32x4_t acc[DT];
#pragma unroll
  for (int i = 0; i < DT; ++i) acc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;

  auto info_of = [&](int i) {
    const uint32_t lo = __builtin_amdgcn_readlane(static_cast<uint32_t>(cbase), i);
    const uint32_t hi = __builtin_amdgcn_readlane(static_cast<uint32_t>(cbase >> 32), i);
    return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
  };
  u32x4_t kcur[DT], vcur[DT], knxt[DT], vnxt[DT];
  if (c0 < c1) decode_load_chunk<HD>(P, info_of(0), kcur, vcur);
  for (int c = c0; c < c1; ++c) {
    const int cn = c + 1 < c1 ? c + 1 : c;  // straight-line prefetch (the last one re-reads)
    decode_load_chunk<HD>(P, info_of(cn - c0), knxt, vnxt);
    const int i = c - c0;
    decode_chunk_math<HD>(P, kcur, vcur, qb, __builtin_amdgcn_readlane(tok_lo, i), __builtin_amdgcn_readlane(tok_hi, i),
                          m_run, l_run, acc);
#pragma unroll
    for (int t = 0; t < DT; ++t) kcur[t] = knxt[t];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) vcur[dt] = vnxt[dt];
  }
  decode_store_partial<HD>(P, b, g, s, m_run, l_run, acc);
}

template <int HD>
__global__ __launch_bounds__(64 * DA_WAVES) void decode_attn_partial_kernel(DecodeParams P) {
  decode_partial_wave<HD>(P, blockIdx.x * DA_WAVES + (threadIdx.x >> 6));
}

// One wave per (sequence, query head) item: lanes read the split maxima and
// sums in parallel, then every lane merges HD / 64 dimensions over the splits.
template <int HD>
__device__ __forceinline__ void decode_merge_wave(const float* __restrict__ m_part, const float* __restrict__ l_part,
                                                  const float* __restrict__ o_part, int Hq, int Hkv, int G, int S,
                                                  bf16_t* __restrict__ out, int item) {
  constexpr int DPL = HD / 64;  // dimensions per lane
  const int lane = threadIdx.x & 63;
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
      // 16 slots' rows are loaded before any is summed (one memory latency per
      // 16 slots); the sum still runs over k in order
      for (int k0 = 0; k0 < n; k0 += 16) {
        float v[16][DPL], wk[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) {
          const int k = k0 + u < n ? k0 + u : n - 1;
          wk[u] = k0 + u < n ? __shfl(w, k, 64) : 0.f;
          const float* src = o_part + ((part0 + s0 + k) * G + h) * HD + lane * DPL;
#pragma unroll
          for (int i = 0; i < DPL; ++i) v[u][i] = src[i];
        }
#pragma unroll
        for (int u = 0; u < 16; ++u)
#pragma unroll
          for (int i = 0; i < DPL; ++i) o[i] = k0 + u < n ? fmaf(v[u][i], wk[u], o[i]) : o[i];
      }
    }
  }
  bf16_t* dst = out + (static_cast<int64_t>(b) * Hq + hq) * HD + lane * DPL;
#pragma unroll
  for (int i = 0; i < DPL; ++i) dst[i] = f32_to_bf16(L > 0.f ? o[i] / L : 0.f);
}

constexpr int MG_WAVES = 4;

template <int HD>
__global__ __launch_bounds__(64 * MG_WAVES) void decode_attn_merge_kernel(const float* __restrict__ m_part,
                                                                         const float* __restrict__ l_part,
                                                                         const float* __restrict__ o_part, int B,
                                                                         int Hq, int Hkv, int G, int S,
                                                                         bf16_t* __restrict__ out) {
  const int item = blockIdx.x * MG_WAVES + (threadIdx.x >> 6);
  if (item >= B * Hq) return;
  decode_merge_wave<HD>(m_part, l_part, o_part, Hq, Hkv, G, S, out, item);
}

// Partials and merge in one launch: one workgroup of S_sub waves per (sequence,
// KV head).  Wave s computes partial slot s_off + s as decode_partial_wave does
// in its own launch; after the workgroup barrier (workgroup-scope release and
// acquire: the slots just written are read back by waves of the same
// workgroup, the slots of an earlier launch are complete) waves merge the
// group's query heads over all S slots of the pair.  Removes the merge launch
// and its ramp; taken when S_sub <= FA_MAX_WAVES.
constexpr int FA_MAX_WAVES = 8;

template <int HD>
__global__ __launch_bounds__(64 * FA_MAX_WAVES) void decode_attn_fused_kernel(DecodeParams P, bf16_t* out) {
  const int wave = threadIdx.x >> 6;
  decode_partial_wave<HD>(P, static_cast<int>(blockIdx.x) * P.S_sub + wave);
  __syncthreads();
  const int b = static_cast<int>(blockIdx.x) / P.Hkv, g = static_cast<int>(blockIdx.x) % P.Hkv;
  for (int h = wave; h < P.G; h += P.S_sub)
    decode_merge_wave<HD>(P.m_part, P.l_part, P.o_part, P.Hq, P.Hkv, P.G, P.S, out, b * P.Hq + g * P.G + h);
}

// Partial waves a decode launch aims for: one round of resident waves on the chip
// (256 CUs x 8 waves of these kernels).
#ifndef FSI_DA_TARGET_WAVES
#define FSI_DA_TARGET_WAVES 2048
#endif

int split_count(int64_t B, int64_t Hkv, int64_t max_chunks) {
  // enough waves to cover the chip, at most 64 chunks per wave
  int64_t S = (FSI_DA_TARGET_WAVES + B * Hkv - 1) / (B * Hkv);
  const int64_t min_s = (max_chunks + MAX_CHUNKS_PER_WAVE - 1) / MAX_CHUNKS_PER_WAVE;
  if (S < min_s) S = min_s;
  if (S > max_chunks) S = max_chunks;
  if (S < 1) S = 1;
  return static_cast<int>(S);
}

// Upper bound on a sequence's local-window chunks: the window spans at most
// ceil(W / 32) + 1 halves and never more than the page table holds.
int64_t local_chunks_of(int64_t window, int64_t max_pages) {
  const int64_t local = (window + CHUNK - 1) / CHUNK + 1;
  return local > 2 * max_pages ? 2 * max_pages : local;
}

// Upper bound on a sequence's chunks (local window, then two per remote page).
int64_t max_chunks_of(int64_t window, int64_t cap, int64_t max_pages) {
  return local_chunks_of(window, max_pages) + 2 * cap;
}

// Partial slots per (sequence, KV head): S for the one-launch form, and
// S_local + S_remote for the local / remote launches, each of which is sized on
// its own to put about FSI_DA_TARGET_WAVES waves on the chip (at most MAX_CHUNKS_PER_WAVE
// chunks per wave, at least one chunk per wave).
struct DecodeSplit {
  int S, S_local, S_remote;
  int slots() const { return S > S_local + S_remote ? S : S_local + S_remote; }
};

int part_waves(int64_t B, int64_t Hkv, int64_t chunks) {
  int64_t s = (FSI_DA_TARGET_WAVES + B * Hkv - 1) / (B * Hkv);
  s = std::max<int64_t>(s, (chunks + MAX_CHUNKS_PER_WAVE - 1) / MAX_CHUNKS_PER_WAVE);
  s = std::min<int64_t>(s, std::max<int64_t>(chunks, 1));
  return static_cast<int>(std::max<int64_t>(s, 1));
}

DecodeSplit decode_split(int64_t B, int64_t Hkv, int64_t window, int64_t cap, int64_t max_pages) {
  DecodeSplit d;
  d.S = split_count(B, Hkv, max_chunks_of(window, cap, max_pages));
  d.S_local = part_waves(B, Hkv, local_chunks_of(window, max_pages));
  d.S_remote = part_waves(B, Hkv, 2 * cap);
  return d;
}



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

// Partial slots per (sequence, KV head) of the one-launch decode step
// (routing.hip, decode_step_fused_kernel: one per wave), which runs only with
// at least FS_MIN_PAIRS pairs.
constexpr int FS_SLOTS = 8;
constexpr int64_t FS_MIN_PAIRS = 128;

// Bytes of per-wave partials (max, sum, O) the partial and merge kernels exchange.
size_t decode_attn_partials_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t head_dim, int64_t window,
                                  int64_t capacity, int64_t max_pages) {
  int64_t slots = decode_split(B, Hkv, window, capacity, max_pages).slots();
  if (B * Hkv >= FS_MIN_PAIRS && slots < FS_SLOTS) slots = FS_SLOTS;
  const int64_t parts = B * Hkv * slots;
  return static_cast<size_t>(parts) * (2 * 16 + (Hq / Hkv) * head_dim) * sizeof(float);
}

// Kernel parameters of one launch in `mode` with the partials at ws (16-byte
// aligned, decode_attn_partials_bytes long).  DA_ALL uses partial slots [0, S);
// DA_LOCAL and DA_REMOTE use [0, S_local) and [S_local, S_local + S_remote) of
// the same layout, so the remote launch's merge sees both.  remote_stride:
// elements between sequences' rows of remote_pages and remote_counts (capacity
// and 1 normally; 0 makes every sequence read row 0).  s_local > 0 lowers the
// local launch's waves per (sequence, KV head); the remote launch of the same
// call must pass the same value.
DecodeParams decode_params(const void* q, const void* k_pool, const void* v_pool, const int32_t* page_table,
                           int64_t max_pages, int64_t n_phys_pages, const int32_t* pos_rows, int64_t pos,
                           int64_t window, const int32_t* remote_pages, const int32_t* remote_counts,
                           int64_t remote_stride, int64_t capacity, int64_t B, int64_t Hq, int64_t Hkv, float scale,
                           char* ws, int* err, int mode, int s_local = 0) {
  DecodeSplit split = decode_split(B, Hkv, window, capacity, max_pages);
  if (s_local > 0 && s_local < split.S_local) {
    // fewer local waves, same layout, but never so few that a wave would get
    // more than MAX_CHUNKS_PER_WAVE chunks of the window (the wave stops there)
    const int64_t min_s = (local_chunks_of(window, max_pages) + MAX_CHUNKS_PER_WAVE - 1) / MAX_CHUNKS_PER_WAVE;
    split.S_local = static_cast<int>(std::max<int64_t>(s_local, min_s));
  }
  const int S = mode == DA_ALL ? split.S : split.S_local + split.S_remote;
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
  P.remote_stride = (int)remote_stride;
  P.mode = mode;
  P.s_off = mode == DA_REMOTE ? split.S_local : 0;
  P.S_sub = mode == DA_ALL ? split.S : (mode == DA_LOCAL ? split.S_local : split.S_remote);
  P.scale_log2 = scale * LOG2E;
  return P;
}

int decode_partial_launch(const DecodeParams& P, int64_t head_dim, hipStream_t st) {
  const unsigned grid = static_cast<unsigned>((static_cast<int64_t>(P.B) * P.Hkv * P.S_sub + DA_WAVES - 1) / DA_WAVES);
  if (head_dim == 128) decode_attn_partial_kernel<128><<<grid, 64 * DA_WAVES, 0, st>>>(P);
  else decode_attn_partial_kernel<64><<<grid, 64 * DA_WAVES, 0, st>>>(P);
  FSI_HIP_LAUNCH_CHECK("decode_attn partial");
  return FSI_OK;
}

int decode_merge_launch(const DecodeParams& P, int64_t head_dim, void* out, hipStream_t st) {
  const unsigned grid = static_cast<unsigned>((static_cast<int64_t>(P.B) * P.Hq + MG_WAVES - 1) / MG_WAVES);
  if (head_dim == 128)
    decode_attn_merge_kernel<128><<<grid, 64 * MG_WAVES, 0, st>>>(P.m_part, P.l_part, P.o_part, P.B, P.Hq, P.Hkv, P.G,
                                                                  P.S, static_cast<bf16_t*>(out));
  else
    decode_attn_merge_kernel<64><<<grid, 64 * MG_WAVES, 0, st>>>(P.m_part, P.l_part, P.o_part, P.B, P.Hq, P.Hkv, P.G,
                                                                 P.S, static_cast<bf16_t*>(out));
  FSI_HIP_LAUNCH_CHECK("decode_attn merge");
  return FSI_OK;
}

// This launch's partials and the merge of all S slots: one fused launch when a
// workgroup holds the launch's waves of a (sequence, KV head), otherwise the
// partial kernel, then the merge kernel.
int decode_partial_merge_launch(const DecodeParams& P, int64_t head_dim, void* out, hipStream_t st) {
  if (P.S_sub > FA_MAX_WAVES) {
    const int c = decode_partial_launch(P, head_dim, st);
    return c != FSI_OK ? c : decode_merge_launch(P, head_dim, out, st);
  }
  const unsigned grid = static_cast<unsigned>(static_cast<int64_t>(P.B) * P.Hkv);
  const unsigned threads = static_cast<unsigned>(64 * P.S_sub);
  if (head_dim == 128) decode_attn_fused_kernel<128><<<grid, threads, 0, st>>>(P, static_cast<bf16_t*>(out));
  else decode_attn_fused_kernel<64><<<grid, threads, 0, st>>>(P, static_cast<bf16_t*>(out));
  FSI_HIP_LAUNCH_CHECK("decode_attn partial + merge");
  return FSI_OK;
}

// The partial and merge kernels in one stream with the partials at `ws`
// (every byte read is written first in the same call, so it needs no clearing).
int decode_attn_launch(const void* q, const void* k_pool, const void* v_pool, const int32_t* page_table,
                       int64_t max_pages, int64_t n_phys_pages, const int32_t* pos_rows, int64_t pos, int64_t window,
                       const int32_t* remote_pages, const int32_t* remote_counts, int64_t capacity, int64_t B,
                       int64_t Hq, int64_t Hkv, int64_t head_dim, float scale, void* out, char* ws, int* err,
                       void* stream) {
  const DecodeParams P = decode_params(q, k_pool, v_pool, page_table, max_pages, n_phys_pages, pos_rows, pos, window,
                                       remote_pages, remote_counts, capacity, capacity, B, Hq, Hkv, scale, ws, err,
                                       DA_ALL);
  return decode_partial_merge_launch(P, head_dim, out, reinterpret_cast<hipStream_t>(stream));
}

}  // namespace
