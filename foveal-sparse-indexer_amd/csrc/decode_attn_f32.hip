// fp32 decode attention over the reference's contiguous cache layout
// (FovealKVCache k_cache / v_cache (B, Hkv, S, hd), its default dtype;
// foveal_indexer/attention.py:45-57, 339-367), split over the keys:
//
//   out[b, h] = sum_i exp(scale q . k_i - m) v_i / sum_i exp(scale q . k_i - m)
//
// over the key list of sequence b: tokens [max(0, pos + 1 - W), pos], then every
// token of each page remote_pages[b, :count] (concatenated, as the reference
// gathers them).
//
//   dec32_partial_kernel: wave (split s, b Hkv + g, head group) takes keys
//     [128 s, 128 s + 128) of that list for up to 16 query heads of KV head g.
//     Scores and products on v_mfma_f32_16x16x4_f32: S^T[key][head] with
//     A = K rows (16-byte loads: 4 dims a lane) and B = q^T; the softmax
//     probabilities of the lane's accumulator are, element by element, the A
//     operand of O[head][dim] += P[head][key] V[key][dim] (k-step kk of a
//     16-key tile takes keys 4 (lane / 16) + kk), B = V rows read 16 dims
//     at a time.  The split's max, sum and unnormalised output go to the
//     workspace (log2 units).
//   dec32_merge_kernel: wave (b, h) combines the splits of its sequence.
// The K / V stream is read once per KV head (the query heads of a group share
// it), which makes the step HBM-bound; the unused MFMA columns of groups of
// fewer than 16 heads cost MFMA time the stream leaves free.
#include "fsi_common.h"

using namespace fsi;

namespace {

// 96 keys per wave: at the C4 shape (3072 keys per sequence and KV head) 32 splits fill
// the chip's 4096 wave slots (four per SIMD) in two whole rounds; 128 (1.5 rounds)
// measured 0.197-0.203 ms against 0.188-0.189, 64 / 80 / 112 no better than 128 and
// 192 (two waves per SIMD) 0.245.
#ifndef FSI_D32_SPLIT
#define FSI_D32_SPLIT 96
#endif
constexpr int D_SPLIT = FSI_D32_SPLIT;  // keys per split (one wave)
constexpr int D_TILES = D_SPLIT / 16;
static_assert(D_SPLIT % 16 == 0 && D_SPLIT >= 16, "a split is whole 16-key tiles");
constexpr int D_WAVES = 4;    // splits per workgroup
constexpr int D_HG = 16;      // query heads per MFMA column block
constexpr float D_LOG2E = 1.4426950408889634f;

struct D32Params {
  const float* q;  // (B, Hq, hd) contiguous
  const float* k;
  const float* v;
  int64_t ks_b, ks_h, ks_t, vs_b, vs_h, vs_t;
  int S;
  const int32_t* pos_rows;
  int pos, window, page;
  int page_shift;         // log2(page) for a power-of-two page, else -1
  const int32_t* remote;  // (B, cap)
  const int32_t* counts;  // (B)
  int cap;
  int B, Hq, Hkv, G, hd, n_split;
  float scale_log2;
  float* part;  // (B, Hq, n_split, hd + 2): m, l, o
  float* out;   // (B, Hq, hd)
  int* err;
};

// Keys of sequence b: n_local window tokens from ls, then cnt pages.
struct KeyList {
  int ls, n_local, cnt, total;
};
__device__ __forceinline__ KeyList key_list(const D32Params& P, int b) {
  KeyList L;
  const int pos = P.pos_rows ? P.pos_rows[b] : P.pos;
  L.ls = pos + 1 - P.window > 0 ? pos + 1 - P.window : 0;
  L.n_local = pos >= 0 ? pos - L.ls + 1 : 0;
  int cnt = P.cap > 0 ? P.counts[b] : 0;
  L.cnt = cnt < 0 ? 0 : (cnt > P.cap ? P.cap : cnt);
  L.total = L.n_local + L.cnt * P.page;
  return L;
}

// Token of list entry i, or -1 (past the list, or a page outside the cache: *bad).
// (Branch-free selects here measured slower: their live values took the kernel
// from 120 to 196 VGPRs, i.e. from four to two waves per SIMD.)
__device__ __forceinline__ int key_token(const D32Params& P, const KeyList& L, int b, int i, bool& bad) {
  if (i < L.n_local) return L.ls + i < P.S ? L.ls + i : -1;
  if (i >= L.total) return -1;
  const int ir = i - L.n_local;
  int j, w;
  if (P.page_shift >= 0) {  // uniform
    j = ir >> P.page_shift;
    w = ir & (P.page - 1);
  } else {
    j = ir / P.page;
    w = ir % P.page;
  }
  const int pg = P.remote[static_cast<int64_t>(b) * P.cap + j];
  const int t = pg * P.page + w;
  if (pg >= 0 && t < P.S) return t;
  bad = true;
  return -1;
}

__device__ __forceinline__ f32x4_t mfma4(float a, float b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

template <int HD>
__global__ __launch_bounds__(64 * D_WAVES) void dec32_partial_kernel(D32Params P) {
  constexpr int DG = HD / 16;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, kg = lane >> 4;
  const int s = blockIdx.x * D_WAVES + wave;  // split
  const int bg = blockIdx.y;
  const int b = bg / P.Hkv, g = bg % P.Hkv;
  const int h0 = g * P.G + blockIdx.z * D_HG;  // first query head of this column block
  const int nh = P.G - blockIdx.z * D_HG < D_HG ? P.G - blockIdx.z * D_HG : D_HG;
  const KeyList L = key_list(P, b);
  if (s * D_SPLIT >= L.total) return;  // whole wave; no barriers in this kernel
  const float* kb = P.k + b * P.ks_b + g * P.ks_h;
  const float* vb = P.v + b * P.vs_b + g * P.vs_h;

  // q^T operand: lane (head r, kg) holds q[h0 + r][16 dg + 4 kg .. +4] (0 past the group)
  f32x4_t qf[DG];
#pragma unroll
  for (int dg = 0; dg < DG; ++dg) {
    qf[dg] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    if (r < nh) qf[dg] = *reinterpret_cast<const f32x4_t*>(P.q + (static_cast<int64_t>(b) * P.Hq + h0 + r) * HD +
                                                          16 * dg + 4 * kg);
  }
  bool bad = false;
  // scores: st[t] holds keys 16 t + 4 kg + e of the split, head r
  f32x4_t st[D_TILES];
  int tok[D_TILES][4];  // token of key 16 t + 4 kg + e (-1: masked)
#pragma unroll
  for (int t = 0; t < D_TILES; ++t) {
    const int i0 = s * D_SPLIT + 16 * t;
    const int tr = key_token(P, L, b, i0 + r, bad);  // the K row this lane loads
    const float* krow = kb + static_cast<int64_t>(tr >= 0 ? tr : 0) * P.ks_t + 4 * kg;
    f32x4_t kf[DG];
#pragma unroll
    for (int dg = 0; dg < DG; ++dg) kf[dg] = *reinterpret_cast<const f32x4_t*>(krow + 16 * dg);
    st[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int dg = 0; dg < DG; ++dg)
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) st[t] = mfma4(kf[dg][kk], qf[dg][kk], st[t]);
#pragma unroll
    for (int e = 0; e < 4; ++e) tok[t][e] = key_token(P, L, b, i0 + 4 * kg + e, bad);
  }
  // split max (log2 units) and probabilities
  float mx = -INFINITY;
#pragma unroll
  for (int t = 0; t < D_TILES; ++t)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float x = tok[t][e] >= 0 ? st[t][e] * P.scale_log2 : -INFINITY;
      st[t][e] = x;
      mx = __builtin_fmaxf(mx, x);
    }
  mx = max_rows4(mx);  // over the lanes of head r
  const float m_use = mx == -INFINITY ? 0.f : mx;
  float lpart = 0.f;
#pragma unroll
  for (int t = 0; t < D_TILES; ++t)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float p = __builtin_amdgcn_exp2f(st[t][e] - m_use);
      st[t][e] = p;
      lpart += p;
    }
  const float l = sum_rows4(lpart);
  // O[head][dim] += P[head][key] V[key][dim]: lane (dim r, kg) loads V[key 16 t + 4 kg + kk][16 dt + r]
  f32x4_t acc[DG];
#pragma unroll
  for (int dt = 0; dt < DG; ++dt) acc[dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int t = 0; t < D_TILES; ++t)
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int tv = tok[t][kk];
      const float* vrow = vb + static_cast<int64_t>(tv >= 0 ? tv : 0) * P.vs_t + r;
      // loads from the clamped row (always inside the cache), then a select: a
      // masked token's V is 0 (an unwritten row may hold anything)
      float vv[DG];
#pragma unroll
      for (int dt = 0; dt < DG; ++dt) vv[dt] = vrow[16 * dt];
#pragma unroll
      for (int dt = 0; dt < DG; ++dt) vv[dt] = tv >= 0 ? vv[dt] : 0.f;
#pragma unroll
      for (int dt = 0; dt < DG; ++dt) acc[dt] = mfma4(st[t][kk], vv[dt], acc[dt]);
    }
  if (bad) set_error(P.err, FSI_ERR_INDEX_RANGE);
  // lane (r, kg) holds O[head 4 kg + e][dim 16 dt + r]; m and l of head r sit in every lane of head r
  const int64_t stride = HD + 2;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int hl = 4 * kg + e;
    if (hl >= nh) continue;
    float* pp = P.part + ((static_cast<int64_t>(b) * P.Hq + h0 + hl) * P.n_split + s) * stride;
#pragma unroll
    for (int dt = 0; dt < DG; ++dt) pp[2 + 16 * dt + r] = acc[dt][e];
  }
  if (kg == 0 && r < nh) {
    float* pp = P.part + ((static_cast<int64_t>(b) * P.Hq + h0 + r) * P.n_split + s) * stride;
    pp[0] = mx;
    pp[1] = l;
  }
}

// Lane j of the wave takes splits j, j + 64, ...: the maximum and the split
// weights exp2(m_s - M) come out of two wave reductions, then every lane adds
// its dims of the weighted split outputs, the splits' loads issued together.
template <int HD>
__global__ __launch_bounds__(64 * D_WAVES) void dec32_merge_kernel(D32Params P) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * D_WAVES + (threadIdx.x >> 6);  // (b, h)
  if (row >= static_cast<int64_t>(P.B) * P.Hq) return;
  const int b = static_cast<int>(row / P.Hq);
  const KeyList L = key_list(P, b);
  const int ns = (L.total + D_SPLIT - 1) / D_SPLIT;
  const float* pp = P.part + row * P.n_split * (HD + 2);
  float M = -INFINITY;
  for (int s = lane; s < ns; s += 64) M = __builtin_fmaxf(M, pp[s * (HD + 2)]);
  M = wave_max(M);
  constexpr int DPL = (HD + 63) / 64;
  float o[DPL] = {};
  float lsum = 0.f;
  if (M != -INFINITY) {
    for (int s0 = 0; s0 < ns; s0 += 64) {
      // lane j: weight of split s0 + j (0 for splits with no key or past the count)
      float wj = 0.f, lj = 0.f;
      if (s0 + lane < ns) {
        const float ms = pp[(s0 + lane) * (HD + 2)];
        wj = ms == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(ms - M);
        lj = pp[(s0 + lane) * (HD + 2) + 1];
      }
      lsum += wave_sum(wj * lj);
      const int n = ns - s0 < 64 ? ns - s0 : 64;
      // eight splits' loads issued together, then added in split order (the same
      // fmaf chain as one split at a time; one at a time left a load latency per split)
      int j = 0;
      for (; j + 8 <= n; j += 8) {
        float qv[8][DPL];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const float* q = pp + (s0 + j + u) * (HD + 2) + 2;
#pragma unroll
          for (int e = 0; e < DPL; ++e) {
            const int d = lane + 64 * e;
            qv[u][e] = d < HD ? q[d] : 0.f;
          }
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const float w = __shfl(wj, j + u, 64);
#pragma unroll
          for (int e = 0; e < DPL; ++e) {
            const int d = lane + 64 * e;
            if (d < HD) o[e] = fmaf(w, qv[u][e], o[e]);
          }
        }
      }
      for (; j < n; ++j) {
        const float w = __shfl(wj, j, 64);
        const float* q = pp + (s0 + j) * (HD + 2) + 2;
#pragma unroll
        for (int e = 0; e < DPL; ++e) {
          const int d = lane + 64 * e;
          if (d < HD) o[e] = fmaf(w, q[d], o[e]);
        }
      }
    }
  }
  const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
#pragma unroll
  for (int e = 0; e < DPL; ++e) {
    const int d = lane + 64 * e;
    if (d < HD) P.out[row * HD + d] = o[e] * inv;
  }
}

}  // namespace

namespace fsi_dec32 {

// Split-key count and workspace bytes for a call (an upper bound over the batch).
int64_t n_split(int64_t window, int64_t capacity, int64_t page_size, int64_t max_seq) {
  const int64_t keys = (window < max_seq ? window : max_seq) + capacity * page_size;
  return keys <= 0 ? 1 : (keys + D_SPLIT - 1) / D_SPLIT;
}
size_t workspace_bytes(int64_t B, int64_t Hq, int64_t head_dim, int64_t window, int64_t capacity, int64_t page_size,
                       int64_t max_seq) {
  return static_cast<size_t>(B * Hq * n_split(window, capacity, page_size, max_seq) * (head_dim + 2)) * sizeof(float);
}

// fp32, head_dim 64 or 128, 16-byte aligned K rows: the split kernels; returns 1
// otherwise (the caller runs the per-head kernel), else an FSI status.
int run(const float* q, const float* k, const float* v, int64_t ks_b, int64_t ks_h, int64_t ks_t, int64_t vs_b,
        int64_t vs_h, int64_t vs_t, int64_t max_seq, const int32_t* pos_rows, int64_t pos, int64_t window,
        int64_t page_size, const int32_t* remote_pages, const int32_t* remote_counts, int64_t capacity, int64_t B,
        int64_t Hq, int64_t Hkv, int64_t head_dim, float scale, float* out, float* part, size_t part_bytes, int* err,
        hipStream_t st) {
  const int64_t ns = n_split(window, capacity, page_size, max_seq);
  const int64_t G = Hq / Hkv;
  const bool fits = (head_dim == 64 || head_dim == 128) && ks_t % 4 == 0 && ks_h % 4 == 0 && ks_b % 4 == 0 &&
                    reinterpret_cast<uintptr_t>(k) % 16 == 0 && reinterpret_cast<uintptr_t>(q) % 16 == 0 &&
                    part != nullptr &&
                    part_bytes >= workspace_bytes(B, Hq, head_dim, window, capacity, page_size, max_seq) &&
                    (ns + D_WAVES - 1) / D_WAVES <= 0x7fffffff && B * Hkv <= 65535 && (G + D_HG - 1) / D_HG <= 65535;
  if (!fits) return 1;
  D32Params P{};
  P.q = q;
  P.k = k;
  P.v = v;
  P.ks_b = ks_b;
  P.ks_h = ks_h;
  P.ks_t = ks_t;
  P.vs_b = vs_b;
  P.vs_h = vs_h;
  P.vs_t = vs_t;
  P.S = static_cast<int>(max_seq);
  P.pos_rows = pos_rows;
  P.pos = static_cast<int>(pos);
  P.window = static_cast<int>(window);
  P.page = static_cast<int>(page_size);
  P.page_shift = page_size > 0 && (page_size & (page_size - 1)) == 0 ? __builtin_ctzll(static_cast<uint64_t>(page_size)) : -1;
  P.remote = remote_pages;
  P.counts = remote_counts;
  P.cap = static_cast<int>(capacity);
  P.B = static_cast<int>(B);
  P.Hq = static_cast<int>(Hq);
  P.Hkv = static_cast<int>(Hkv);
  P.G = static_cast<int>(G);
  P.hd = static_cast<int>(head_dim);
  P.n_split = static_cast<int>(ns);
  P.scale_log2 = scale * D_LOG2E;
  P.part = part;
  P.out = out;
  P.err = err;
  const dim3 g1(static_cast<unsigned>((ns + D_WAVES - 1) / D_WAVES), static_cast<unsigned>(B * Hkv),
                static_cast<unsigned>((G + D_HG - 1) / D_HG));
  const dim3 g2(static_cast<unsigned>((B * Hq + D_WAVES - 1) / D_WAVES));
  if (head_dim == 64) {
    dec32_partial_kernel<64><<<g1, 64 * D_WAVES, 0, st>>>(P);
    FSI_HIP_LAUNCH_CHECK("decode_attn_dense fp32 partials");
    dec32_merge_kernel<64><<<g2, 64 * D_WAVES, 0, st>>>(P);
  } else {
    dec32_partial_kernel<128><<<g1, 64 * D_WAVES, 0, st>>>(P);
    FSI_HIP_LAUNCH_CHECK("decode_attn_dense fp32 partials");
    dec32_merge_kernel<128><<<g2, 64 * D_WAVES, 0, st>>>(P);
  }
  FSI_HIP_LAUNCH_CHECK("decode_attn_dense fp32 merge");
  return FSI_OK;
}

}  // namespace fsi_dec32
