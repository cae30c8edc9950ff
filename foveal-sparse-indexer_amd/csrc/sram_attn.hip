// Fused block indexer + greedy block selection + block attention, one workgroup
// per (query block, batch * head).  Replaces triton_fused_sram_indexer_attention
// (foveal_indexer/triton_ops.py:142-249 kernel, :373-435 wrapper).
//
// Per workgroup, all in LDS / registers (nothing but q, k, v, q16, k16 is read
// from HBM and only the output is written):
//   1. 16-D scores s_j = <q16[b, m], k16[b, j]> * 0.25 of query block m against
//      every block j; a softmax over the remote blocks (j != m; the self block
//      gets probability 0) with the sum padded by 1e-6 (triton_ops.py:170-182).
//   2. Greedy selection, max_remote rounds: take the largest remaining
//      probability (lowest index among equal values); the pick attends iff the
//      mass taken before it is < top_p and its own probability is > 1e-4; its
//      probability is then retired (triton_ops.py:219-245).  Every round adds
//      its probability to the mass, attended or not.
//   3. Online-softmax attention of the block's queries over the self block and
//      then the attended picks in pick order: scores (q . k) * scale in fp32,
//      running max starting at -1e4, the row sum taken over the fp32
//      probabilities and the PV product over the probabilities rounded to the
//      storage dtype (triton_ops.py:200-243), output acc / max(l, 1e-6).
// A non-attended round of the reference leaves the running state unchanged
// (its scores are -1e4, never above the running max), so it is skipped here.
//
// fp16 / bf16 with block_size 16 / 32 / 64 and head_dim a multiple of 16 up to
// 128 run step 3 on MFMA tiles (sram_attn_mfma_kernel below); fp32 and other
// shapes use plain fp32 VALU over LDS tiles (q and k rows padded by one float:
// lanes of a score row read distinct banks).
#include <climits>

#include "fsi_common.h"

namespace {

using namespace fsi;

constexpr int SR_THREADS = 256;
constexpr int SR_MAX_BLOCK = 64;
constexpr int SR_MAX_HEAD_DIM = 256;
constexpr int SR_MAX_TILE = 8192;  // block_size * head_dim
constexpr int SR_MAX_BLOCKS = 8192;
constexpr int SR_MAX_REMOTE = 64;
constexpr float SR_NEG = -1.0e4f;

typedef _Float16 f16_t;

template <typename T>
__device__ __forceinline__ float to_f32(T v);
template <>
__device__ __forceinline__ float to_f32<float>(float v) { return v; }
template <>
__device__ __forceinline__ float to_f32<bf16_t>(bf16_t v) { return bf16_to_f32(v); }
template <>
__device__ __forceinline__ float to_f32<f16_t>(f16_t v) { return static_cast<float>(v); }

template <typename T>
__device__ __forceinline__ T from_f32(float v);
template <>
__device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <>
__device__ __forceinline__ bf16_t from_f32<bf16_t>(float v) { return f32_to_bf16(v); }
template <>
__device__ __forceinline__ f16_t from_f32<f16_t>(float v) { return static_cast<f16_t>(v); }

// Probability as the PV product consumes it: rounded to the storage dtype.
template <typename T>
__device__ __forceinline__ float round_to(float v) { return to_f32<T>(from_f32<T>(v)); }

struct SramArgs {
  const void* q;
  const void* k;
  const void* v;
  const void* q16;
  const void* k16;
  void* out;
  int32_t* sel_out;  // [B, n_blocks, max_remote] or null
  int H, N, D, BS, n_blocks, max_remote;
  float scale, top_p;
};

// (value, index) argmax step: larger value wins, equal values keep the lower index.
__device__ __forceinline__ void argmax_merge(float& v, int& i, float ov, int oi) {
  if (ov > v || (ov == v && oi < i)) {
    v = ov;
    i = oi;
  }
}

// Steps 1 and 2 for query block m of (b, h): probs [M], the selection in
// sel[0 .. *n_sel) (the self block first, then the attended picks in pick order)
// and, for h == 0, the per-round picks in sel_out.  Ends with a barrier.
template <typename TI>
__device__ void sram_route(const SramArgs& a, int b, int h, int m, float* probs, float* red_v, int* red_i,
                           int* sel, int* n_sel) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int M = a.n_blocks;
  const TI* q16 = static_cast<const TI*>(a.q16) + (static_cast<int64_t>(b) * M + m) * 16;
  const TI* k16 = static_cast<const TI*>(a.k16) + static_cast<int64_t>(b) * M * 16;

  // ---- 1. 16-D scores and the remote softmax ----
  float qv[16];
#pragma unroll
  for (int d = 0; d < 16; ++d) qv[d] = to_f32<TI>(q16[d]);
  float mx = -INFINITY;
  for (int j = tid; j < M; j += SR_THREADS) {
    float s = 0.f;
#pragma unroll
    for (int d = 0; d < 16; ++d) s = fmaf(qv[d], to_f32<TI>(k16[j * 16 + d]), s);
    s = j != m ? s * 0.25f : SR_NEG;
    probs[j] = s;
    mx = fmaxf(mx, s);
  }
  mx = wave_max(mx);
  if (lane == 0) red_v[wave] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red_v[0], red_v[1]), fmaxf(red_v[2], red_v[3]));
  float sum = 0.f;
  for (int j = tid; j < M; j += SR_THREADS) {
    const float e = j != m ? expf(probs[j] - mx) : 0.f;
    probs[j] = e;
    sum += e;
  }
  sum = wave_sum(sum);
  __syncthreads();  // every wave has read red_v
  if (lane == 0) red_v[wave] = sum;
  __syncthreads();
  const float denom = (red_v[0] + red_v[1]) + (red_v[2] + red_v[3]) + 1e-6f;
  for (int j = tid; j < M; j += SR_THREADS) probs[j] /= denom;
  if (tid == 0) {
    sel[0] = m;
    *n_sel = 1;
  }
  __syncthreads();

  // ---- 2. greedy selection ----
  float mass = 0.f;  // identical in every thread
  for (int r = 0; r < a.max_remote; ++r) {
    float bv = -INFINITY;
    int bi = INT_MAX;
    for (int j = tid; j < M; j += SR_THREADS) argmax_merge(bv, bi, probs[j], j);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      const float ov = __shfl_xor(bv, off, 64);
      const int oi = __shfl_xor(bi, off, 64);
      argmax_merge(bv, bi, ov, oi);
    }
    __syncthreads();  // previous round's readers of red_v / red_i are done
    if (lane == 0) {
      red_v[wave] = bv;
      red_i[wave] = bi;
    }
    __syncthreads();
    bv = red_v[0];
    bi = red_i[0];
#pragma unroll
    for (int w = 1; w < 4; ++w) argmax_merge(bv, bi, red_v[w], red_i[w]);
    const bool attend = bi < M && mass < a.top_p && bv > 1e-4f;
    mass += bv;
    if (tid == 0) {
      if (bi < M) probs[bi] = -1.f;
      if (attend) sel[(*n_sel)++] = bi;
      if (a.sel_out && h == 0)
        a.sel_out[(static_cast<int64_t>(b) * M + m) * a.max_remote + r] = attend ? bi : -1;
    }
    __syncthreads();
  }
}

template <typename T, typename TI, int NACC>
__global__ __launch_bounds__(SR_THREADS) void sram_attn_kernel(SramArgs a) {
  extern __shared__ __attribute__((aligned(16))) float sm[];
  const int tid = threadIdx.x;
  const int m = blockIdx.x, bh = blockIdx.y;
  const int b = bh / a.H, h = bh % a.H;
  const int M = a.n_blocks, BS = a.BS, D = a.D, DP = D + 1;

  float* probs = sm;                   // [M]
  float* qs = probs + ((M + 3) & ~3);  // [BS][DP]
  float* ks = qs + BS * DP;            // [BS][DP]
  float* vs = ks + BS * DP;            // [BS][D]
  float* ps = vs + BS * D;             // [BS][BS]
  float* row_m = ps + BS * BS;         // [BS]
  float* row_l = row_m + BS;           // [BS]
  float* row_a = row_l + BS;           // [BS]
  float* red_v = row_a + BS;           // [4]
  int* red_i = reinterpret_cast<int*>(red_v + 4);  // [4]
  int* sel = red_i + 4;                // [max_remote + 1]: attended blocks, self first
  __shared__ int n_sel;
  sram_route<TI>(a, b, h, m, probs, red_v, red_i, sel, &n_sel);

  // ---- 3. attention over the self block and the attended picks ----
  const int64_t head = (static_cast<int64_t>(b) * a.H + h) * a.N * D;
  const T* qg = static_cast<const T*>(a.q) + head + static_cast<int64_t>(m) * BS * D;
  for (int e = tid; e < BS * D; e += SR_THREADS) qs[(e / D) * DP + e % D] = to_f32<T>(qg[e]);
  if (tid < BS) {
    row_m[tid] = SR_NEG;
    row_l[tid] = 0.f;
  }
  float acc[NACC];
#pragma unroll
  for (int c = 0; c < NACC; ++c) acc[c] = 0.f;
  const int n_att = n_sel;
  for (int s = 0; s < n_att; ++s) {
    const int64_t kb = head + static_cast<int64_t>(sel[s]) * BS * D;
    const T* kg = static_cast<const T*>(a.k) + kb;
    const T* vg = static_cast<const T*>(a.v) + kb;
    for (int e = tid; e < BS * D; e += SR_THREADS) {
      ks[(e / D) * DP + e % D] = to_f32<T>(kg[e]);
      vs[e] = to_f32<T>(vg[e]);
    }
    __syncthreads();
    for (int e = tid; e < BS * BS; e += SR_THREADS) {
      const float* qr = qs + (e / BS) * DP;
      const float* kr = ks + (e % BS) * DP;
      float dot = 0.f;
      for (int d = 0; d < D; ++d) dot = fmaf(qr[d], kr[d], dot);
      ps[e] = dot * a.scale;
    }
    __syncthreads();
    if (tid < BS) {
      float* pr = ps + tid * BS;
      float rm = -INFINITY;
      for (int j = 0; j < BS; ++j) rm = fmaxf(rm, pr[j]);
      const float m_old = row_m[tid];
      const float m_new = fmaxf(m_old, rm);
      float psum = 0.f;
      for (int j = 0; j < BS; ++j) {
        const float p = expf(pr[j] - m_new);
        psum += p;
        pr[j] = round_to<T>(p);
      }
      const float alpha = expf(m_old - m_new);
      row_l[tid] = row_l[tid] * alpha + psum;
      row_a[tid] = alpha;
      row_m[tid] = m_new;
    }
    __syncthreads();
#pragma unroll
    for (int c = 0; c < NACC; ++c) {
      const int e = tid + c * SR_THREADS;
      if (e < BS * D) {
        const int i = e / D, d = e % D;
        const float* pr = ps + i * BS;
        float pv = 0.f;
        for (int j = 0; j < BS; ++j) pv = fmaf(pr[j], vs[j * D + d], pv);
        acc[c] = acc[c] * row_a[i] + pv;
      }
    }
    __syncthreads();  // ks / vs / ps are overwritten by the next block
  }
  T* og = static_cast<T*>(a.out) + head + static_cast<int64_t>(m) * BS * D;
#pragma unroll
  for (int c = 0; c < NACC; ++c) {
    const int e = tid + c * SR_THREADS;
    if (e < BS * D) og[e] = from_f32<T>(acc[c] / fmaxf(row_l[e / D], 1e-6f));
  }
}

// ---------------------------------------------------------------------------
// MFMA path: fp16 / bf16, block_size 16 / 32 / 64, head_dim a multiple of 16 up
// to 128.  Step 3 on v_mfma_f32_16x16x16 tiles, computed transposed so that every
// lane keeps one query: S^T = K Q^T leaves lane l (q = l / 16, r = l % 16) the
// scores of query r of its query tile against keys 4 q .. 4 q + 3 of each key
// tile, which is also the lane layout of the B operand of O^T = V^T P^T.  The
// row max and sum are taken over a lane's values and then across the four lane
// groups of a query; alpha rescales a lane's own O^T accumulators.  Q and K
// fragments (4 consecutive head dims of one row: 8 bytes) come straight from
// global memory; V is staged transposed in LDS (double buffered, one barrier per
// attended block).  Q, the self block's K fragments and its V rows are loaded
// before the selection, so their latency overlaps steps 1-2.
// Wave w owns query tile w / (4 / QT) and every (4 / QT)-th dim tile of it; with
// block_size 16 four waves share the query tile and split its dim tiles.
// ---------------------------------------------------------------------------
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef short short4_t __attribute__((ext_vector_type(4)));

template <typename T>
__device__ __forceinline__ f32x4_t mfma16x16x16(uint2 a, uint2 b, f32x4_t c);
template <>
__device__ __forceinline__ f32x4_t mfma16x16x16<f16_t>(uint2 a, uint2 b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(half4_t, a), __builtin_bit_cast(half4_t, b), c,
                                              0, 0, 0);
}
template <>
__device__ __forceinline__ f32x4_t mfma16x16x16<bf16_t>(uint2 a, uint2 b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(short4_t, a), __builtin_bit_cast(short4_t, b),
                                                  c, 0, 0, 0);
}

template <typename T>
__device__ __forceinline__ uint32_t bits16(float v);
template <>
__device__ __forceinline__ uint32_t bits16<f16_t>(float v) {
  return __builtin_bit_cast(uint16_t, static_cast<f16_t>(v));
}
template <>
__device__ __forceinline__ uint32_t bits16<bf16_t>(float v) { return f32_to_bf16(v); }

template <typename T>
__device__ __forceinline__ uint2 pack4(float a0, float a1, float a2, float a3) {
  return uint2{bits16<T>(a0) | (bits16<T>(a1) << 16), bits16<T>(a2) | (bits16<T>(a3) << 16)};
}

constexpr int SRM_MAX_DT = 8;  // head_dim <= 128

template <typename T, typename TI, int BS>
__global__ __launch_bounds__(SR_THREADS) void sram_attn_mfma_kernel(SramArgs a) {
  constexpr int QT = BS / 16;             // query tiles = key tiles of a block
  constexpr int WPQ = 4 / QT;             // waves per query tile
  constexpr int VT_LD = BS + 4;           // V^T row stride (halfs; rows stay 8-byte aligned)
  constexpr int VCH = (BS * SRM_MAX_DT * 16 / 8 + SR_THREADS - 1) / SR_THREADS;  // V rows' 16-byte chunks per thread
  extern __shared__ __attribute__((aligned(16))) float sm[];
  __shared__ __attribute__((aligned(16))) uint16_t vt[2][SRM_MAX_DT * 16 * VT_LD];
  __shared__ int n_sel;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int q4 = lane >> 4, r16 = lane & 15;
  const int m = blockIdx.x, bh = blockIdx.y;
  const int b = bh / a.H, h = bh % a.H;
  const int M = a.n_blocks, D = a.D, ndt = D / 16;
  const int it = wave / WPQ, sub = wave % WPQ;

  float* probs = sm;                               // [M]
  float* red_v = probs + ((M + 3) & ~3);           // [4]
  int* red_i = reinterpret_cast<int*>(red_v + 4);  // [4]
  int* sel = red_i + 4;                            // [max_remote + 1]

  const int64_t head = (static_cast<int64_t>(b) * a.H + h) * a.N * D;
  const T* qb = static_cast<const T*>(a.q) + head;
  const T* kbase = static_cast<const T*>(a.k) + head;
  const T* vbase = static_cast<const T*>(a.v) + head;

  // ---- loads issued before the selection: Q, the self block's K and V ------
  uint2 qf[SRM_MAX_DT];
  uint2 kf[QT][SRM_MAX_DT];
  uint4 vraw[VCH];
  auto load_k = [&](int blk) {
    const T* kg = kbase + static_cast<int64_t>(blk) * BS * D;
#pragma unroll
    for (int jt = 0; jt < QT; ++jt)
#pragma unroll
      for (int c = 0; c < SRM_MAX_DT; ++c)
        if (c < ndt) kf[jt][c] = *reinterpret_cast<const uint2*>(kg + (16 * jt + r16) * D + 16 * c + 4 * q4);
  };
  auto load_v = [&](int blk) {
    const T* vg = vbase + static_cast<int64_t>(blk) * BS * D;
#pragma unroll
    for (int u = 0; u < VCH; ++u) {
      const int ch = tid + u * SR_THREADS;
      if (ch * 8 < BS * D) vraw[u] = *reinterpret_cast<const uint4*>(vg + ch * 8);
    }
  };
  {
    const T* qg = qb + static_cast<int64_t>(m) * BS * D;
#pragma unroll
    for (int c = 0; c < SRM_MAX_DT; ++c)
      if (c < ndt) qf[c] = *reinterpret_cast<const uint2*>(qg + (16 * it + r16) * D + 16 * c + 4 * q4);
  }
  load_k(m);
  load_v(m);

  sram_route<TI>(a, b, h, m, probs, red_v, red_i, sel, &n_sel);

  // ---- 3. online softmax attention over the attended blocks ----------------
  float m_run = SR_NEG, l_run = 0.f;
  f32x4_t o[SRM_MAX_DT];
#pragma unroll
  for (int c = 0; c < SRM_MAX_DT; ++c) o[c] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const int n_att = n_sel;
  for (int s = 0; s < n_att; ++s) {
    if (s > 0) {
      load_k(sel[s]);
      load_v(sel[s]);
    }
    uint16_t* vts = vt[s & 1];
#pragma unroll
    for (int u = 0; u < VCH; ++u) {  // V rows -> V^T
      const int ch = tid + u * SR_THREADS;
      if (ch * 8 < BS * D) {
        const int j = (ch * 8) / D, d0 = (ch * 8) % D;
        const uint32_t w[4] = {vraw[u].x, vraw[u].y, vraw[u].z, vraw[u].w};
#pragma unroll
        for (int e = 0; e < 8; ++e) vts[(d0 + e) * VT_LD + j] = static_cast<uint16_t>(w[e >> 1] >> (16 * (e & 1)));
      }
    }
    // S^T tiles of this wave's query tile
    f32x4_t st[QT];
#pragma unroll
    for (int jt = 0; jt < QT; ++jt) {
      st[jt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < SRM_MAX_DT; ++c)
        if (c < ndt) st[jt] = mfma16x16x16<T>(kf[jt][c], qf[c], st[jt]);
    }
    float rm = -INFINITY;
#pragma unroll
    for (int jt = 0; jt < QT; ++jt)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        st[jt][e] *= a.scale;
        rm = fmaxf(rm, st[jt][e]);
      }
    rm = fmaxf(rm, __shfl_xor(rm, 16, 64));
    rm = fmaxf(rm, __shfl_xor(rm, 32, 64));
    const float m_new = fmaxf(m_run, rm);
    const float alpha = expf(m_run - m_new);
    float psum = 0.f;
    uint2 pf[QT];
#pragma unroll
    for (int jt = 0; jt < QT; ++jt) {
      float p[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        p[e] = expf(st[jt][e] - m_new);
        psum += p[e];
      }
      pf[jt] = pack4<T>(p[0], p[1], p[2], p[3]);  // probabilities rounded to the storage dtype
    }
    psum += __shfl_xor(psum, 16, 64);
    psum += __shfl_xor(psum, 32, 64);
    l_run = l_run * alpha + psum;
    m_run = m_new;
    __syncthreads();  // V^T of this block staged
#pragma unroll
    for (int c = 0; c < SRM_MAX_DT; ++c) {
      const int dt = sub + WPQ * c;
      if (dt < ndt) {
        o[c] *= alpha;
#pragma unroll
        for (int jt = 0; jt < QT; ++jt) {
          const uint2 vf = *reinterpret_cast<const uint2*>(&vts[(16 * dt + r16) * VT_LD + 16 * jt + 4 * q4]);
          o[c] = mfma16x16x16<T>(vf, pf[jt], o[c]);
        }
      }
    }
  }
  // lane: dims 16 dt + 4 q .. + 3 of query 16 it + r
  T* og = static_cast<T*>(a.out) + head + (static_cast<int64_t>(m) * BS + 16 * it + r16) * D;
  const float den = fmaxf(l_run, 1e-6f);
#pragma unroll
  for (int c = 0; c < SRM_MAX_DT; ++c) {
    const int dt = sub + WPQ * c;
    if (dt < ndt) *reinterpret_cast<uint2*>(og + 16 * dt + 4 * q4) = pack4<T>(o[c][0] / den, o[c][1] / den,
                                                                               o[c][2] / den, o[c][3] / den);
  }
}

size_t sram_mfma_lds_bytes(int64_t M, int64_t max_remote) {
  return (static_cast<size_t>((M + 3) & ~int64_t(3)) + 8 + static_cast<size_t>(max_remote) + 1) * 4;
}

bool sram_mfma_ok(int dtype, int64_t BS, int64_t D) {
  return dtype != FSI_DTYPE_F32 && (BS == 16 || BS == 32 || BS == 64) && D % 16 == 0 && D <= 16 * SRM_MAX_DT;
}

template <typename T, typename TI, int BS>
int launch_mfma_bs(const SramArgs& a, int64_t B, size_t lds, hipStream_t st) {
  if (lds > 32 * 1024 &&
      hipFuncSetAttribute(reinterpret_cast<const void*>(&sram_attn_mfma_kernel<T, TI, BS>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)) != hipSuccess) {
    fsi_host::set_last_error("sram_indexer_attention: %zu bytes of dynamic LDS refused", lds);
    return FSI_ERR_HIP;
  }
  dim3 grid(static_cast<unsigned>(a.n_blocks), static_cast<unsigned>(B * a.H));
  sram_attn_mfma_kernel<T, TI, BS><<<grid, SR_THREADS, lds, st>>>(a);
  FSI_HIP_LAUNCH_CHECK("sram_indexer_attention");
  return FSI_OK;
}

template <typename T, typename TI>
int launch_mfma(const SramArgs& a, int64_t B, size_t lds, hipStream_t st) {
  if (a.BS == 16) return launch_mfma_bs<T, TI, 16>(a, B, lds, st);
  if (a.BS == 32) return launch_mfma_bs<T, TI, 32>(a, B, lds, st);
  return launch_mfma_bs<T, TI, 64>(a, B, lds, st);
}

size_t sram_lds_bytes(int64_t M, int64_t BS, int64_t D, int64_t max_remote) {
  const size_t floats = static_cast<size_t>((M + 3) & ~int64_t(3)) + 2 * BS * (D + 1) + BS * D + BS * BS + 3 * BS + 4;
  return (floats + 4 + static_cast<size_t>(max_remote) + 1) * 4;
}

template <typename T, typename TI, int NACC>
int launch_nacc(const SramArgs& a, int64_t B, size_t lds, hipStream_t st) {
  if (lds > 64 * 1024 &&
      hipFuncSetAttribute(reinterpret_cast<const void*>(&sram_attn_kernel<T, TI, NACC>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)) != hipSuccess) {
    fsi_host::set_last_error("sram_indexer_attention: %zu bytes of dynamic LDS refused", lds);
    return FSI_ERR_HIP;
  }
  dim3 grid(static_cast<unsigned>(a.n_blocks), static_cast<unsigned>(B * a.H));
  sram_attn_kernel<T, TI, NACC><<<grid, SR_THREADS, lds, st>>>(a);
  FSI_HIP_LAUNCH_CHECK("sram_indexer_attention");
  return FSI_OK;
}

template <typename T, typename TI>
int launch_typed(const SramArgs& a, int64_t B, size_t lds, hipStream_t st) {
  const int64_t per = (static_cast<int64_t>(a.BS) * a.D + SR_THREADS - 1) / SR_THREADS;
  if (per <= 1) return launch_nacc<T, TI, 1>(a, B, lds, st);
  if (per <= 2) return launch_nacc<T, TI, 2>(a, B, lds, st);
  if (per <= 4) return launch_nacc<T, TI, 4>(a, B, lds, st);
  if (per <= 8) return launch_nacc<T, TI, 8>(a, B, lds, st);
  if (per <= 16) return launch_nacc<T, TI, 16>(a, B, lds, st);
  return launch_nacc<T, TI, 32>(a, B, lds, st);
}

template <typename T>
int launch_idx(const SramArgs& a, int idx_f32, int64_t B, size_t lds, hipStream_t st) {
  return idx_f32 ? launch_typed<T, float>(a, B, lds, st) : launch_typed<T, T>(a, B, lds, st);
}

}  // namespace

extern "C" {

FSI_API int fsi_sram_indexer_attention(const void* q, const void* k, const void* v, int dtype, const void* q16,
                                       const void* k16, int idx_dtype, int64_t B, int64_t H, int64_t N, int64_t head_dim,
                                       int64_t block_size, int64_t max_remote, float scale, float top_p, void* out,
                                       int32_t* selected, void* stream) {
  FSI_CHECK_ARG(q && k && v && q16 && k16 && out, FSI_ERR_INVALID_ARG, "sram_indexer_attention: null pointer");
  FSI_CHECK_ARG(dtype == FSI_DTYPE_F32 || dtype == FSI_DTYPE_BF16 || dtype == FSI_DTYPE_F16, FSI_ERR_DTYPE,
                "sram_indexer_attention: dtype %d unsupported", dtype);
  FSI_CHECK_ARG(idx_dtype == dtype || idx_dtype == FSI_DTYPE_F32, FSI_ERR_DTYPE,
                "sram_indexer_attention: q16 / k16 dtype %d must be the dtype of q or F32", idx_dtype);
  FSI_CHECK_ARG(B >= 0 && H > 0 && N >= 0 && head_dim > 0 && block_size > 0 && max_remote >= 0, FSI_ERR_SHAPE,
                "sram_indexer_attention: bad sizes");
  FSI_CHECK_ARG(N % block_size == 0, FSI_ERR_SHAPE, "sram_indexer_attention: N (%lld) %% block_size (%lld) != 0",
                static_cast<long long>(N), static_cast<long long>(block_size));
  FSI_CHECK_ARG(block_size <= SR_MAX_BLOCK && head_dim <= SR_MAX_HEAD_DIM && block_size * head_dim <= SR_MAX_TILE &&
                    N / block_size <= SR_MAX_BLOCKS && max_remote <= SR_MAX_REMOTE,
                FSI_ERR_CAPACITY,
                "sram_indexer_attention: block_size <= %d, head_dim <= %d, block_size * head_dim <= %d, "
                "N / block_size <= %d and max_remote <= %d",
                SR_MAX_BLOCK, SR_MAX_HEAD_DIM, SR_MAX_TILE, SR_MAX_BLOCKS, SR_MAX_REMOTE);
  FSI_CHECK_ARG(B * H <= 65535, FSI_ERR_CAPACITY, "sram_indexer_attention: B * H (%lld) > 65535",
                static_cast<long long>(B * H));
  if (B == 0 || N == 0) return FSI_OK;
  SramArgs a{q, k, v, q16, k16, out, selected, static_cast<int>(H), static_cast<int>(N), static_cast<int>(head_dim),
             static_cast<int>(block_size), static_cast<int>(N / block_size), static_cast<int>(max_remote), scale,
             top_p};
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int idx_f32 = idx_dtype == FSI_DTYPE_F32;
  const bool aligned = ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) |
                         reinterpret_cast<uintptr_t>(v) | reinterpret_cast<uintptr_t>(out)) & 15) == 0;
  if (aligned && sram_mfma_ok(dtype, block_size, head_dim)) {
    const size_t lds = sram_mfma_lds_bytes(a.n_blocks, max_remote);
    if (dtype == FSI_DTYPE_BF16)
      return idx_f32 ? launch_mfma<bf16_t, float>(a, B, lds, st) : launch_mfma<bf16_t, bf16_t>(a, B, lds, st);
    return idx_f32 ? launch_mfma<f16_t, float>(a, B, lds, st) : launch_mfma<f16_t, f16_t>(a, B, lds, st);
  }
  const size_t lds = sram_lds_bytes(a.n_blocks, block_size, head_dim, max_remote);
  FSI_CHECK_ARG(lds <= 160 * 1024, FSI_ERR_CAPACITY, "sram_indexer_attention: %zu bytes of LDS needed", lds);
  if (dtype == FSI_DTYPE_F32) return launch_idx<float>(a, idx_f32, B, lds, st);
  if (dtype == FSI_DTYPE_BF16) return launch_idx<bf16_t>(a, idx_f32, B, lds, st);
  return launch_idx<f16_t>(a, idx_f32, B, lds, st);
}

}  // extern "C"
