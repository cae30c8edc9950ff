// fp32 block-sparse prefill attention on MFMA (gfx950): the fp32 form of the
// 64-query LDS kernel of sparse_attn.hip, for fsi_sparse_attn with dtype fp32
// (FovealSparseAttention's default dtype, foveal_indexer/attention.py:35,
// 148-269; triton_foveal_sparse_attention, triton_ops.py:26-93).
//
//   out[t] = sum_s w(t, s) exp(scale q_t . k_s - m_t) v_s / l_t
//
// over the keys of the pattern: FSI_SATTN_LOCAL_REMOTE takes the union of the
// window (t - W, t] and the listed pages, FSI_SATTN_BLOCK_LIST every key of each
// listed block, counted as often as it is listed.
//
// Layout of the work: one workgroup per (sequence, GQA group of up to 4 query
// heads, 64 queries), 8 waves of one head x 32 queries (two 16-query tiles).
// 32-key chunks (K rows and a dim-major fp32 V^T copy) go once per workgroup
// into a ring of LDS slots with direct-to-LDS loads, F_AHEAD chunks ahead, and
// are read from there by all 8 waves.  Both products run on
// v_mfma_f32_16x16x4_f32 with fp32 operands, so scores, probabilities and
// sums are fp32 throughout:
//   S^T[key][query] = sum_d K[key][d] Q[query][d]     (A = K from LDS, B = Q^T
//                                                     held in registers)
//   O^T[d][query] += sum_key V^T[d][key] P^T[key][query]
// A 16-byte fragment read gives a lane 4 consecutive k values, used by four
// MFMAs (k-step kk takes k = 4 (lane / 16) + kk in every operand), and the P^T
// operand of step kk is element kk of the lane's S^T accumulator: the softmax
// needs no data movement between the products.  The row sums are kept per lane
// (a partial over its 8 keys of each chunk) and reduced across the four lane
// groups once at the end.  The running max moves only when a score passes it by
// more than 8 (log2 units), so the accumulators are rescaled rarely.
#include "fsi_common.h"

using namespace fsi;

namespace {

constexpr int F_CHUNK = 32;      // keys per chunk
constexpr int F_WAVES = 8;       // 4 query heads x 2 halves of the 64 queries
constexpr int F_QT = 2;          // 16-query tiles per wave
constexpr int F_MAX_CAP = 64;    // listed pages per query block
constexpr int F_AHEAD = 2;       // chunks in flight ahead of the one computed
constexpr int F_SLOTS = F_AHEAD + 1;
constexpr float F_LOG2E = 1.4426950408889634f;
typedef __attribute__((address_space(3))) void f_lds_t;
typedef __attribute__((address_space(1))) void f_glb_t;

struct F32Params {
  const float* q;
  int64_t qs_b, qs_h, qs_t;
  const float* k;
  int64_t ks_b, ks_h, ks_t;
  const float* vt;  // workspace: dim-major V^T per 32-key chunk (vt32_kernel)
  int B, Hq, Hkv, G, T, n32, block, mode, window;
  const int32_t* lists;
  int64_t ls_b, ls_q;
  const int32_t* counts;
  int64_t cs_b, cs_q;
  int cap, n_blocks;
  float scale_log2;
  float* out;
  int64_t os_b, os_h, os_t;
  int* err;
};

// vt[((b Hkv + g) n32 + c) HD 32 + d 32 + tau] = v[b][g][32 c + tau][d], 0 past T.
// Workgroup (c, b Hkv + g): the chunk's 32 rows in through LDS, out dim-major.
template <int HD>
__global__ __launch_bounds__(256) void vt32_kernel(const float* __restrict__ v, int64_t vs_b, int64_t vs_g,
                                                   int64_t vs_t, int Hkv, int T, int n32, float* __restrict__ vt) {
  __shared__ float tile[F_CHUNK][HD + 1];
  const int c = blockIdx.x, bg = blockIdx.y;
  const int b = bg / Hkv, g = bg % Hkv;
  const float* src = v + b * vs_b + g * vs_g;
  for (int i = threadIdx.x; i < F_CHUNK * HD / 4; i += 256) {
    const int row = i / (HD / 4), piece = i % (HD / 4);
    const int t = c * F_CHUNK + row;
    f32x4_t x = f32x4_t{0.f, 0.f, 0.f, 0.f};
    if (t < T) x = *reinterpret_cast<const f32x4_t*>(src + t * vs_t + 4 * piece);
#pragma unroll
    for (int j = 0; j < 4; ++j) tile[row][4 * piece + j] = x[j];
  }
  __syncthreads();
  float* dst = vt + (static_cast<int64_t>(bg) * n32 + c) * HD * F_CHUNK;
  for (int i = threadIdx.x; i < HD * F_CHUNK; i += 256) dst[i] = tile[i % F_CHUNK][i / F_CHUNK];
}

template <int N>
__device__ __forceinline__ void f_wait_vmcnt() {
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}
__device__ __forceinline__ void f_barrier() { asm volatile("s_barrier" ::: "memory"); }

__device__ __forceinline__ f32x4_t mfma4(float a, float b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

template <int HD>
__global__ __launch_bounds__(64 * F_WAVES) void sparse_attn_f32_kernel(F32Params P) {
  constexpr int DG = HD / 16;               // 16-dim groups
  constexpr int KROW = HD * 4;              // bytes of a K row
  constexpr int KBYTES = F_CHUNK * KROW;
  constexpr int VROW = F_CHUNK * 4;         // bytes of a V^T row (32 keys)
  constexpr int VBYTES = HD * VROW;
  constexpr int SLOT = KBYTES + VBYTES;     // one chunk in LDS
  constexpr int LOADS = SLOT / 1024;        // 1 KiB direct loads per chunk
  constexpr int LPW = LOADS / F_WAVES;
  static_assert(LPW >= 1 && LOADS % F_WAVES == 0, "chunk loads must split over the waves");
  static_assert(KBYTES % (1024 * LPW) == 0, "a wave's loads of a chunk are all K or all V^T");
  // One LDS array for the ring and the block list: separate __shared__ arrays get
  // alias scopes, and the compiler would then wait for every direct load in
  // flight before each ring read.
  __shared__ __attribute__((aligned(1024))) char smem[F_SLOTS * SLOT + F_MAX_CAP * 4];
  char (*ring)[SLOT] = reinterpret_cast<char (*)[SLOT]>(smem);
  int* wl = reinterpret_cast<int*>(smem + F_SLOTS * SLOT);

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int qblk0 = (gridDim.x - 1 - blockIdx.x) * 64;  // query blocks from the last (most keys)
  const int half = wave / 4;
  const int q0 = qblk0 + half * 16 * F_QT;
  const int per_g = (P.G + 3) / 4;
  int y = blockIdx.y;
  const int hsub = y % per_g;
  y /= per_g;
  const int g = y % P.Hkv;
  const int b = y / P.Hkv;
  const int hg = hsub * 4 + (wave & 3);
  const bool head_live = hg < P.G;  // idle waves still load and meet the barriers
  const int h = g * P.G + (head_live ? hg : 0);
  const int r = lane & 15, kg = lane >> 4;
  const int qb = qblk0 / P.block;
  const float sl2 = P.scale_log2, inv_sl2 = 1.f / P.scale_log2;

  // ---- listed pages: validity, first-listing de-duplication, compaction ----
  int cnt = P.counts[b * P.cs_b + qb * P.cs_q];
  cnt = cnt < 0 ? 0 : (cnt > P.cap ? P.cap : cnt);
  const int32_t* list = P.lists + b * P.ls_b + qb * P.ls_q;
  const int myblk = lane < cnt ? list[lane] : -1;
  bool okl = lane < cnt && myblk >= 0 && myblk < P.n_blocks;
  if (wave == 0 && lane < cnt && !okl && P.err) set_error(P.err, FSI_ERR_INDEX_RANGE);
  if (P.mode == FSI_SATTN_LOCAL_REMOTE) {
    for (int s2 = 0; s2 < F_MAX_CAP; ++s2) {  // a union: a page listed twice counts once
      if (s2 >= cnt) break;
      const int other = __builtin_amdgcn_readlane(myblk, s2);
      okl = okl && !(s2 < lane && other == myblk);
    }
  }
  const uint64_t vmask = __ballot(okl);
  if (wave == 0 && okl) wl[__popcll(vmask & ((uint64_t(1) << lane) - 1))] = myblk;
  const int n_remote = __popcll(vmask);

  int n_local = 0, c_lo = 0;
  if (P.mode == FSI_SATTN_LOCAL_REMOTE) {
    const int klo = qblk0 - P.window + 1 > 0 ? qblk0 - P.window + 1 : 0;
    const int khi = qblk0 + 63 < P.T - 1 ? qblk0 + 63 : P.T - 1;
    c_lo = klo / F_CHUNK;
    n_local = khi / F_CHUNK - c_lo + 1;
  }
  const int per_block = P.block / F_CHUNK;  // a power of two (host-checked)
  const int pb_shift = __builtin_ctz(per_block);
  const int n_chunks = n_local + n_remote * per_block;
  __syncthreads();  // wl is written
  // page list in a register (lane i: entry i), read with v_readlane: an LDS read in
  // the loop would wait for every direct load in flight
  const int wl_reg = lane < n_remote ? wl[lane] : 0;

  // chunk i: absolute chunk c, keys [0, hi) of it taken, window or page chunk
  auto describe = [&](int i, int& c, int& hi, bool& local) {
    if (i < n_local) {
      c = c_lo + i;
      hi = F_CHUNK;
      local = true;
    } else {
      const int j = i - n_local;
      const int blk = __builtin_amdgcn_readlane(wl_reg, j >> pb_shift);
      const int k0 = blk * P.block;
      const int k1 = k0 + P.block < P.T ? k0 + P.block : P.T;
      c = k0 / F_CHUNK + (j & (per_block - 1));
      hi = k1 - c * F_CHUNK;
      hi = hi > F_CHUNK ? F_CHUNK : hi;
      if (hi <= 0) {  // past the sequence: load the page's first chunk, use nothing
        c = k0 / F_CHUNK;
        hi = 0;
      }
      local = false;
    }
  };

  // ---- direct loads: this wave's LPW KiB of a chunk, K rows or V^T rows.  The
  // 16-byte pieces of each LDS row are XOR-swizzled with the row's low 3 bits, so
  // the 8 rows a 128-bit fragment read serves at once fall on 8 bank groups. ----
  const char* kbase = reinterpret_cast<const char*>(P.k + b * P.ks_b + g * P.ks_h);
  const char* vtbase =
      reinterpret_cast<const char*>(P.vt + (static_cast<int64_t>(b) * P.Hkv + g) * P.n32 * HD * F_CHUNK);
  const bool wave_k = wave * LPW * 1024 < KBYTES;
  uint32_t loff[LPW];
  int krow[LPW];
#pragma unroll
  for (int i = 0; i < LPW; ++i) {
    const int off = (wave * LPW + i) * 1024 + lane * 16;
    if (wave_k) {
      const int row = off / KROW, piece = (off % KROW) / 16;
      krow[i] = row;
      loff[i] = static_cast<uint32_t>(row * P.ks_t * 4 + 16 * (piece ^ (row & 7)));
    } else {
      const int vo = off - KBYTES;
      const int row = vo / VROW, piece = (vo % VROW) / 16;
      krow[i] = 0;
      loff[i] = static_cast<uint32_t>(row * VROW + 16 * (piece ^ (row & 7)));
    }
  }
  auto issue = [&](int c, int sl) {
    const char* base = wave_k ? kbase + static_cast<int64_t>(c) * F_CHUNK * P.ks_t * 4
                              : vtbase + static_cast<int64_t>(c) * VBYTES;
    char __attribute__((address_space(3)))* dst =
        (char __attribute__((address_space(3)))*)(&ring[sl][wave * LPW * 1024]);
    if (!wave_k || (c + 1) * F_CHUNK <= P.T) {
#pragma unroll
      for (int i = 0; i < LPW; ++i)
        __builtin_amdgcn_global_load_lds((f_glb_t*)(base + loff[i]), (f_lds_t*)(dst + i * 1024), 16, 0, 0);
    } else {  // the sequence's last chunk: K rows past T read row T - 1
#pragma unroll
      for (int i = 0; i < LPW; ++i) {
        const int row = c * F_CHUNK + krow[i] < P.T ? krow[i] : P.T - 1 - c * F_CHUNK;
        const char* src = base + loff[i] + static_cast<int64_t>(row - krow[i]) * P.ks_t * 4;
        __builtin_amdgcn_global_load_lds((f_glb_t*)src, (f_lds_t*)(dst + i * 1024), 16, 0, 0);
      }
    }
  };

  // Q^T operands for the whole kernel: lane (r, kg) holds Q[query 16 qt + r][16 dg + 4 kg .. +4]
  f32x4_t qreg[F_QT][DG];
#pragma unroll
  for (int qt = 0; qt < F_QT; ++qt) {
    const int myq = q0 + 16 * qt + r;
    const int qq = myq < P.T ? myq : P.T - 1;
    const float* qp = P.q + b * P.qs_b + h * P.qs_h + static_cast<int64_t>(qq) * P.qs_t + 4 * kg;
#pragma unroll
    for (int dg = 0; dg < DG; ++dg) qreg[qt][dg] = *reinterpret_cast<const f32x4_t*>(qp + 16 * dg);
  }
  f32x4_t acc[F_QT][DG];
  float m_run[F_QT], m_thr[F_QT], lpart[F_QT];
#pragma unroll
  for (int qt = 0; qt < F_QT; ++qt) {
    m_run[qt] = -1e30f;  // finite: masked scores (-inf) give p = 0 without a special case
    m_thr[qt] = (-1e30f + 8.f) * inv_sl2;
    lpart[qt] = 0.f;
#pragma unroll
    for (int dg = 0; dg < DG; ++dg) acc[qt][dg] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }

  f_wait_vmcnt<0>();  // the Q loads land before the ring's vmcnt accounting starts
  for (int i = 0; i < F_AHEAD; ++i) {
    if (i >= n_chunks) break;
    int c, hi;
    bool lc;
    describe(i, c, hi, lc);
    issue(c < P.n32 - 1 ? c : P.n32 - 1, i);
  }

  for (int i = 0; i < n_chunks; ++i) {
    // chunk i landed: at most the loads of chunks i + 1 .. i + AHEAD - 1 remain
    const int later = (i + F_AHEAD - 1 < n_chunks - 1 ? i + F_AHEAD - 1 : n_chunks - 1) - i;
    if (later >= 1) f_wait_vmcnt<LPW>();
    else f_wait_vmcnt<0>();
    f_barrier();
    if (i + F_AHEAD < n_chunks) {  // into the slot chunk i - 1 used
      int c, hi;
      bool lc;
      describe(i + F_AHEAD, c, hi, lc);
      issue(c < P.n32 - 1 ? c : P.n32 - 1, (i + F_AHEAD) % F_SLOTS);
    }
    int c, hi;
    bool local;
    describe(i, c, hi, local);
    if (hi <= 0 || !head_live) continue;  // uniform
    const char* stg = ring[i % F_SLOTS];
    const int kc0 = c * F_CHUNK;

    // S^T tiles: st[qt][t] holds keys 16 t + 4 kg + e, query 16 qt + r
    f32x4_t st[F_QT][2];
#pragma unroll
    for (int qt = 0; qt < F_QT; ++qt) st[qt][0] = st[qt][1] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int dg = 0; dg < DG; ++dg) {
      f32x4_t kf[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int row = 16 * t + r;
        kf[t] = *reinterpret_cast<const f32x4_t*>(stg + row * KROW + 16 * ((4 * dg + kg) ^ (row & 7)));
      }
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
#pragma unroll
        for (int qt = 0; qt < F_QT; ++qt)
#pragma unroll
          for (int t = 0; t < 2; ++t) st[qt][t] = mfma4(kf[t][kk], qreg[qt][dg][kk], st[qt][t]);
    }

    // online softmax; chunks every query of the wave sees skip the per-key mask
    const bool nomask = local ? (kc0 + F_CHUNK - 1 <= q0 && kc0 > q0 + 16 * F_QT - 1 - P.window &&
                                 kc0 + F_CHUNK <= P.T)
                              : (hi == F_CHUNK && (P.mode != FSI_SATTN_LOCAL_REMOTE ||
                                                   kc0 + F_CHUNK - 1 <= q0 - P.window));
#pragma unroll
    for (int qt = 0; qt < F_QT; ++qt) {
      const int myq = q0 + 16 * qt + r;
      float sv[8];  // key 16 t + 4 kg + e at 4 t + e
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e) sv[4 * t + e] = st[qt][t][e];
      if (!nomask) {
        // Branch-free: a score is kept when its sign word is negative (a taken key
        // inside T, and inside / outside the window for a local / listed chunk);
        // wlo >= -1 keeps every difference inside int range.
        int lk = 4 * kg;
        asm volatile("" : "+v"(lk));  // formed here, not held across the loop
        const int wlo = myq - (P.window < myq + 1 ? P.window : myq + 1);  // window: wlo < key <= myq
        const int wmode = P.mode == FSI_SATTN_LOCAL_REMOTE ? (local ? 1 : 2) : 0;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int tau = 16 * t + lk + e;
            const int key = kc0 + tau;
            int keep = (tau - hi) & (key - P.T);
            const int inw = (key - myq - 1) & (wlo - key);
            keep &= wmode == 0 ? -1 : (wmode == 1 ? inw : ~inw);
            sv[4 * t + e] = keep < 0 ? sv[4 * t + e] : -INFINITY;
          }
      }
      const float mx = max3_raw(max3_raw(sv[0], sv[1], sv[2]), max3_raw(sv[3], sv[4], sv[5]), max3_raw(sv[6], sv[7], sv[7]));
      if (__ballot(mx > m_thr[qt]) != 0) {  // uniform, rare: the running max moves
        const float m_cand = max_rows4(mx) * sl2;
        const bool bump = m_cand > m_run[qt] + 8.f;
        const float m_new = bump ? m_cand : m_run[qt];
        const float alpha = bump ? __builtin_amdgcn_exp2f(m_run[qt] - m_new) : 1.f;
        m_run[qt] = m_new;
        m_thr[qt] = (m_new + 8.f) * inv_sl2;  // scale_log2 > 0 on this path
        if (__ballot(bump) != 0) {
#pragma unroll
          for (int dg = 0; dg < DG; ++dg)
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[qt][dg][e] *= alpha;
          lpart[qt] *= alpha;
        }
      }
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float p = __builtin_amdgcn_exp2f(fmaf(sv[4 * t + e], sl2, -m_run[qt]));
          st[qt][t][e] = p;
          lpart[qt] += p;
        }
    }

    // O^T += V^T P^T: lane (r, kg) reads V^T[dim 16 dt + r][keys 16 t + 4 kg .. +4]
#pragma unroll
    for (int dt = 0; dt < DG; ++dt) {
      const int row = 16 * dt + r;
      f32x4_t vf[2];
#pragma unroll
      for (int t = 0; t < 2; ++t)
        vf[t] = *reinterpret_cast<const f32x4_t*>(stg + KBYTES + row * VROW + 16 * ((4 * t + kg) ^ (row & 7)));
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
#pragma unroll
          for (int qt = 0; qt < F_QT; ++qt) acc[qt][dt] = mfma4(vf[t][kk], st[qt][t][kk], acc[qt][dt]);
    }
  }

  if (!head_live) return;
#pragma unroll
  for (int qt = 0; qt < F_QT; ++qt) {
    const float l = sum_rows4(lpart[qt]);
    const int myq = q0 + 16 * qt + r;
    if (myq < P.T) {
      const float inv = l > 0.f ? 1.f / l : 0.f;
      float* o = P.out + b * P.os_b + h * P.os_h + static_cast<int64_t>(myq) * P.os_t + 4 * kg;
#pragma unroll
      for (int dt = 0; dt < DG; ++dt) {
        f32x4_t w = acc[qt][dt];
#pragma unroll
        for (int e = 0; e < 4; ++e) w[e] *= inv;
        *reinterpret_cast<f32x4_t*>(o + 16 * dt) = w;
      }
    }
  }
}

}  // namespace

namespace fsi_attn_f32 {

// fp32 prefill on MFMA when the shape fits the 64-query kernel: pages / blocks a
// power-of-two multiple of 64, at most 64 listed per query block, head_dim 64 or
// 128, 16-byte aligned rows, positive scale.  Returns 1 when it does not fit (the
// caller runs the generic kernel), else an FSI status.  `vt` holds the fp32 V^T
// copy (B Hkv ceil(T / 32) 32 head_dim floats).
int sparse_attn(const float* q, int64_t qs_b, int64_t qs_h, int64_t qs_t, const float* k, int64_t ks_b, int64_t ks_h,
                int64_t ks_t, const float* v, int64_t vs_b, int64_t vs_h, int64_t vs_t, int64_t B, int64_t Hq,
                int64_t Hkv, int64_t T, int64_t head_dim, int64_t block, int mode, int64_t window,
                const int32_t* lists, int64_t ls_b, int64_t ls_q, int64_t capacity, const int32_t* counts,
                int64_t cs_b, int64_t cs_q, float scale, float* out, int64_t os_b, int64_t os_h, int64_t os_t,
                float* vt, int* err, hipStream_t st) {
  using namespace fsi_host;
  const bool fits = (head_dim == 64 || head_dim == 128) && block % 64 == 0 && is_pow2(block) &&
                    capacity <= F_MAX_CAP && scale > 0.f && Hq % Hkv == 0 && qs_t % 4 == 0 && qs_h % 4 == 0 &&
                    qs_b % 4 == 0 && ks_t % 4 == 0 && ks_h % 4 == 0 && ks_b % 4 == 0 && vs_t % 4 == 0 &&
                    vs_h % 4 == 0 && vs_b % 4 == 0 && os_t % 4 == 0 && os_h % 4 == 0 && os_b % 4 == 0 &&
                    reinterpret_cast<uintptr_t>(q) % 16 == 0 && reinterpret_cast<uintptr_t>(k) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(v) % 16 == 0 && reinterpret_cast<uintptr_t>(out) % 16 == 0 &&
                    ks_t <= (int64_t(1) << 24) && T <= (int64_t(1) << 30) &&
                    B * Hkv * ((Hq / Hkv + 3) / 4) <= 65535 && B * Hkv <= 65535 && (T + F_CHUNK - 1) / F_CHUNK <= (1 << 30);
  if (!fits) return 1;
  const int n32 = static_cast<int>((T + F_CHUNK - 1) / F_CHUNK);
  F32Params P{};
  P.q = q;
  P.qs_b = qs_b;
  P.qs_h = qs_h;
  P.qs_t = qs_t;
  P.k = k;
  P.ks_b = ks_b;
  P.ks_h = ks_h;
  P.ks_t = ks_t;
  P.vt = vt;
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
  P.scale_log2 = scale * F_LOG2E;
  P.out = out;
  P.os_b = os_b;
  P.os_h = os_h;
  P.os_t = os_t;
  P.err = err;
  const dim3 g_vt(static_cast<unsigned>(n32), static_cast<unsigned>(B * Hkv));
  const dim3 grid(static_cast<unsigned>((T + 63) / 64), static_cast<unsigned>(B * Hkv * ((P.G + 3) / 4)));
  if (head_dim == 64) {
    vt32_kernel<64><<<g_vt, 256, 0, st>>>(v, vs_b, vs_h, vs_t, P.Hkv, P.T, n32, vt);
    FSI_HIP_LAUNCH_CHECK("sparse_attn fp32 v copy");
    sparse_attn_f32_kernel<64><<<grid, 64 * F_WAVES, 0, st>>>(P);
  } else {
    vt32_kernel<128><<<g_vt, 256, 0, st>>>(v, vs_b, vs_h, vs_t, P.Hkv, P.T, n32, vt);
    FSI_HIP_LAUNCH_CHECK("sparse_attn fp32 v copy");
    sparse_attn_f32_kernel<128><<<grid, 64 * F_WAVES, 0, st>>>(P);
  }
  FSI_HIP_LAUNCH_CHECK("sparse_attn fp32");
  return FSI_OK;
}

}  // namespace fsi_attn_f32
