// Block-sparse non-softmax Pattention forward for MI355X (gfx950).
//
//   out[M, D_out] = act(x K_gate[S]^T [, x K_up[S]^T]) V[S]
//
// Semantics follow foveal_indexer/pattention_triton.py:108-311 (fused kernel and
// PyTorch fallback) and the eval body of FovealPattentionMLP.forward
// (foveal_indexer/foveal_pattention.py:278-288,328-335).
//
// bf16 has three paths, chosen per call:
//   decode   (up to 64 tokens, V in down_proj layout, K % 256 == 0): split-K
//            kernels of pattention_decode.hip (LDS-shared token tile, weight
//            rows streamed once through a register ring).
//   GEMM     (256+ tokens, SwiGLU): the tiled MFMA engine of bsgemm.hip, with
//            the gather of active blocks in its loaders and SwiGLU fused in
//            the gate/up epilogue.
//   skinny   (everything else, below): one workgroup per (16 weight rows,
//            64-token tile) stages x and the weight rows through LDS and
//            splits K across its own waves, combined in LDS in a fixed order;
//            the down kernel reads V or V^T the same way.  H = act(...) is
//            written once as bf16 with the requested rounding points.
// Gate/up are computed exactly once per (token, channel); the reference fused
// kernel recomputes them for every 64-wide output tile
// (pattention_triton.py:127-169).
#include <stdlib.h>

#include "fsi_common.h"

namespace fsi_gemm {
int gateup_swiglu(const fsi::bf16_t* x, int64_t ldx, const fsi::bf16_t* kg, const fsi::bf16_t* ku, int64_t ldk,
                  int N_p, const int32_t* blocks, int n_active, int block_n, int M, int K, int rounding,
                  fsi::bf16_t* H, int64_t ldh, int* err, hipStream_t st);
int down_gather(const fsi::bf16_t* H, int64_t ldh, const fsi::bf16_t* wd, int64_t ldw, int N_p, const int32_t* blocks,
                int n_active, int block_n, int M, int D, fsi::bf16_t* out, int64_t ldo, int* err, hipStream_t st);
}  // namespace fsi_gemm

namespace fsi_dec {
size_t workspace_bytes(int64_t M, int64_t K, int64_t D, int64_t n_ch, int log2bn);
int run(const fsi::bf16_t* x, int64_t ldx, const fsi::bf16_t* kg, const fsi::bf16_t* ku, int64_t ldk,
        const fsi::bf16_t* vt, int64_t ldv, const int32_t* active, int64_t n_blocks_valid, int log2bn, int64_t N_p,
        int M, int K, int64_t n_ch, int D, int activation, int rounding, fsi::bf16_t* out, int64_t ldo,
        void* workspace, size_t ws_bytes, int* err, hipStream_t st);
}  // namespace fsi_dec

// Token count from which the tiled MFMA GEMM path replaces the skinny kernels.
constexpr int64_t GEMM_MIN_M = 256;
// Most active blocks the K-gathered down GEMM keeps in its LDS table.
constexpr int64_t GEMM_MAX_BLOCKS = 2048;

using namespace fsi;

namespace {

constexpr int TM = 64;   // tokens per tile
constexpr int TC = 64;   // channels (or output columns) per tile
constexpr int KCH = 64;  // K elements consumed per wave iteration in phase 1
constexpr int MAX_STAGES = 512;  // 64-channel stages with an LDS row table in the down kernel

// Logical channel -> weight row.  Channel c of the active set is row
// active[c >> log2bn] * bn + (c & (bn - 1)); dense when active == nullptr.
struct ChanMap {
  const int32_t* active;
  int64_t n_channels;
  int64_t N_p;
  int64_t n_blocks;  // number of valid block indices: ceil(N_p / bn)
  int log2bn;
};

__device__ __forceinline__ int64_t chan_row(const ChanMap& cm, int64_t c, int* err) {
  if (c >= cm.n_channels) return -1;
  if (cm.active == nullptr) return c;
  const int32_t blk = cm.active[c >> cm.log2bn];
  if (blk < 0 || blk >= cm.n_blocks) {
    set_error(err, FSI_ERR_INDEX_RANGE);
    return -1;
  }
  const int64_t r = (static_cast<int64_t>(blk) << cm.log2bn) | (c & ((int64_t(1) << cm.log2bn) - 1));
  return r < cm.N_p ? r : -1;  // tail rows of a partial last block are masked (pattention_triton.py:151)
}

// Workgroups with consecutive logical ids are placed on the same XCD: hardware
// dispatches workgroup w to XCD (w mod 8).  Neighbouring column groups of the
// down kernel share 128-byte lines of V, so they should share an L2.
__device__ __forceinline__ int xcd_logical_id(int w, int n) {
  if ((n & 7) != 0) return w;
  return (w & 7) * (n >> 3) + (w >> 3);
}

// Keeps the compiler's scheduler from moving instructions across a software
// pipeline stage boundary (loads of the next buffer vs. MFMAs on the current one).
#define SCHED_FENCE() __builtin_amdgcn_sched_barrier(0)

__device__ __forceinline__ u32x4_t ld16(const void* p) { return *reinterpret_cast<const u32x4_t*>(p); }

// ---------------------------------------------------------------------------
// Decode-shaped bf16 path.  No workgroup ever waits for another one: every
// workgroup produces complete outputs and splits the reduction dimension
// across its own waves, combined in LDS in a fixed order (deterministic).
// Device-scope fences between workgroups cost ~0.1 us each on MI355X and
// serialise, so split-K across workgroups is not used.
// ---------------------------------------------------------------------------
constexpr int NW2 = 16;  // waves per gather-down workgroup
constexpr int GC = 16;   // output columns per gather-down workgroup
constexpr int RED_LD = GC + 1;

// ---------------------------------------------------------------------------
// Phase 2 (down): workgroup = 16 output columns x 64 tokens, all channels.
// Wave w takes the 64-channel stages w, w + NW2, ...; a stage is two MFMA
// k-steps of 32 channels.  A operand: lane (r, q) holds H[16i + r][c0 + 8q, +8].
// B operand: lane (r, q) holds V[c0 + 8q + e][d0 + r], e < 8, gathered with
// 16-bit loads straight into the packed operand (V rows are D-contiguous).
// Masked channels have H == 0 and their V row is clamped to row 0.
// ---------------------------------------------------------------------------
template <bool ROW_LOOKUP>
__global__ __launch_bounds__(NW2 * 64) void patt_dec_down(
    const bf16_t* __restrict__ h, int64_t ldh, int M, const bf16_t* __restrict__ v, int64_t ldv,
    ChanMap cm, int n_ch_pad, int D_out, int d_groups, void* __restrict__ out, int64_t ldo, int out_f32,
    int* err) {
  __shared__ float red[NW2][TM][RED_LD];
  __shared__ int32_t rowtab[MAX_STAGES * 8];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15, q = lane >> 4;
  const int dg = xcd_logical_id(blockIdx.x, d_groups);
  const int mt = blockIdx.y;
  const int n_stages = n_ch_pad / TC;

  // Weight row of the first channel of each 8-channel group of every stage
  // (block_n >= 8 keeps such a group inside one block), or -1; built once.
  if (!ROW_LOOKUP) {
    for (int idx = threadIdx.x; idx < n_stages * 8; idx += NW2 * 64) {
      const int64_t c = static_cast<int64_t>(idx) * 8;
      rowtab[idx] = static_cast<int32_t>(chan_row(cm, c, err));
    }
    __syncthreads();
  }

  const char* hb = reinterpret_cast<const char*>(h);
  const char* vb = reinterpret_cast<const char*>(v);
  uint32_t hoff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int t = mt * TM + 16 * i + r;
    hoff[i] = static_cast<uint32_t>((t < M ? t : 0) * ldh * 2 + 8 * q * 2);
  }
  const int dcol = dg * GC + r;
  const bool dv = dcol < D_out;
  const uint32_t dbyte = static_cast<uint32_t>(dv ? dcol : 0) * 2u;

  f32x4_t acc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) acc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  struct Frag {
    u32x4_t ha[4][2];
    uint32_t vr[2][8];  // raw 16-bit V elements; packed into operands in compute()
  };
  auto load = [&](Frag& f, int st) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        f.ha[i][t] = ld16(hb + (hoff[i] + static_cast<uint32_t>(st * TC + 32 * t) * 2u));
      // 8 consecutive channels c0 .. c0 + 7 of this lane's k-group
      const int64_t c0 = static_cast<int64_t>(st) * TC + 32 * t + 8 * q;
      const int64_t base = ROW_LOOKUP ? -1 : rowtab[c0 >> 3];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        int64_t row;
        if (!ROW_LOOKUP) row = base >= 0 ? base + e : -1;
        else row = chan_row(cm, c0 + e, err);
        const uint32_t off = static_cast<uint32_t>((row >= 0 && row < cm.N_p ? row : 0) * ldv * 2) + dbyte;
        f.vr[t][e] = *reinterpret_cast<const uint16_t*>(vb + off);
      }
    }
  };
  auto compute = [&](const Frag& f) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const u32x4_t b = u32x4_t{f.vr[t][0] | (f.vr[t][1] << 16), f.vr[t][2] | (f.vr[t][3] << 16),
                                f.vr[t][4] | (f.vr[t][5] << 16), f.vr[t][6] | (f.vr[t][7] << 16)};
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] = mfma16x16x32(f.ha[i][t], b, acc[i]);
    }
  };

  const int mine = wave < n_stages ? (n_stages - wave + NW2 - 1) / NW2 : 0;
  if (mine > 0) {
    Frag f0, f1;
    load(f0, wave);
    int i = 0;
    for (; i + 2 < mine; i += 2) {
      load(f1, wave + NW2 * (i + 1));
      SCHED_FENCE();
      compute(f0);
      SCHED_FENCE();
      load(f0, wave + NW2 * (i + 2));
      SCHED_FENCE();
      compute(f1);
      SCHED_FENCE();
    }
    if (i + 1 < mine) {
      load(f1, wave + NW2 * (i + 1));
      SCHED_FENCE();
      compute(f0);
      compute(f1);
    } else {
      compute(f0);
    }
  }

#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) red[wave][16 * i + 4 * q + jj][r] = acc[i][jj];
  __syncthreads();
  for (int idx = threadIdx.x; idx < TM * GC; idx += NW2 * 64) {
    const int tok = idx / GC, col = idx % GC;
    float Y = 0.f;
#pragma unroll
    for (int w = 0; w < NW2; ++w) Y += red[w][tok][col];
    const int t = mt * TM + tok;
    const int d = dg * GC + col;
    if (t < M && d < D_out) {
      if (out_f32) reinterpret_cast<float*>(out)[static_cast<int64_t>(t) * ldo + d] = Y;
      else reinterpret_cast<bf16_t*>(out)[static_cast<int64_t>(t) * ldo + d] = f32_to_bf16(Y);
    }
  }
}

// ---------------------------------------------------------------------------
// LDS-staged skinny GEMM for the decode regime (the fast path).
//
//   acc_m[tok][row] = sum_k A[tok][k] * W_m[row][col(k)]      m < NMAT
//
// One workgroup = 16 weight rows x 64 tokens x all of K; 8 waves = 2 K-halves
// (kh) x 4 token quarters (mq).  A stage is two 64-wide K chunks (one per kh).
// Global loads are full 128-byte lines (lane l -> row 8v + l/8, 16-byte piece
// l%8), prefetched SK_DEPTH stages ahead into registers, then written to a
// two-buffer LDS ring with the piece order XOR-swizzled by (row >> 1) & 7, so
// that the MFMA-layout ds_read_b128 of 16 rows is bank-conflict free.  Loads
// in MFMA lane layout touch 16 half-used lines per instruction and ran at half
// the speed of full-line loads on MI355X.
//   MODE_GATEUP: A = x (M x K), W_0/W_1 = K_gate/K_up rows of 16 channels,
//                epilogue H = act(G, U) -> bf16 (zero on masked channels).
//   MODE_DOWNT : A = H (M x n_ch), W_0 = 16 rows of V^T (V stored [D_out, N_p],
//                the down_proj layout), K mapped through the active-channel
//                table; epilogue out = acc -> bf16 / fp32.
// ---------------------------------------------------------------------------
constexpr int MODE_GATEUP = 0;
constexpr int MODE_DOWNT = 1;
constexpr int SK_WAVES = 8;
constexpr int SK_ROWS = 64 + 2 * 16;  // LDS rows per K-half: 64 A rows + up to 2 x 16 W rows
constexpr int SK_HALF = SK_ROWS * 128;
constexpr int SK_STAGE = 2 * SK_HALF;
constexpr int SK_LOADS = 3;           // 16-byte loads per lane per stage (24 instr / 8 waves)
#ifndef FSI_SK_DEPTH
#define FSI_SK_DEPTH 4
#endif
constexpr int SKD = FSI_SK_DEPTH;     // stages of loads in flight per wave
constexpr int SK_TAB = MAX_STAGES * 8;

template <int MODE, int ACT, bool HAS_UP, int SK_DEPTH>
__global__ __launch_bounds__(SK_WAVES * 64) void patt_skinny(
    const bf16_t* __restrict__ a, int64_t lda, int M, const bf16_t* __restrict__ w0,
    const bf16_t* __restrict__ w1, int64_t ldw, ChanMap cm, int K, int n_rowgroups, int D_out,
    void* __restrict__ out, int64_t ldo, int out_f32, int rounding, int* err) {
  constexpr int NMAT = (MODE == MODE_GATEUP && HAS_UP) ? 2 : 1;
  constexpr int WROWS = 16 * NMAT;
  constexpr int ROWS = 64 + WROWS;  // rows staged per K-half
  __shared__ __attribute__((aligned(16))) unsigned char lds[2 * SK_STAGE];
  __shared__ int32_t coltab[MODE == MODE_DOWNT ? SK_TAB : 1];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kh = wave >> 2, mq = wave & 3;
  const int r = lane & 15, q = lane >> 4;
  const int rg = xcd_logical_id(blockIdx.x, n_rowgroups);  // group of 16 weight rows
  const int mt = blockIdx.y;
  const int n_chunks = (K + KCH - 1) / KCH;
  const int n_stages = (n_chunks + 1) / 2;

  if (MODE == MODE_DOWNT) {
    // Column (row of V^T's K dimension) of each 8-channel group, or -1 when masked.
    for (int i = threadIdx.x; i < n_chunks * 8; i += SK_WAVES * 64)
      coltab[i] = static_cast<int32_t>(chan_row(cm, static_cast<int64_t>(i) * 8, err));
    __syncthreads();
  }

  // ---- per-lane load descriptors (fixed for the whole kernel) --------------
  // Slot i of this wave loads instruction u = 3 * wave + i of a stage:
  // K-half kh_u = u / 12, 8-row group v_u = u % 12 of that half's ROWS rows.
  const char* lbase[SK_LOADS];
  uint32_t loff[SK_LOADS];   // byte offset of this lane's row
  uint32_t lpiece[SK_LOADS]; // 16-byte piece index in the 64-wide chunk
  int lkh[SK_LOADS];
  bool lvalid[SK_LOADS], lisA[SK_LOADS];
  uint32_t ldsoff[SK_LOADS];
#pragma unroll
  for (int i = 0; i < SK_LOADS; ++i) {
    const int u = SK_LOADS * wave + i;
    const int khu = u / 12, v = u % 12;
    const int R = 8 * v + (lane >> 3);
    const int slot = lane & 7;
    const int piece = slot ^ ((R >> 1) & 7);
    lkh[i] = khu;
    lpiece[i] = piece;
    lvalid[i] = R < ROWS;
    lisA[i] = R < 64;
    ldsoff[i] = static_cast<uint32_t>(khu * SK_HALF + R * 128 + slot * 16);
    if (R < 64) {
      const int t = mt * TM + R;
      lbase[i] = reinterpret_cast<const char*>(a);
      loff[i] = static_cast<uint32_t>((t < M ? t : 0) * lda * 2);
    } else {
      const int m = (R - 64) >> 4, wr = (R - 64) & 15;
      int64_t row;
      if (MODE == MODE_GATEUP) row = chan_row(cm, static_cast<int64_t>(rg) * 16 + wr, err);
      else row = (rg * 16 + wr < D_out) ? rg * 16 + wr : -1;
      lbase[i] = reinterpret_cast<const char*>(m == 0 ? w0 : w1);
      loff[i] = static_cast<uint32_t>((row >= 0 && R < ROWS ? row : 0) * ldw * 2);
    }
  }

  // Loads of stage st (clamped to the last stage at the tail; the duplicate is discarded).
  auto load_stage = [&](u32x4_t (&buf)[SK_LOADS], int st) {
    st = st < n_stages ? st : n_stages - 1;
#pragma unroll
    for (int i = 0; i < SK_LOADS; ++i) {
      const int c = 2 * st + lkh[i];
      uint32_t colb;
      bool kv;
      if (MODE == MODE_GATEUP || lisA[i]) {
        const int k = c * KCH + 8 * static_cast<int>(lpiece[i]);
        kv = k < K;
        colb = static_cast<uint32_t>(kv ? k : 0) * 2u;
      } else {
        const int g8 = c * 8 + static_cast<int>(lpiece[i]);
        const int32_t col = g8 < n_chunks * 8 ? coltab[g8] : -1;
        kv = true;  // masked channels have H == 0; clamp the column into the row
        colb = static_cast<uint32_t>(col >= 0 ? col : 0) * 2u;
      }
      u32x4_t vv = ld16(lbase[i] + (loff[i] + colb));
      // Past K the A operand must be zero (weights at the clamped address are finite).
      if (lisA[i] && !kv) vv = u32x4_t{0u, 0u, 0u, 0u};
      buf[i] = vv;
    }
  };
  auto store_stage = [&](const u32x4_t (&buf)[SK_LOADS], int b) {
#pragma unroll
    for (int i = 0; i < SK_LOADS; ++i)
      if (lvalid[i]) *reinterpret_cast<u32x4_t*>(lds + b * SK_STAGE + ldsoff[i]) = buf[i];
  };

  f32x4_t acc[NMAT];
#pragma unroll
  for (int m = 0; m < NMAT; ++m) acc[m] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // MFMA-layout reads: A rows 16 mq + r, W_m rows 64 + 16 m + r; pieces 2q + t.
  const int RA = 16 * mq + r;
  auto compute = [&](int b) {
    const unsigned char* half = lds + b * SK_STAGE + kh * SK_HALF;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const u32x4_t av = *reinterpret_cast<const u32x4_t*>(half + RA * 128 + (((2 * q + t) ^ ((RA >> 1) & 7)) * 16));
#pragma unroll
      for (int m = 0; m < NMAT; ++m) {
        const int RW = 64 + 16 * m + r;
        const u32x4_t wv = *reinterpret_cast<const u32x4_t*>(half + RW * 128 + (((2 * q + t) ^ ((RW >> 1) & 7)) * 16));
        acc[m] = mfma16x16x32(av, wv, acc[m]);
      }
    }
  };

  // SK_DEPTH stages of loads are in flight per wave (register ring, static indices).
  u32x4_t ring[SK_DEPTH][SK_LOADS];
#pragma unroll
  for (int d = 0; d < SK_DEPTH; ++d) load_stage(ring[d], d);
  for (int st = 0; st < n_stages; st += SK_DEPTH) {
#pragma unroll
    for (int d = 0; d < SK_DEPTH; ++d) {
      const int cur = st + d;
      if (cur < n_stages) {
        store_stage(ring[d], cur & 1);
        load_stage(ring[d], cur + SK_DEPTH);
        __syncthreads();
        compute(cur & 1);
      }
    }
  }

  // Combine the two K-halves: kh = 1 waves park their sums in LDS.
  __syncthreads();
  float* red = reinterpret_cast<float*>(lds);
  if (kh == 1) {
#pragma unroll
    for (int m = 0; m < NMAT; ++m)
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) red[(m * 64 + 16 * mq + 4 * q + jj) * 17 + r] = acc[m][jj];
  }
  __syncthreads();
  if (kh == 1) return;
#pragma unroll
  for (int m = 0; m < NMAT; ++m)
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) acc[m][jj] += red[(m * 64 + 16 * mq + 4 * q + jj) * 17 + r];

  // Epilogue: lane holds tokens 16 mq + 4 q + jj (jj < 4) of weight row r.
#pragma unroll
  for (int jj = 0; jj < 4; ++jj) {
    const int t = mt * TM + 16 * mq + 4 * q + jj;
    if (t >= M) continue;
    if (MODE == MODE_GATEUP) {
      const int64_t c = static_cast<int64_t>(rg) * 16 + r;
      const float g = acc[0][jj];
      const float uu = NMAT == 2 ? acc[NMAT - 1][jj] : 0.0f;
      const float av = chan_row(cm, c, nullptr) >= 0 ? pattention_act<ACT>(g, uu, rounding) : 0.0f;
      reinterpret_cast<bf16_t*>(out)[static_cast<int64_t>(t) * ldo + c] = f32_to_bf16(av);
    } else {
      const int d = rg * 16 + r;
      if (d < D_out) {
        if (out_f32) reinterpret_cast<float*>(out)[static_cast<int64_t>(t) * ldo + d] = acc[0][jj];
        else reinterpret_cast<bf16_t*>(out)[static_cast<int64_t>(t) * ldo + d] = f32_to_bf16(acc[0][jj]);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// fp32 path: LDS-tiled 16x16 kernels.  Each 16-wide K tile is summed into a
// fresh fp32 partial that is then added to the running sum (a two-level
// order): the rounding error grows with sqrt(16) + sqrt(K / 16) instead of
// sqrt(K) for one sequential chain, e.g. 2.4e-7 instead of 7.6e-7 rel-L2
// against exact arithmetic at D = 512 (CPU fp32 GEMMs: 5.3e-7).
// ---------------------------------------------------------------------------
template <int ACT, bool HAS_UP>
__global__ __launch_bounds__(256) void patt_gateup_f32(const float* __restrict__ x, int64_t ldx, int M,
                                                       const float* __restrict__ kg,
                                                       const float* __restrict__ ku, int64_t ldk,
                                                       ChanMap cm, int K, float* __restrict__ h,
                                                       int64_t ldh, int* err) {
  __shared__ float xs[16][17], gs[16][17], us[16][17];
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const int m0 = blockIdx.y * 16, c0 = blockIdx.x * 16;
  // Loader roles: thread (ty, tx) loads x[m0+ty][k+tx] and K[row(c0+ty)][k+tx].
  const int lm = m0 + ty;
  const int64_t lrow = chan_row(cm, c0 + ty, err);
  float accg = 0.f, accu = 0.f;
  for (int k0 = 0; k0 < K; k0 += 16) {
    const int k = k0 + tx;
    xs[ty][tx] = (lm < M && k < K) ? x[static_cast<int64_t>(lm) * ldx + k] : 0.f;
    gs[ty][tx] = (lrow >= 0 && k < K) ? kg[lrow * ldk + k] : 0.f;
    if (HAS_UP) us[ty][tx] = (lrow >= 0 && k < K) ? ku[lrow * ldk + k] : 0.f;
    __syncthreads();
    float pg = 0.f, pu = 0.f;
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) {
      pg = fmaf(xs[ty][kk], gs[tx][kk], pg);
      if (HAS_UP) pu = fmaf(xs[ty][kk], us[tx][kk], pu);
    }
    accg += pg;
    if (HAS_UP) accu += pu;
    __syncthreads();
  }
  const int m = m0 + ty, c = c0 + tx;
  if (m < M && c < cm.n_channels) h[static_cast<int64_t>(m) * ldh + c] = pattention_act<ACT>(accg, accu, FSI_ROUND_FP32);
}

__global__ __launch_bounds__(256) void patt_down_f32(const float* __restrict__ h, int64_t ldh, int M,
                                                     const float* __restrict__ v, int64_t ldv,
                                                     ChanMap cm, int D_out, float* __restrict__ out,
                                                     int64_t ldo, int* err) {
  __shared__ float hs[16][17], vs[16][17];
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const int m0 = blockIdx.y * 16, d0 = blockIdx.x * 16;
  float acc = 0.f;
  const int64_t C = cm.n_channels;
  for (int64_t c0 = 0; c0 < C; c0 += 16) {
    const int lm = m0 + ty;
    hs[ty][tx] = (lm < M && c0 + tx < C) ? h[static_cast<int64_t>(lm) * ldh + c0 + tx] : 0.f;
    const int64_t row = chan_row(cm, c0 + ty, err);
    vs[ty][tx] = (row >= 0 && d0 + tx < D_out) ? v[row * ldv + d0 + tx] : 0.f;
    __syncthreads();
    float p = 0.f;
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) p = fmaf(hs[ty][kk], vs[kk][tx], p);
    acc += p;
    __syncthreads();
  }
  const int m = m0 + ty, d = d0 + tx;
  if (m < M && d < D_out) out[static_cast<int64_t>(m) * ldo + d] = acc;
}

// ---------------------------------------------------------------------------
// Elementwise SwiGLU (pattention_triton.py:30-47 forward, 98-104).
// ---------------------------------------------------------------------------
__global__ void swiglu_bf16(const bf16_t* __restrict__ g, const bf16_t* __restrict__ u,
                            bf16_t* __restrict__ out, int64_t n, int rounding) {
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const float gv = bf16_to_f32(g[i]), uv = bf16_to_f32(u[i]);
    float s = silu_f32(gv);
    if (rounding == FSI_ROUND_EAGER) s = round_bf16(s);
    out[i] = f32_to_bf16(s * uv);
  }
}
__global__ void swiglu_f32(const float* __restrict__ g, const float* __restrict__ u, float* __restrict__ out,
                           int64_t n) {
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x)
    out[i] = silu_f32(g[i]) * u[i];
}

// SwiGLU backward (pattention_triton.py:49-71): with s = sigmoid(g),
//   du = dout * g s,   dg = dout * u * s (1 + g (1 - s)),
// in fp32, each rounded once to the storage dtype.
template <typename T>
__device__ __forceinline__ float ld_as_f32(const T* p, int64_t i) {
  if constexpr (sizeof(T) == 2) return bf16_to_f32(reinterpret_cast<const bf16_t*>(p)[i]);
  else return reinterpret_cast<const float*>(p)[i];
}
template <typename T>
__device__ __forceinline__ void st_from_f32(T* p, int64_t i, float v) {
  if constexpr (sizeof(T) == 2) reinterpret_cast<bf16_t*>(p)[i] = f32_to_bf16(v);
  else reinterpret_cast<float*>(p)[i] = v;
}
template <typename T>
__global__ void swiglu_bwd_kernel(const T* __restrict__ dout, const T* __restrict__ g, const T* __restrict__ u,
                                  T* __restrict__ dg, T* __restrict__ du, int64_t n) {
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const float d = ld_as_f32(dout, i), gv = ld_as_f32(g, i), uv = ld_as_f32(u, i);
    const float s = 1.0f / (1.0f + expf(-gv));
    st_from_f32(du, i, d * (gv * s));
    st_from_f32(dg, i, d * uv * (s * (1.0f + gv * (1.0f - s))));
  }
}

// Byte-wise zero fill of `rows` rows of `row_bytes` bytes (stride `ld_bytes`).
// A kernel rather than hipMemsetAsync so the call stays safe inside graph capture.
__global__ void zero_rows(char* __restrict__ p, int64_t ld_bytes, int64_t row_bytes) {
  const int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
  if (i < row_bytes) p[static_cast<int64_t>(blockIdx.y) * ld_bytes + i] = 0;
}

// ---------------------------------------------------------------------------
// Host-side planning.
// ---------------------------------------------------------------------------
struct Plan {
  int m_tiles, n_groups, d_groups;
  int64_t n_ch_pad;  // channels rounded up to whole 64-channel stages
  size_t off_h, total;
};

Plan make_plan_bf16(int64_t M, int64_t D_out, int64_t n_channels) {
  Plan p{};
  p.m_tiles = static_cast<int>((M + TM - 1) / TM);
  p.n_ch_pad = (n_channels + TC - 1) / TC * TC;
  p.n_groups = static_cast<int>(p.n_ch_pad / GC);
  p.d_groups = static_cast<int>((D_out + GC - 1) / GC);
  p.off_h = FSI_WORKSPACE_COUNTER_BYTES;
  p.total = p.off_h + fsi_host::align_up(sizeof(bf16_t) * static_cast<size_t>(M) * p.n_ch_pad, 256);
  return p;
}

size_t workspace_f32(int64_t M, int64_t n_channels) {
  return FSI_WORKSPACE_COUNTER_BYTES +
         fsi_host::align_up(sizeof(float) * static_cast<size_t>(M) * static_cast<size_t>(n_channels), 256);
}

template <int ACT>
void launch_gateup_f32(bool has_up, dim3 grid, hipStream_t st, const float* x, int64_t ldx, int M,
                       const float* kg, const float* ku, int64_t ldk, ChanMap cm, int K, float* h, int64_t ldh,
                       int* err) {
  if (has_up)
    patt_gateup_f32<ACT, true><<<grid, 256, 0, st>>>(x, ldx, M, kg, ku, ldk, cm, K, h, ldh, err);
  else
    patt_gateup_f32<ACT, false><<<grid, 256, 0, st>>>(x, ldx, M, kg, ku, ldk, cm, K, h, ldh, err);
}

}  // namespace

extern "C" {

size_t fsi_pattention_workspace_size(int64_t M, int64_t K, int64_t D_out, int64_t n_channels, int dtype) {
  if (M <= 0 || K <= 0 || D_out <= 0 || n_channels <= 0) return FSI_WORKSPACE_COUNTER_BYTES;
  if (dtype == FSI_DTYPE_F32) return workspace_f32(M, n_channels);
  const size_t skinny = make_plan_bf16(M, D_out, n_channels).total;
  // the decode path (M <= 64) needs its split partials too; block sizes >= 32 only
  const size_t dec = fsi_dec::workspace_bytes(M, K, D_out, n_channels, 5);
  return skinny > dec ? skinny : dec;
}

int fsi_pattention_fwd(const void* x, int64_t ldx, const void* k_gate, const void* k_up, int64_t ldk,
                       const void* v, int64_t ldv, int v_transposed, const int32_t* active_blocks, int64_t n_active,
                       int64_t block_n, int64_t M, int64_t K, int64_t N_p, int64_t D_out, int dtype,
                       int activation, int rounding, void* out, int64_t ldo, void* workspace,
                       size_t workspace_bytes, int* err, void* stream) {
  FSI_CHECK_ARG(dtype == FSI_DTYPE_BF16 || dtype == FSI_DTYPE_F32, FSI_ERR_DTYPE, "pattention: dtype %d", dtype);
  FSI_CHECK_ARG(activation >= FSI_ACT_SWIGLU && activation <= FSI_ACT_RELU2, FSI_ERR_INVALID_ARG,
                "pattention: activation code %d", activation);
  FSI_CHECK_ARG(rounding >= FSI_ROUND_EAGER && rounding <= FSI_ROUND_FP32, FSI_ERR_INVALID_ARG,
                "pattention: rounding mode %d", rounding);
  FSI_CHECK_ARG(M >= 0 && K > 0 && N_p > 0 && D_out > 0, FSI_ERR_SHAPE,
                "pattention: M=%lld K=%lld N_p=%lld D_out=%lld", (long long)M, (long long)K, (long long)N_p,
                (long long)D_out);
  FSI_CHECK_ARG(M < (int64_t(1) << 30) && K < (int64_t(1) << 30) && D_out < (int64_t(1) << 30), FSI_ERR_SHAPE,
                "pattention: dimension too large");
  FSI_CHECK_ARG(fsi_host::is_pow2(block_n), FSI_ERR_SHAPE, "pattention: block_n=%lld must be a power of two",
                (long long)block_n);
  FSI_CHECK_ARG(x && k_gate && v && out, FSI_ERR_INVALID_ARG, "pattention: null tensor pointer");
  FSI_CHECK_ARG(activation != FSI_ACT_SWIGLU || k_up != nullptr, FSI_ERR_INVALID_ARG,
                "pattention: k_up required for swiglu");
  FSI_CHECK_ARG(ldx >= K && ldk >= K && ldo >= D_out && ldv >= (v_transposed ? N_p : D_out), FSI_ERR_SHAPE,
                "pattention: leading dimension smaller than row length");
  FSI_CHECK_ARG(active_blocks != nullptr || n_active == 0, FSI_ERR_INVALID_ARG,
                "pattention: n_active > 0 with null active_blocks");
  FSI_CHECK_ARG(n_active >= 0, FSI_ERR_SHAPE, "pattention: n_active < 0");

  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const bool has_up = (activation == FSI_ACT_SWIGLU);
  const bool dense = (active_blocks == nullptr);
  const int64_t n_channels = dense ? N_p : n_active * block_n;

  ChanMap cm;
  cm.active = active_blocks;
  cm.n_channels = n_channels;
  cm.N_p = N_p;
  cm.log2bn = fsi_host::ilog2(block_n);
  cm.n_blocks = (N_p + block_n - 1) / block_n;

  const size_t elt = dtype == FSI_DTYPE_BF16 ? 2 : 4;
  if (M == 0) return FSI_OK;
  if (n_channels == 0) {
    // No active channels: the output is exactly zero (pattention_triton.py:141 loop never runs).
    const dim3 gz((unsigned)((D_out * (int64_t)elt + 255) / 256), (unsigned)M);
    zero_rows<<<gz, 256, 0, st>>>(static_cast<char*>(out), ldo * (int64_t)elt, D_out * (int64_t)elt);
    FSI_HIP_LAUNCH_CHECK("pattention zero fill");
    return FSI_OK;
  }

  if (dtype == FSI_DTYPE_F32) {
    FSI_CHECK_ARG(!v_transposed, FSI_ERR_SHAPE, "pattention f32: V must be [N_p, D_out] row-major");
    const size_t need = workspace_f32(M, n_channels);
    FSI_CHECK_ARG(workspace && workspace_bytes >= need, FSI_ERR_WORKSPACE,
                  "pattention: workspace %zu < required %zu", workspace_bytes, need);
    float* h = reinterpret_cast<float*>(static_cast<char*>(workspace) + FSI_WORKSPACE_COUNTER_BYTES);
    const dim3 g1((unsigned)((n_channels + 15) / 16), (unsigned)((M + 15) / 16));
    const float* xf = static_cast<const float*>(x);
    const float* kgf = static_cast<const float*>(k_gate);
    const float* kuf = static_cast<const float*>(k_up);
    switch (activation) {
      case FSI_ACT_SWIGLU: launch_gateup_f32<ACT_SWIGLU>(true, g1, st, xf, ldx, (int)M, kgf, kuf, ldk, cm, (int)K, h, n_channels, err); break;
      case FSI_ACT_SILU: launch_gateup_f32<ACT_SILU>(false, g1, st, xf, ldx, (int)M, kgf, kuf, ldk, cm, (int)K, h, n_channels, err); break;
      case FSI_ACT_GELU: launch_gateup_f32<ACT_GELU>(false, g1, st, xf, ldx, (int)M, kgf, kuf, ldk, cm, (int)K, h, n_channels, err); break;
      case FSI_ACT_RELU: launch_gateup_f32<ACT_RELU>(false, g1, st, xf, ldx, (int)M, kgf, kuf, ldk, cm, (int)K, h, n_channels, err); break;
      default: launch_gateup_f32<ACT_RELU2>(false, g1, st, xf, ldx, (int)M, kgf, kuf, ldk, cm, (int)K, h, n_channels, err); break;
    }
    FSI_HIP_LAUNCH_CHECK("pattention gateup f32");
    const dim3 g2((unsigned)((D_out + 15) / 16), (unsigned)((M + 15) / 16));
    patt_down_f32<<<g2, 256, 0, st>>>(h, n_channels, (int)M, static_cast<const float*>(v), ldv, cm, (int)D_out,
                                      static_cast<float*>(out), ldo, err);
    FSI_HIP_LAUNCH_CHECK("pattention down f32");
    return FSI_OK;
  }

  // bf16: 16-byte operand loads need K % 8 == 0 and aligned rows; V uses 8-byte loads.
  FSI_CHECK_ARG(K % 8 == 0 && ldx % 8 == 0 && ldk % 8 == 0, FSI_ERR_ALIGN,
                "pattention bf16: K, ldx, ldk must be multiples of 8");
  FSI_CHECK_ARG(((uintptr_t)x % 16 == 0) && ((uintptr_t)k_gate % 16 == 0) &&
                    (k_up == nullptr || (uintptr_t)k_up % 16 == 0) && ((uintptr_t)v % 2 == 0) &&
                    ((uintptr_t)out % 2 == 0),
                FSI_ERR_ALIGN, "pattention bf16: misaligned base pointer");
  const uint64_t lim = uint64_t(1) << 32;
  FSI_CHECK_ARG(uint64_t(M) * ldx * 2 < lim && uint64_t(N_p) * ldk * 2 < lim &&
                    uint64_t(v_transposed ? D_out : N_p) * ldv * 2 < lim,
                FSI_ERR_SHAPE, "pattention bf16: each tensor must be smaller than 4 GiB");
  const Plan p = make_plan_bf16(M, D_out, n_channels);
  FSI_CHECK_ARG(workspace && workspace_bytes >= p.total, FSI_ERR_WORKSPACE,
                "pattention: workspace %zu < required %zu", workspace_bytes, p.total);
  FSI_CHECK_ARG((uintptr_t)workspace % 256 == 0, FSI_ERR_ALIGN, "pattention: workspace must be 256-byte aligned");
  FSI_CHECK_ARG(uint64_t(M) * p.n_ch_pad * 2 < lim, FSI_ERR_SHAPE, "pattention bf16: intermediate larger than 4 GiB");

  bf16_t* h = reinterpret_cast<bf16_t*>(static_cast<char*>(workspace) + p.off_h);
  const int64_t ldh = p.n_ch_pad;
  const bf16_t* xb = static_cast<const bf16_t*>(x);
  const bf16_t* kgb = static_cast<const bf16_t*>(k_gate);
  const bf16_t* kub = static_cast<const bf16_t*>(k_up);

  // Decode (up to 64 tokens): split-K MFMA kernels with every operand loaded
  // straight into registers; falls through when its shape conditions do not hold.
  if (M <= 64 && v_transposed && cm.log2bn >= 5) {
    const int r = fsi_dec::run(xb, ldx, kgb, kub, ldk, static_cast<const bf16_t*>(v), ldv, active_blocks,
                               cm.n_blocks, cm.log2bn, N_p, (int)M, (int)K, n_channels, (int)D_out, activation,
                               rounding, static_cast<bf16_t*>(out), ldo, workspace, workspace_bytes, err, st);
    if (r < 0) {
      fsi_host::set_last_error("pattention: decode launch failed: %s", hipGetErrorString(hipGetLastError()));
      return FSI_ERR_HIP;
    }
    if (r == 0) return FSI_OK;
  }

  // Many tokens: tiled MFMA GEMMs (gathered gate/up with the SwiGLU fused in the
  // epilogue, then the down projection gathered along K).
  if (M >= GEMM_MIN_M && activation == FSI_ACT_SWIGLU && kub && block_n % 64 == 0 && N_p % block_n == 0 &&
      (active_blocks ? n_active : N_p / block_n) <= GEMM_MAX_BLOCKS &&
      v_transposed && ldv % 8 == 0 && (uintptr_t)v % 16 == 0 && ldo % 8 == 0 && (uintptr_t)out % 16 == 0) {
    const int n_act = active_blocks ? (int)n_active : (int)(N_p / block_n);
    if (fsi_gemm::gateup_swiglu(xb, ldx, kgb, kub, ldk, (int)N_p, active_blocks, n_act, (int)block_n, (int)M,
                                (int)K, rounding, h, ldh, err, st) != 0) {
      fsi_host::set_last_error("pattention: gate/up GEMM launch failed: %s", hipGetErrorString(hipGetLastError()));
      return FSI_ERR_HIP;
    }
    if (fsi_gemm::down_gather(h, ldh, static_cast<const bf16_t*>(v), ldv, (int)N_p, active_blocks, n_act,
                              (int)block_n, (int)M, (int)D_out, static_cast<bf16_t*>(out), ldo, err, st) != 0) {
      fsi_host::set_last_error("pattention: down GEMM launch failed: %s", hipGetErrorString(hipGetLastError()));
      return FSI_ERR_HIP;
    }
    return FSI_OK;
  }
  const dim3 g1((unsigned)p.n_groups, (unsigned)p.m_tiles);
  const bf16_t* kub2 = kub ? kub : kgb;
  switch (activation) {
    case FSI_ACT_SWIGLU: patt_skinny<MODE_GATEUP, ACT_SWIGLU, true, SKD><<<g1, SK_WAVES * 64, 0, st>>>(xb, ldx, (int)M, kgb, kub2, ldk, cm, (int)K, p.n_groups, 0, h, ldh, 0, rounding, err); break;
    case FSI_ACT_SILU: patt_skinny<MODE_GATEUP, ACT_SILU, false, SKD><<<g1, SK_WAVES * 64, 0, st>>>(xb, ldx, (int)M, kgb, kgb, ldk, cm, (int)K, p.n_groups, 0, h, ldh, 0, rounding, err); break;
    case FSI_ACT_GELU: patt_skinny<MODE_GATEUP, ACT_GELU, false, SKD><<<g1, SK_WAVES * 64, 0, st>>>(xb, ldx, (int)M, kgb, kgb, ldk, cm, (int)K, p.n_groups, 0, h, ldh, 0, rounding, err); break;
    case FSI_ACT_RELU: patt_skinny<MODE_GATEUP, ACT_RELU, false, SKD><<<g1, SK_WAVES * 64, 0, st>>>(xb, ldx, (int)M, kgb, kgb, ldk, cm, (int)K, p.n_groups, 0, h, ldh, 0, rounding, err); break;
    default: patt_skinny<MODE_GATEUP, ACT_RELU2, false, SKD><<<g1, SK_WAVES * 64, 0, st>>>(xb, ldx, (int)M, kgb, kgb, ldk, cm, (int)K, p.n_groups, 0, h, ldh, 0, rounding, err); break;
  }
  FSI_HIP_LAUNCH_CHECK("pattention gateup bf16");
  const bf16_t* vbp = static_cast<const bf16_t*>(v);
  if (v_transposed) {
    FSI_CHECK_ARG(cm.log2bn >= 3 && p.n_ch_pad / TC <= MAX_STAGES, FSI_ERR_SHAPE,
                  "pattention bf16: transposed V needs block_n >= 8 and at most %d active channels", MAX_STAGES * TC);
    const dim3 g2((unsigned)p.d_groups, (unsigned)p.m_tiles);
    patt_skinny<MODE_DOWNT, ACT_SWIGLU, false, SKD><<<g2, SK_WAVES * 64, 0, st>>>(
        h, ldh, (int)M, vbp, vbp, ldv, cm, (int)p.n_ch_pad, p.d_groups, (int)D_out, out, ldo, 0, rounding, err);
  } else {
    const dim3 g2((unsigned)p.d_groups, (unsigned)p.m_tiles);
    const bool table = cm.log2bn >= 3 && p.n_ch_pad / TC <= MAX_STAGES;
    if (table)
      patt_dec_down<false><<<g2, NW2 * 64, 0, st>>>(h, ldh, (int)M, vbp, ldv, cm, (int)p.n_ch_pad, (int)D_out,
                                                    p.d_groups, out, ldo, 0, err);
    else
      patt_dec_down<true><<<g2, NW2 * 64, 0, st>>>(h, ldh, (int)M, vbp, ldv, cm, (int)p.n_ch_pad, (int)D_out,
                                                   p.d_groups, out, ldo, 0, err);
  }
  FSI_HIP_LAUNCH_CHECK("pattention down bf16");
  return FSI_OK;
}

int fsi_swiglu(const void* g, const void* u, void* out, int64_t n, int dtype, int rounding, void* stream) {
  FSI_CHECK_ARG(dtype == FSI_DTYPE_BF16 || dtype == FSI_DTYPE_F32, FSI_ERR_DTYPE, "swiglu: dtype %d", dtype);
  FSI_CHECK_ARG(n >= 0, FSI_ERR_SHAPE, "swiglu: n < 0");
  if (n == 0) return FSI_OK;
  FSI_CHECK_ARG(g && u && out, FSI_ERR_INVALID_ARG, "swiglu: null pointer");
  FSI_CHECK_ARG(rounding == FSI_ROUND_EAGER || rounding == FSI_ROUND_FUSED, FSI_ERR_INVALID_ARG,
                "swiglu: rounding %d", rounding);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int64_t blocks64 = (n + 255) / 256;
  const unsigned blocks = (unsigned)(blocks64 > 16384 ? 16384 : blocks64);
  if (dtype == FSI_DTYPE_BF16)
    swiglu_bf16<<<blocks, 256, 0, st>>>(static_cast<const bf16_t*>(g), static_cast<const bf16_t*>(u),
                                        static_cast<bf16_t*>(out), n, rounding);
  else
    swiglu_f32<<<blocks, 256, 0, st>>>(static_cast<const float*>(g), static_cast<const float*>(u),
                                       static_cast<float*>(out), n);
  FSI_HIP_LAUNCH_CHECK("swiglu");
  return FSI_OK;
}

int fsi_swiglu_bwd(const void* dout, const void* g, const void* u, void* dg, void* du, int64_t n, int dtype,
                   void* stream) {
  FSI_CHECK_ARG(dtype == FSI_DTYPE_BF16 || dtype == FSI_DTYPE_F32, FSI_ERR_DTYPE, "swiglu_bwd: dtype %d", dtype);
  FSI_CHECK_ARG(n >= 0, FSI_ERR_SHAPE, "swiglu_bwd: n < 0");
  if (n == 0) return FSI_OK;
  FSI_CHECK_ARG(dout && g && u && dg && du, FSI_ERR_INVALID_ARG, "swiglu_bwd: null pointer");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int64_t blocks64 = (n + 255) / 256;
  const unsigned blocks = (unsigned)(blocks64 > 16384 ? 16384 : blocks64);
  if (dtype == FSI_DTYPE_BF16)
    swiglu_bwd_kernel<bf16_t><<<blocks, 256, 0, st>>>(
        static_cast<const bf16_t*>(dout), static_cast<const bf16_t*>(g), static_cast<const bf16_t*>(u),
        static_cast<bf16_t*>(dg), static_cast<bf16_t*>(du), n);
  else
    swiglu_bwd_kernel<float><<<blocks, 256, 0, st>>>(static_cast<const float*>(dout), static_cast<const float*>(g),
                                                     static_cast<const float*>(u), static_cast<float*>(dg),
                                                     static_cast<float*>(du), n);
  FSI_HIP_LAUNCH_CHECK("swiglu_bwd");
  return FSI_OK;
}

}  // extern "C"
