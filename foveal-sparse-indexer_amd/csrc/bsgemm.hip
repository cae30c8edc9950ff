// Gather-driven block-sparse bf16 GEMM engine for MI355X (gfx950).
//
// One workgroup (4 waves) computes a 128 x 128 tile of C[M, N] = A[M, K] B[N, K]^T
// (both operands K-contiguous, the F.linear layout) with fp32 accumulation on
// v_mfma_f32_16x16x32_bf16.  What makes it block-sparse is how a tile finds its
// operands:
//   * N is gathered in 32-column sub-blocks: each of the tile's four
//     sub-blocks has its own B pointer and row base and its own C column base
//     (active column blocks of BlockSparseLinear, gate/up rows of the active
//     Pattention blocks);
//   * K advances in 64-wide steps, each with its own A and B column offset
//     (dense K, or K gathered by active blocks for the Pattention down
//     projection).  2-D tile-sparse products run on csrc/tile_gemm.hip.
// Per K-step the workgroup stages A and B (16 KiB each) through a double-
// buffered, XOR-swizzled LDS tile: the global loads are 1 KiB contiguous per
// wave instruction and the MFMA fragment reads are free of bank conflicts.
// Wave (wm, wn) owns rows 64 wm .. +64 and tile columns {32 wn .. +32} of both
// 64-column halves, so a gate column and its up column land in the same lane.
#include <algorithm>

#include <type_traits>

#include "fsi_common.h"

using namespace fsi;

namespace fsi_bs_generic {  // csrc/bsgemm_generic.hip: fp32 and the bf16 tilings below do not take
int column_gemm(const void* x, int64_t ldx, const void* w, int64_t ldw, const void* bias,
                const int32_t* active_blocks, int64_t n_active, int64_t block_size, int64_t M, int64_t N, int64_t K,
                int dtype, void* out, int64_t ldo, uint8_t* mask_ws, int* err, hipStream_t st);
}  // namespace fsi_bs_generic

namespace {

constexpr int TM = 128, TN = 128, TK = 64;

// Global-load lead of the software pipeline in K-steps (1: loads for step s + 1
// issued at the start of step s, two workgroups per CU; 2: two register stages,
// one workgroup per CU with the full register file).
#ifndef FSI_GEMM_DEPTH
#define FSI_GEMM_DEPTH 1
#endif
constexpr int GEMM_DEPTH = FSI_GEMM_DEPTH;
constexpr int GEMM_WG_PER_CU = GEMM_DEPTH == 1 ? 2 : 1;
constexpr int GT = 256;  // threads per workgroup
constexpr int SUB = 32;  // N gather granularity
// K-gathered problems keep the column offset of every active K block in LDS
// (a per-step global lookup would make each step wait for all loads in flight).
constexpr int KTAB_MAX = 2048;

enum NMode { N_DIRECT = 0, N_GATHER = 1, N_DUAL = 2 };
enum KMode { K_DENSE = 0, K_GATHER_B = 1 };
enum Epi { EPI_STORE = 0, EPI_SWIGLU = 1, EPI_ENERGY = 2 };

struct GemmArgs {
  const bf16_t* A;  // [M, lda]
  const bf16_t* B0; // [rows, ldb]
  const bf16_t* B1; // second B (up projection) for N_DUAL
  const bf16_t* bias;
  bf16_t* C;
  float* E;         // EPI_ENERGY: [M, N / 32] per-row sums of |act| over 32-channel groups (row stride ldc)
  int64_t lda, ldb, ldc;
  int M, N, K;                 // N: logical columns of the gathered problem, K: reduction length
  const int32_t* blocks;       // N_GATHER / N_DUAL: active block ids; K_GATHER_B: active blocks along K
  int n_blocks;                // entries in `blocks`
  int block;                   // block size in columns (multiple of 32)
  int n_rows_total;            // rows of B (bounds for gathered ids)
  int scatter_c;               // N_GATHER: write C at the gathered column (1) or compactly (0)
  int m_tiles, n_tiles;        // dense grid (non-list modes)
  int act, rounding;           // EPI_SWIGLU
  int* err;
  // Packed B (the decode weight layout: 16 x 32 MFMA operand tiles of 1 KiB in lane
  // order).  N_DUAL / K_DENSE: tile (ct, s) of 16 rows at (ct pk_S + s) KiB of Bp0
  // (gate) / Bp1 (up).  N_DIRECT / K_GATHER_B: tile (b, dt, cl) of block b, 16 output
  // dims dt, 32-channel slice cl at ((b pk_DT + dt) pk_CB + cl) KiB of Bp0.
  const bf16_t* Bp0;
  const bf16_t* Bp1;
  int pk_S, pk_DT, pk_CB;
};

__device__ __forceinline__ int swz(int row, int chunk) { return chunk ^ ((row >> 1) & 7); }

// Sum over the 16 lanes that hold one row of a 16 x 16 MFMA result (lanes 16 q .. 16 q + 15).
__device__ __forceinline__ float sum16(float v) {
  v += __shfl_xor(v, 8, 16);
  v += __shfl_xor(v, 4, 16);
  v += __shfl_xor(v, 2, 16);
  v += __shfl_xor(v, 1, 16);
  return v;
}

// |act(g, u)| of one gate/up accumulator pair, rounded as the stored activation
// would be unless the rounding mode is fp32 (EPI_ENERGY).
__device__ __forceinline__ float energy_term(float gv, float uv, int rounding) {
  const float h = pattention_act<ACT_SWIGLU>(gv, uv, rounding);
  return fabsf(rounding == FSI_ROUND_FP32 ? h : round_bf16(h));
}

// Two fp32 values to a packed bf16 pair with v_cvt_pk_bf16_f32 (round to nearest even).
__device__ __forceinline__ uint32_t hw_pack_bf16x2(float a, float b) {
  typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2_t;
  const bf16x2_t v = {static_cast<__bf16>(a), static_cast<__bf16>(b)};
  return __builtin_bit_cast(uint32_t, v);
}

// SwiGLU of the GEMM epilogue with the rounding mode R fixed at compile time:
// silu from the hardware exp2 and reciprocal (about 1 ulp each in fp32; the result
// is rounded to bf16).  The library expf / IEEE divide expand to ~25 instructions
// per element, and the epilogue runs once per tile from a cold instruction cache.
template <int R>
__device__ __forceinline__ float swiglu_epi(float gv, float uv) {
  if (R != FSI_ROUND_FP32) {
    gv = round_bf16(gv);
    uv = round_bf16(uv);
  }
  float s = gv * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-1.4426950408889634f * gv));
  if (R == FSI_ROUND_EAGER) s = round_bf16(s);
  return s * uv;
}

// Epilogue fast path: four outputs known to be inside the matrix, 8-byte aligned.
__device__ __forceinline__ void store4_fast(bf16_t* C, int64_t off, const float (&v)[4]) {
  uint2 w;
  w.x = hw_pack_bf16x2(v[0], v[1]);
  w.y = hw_pack_bf16x2(v[2], v[3]);
  *reinterpret_cast<uint2*>(C + off) = w;
}

// Four consecutive bf16 outputs C[off .. off + 3] (n of them inside the matrix): one
// 8-byte store when all four exist and `vec` (8-byte aligned rows) holds.
__device__ __forceinline__ void store4_bf16(bf16_t* C, int64_t off, const float (&v)[4], int n, bool vec) {
  if (vec && n >= 4) {
    uint2 w;
    w.x = pack_bf16x2(v[0], v[1]);
    w.y = pack_bf16x2(v[2], v[3]);
    *reinterpret_cast<uint2*>(C + off) = w;
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (j < n) C[off + j] = f32_to_bf16(v[j]);
  }
}

// ktab[i] = first B column of active K block i, or -1 when its id is out of range.
__device__ __forceinline__ void fill_ktab(const GemmArgs& g, int32_t* ktab, int nthreads) {
  for (int i = threadIdx.x; i < g.n_blocks; i += nthreads) {
    const int blk = g.blocks ? g.blocks[i] : i;
    ktab[i] = (blk < 0 || static_cast<int64_t>(blk + 1) * g.block > g.n_rows_total) ? -1 : blk * g.block;
  }
}

template <int NM, int KM, int EPI>
__global__ __launch_bounds__(GT, GEMM_WG_PER_CU) void bsgemm_kernel(GemmArgs g) {
  __shared__ __attribute__((aligned(16))) bf16_t lds[2][2][TM * TK];  // [buf][A/B][row * 64 + k]
  __shared__ int32_t ktab[KM == K_GATHER_B ? KTAB_MAX : 1];
  const int tid = threadIdx.x;
  if (KM == K_GATHER_B) {
    fill_ktab(g, ktab, GT);
    __syncthreads();
  }
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  // ---- which tile ----------------------------------------------------------
  // consecutive workgroups walk down M for one N tile: the B tile stays hot in L2
  const int mt = blockIdx.x % g.m_tiles;
  const int nt = blockIdx.x / g.m_tiles;
  const int kcount = KM == K_GATHER_B ? g.n_blocks * (g.block / TK) : (g.K + TK - 1) / TK;
  const int m0 = mt * TM;

  // ---- per 32-column sub-block: B row base (and pointer) and C column base --
  // (computed by every thread for all four sub-blocks; cheap scalar work)
  int64_t brow[4];
  int ccol[4];
  bool bval[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    if (NM == N_DUAL) {
      // tile nt covers channel block half: 64 channels = [gate 64 | up 64]
      const int ch = nt * 64 + (s & 1) * SUB;  // compact channel index
      const int bi = ch / g.block;
      const int blk = bi < g.n_blocks ? (g.blocks ? g.blocks[bi] : bi) : -1;
      const int64_t row = static_cast<int64_t>(blk) * g.block + ch % g.block;
      bval[s] = blk >= 0 && row + SUB <= g.n_rows_total;
      brow[s] = bval[s] ? row : 0;
      ccol[s] = ch;
    } else if (NM == N_GATHER) {
      const int col = nt * TN + s * SUB;  // compact column
      const int bi = col / g.block;
      const int blk = bi < g.n_blocks ? (g.blocks ? g.blocks[bi] : bi) : -1;
      const int64_t row = static_cast<int64_t>(blk) * g.block + col % g.block;
      bval[s] = blk >= 0 && row + SUB <= g.n_rows_total;
      brow[s] = bval[s] ? row : 0;
      ccol[s] = g.scatter_c ? static_cast<int>(row) : col;
    } else {
      const int col = nt * TN + s * SUB;
      bval[s] = col < g.N;
      brow[s] = bval[s] ? col : 0;
      ccol[s] = col;
    }
    if (NM != N_DIRECT && !bval[s] && g.err && ((NM == N_DUAL ? nt * 64 + (s & 1) * SUB : nt * TN + s * SUB) < g.N))
      set_error(g.err, FSI_ERR_INDEX_RANGE);
  }

  // ---- global -> register staging: thread loads 4 A chunks and 4 B chunks ----
  // chunk q = tid + 256 i: row q / 8, k chunk q % 8 (16 B)
  const int lrow0 = tid >> 3, lchunk = tid & 7;
  // K_GATHER_B: kb_rows = columns of B (bounds for the gathered blocks)
  auto k_cols = [&](int step, int64_t& a_k, int64_t& b_k) -> bool {
    if (KM == K_GATHER_B) {
      const int per = g.block / TK;
      const int col = ktab[step / per];
      a_k = static_cast<int64_t>(step) * TK;
      if (col < 0) {
        b_k = 0;
        return false;
      }
      b_k = col + (step % per) * TK;
    } else {
      a_k = b_k = static_cast<int64_t>(step) * TK;
    }
    return true;
  };
  auto load_step = [&](int step, u32x4_t (&ra)[4], u32x4_t (&rb)[4]) {
    int64_t a_k, b_k;
    const bool kval = k_cols(step, a_k, b_k);
    if (!kval && g.err) set_error(g.err, FSI_ERR_INDEX_RANGE);
    const int kk = static_cast<int>((KM == K_DENSE ? a_k : 0) + lchunk * 8);  // element k within the problem
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = lrow0 + 32 * i;
      const int m = m0 + r;
      const bool kin = KM == K_DENSE ? (kk < g.K) : true;
      if (m < g.M && kin) ra[i] = *reinterpret_cast<const u32x4_t*>(g.A + m * g.lda + a_k + lchunk * 8);
      else ra[i] = u32x4_t{0u, 0u, 0u, 0u};
      const int s = r / SUB;  // sub-block of this tile row
      const bf16_t* bp = (NM == N_DUAL && s >= 2) ? g.B1 : g.B0;
      const int64_t row = brow[s] + (r % SUB);
      const bool rin = NM != N_DIRECT || row < g.N;  // direct N: rows past N (N % 32 != 0) are not read
      if (bval[s] && rin && kin && kval)
        rb[i] = *reinterpret_cast<const u32x4_t*>(bp + row * g.ldb + b_k + lchunk * 8);
      else rb[i] = u32x4_t{0u, 0u, 0u, 0u};
    }
  };
  auto store_step = [&](int buf, const u32x4_t (&ra)[4], const u32x4_t (&rb)[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = lrow0 + 32 * i;
      const int off = r * TK + swz(r, lchunk) * 8;
      *reinterpret_cast<u32x4_t*>(&lds[buf][0][off]) = ra[i];
      *reinterpret_cast<u32x4_t*>(&lds[buf][1][off]) = rb[i];
    }
  };

  f32x4_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // wave's B fragment rows: tile columns {32 wn + 16 f} (f = 0, 1) and {64 + 32 wn + 16 (f - 2)}
  const int frow = lane & 15, fchunk = lane >> 4;
  // Software pipeline: LDS holds steps s and s + 1 (double buffer); with depth 2
  // registers hold step s + 2, issued two compute steps before it is written to
  // LDS, so the global-load latency is covered by two steps of MFMA work.
  auto compute = [&](int buf) {
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      u32x4_t fa[4], fb[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 64 * wm + 16 * i + frow;
        fa[i] = *reinterpret_cast<const u32x4_t*>(&lds[buf][0][r * TK + swz(r, ks * 4 + fchunk) * 8]);
      }
#pragma unroll
      for (int f = 0; f < 4; ++f) {
        const int c = (f < 2 ? 32 * wn + 16 * f : 64 + 32 * wn + 16 * (f - 2)) + frow;
        fb[f] = *reinterpret_cast<const u32x4_t*>(&lds[buf][1][c * TK + swz(c, ks * 4 + fchunk) * 8]);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int f = 0; f < 4; ++f) acc[i][f] = mfma16x16x32(fb[f], fa[i], acc[i][f]);  // C^T fragment
    }
  };
  auto clampk = [&](int st) { return st < kcount ? st : (kcount > 0 ? kcount - 1 : 0); };
  if (GEMM_DEPTH == 1) {
    u32x4_t ra[4], rb[4];
    if (kcount > 0) {
      load_step(0, ra, rb);
      store_step(0, ra, rb);
    }
    __syncthreads();
    for (int step = 0; step < kcount; ++step) {
      load_step(clampk(step + 1), ra, rb);  // straight-line prefetch; the last one is redundant
      compute(step & 1);
      if (step + 1 < kcount) store_step((step & 1) ^ 1, ra, rb);
      __syncthreads();
    }
  } else {
    u32x4_t ra0[4], rb0[4], ra1[4], rb1[4];
    if (kcount > 0) {
      load_step(0, ra0, rb0);
      store_step(0, ra0, rb0);
      load_step(clampk(1), ra1, rb1);
    }
    __syncthreads();
    // one iteration = two K-steps: regs1 hold step + 1, regs0 receive step + 2, and so on
    for (int step = 0; step < kcount; step += 2) {
      load_step(clampk(step + 2), ra0, rb0);  // redundant past the end (straight-line code)
      compute(0);
      if (step + 1 < kcount) store_step(1, ra1, rb1);
      __syncthreads();
      if (step + 1 >= kcount) break;
      load_step(clampk(step + 3), ra1, rb1);
      compute(1);
      if (step + 2 < kcount) store_step(0, ra0, rb0);
      __syncthreads();
    }
  }

  // ---- epilogue: the fragments hold C^T, so lane (q = lane / 16, r = lane % 16) of
  // fragment (i, f) holds row 16 i + r of the wave's rows and the four consecutive
  // columns 4 q .. 4 q + 3 of the fragment: one 8-byte store per fragment; interior
  // tiles take a branch-free path (see the 256 x 256 kernels)
  const int crow = m0 + 64 * wm + frow;
  const int cq = 4 * fchunk;
  const bool vec = (reinterpret_cast<uintptr_t>(g.C) & 7) == 0 && (g.ldc & 3) == 0;
  const bool rows_in = m0 + TM <= g.M;
  if (EPI == EPI_SWIGLU) {
    // gate fragments f = 0, 1 pair with up fragments f = 2, 3 (same channel); both
    // gate fragments of wave wn lie in sub-block wn
    const bool live = g.act == ACT_SWIGLU && bval[wn] && bval[2 + wn];
    const int ch0 = ccol[0] + 32 * wn + cq;
    auto interior = [&](auto rnd) {
      constexpr int R = decltype(rnd)::value;
#pragma unroll
      for (int f = 0; f < 2; ++f)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float h[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) h[j] = swiglu_epi<R>(acc[i][f][j], acc[i][f + 2][j]);
          store4_fast(g.C, static_cast<int64_t>(crow + 16 * i) * g.ldc + ch0 + 16 * f, h);
        }
    };
    if (vec && rows_in && live && ccol[0] + 64 <= g.N) {
      if (g.rounding == FSI_ROUND_FP32) interior(std::integral_constant<int, FSI_ROUND_FP32>{});
      else if (g.rounding == FSI_ROUND_FUSED) interior(std::integral_constant<int, FSI_ROUND_FUSED>{});
      else interior(std::integral_constant<int, FSI_ROUND_EAGER>{});
    } else {
#pragma unroll
      for (int f = 0; f < 2; ++f) {
        const int ch = ch0 + 16 * f;
        if (ch >= g.N) continue;
        const int n = g.N - ch;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int m = crow + 16 * i;
          if (m >= g.M) continue;
          float h[4];
#pragma unroll
          for (int j = 0; j < 4; ++j)
            h[j] = live ? pattention_act<ACT_SWIGLU>(acc[i][f][j], acc[i][f + 2][j], g.rounding) : 0.f;
          store4_bf16(g.C, static_cast<int64_t>(m) * g.ldc + ch, h, n, vec);
        }
      }
    }
  } else if (EPI == EPI_ENERGY) {
    // wave wn holds the tile's channels 32 wn .. 32 wn + 31 (gate fragments f = 0, 1):
    // each lane sums its 8 channels of row 16 i + r, then the four lanes r, r + 16,
    // r + 32, r + 48 of the row are added
    const int grp_ch = ccol[0] + 32 * wn;
    if (grp_ch < g.N) {
      const bool live = bval[wn] && bval[2 + wn];
      auto sums = [&](auto rnd) {
        constexpr int R = decltype(rnd)::value;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float e = 0.f;
          if (live) {
#pragma unroll
            for (int j = 0; j < 4; ++j)
              e += energy_term(acc[i][0][j], acc[i][2][j], R) + energy_term(acc[i][1][j], acc[i][3][j], R);
          }
          e = sum_rows4(e);
          const int m = crow + 16 * i;
          if (fchunk == 0 && m < g.M) g.E[static_cast<int64_t>(m) * g.ldc + grp_ch / SUB] = e;
        }
      };
      if (g.rounding == FSI_ROUND_FP32) sums(std::integral_constant<int, FSI_ROUND_FP32>{});
      else if (g.rounding == FSI_ROUND_FUSED) sums(std::integral_constant<int, FSI_ROUND_FUSED>{});
      else sums(std::integral_constant<int, FSI_ROUND_EAGER>{});
    }
  } else {
    auto tcol = [&](int f) { return f < 2 ? 32 * wn + 16 * f : 64 + 32 * wn + 16 * (f - 2); };
    bool all = vec && rows_in;
#pragma unroll
    for (int sb = 0; sb < 4; ++sb) all = all && (NM == N_DIRECT ? ccol[sb] + SUB <= g.N : bval[sb]);
    if (all) {
#pragma unroll
      for (int f = 0; f < 4; ++f) {
        const int tc = tcol(f);
        const int s = tc / SUB;
        const int col = ccol[s] + (tc % SUB) + cq;
        float bv[4] = {0.f, 0.f, 0.f, 0.f};
        if (g.bias) {
#pragma unroll
          for (int j = 0; j < 4; ++j)
            bv[j] = bf16_to_f32(g.bias[NM == N_GATHER ? brow[s] + (tc % SUB) + cq + j : col + j]);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float o[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) o[j] = acc[i][f][j] + bv[j];
          store4_fast(g.C, static_cast<int64_t>(crow + 16 * i) * g.ldc + col, o);
        }
      }
    } else {
#pragma unroll
      for (int f = 0; f < 4; ++f) {
        const int tc = tcol(f);
        const int s = tc / SUB;
        if (NM != N_DIRECT && !bval[s]) continue;
        const int col = ccol[s] + (tc % SUB) + cq;
        if (NM == N_DIRECT && col >= g.N) continue;
        const int n = NM == N_DIRECT ? g.N - col : 4;
        float bv[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
          bv[j] = g.bias && j < n ? bf16_to_f32(g.bias[NM == N_GATHER ? brow[s] + (tc % SUB) + cq + j : col + j]) : 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int m = crow + 16 * i;
          if (m >= g.M) continue;
          float o[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) o[j] = acc[i][f][j] + bv[j];
          store4_bf16(g.C, static_cast<int64_t>(m) * g.ldc + col, o, n, vec);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Large-tile variant for many-row problems (prefill): 256 x 256 tile, 4 waves
// of 128 x 128 (one wave per SIMD, accumulators in AGPRs), K in 32-wide
// steps.  A wave reads 16 fragments per 64 MFMAs from LDS (vs. 8 per 16 in the
// 128 x 128 kernel), and a tile re-reads A and B half as often from L2.
// LDS: 2 stages x (A + B) x 16 KiB.
// Workgroups with consecutive logical ids share an XCD (and its L2); a
// logical id walks down M first, so the B tile of an XCD's group stays hot.
// ---------------------------------------------------------------------------
#ifndef FSI_GEMM_BIG_WAVES
#define FSI_GEMM_BIG_WAVES 8
#endif
#ifndef FSI_GEMM_BIG_PIPE
#define FSI_GEMM_BIG_PIPE 1
#endif
#ifndef FSI_GEMM_BIG_BK
#define FSI_GEMM_BIG_BK 64
#endif
constexpr int BM = 256, BN = 256, BK = FSI_GEMM_BIG_BK;
constexpr int BCPR = BK / 8;                 // 16-byte chunks per LDS row
constexpr int BWN = FSI_GEMM_BIG_WAVES / 2;  // waves along N (2 along M)
constexpr int BT = 64 * 2 * BWN;             // threads per workgroup
constexpr int BHW = 128 / BWN;               // columns of each tile half per wave
constexpr int BNF = 2 * BHW / 16;            // B fragments per wave
constexpr int BLPT = BM * BCPR / BT;        // 16-byte A (and B) chunks per thread and step

// Conflict-free fragment reads: 32-wide rows XOR the chunk with row bits 2-3,
// 64-wide rows with row bits 1-3.
__device__ __forceinline__ int swzb(int row, int chunk) {
  return BCPR == 4 ? chunk ^ ((row >> 2) & 3) : chunk ^ ((row >> 1) & 7);
}

__device__ __forceinline__ int xcd_group_id(int w, int n) {
  if ((n & 7) != 0) return w;
  return (w & 7) * (n >> 3) + (w >> 3);
}

// Logical id -> (m tile, n tile) in groups of GEMM_GROUP_M m tiles: the workgroups an
// XCD runs at once cover a few m tiles x several n tiles, so both operands' tiles
// are shared in its L2 (a plain walk down M shares only the B tile).
#ifndef FSI_GEMM_GROUP_M
#define FSI_GEMM_GROUP_M 4
#endif
__device__ __forceinline__ void grouped_tile(int lid, int m_tiles, int n_tiles, int& mt, int& nt) {
  constexpr int G = FSI_GEMM_GROUP_M;
  if (G <= 1 || m_tiles % G != 0) {
    mt = lid % m_tiles;
    nt = lid / m_tiles;
    return;
  }
  const int group = lid / (G * n_tiles), within = lid % (G * n_tiles);
  mt = group * G + within % G;
  nt = within / G;
}

template <int NM, int KM, int EPI>
__global__ __launch_bounds__(BT, 1) void bsgemm_big_kernel(GemmArgs g) {
  __shared__ __attribute__((aligned(16))) bf16_t lds[2][2][BM * BK];  // [stage][A/B][row * 32 + k]
  __shared__ int32_t ktab[KM == K_GATHER_B ? KTAB_MAX : 1];
  const int tid = threadIdx.x;
  if (KM == K_GATHER_B) {
    fill_ktab(g, ktab, BT);
    __syncthreads();
  }
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave / BWN, wn = wave % BWN;

  const int lid = xcd_group_id(blockIdx.x, gridDim.x);
  int mt, nt;
  grouped_tile(lid, g.m_tiles, g.n_tiles, mt, nt);
  const int kcount = KM == K_GATHER_B ? g.n_blocks * (g.block / BK) : (g.K + BK - 1) / BK;
  const int m0 = mt * BM;

  // ---- per 32-column sub-block: B row base and C column base ----------------
  int64_t brow[8];
  int ccol[8];
  bool bval[8];
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    if (NM == N_DUAL) {
      // tile nt covers 128 channels: tile columns [gate 128 | up 128]
      const int ch = nt * 128 + (s & 3) * SUB;
      const int bi = ch / g.block;
      const int blk = bi < g.n_blocks ? (g.blocks ? g.blocks[bi] : bi) : -1;
      const int64_t row = static_cast<int64_t>(blk) * g.block + ch % g.block;
      bval[s] = blk >= 0 && row + SUB <= g.n_rows_total;
      brow[s] = bval[s] ? row : 0;
      ccol[s] = ch;
    } else if (NM == N_GATHER) {
      const int col = nt * BN + s * SUB;
      const int bi = col / g.block;
      const int blk = bi < g.n_blocks ? (g.blocks ? g.blocks[bi] : bi) : -1;
      const int64_t row = static_cast<int64_t>(blk) * g.block + col % g.block;
      bval[s] = blk >= 0 && row + SUB <= g.n_rows_total;
      brow[s] = bval[s] ? row : 0;
      ccol[s] = g.scatter_c ? static_cast<int>(row) : col;
    } else {
      const int col = nt * BN + s * SUB;
      bval[s] = col < g.N;
      brow[s] = bval[s] ? col : 0;
      ccol[s] = col;
    }
    if (NM != N_DIRECT && !bval[s] && g.err && ((NM == N_DUAL ? nt * 128 + (s & 3) * SUB : nt * BN + s * SUB) < g.N))
      set_error(g.err, FSI_ERR_INDEX_RANGE);
  }

  // ---- global -> register staging: chunk q = tid + BT i: row q / BCPR, 16-byte chunk q % BCPR
  const int lrow0 = tid / BCPR, lchunk = tid % BCPR;
  auto k_cols = [&](int step, int64_t& a_k, int64_t& b_k) -> bool {
    if (KM == K_GATHER_B) {
      const int per = g.block / BK;
      const int col = ktab[step / per];
      a_k = static_cast<int64_t>(step) * BK;
      if (col < 0) {
        b_k = 0;
        return false;
      }
      b_k = col + (step % per) * BK;
    } else {
      a_k = b_k = static_cast<int64_t>(step) * BK;
    }
    return true;
  };
  auto load_step = [&](int step, u32x4_t (&ra)[BLPT], u32x4_t (&rb)[BLPT]) {
    int64_t a_k, b_k;
    const bool kval = k_cols(step, a_k, b_k);
    if (!kval && g.err) set_error(g.err, FSI_ERR_INDEX_RANGE);
    const int kk = static_cast<int>((KM == K_DENSE ? a_k : 0) + lchunk * 8);
    const bool kin = KM == K_DENSE ? (kk < g.K) : true;
#pragma unroll
    for (int i = 0; i < BLPT; ++i) {
      const int r = lrow0 + (BT / BCPR) * i;
      const int m = m0 + r;
      if (m < g.M && kin) ra[i] = *reinterpret_cast<const u32x4_t*>(g.A + static_cast<int64_t>(m) * g.lda + a_k + lchunk * 8);
      else ra[i] = u32x4_t{0u, 0u, 0u, 0u};
      const int s = r / SUB;
      const bf16_t* bp = (NM == N_DUAL && s >= 4) ? g.B1 : g.B0;
      const int64_t row = brow[s] + (r % SUB);
      const bool rin = NM != N_DIRECT || row < g.N;
      if (bval[s] && rin && kin && kval)
        rb[i] = *reinterpret_cast<const u32x4_t*>(bp + row * g.ldb + b_k + lchunk * 8);
      else rb[i] = u32x4_t{0u, 0u, 0u, 0u};
    }
  };
  auto store_step = [&](int buf, const u32x4_t (&ra)[BLPT], const u32x4_t (&rb)[BLPT]) {
#pragma unroll
    for (int i = 0; i < BLPT; ++i) {
      const int r = lrow0 + (BT / BCPR) * i;
      const int off = r * BK + swzb(r, lchunk) * 8;
      *reinterpret_cast<u32x4_t*>(&lds[buf][0][off]) = ra[i];
      *reinterpret_cast<u32x4_t*>(&lds[buf][1][off]) = rb[i];
    }
  };

  f32x4_t acc[8][BNF];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < BNF; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // wave fragments: A rows 128 wm + 16 i; B tile columns {BHW wn + 16 f} (f < BNF / 2)
  // and {128 + BHW wn + 16 (f - BNF / 2)}: a gate column and its up column share a lane
  const int frow = lane & 15, fchunk = lane >> 4;
  auto bcol = [&](int f) { return f < BNF / 2 ? BHW * wn + 16 * f : 128 + BHW * wn + 16 * (f - BNF / 2); };
  auto compute = [&](int buf) {
#pragma unroll
    for (int ks = 0; ks < BK / 32; ++ks) {
      u32x4_t fa[8], fb[BNF];
#pragma unroll
      for (int f = 0; f < BNF; ++f) {
        const int c = bcol(f) + frow;
        fb[f] = *reinterpret_cast<const u32x4_t*>(&lds[buf][1][c * BK + swzb(c, 4 * ks + fchunk) * 8]);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int r = 128 * wm + 16 * i + frow;
        fa[i] = *reinterpret_cast<const u32x4_t*>(&lds[buf][0][r * BK + swzb(r, 4 * ks + fchunk) * 8]);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int f = 0; f < BNF; ++f) acc[i][f] = mfma16x16x32(fb[f], fa[i], acc[i][f]);  // C^T fragment
    }
  };

#if FSI_GEMM_BIG_PIPE == 2
  // Loads run three K-steps ahead: at iteration s the registers of step s + 1
  // go to the free LDS stage, step s + 3 is issued into them, then step s is
  // computed.  A load has two steps of MFMA work to arrive.
  u32x4_t ra0[BLPT], rb0[BLPT], ra1[BLPT], rb1[BLPT];
  if (kcount > 0) {
    load_step(0, ra0, rb0);
    store_step(0, ra0, rb0);
  }
  if (kcount > 1) load_step(1, ra1, rb1);
  if (kcount > 2) load_step(2, ra0, rb0);
  __syncthreads();
  int step = 0;
  for (; step + 1 < kcount; step += 2) {
    store_step(1, ra1, rb1);
    if (step + 3 < kcount) load_step(step + 3, ra1, rb1);
    __builtin_amdgcn_sched_barrier(0);
    compute(0);
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    if (step + 2 < kcount) store_step(0, ra0, rb0);
    if (step + 4 < kcount) load_step(step + 4, ra0, rb0);
    __builtin_amdgcn_sched_barrier(0);
    compute(1);
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
  }
  if (step < kcount) compute(0);  // odd step count: the last step sits in stage 0
#else
  // loads for step s + 1 are issued before step s is computed and written to
  // the other LDS stage after it
  u32x4_t ra0[BLPT], rb0[BLPT];
  if (kcount > 0) {
    load_step(0, ra0, rb0);
    store_step(0, ra0, rb0);
  }
  __syncthreads();
  for (int step = 0; step < kcount; ++step) {
    if (step + 1 < kcount) load_step(step + 1, ra0, rb0);
    compute(step & 1);
    if (step + 1 < kcount) store_step((step & 1) ^ 1, ra0, rb0);
    __syncthreads();
  }
#endif

  // ---- epilogue: the fragments hold C^T, so lane (q = lane / 16, r = lane % 16) of
  // fragment (i, f) holds row 16 i + r of the wave's rows and the four consecutive
  // columns 4 q .. 4 q + 3 of the fragment: one 8-byte store per fragment
  const int crow = m0 + 128 * wm + frow;
  const int cq = 4 * fchunk;
  const bool vec = (reinterpret_cast<uintptr_t>(g.C) & 7) == 0 && (g.ldc & 3) == 0;
  if (EPI == EPI_SWIGLU) {
#pragma unroll
    for (int f = 0; f < BNF / 2; ++f) {
      const int ch = ccol[0] + BHW * wn + 16 * f + cq;  // ccol[0] = first channel of the tile
      if (ch >= g.N) continue;
      const int n = g.N - ch;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int m = crow + 16 * i;
        if (m >= g.M) continue;
        float h[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) h[j] = pattention_act<ACT_SWIGLU>(acc[i][f][j], acc[i][f + BNF / 2][j], g.rounding);
        store4_bf16(g.C, static_cast<int64_t>(m) * g.ldc + ch, h, n, vec);
      }
    }
  } else {
    bool all = vec && m0 + BM <= g.M;
#pragma unroll
    for (int sb = 0; sb < 8; ++sb) all = all && (NM == N_DIRECT ? ccol[sb] + SUB <= g.N : bval[sb]);
    if (all) {  // interior tile: no per-element checks (the epilogue's code size is its cost)
#pragma unroll
      for (int f = 0; f < BNF; ++f) {
        const int tc = bcol(f);
        const int s = tc / SUB;
        const int col = ccol[s] + (tc % SUB) + cq;
        float bv[4] = {0.f, 0.f, 0.f, 0.f};
        if (g.bias) {
#pragma unroll
          for (int j = 0; j < 4; ++j)
            bv[j] = bf16_to_f32(g.bias[NM == N_GATHER ? brow[s] + (tc % SUB) + cq + j : col + j]);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          float o[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) o[j] = acc[i][f][j] + bv[j];
          store4_fast(g.C, static_cast<int64_t>(crow + 16 * i) * g.ldc + col, o);
        }
      }
      return;
    }
#pragma unroll
    for (int f = 0; f < BNF; ++f) {
      const int tc = bcol(f);
      const int s = tc / SUB;
      if (NM != N_DIRECT && !bval[s]) continue;
      const int col = ccol[s] + (tc % SUB) + cq;
      if (NM == N_DIRECT && col >= g.N) continue;
      const int n = NM == N_DIRECT ? g.N - col : 4;
      float bv[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        bv[j] = g.bias && j < n ? bf16_to_f32(g.bias[NM == N_GATHER ? brow[s] + (tc % SUB) + cq + j : col + j]) : 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int m = crow + 16 * i;
        if (m >= g.M) continue;
        float o[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] = acc[i][f][j] + bv[j];
        store4_bf16(g.C, static_cast<int64_t>(m) * g.ldc + col, o, n, vec);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Direct-to-LDS variant of the 256 x 256 kernel.  Operands go from global
// memory straight into LDS with global_load_lds_dwordx4 (lane l's 16 bytes
// land at M0 + 16 l), so the pipeline holds four LDS stages without staging
// registers and loads run three 32-wide K-steps ahead of the MFMAs.  Each load
// fills one MFMA fragment (16 rows x 64 bytes) in lane order.
// Rows that must read as zero (past M, past N, inactive blocks) are never
// masked on the load side: they read a valid row, and the epilogue drops or
// zeroes what they produce.  Dense K needs K % 32 == 0.
// ---------------------------------------------------------------------------
// Direct-to-LDS loads for the 256 x 256 tiles (0: register-staged kernel).
#ifndef FSI_GEMM_DMA
#define FSI_GEMM_DMA 1
#endif
#ifndef FSI_GEMM_DMA_SCHED
#define FSI_GEMM_DMA_SCHED 1
#endif
#ifndef FSI_GEMM_DMA_STAGES
#define FSI_GEMM_DMA_STAGES 4
#endif
#ifndef FSI_GEMM_DMA_PREFETCH
#define FSI_GEMM_DMA_PREFETCH 1
#endif
// K-gathered problems (the Pattention down projection) on the DMA kernel: 174 vs
// 168 us for the register-staged 64-wide-step kernel at the 8B prefill shape.
#ifndef FSI_GEMM_DMA_KGATHER
#define FSI_GEMM_DMA_KGATHER 0
#endif
// Waves of the direct-to-LDS kernel: 8 (2 x 4 waves of 128 x 64) or 4 (2 x 2 waves
// of 128 x 128, accumulators in AGPRs: 16 fragment reads per 64 MFMAs instead of
// 12 per 32).  Measured at the 8B prefill shape, 4 waves run the K-gathered down
// projection no faster (131.6 vs 131.4 us: one wave per SIMD leaves the barrier and
// load waits exposed) and spill in the gate/up SwiGLU epilogue, so 8 is the default.
#ifndef FSI_GEMM_DMA_WAVES
#define FSI_GEMM_DMA_WAVES 8
#endif
constexpr int DK = 32, DSTAGES = FSI_GEMM_DMA_STAGES, DWAVES = FSI_GEMM_DMA_WAVES, DTHREADS = 64 * DWAVES;
static_assert(DWAVES == 4 || DWAVES == 8, "direct-to-LDS GEMM waves");
static_assert(DSTAGES >= 3, "the fragment prefetch reads the stage after the one being multiplied");
constexpr int PK_TILE_ELEMS = 512;  // bf16 elements of one packed 16 x 32 operand tile

// Chunk swizzle of 64-byte LDS rows.  A 128-bit LDS read is served eight lanes at a
// time over a 128-byte bank period, so the eight rows r .. r + 7 of one fragment
// column must fall on distinct 16-byte slots: rows r and r + 1 differ in their
// 64-byte half, and XOR-ing the chunk with row bits 1-2 separates the four pairs.
// Measured on gfx950 with the fragment read pattern: 145 B/clk per CU against
// 100 B/clk for a swizzle on row bits 2-3 (the SQ_LDS_BANK_CONFLICT count of the
// GEMM drops to zero).
__device__ __forceinline__ int dswz(int r) { return (r >> 1) & 3; }
constexpr int DFPW = 16 / DWAVES;      // fragments of A (and of B) each wave loads per K-step
constexpr int DLOADS = 2 * DFPW;       // global_load_lds per wave and K-step
constexpr int DFB = 32 / DWAVES;       // B fragments a wave multiplies (A: 8)
constexpr int DFBH = DFB / 2;          // of them in each 128-column half (gate / up)
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void glb_void_t;

// s_waitcnt vmcnt(N) leaving expcnt and lgkmcnt alone (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Workgroup barrier without the release fence of __syncthreads(), which would
// wait for every direct-to-LDS load in flight.  The caller has waited for the
// loads the next step reads; the memory clobber keeps the compiler from moving
// LDS accesses across it.
__device__ __forceinline__ void stage_barrier() { asm volatile("s_barrier" ::: "memory"); }

template <int NM, int KM, int EPI, bool PB = false>
__global__ __launch_bounds__(DTHREADS, 1) void bsgemm_dma_kernel(GemmArgs g) {
  static_assert(!PB || (NM == N_DUAL && KM == K_DENSE) || (NM == N_DIRECT && KM == K_GATHER_B),
                "packed B: gate/up (dual, dense K) or down (direct, gathered K)");
  __shared__ __attribute__((aligned(1024))) bf16_t lds[DSTAGES][2][BM * DK];  // [stage][A/B][row * 32 + k]
  __shared__ int32_t ktab[KM == K_GATHER_B ? KTAB_MAX : 1];
  const int tid = threadIdx.x;
  if (KM == K_GATHER_B && !PB) {  // packed B reads the block ids from global memory
    fill_ktab(g, ktab, DTHREADS);
    __syncthreads();
  }
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / (DWAVES / 2), wn = wave % (DWAVES / 2);  // 2 x (DWAVES / 2) waves

  const int lid = xcd_group_id(blockIdx.x, gridDim.x);
  int mt, nt;
  grouped_tile(lid, g.m_tiles, g.n_tiles, mt, nt);
  const int kcount = KM == K_GATHER_B ? g.n_blocks * (g.block / DK) : g.K / DK;
  const int m0 = mt * BM;

  // ---- per 32-column sub-block: B row base and C column base ----------------
  int64_t brow[8];
  int ccol[8];
  bool bval[8];
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    if (NM == N_DUAL) {
      const int ch = nt * 128 + (s & 3) * SUB;  // tile columns [gate 128 | up 128]
      const int bi = ch / g.block;
      const int blk = bi < g.n_blocks ? (g.blocks ? g.blocks[bi] : bi) : -1;
      const int64_t row = static_cast<int64_t>(blk) * g.block + ch % g.block;
      bval[s] = blk >= 0 && row + SUB <= g.n_rows_total;
      brow[s] = bval[s] ? row : 0;
      ccol[s] = ch;
    } else if (NM == N_GATHER) {
      const int col = nt * BN + s * SUB;
      const int bi = col / g.block;
      const int blk = bi < g.n_blocks ? (g.blocks ? g.blocks[bi] : bi) : -1;
      const int64_t row = static_cast<int64_t>(blk) * g.block + col % g.block;
      bval[s] = blk >= 0 && row + SUB <= g.n_rows_total;
      brow[s] = bval[s] ? row : 0;
      ccol[s] = g.scatter_c ? static_cast<int>(row) : col;
    } else {
      const int col = nt * BN + s * SUB;
      bval[s] = col < g.N;
      brow[s] = bval[s] ? col : 0;
      ccol[s] = col;
    }
    if (NM != N_DIRECT && !bval[s] && g.err && ((NM == N_DUAL ? nt * 128 + (s & 3) * SUB : nt * BN + s * SUB) < g.N))
      set_error(g.err, FSI_ERR_INDEX_RANGE);
  }

  // ---- this lane's source rows.  A stage holds each operand row-major, 64 bytes
  // (4 chunks of 16) per row, the chunk of row r at physical slot chunk ^ dswz(r).
  // Wave w loads KiB DFPW w .. DFPW w + DFPW - 1 of A and of B (16 rows each): lane l
  // lands at row 16 KiB + l / 4, slot l % 4, so it loads the logical chunk
  // (l % 4) ^ dswz(row).  Packed B: the stage holds B as 16 fragments of 1 KiB in
  // lane order (fragment fi = tile columns 16 fi .. 16 fi + 15) and wave w loads its
  // fragments straight from their packed tiles: one contiguous KiB per load.
  const bf16_t* asrc[DFPW];
  const bf16_t* bsrc[DFPW];
#pragma unroll
  for (int j = 0; j < DFPW; ++j) {
    const int r = 16 * (DFPW * wave + j) + (lane >> 2);
    const int lc = (lane & 3) ^ dswz(r);
    const int m = m0 + r < g.M ? m0 + r : g.M - 1;
    asrc[j] = g.A + static_cast<int64_t>(m) * g.lda + lc * 8;
    if (PB) {
      const int fi = DFPW * wave + j;
      if (NM == N_DUAL) {
        const int sb = fi >> 1;                                     // 32-row sub-block
        const int64_t ct = (brow[sb] >> 4) + (fi & 1);              // 16-row packed tile
        bsrc[j] = (sb >= 4 ? g.Bp1 : g.Bp0) + ct * g.pk_S * PK_TILE_ELEMS + lane * 8;
      } else {
        int dt = (nt * BN) / 16 + fi;
        if (dt >= g.pk_DT) dt = g.pk_DT - 1;                        // columns past N: never stored
        bsrc[j] = g.Bp0 + static_cast<int64_t>(dt) * g.pk_CB * PK_TILE_ELEMS + lane * 8;
      }
    } else {
      const int s = r / SUB;
      const bf16_t* bp = (NM == N_DUAL && s >= 4) ? g.B1 : g.B0;
      int64_t brw = brow[s] + (r % SUB);
      if (NM == N_DIRECT && brw >= g.N) brw = g.N - 1;
      bsrc[j] = bp + brw * g.ldb + lc * 8;
    }
  }
  // K-gathered B: steps are issued in order, so the block and 32-wide sub-step of the
  // next issue are counters, and the block's first column (block id for packed B)
  // comes from a register copy of 64 ktab entries (lane i holds entry 64 c + i) read
  // with v_readlane.  The copy of the next 64 entries is loaded one chunk ahead, so
  // an issue never waits on an LDS read (a wait on it would also hold back the
  // global loads behind the fragment reads in flight).
  const int per = KM == K_GATHER_B ? g.block / DK : 1;
  auto kt_load = [&](int c) {
    const int e = 64 * c + lane;
    if (PB) {  // block ids straight from global memory: an LDS read here would make the
               // compiler wait for every direct-to-LDS load before each fragment read
      const int blk = e < g.n_blocks ? (g.blocks ? g.blocks[e] : e) : -1;
      return blk >= 0 && static_cast<int64_t>(blk + 1) * g.block <= g.n_rows_total ? blk : -1;
    }
    return e < g.n_blocks ? ktab[e] : -1;
  };
  int iss_blk = 0, iss_sub = 0, kt_cur = 0, kt_next = 0;
  if (KM == K_GATHER_B) {
    kt_cur = kt_load(0);
    kt_next = kt_load(1);
  }
  auto issue = [&](int step, int stage) {
    const int64_t a_k = static_cast<int64_t>(step) * DK;
    int64_t b_k = a_k;
    if (KM == K_GATHER_B) {
      const int col = __builtin_amdgcn_readlane(kt_cur, iss_blk & 63);
      if (PB)  // tile (b, dt, cl) at ((b DT + dt) CB + cl) KiB; a dead block reads block 0 (its H is zero)
        b_k = (static_cast<int64_t>(col < 0 ? 0 : col) * g.pk_DT * g.pk_CB + iss_sub) * PK_TILE_ELEMS;
      else
        b_k = col < 0 ? 0 : col + iss_sub * DK;  // an inactive block's H columns are zero
      if (++iss_sub == per) {
        iss_sub = 0;
        if ((++iss_blk & 63) == 0) {
          kt_cur = kt_next;
          kt_next = kt_load((iss_blk >> 6) + 1);
        }
      }
    } else if (PB) {
      b_k = static_cast<int64_t>(step) * PK_TILE_ELEMS;  // k-step s of every row tile
    }
#pragma unroll
    for (int j = 0; j < DFPW; ++j) {
      bf16_t* da = &lds[stage][0][(DFPW * wave + j) * 512];
      bf16_t* db = &lds[stage][1][(DFPW * wave + j) * 512];
      __builtin_amdgcn_global_load_lds((glb_void_t*)(asrc[j] + a_k), (lds_void_t*)da, 16, 0, 0);
      __builtin_amdgcn_global_load_lds((glb_void_t*)(bsrc[j] + b_k), (lds_void_t*)db, 16, 0, 0);
    }
  };

  f32x4_t acc[8][DFB];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < DFB; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // wave fragments: A fragments 8 wm + i; B fragments of tile columns
  // {16 DFBH wn + 16 f} (f < DFBH) and {128 + 16 DFBH wn + 16 (f - DFBH)}: a gate column
  // and its up column share a lane
  const int frow = lane & 15;
  auto bcol = [&](int f) {
    return f < DFBH ? 16 * DFBH * wn + 16 * f : 128 + 16 * DFBH * wn + 16 * (f - DFBH);
  };
  const int fchunk = lane >> 4;
  auto read_frags = [&](int stage, u32x4_t (&fa)[8], u32x4_t (&fb)[DFB]) {
#pragma unroll
    for (int f = 0; f < DFB; ++f) {
      if (PB) {
        fb[f] = *reinterpret_cast<const u32x4_t*>(&lds[stage][1][(bcol(f) >> 4) * PK_TILE_ELEMS + lane * 8]);
      } else {
        const int c = bcol(f) + frow;
        fb[f] = *reinterpret_cast<const u32x4_t*>(&lds[stage][1][c * DK + (fchunk ^ dswz(c)) * 8]);
      }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r = 128 * wm + 16 * i + frow;
      fa[i] = *reinterpret_cast<const u32x4_t*>(&lds[stage][0][r * DK + (fchunk ^ dswz(r)) * 8]);
    }
  };
  auto mfmas = [&](const u32x4_t (&fa)[8], const u32x4_t (&fb)[DFB]) {
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int f = 0; f < DFB; ++f) acc[i][f] = mfma16x16x32(fb[f], fa[i], acc[i][f]);  // C^T fragment
  };
#if FSI_GEMM_DMA_PREFETCH
  // Step s + 2 must have landed at the end of iteration s (its fragments are read
  // during iteration s + 1); later steps may still be in flight.
  auto wait_through = [&](int s) {
    const int last = kcount - 1 < s + DSTAGES - 1 ? kcount - 1 : s + DSTAGES - 1;  // last step issued
    const int after = last - (s + 2);
    if (DSTAGES >= 5 && after >= 2) wait_vmcnt<2 * DLOADS>();
    else if (after >= 1) wait_vmcnt<DLOADS>();
    else wait_vmcnt<0>();
  };
  // One K-step: issue step + DSTAGES - 1, read step + 1's fragments while step's
  // MFMAs run.
  auto iteration = [&](int step, const u32x4_t (&ca)[8], const u32x4_t (&cb)[DFB], u32x4_t (&na)[8],
                       u32x4_t (&nb)[DFB]) {
    // the stage of step + DSTAGES - 1 was last read during iteration step - 2
    if (step + DSTAGES - 1 < kcount) issue(step + DSTAGES - 1, (step + DSTAGES - 1) % DSTAGES);
    // unconditional (past the last step it reads a stale stage that is never
    // used), so the compiler's wait before the MFMAs counts only older reads
    read_frags((step + 1) % DSTAGES, na, nb);
    mfmas(ca, cb);
    // spread the 8 + DFB fragment reads over the 8 DFB MFMAs (a few MFMAs first,
    // then one read per 2 (8 waves) or 3 (4 waves) MFMAs) instead of leaving them
    // to the end of the step
    constexpr int HEAD = DWAVES == 8 ? 2 : 4, PER = DWAVES == 8 ? 2 : 3;
    constexpr int TAIL = 8 * DFB - HEAD - (8 + DFB) * PER;
    __builtin_amdgcn_sched_group_barrier(0x008, HEAD, 0);
#pragma unroll
    for (int r = 0; r < 8 + DFB; ++r) {
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, PER, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, TAIL, 0);
    wait_through(step);
    stage_barrier();
  };

  // prologue: steps 0 .. DSTAGES - 2 into their stages; steps 0 and 1 must land first
  const int pre = kcount < DSTAGES - 1 ? kcount : DSTAGES - 1;
  for (int p = 0; p < pre; ++p) issue(p, p);
  if (DSTAGES >= 5 && pre >= 4) wait_vmcnt<2 * DLOADS>();
  else if (pre >= 3) wait_vmcnt<DLOADS>();
  else wait_vmcnt<0>();
  stage_barrier();
  u32x4_t fa0[8], fb0[DFB], fa1[8], fb1[DFB];
  if (kcount > 0) read_frags(0, fa0, fb0);
  int step = 0;
  for (; step + 1 < kcount; step += 2) {
    iteration(step, fa0, fb0, fa1, fb1);
    iteration(step + 1, fa1, fb1, fa0, fb0);
  }
  if (step < kcount) mfmas(fa0, fb0);  // odd step count: the last step's fragments are in set 0
#else
  // Each iteration reads its own step's fragments; step s + 1 must have landed at
  // the end of iteration s.
  const int pre = kcount < DSTAGES - 1 ? kcount : DSTAGES - 1;
  for (int p = 0; p < pre; ++p) issue(p, p);
  if (DSTAGES >= 5 && pre >= 4) wait_vmcnt<3 * DLOADS>();
  else if (pre >= 3) wait_vmcnt<2 * DLOADS>();
  else if (pre >= 2) wait_vmcnt<DLOADS>();
  else wait_vmcnt<0>();
  stage_barrier();
  for (int step = 0; step < kcount; ++step) {
    if (step + DSTAGES - 1 < kcount) issue(step + DSTAGES - 1, (step + DSTAGES - 1) % DSTAGES);
    u32x4_t fa[8], fb[DFB];
    read_frags(step % DSTAGES, fa, fb);
    mfmas(fa, fb);
    const int last = kcount - 1 < step + DSTAGES - 1 ? kcount - 1 : step + DSTAGES - 1;
    const int after = last - (step + 1);
    if (DSTAGES >= 5 && after >= 3) wait_vmcnt<3 * DLOADS>();
    else if (after >= 2) wait_vmcnt<2 * DLOADS>();
    else if (after >= 1) wait_vmcnt<DLOADS>();
    else wait_vmcnt<0>();
    stage_barrier();
  }
#endif

  // ---- epilogue: the fragments hold C^T, so lane (q = lane / 16, r = lane % 16) of
  // fragment (i, f) holds row 16 i + r of the wave's rows and the four consecutive
  // columns 4 q .. 4 q + 3 of the fragment: one 8-byte store per fragment.  Interior
  // tiles take a branch-free path with the rounding mode fixed at compile time: the
  // epilogue runs once per tile from a cold instruction cache, so its code size is
  // its cost.
  const int crow = m0 + 128 * wm + frow;
  const int cq = 4 * fchunk;
  const bool vec = (reinterpret_cast<uintptr_t>(g.C) & 7) == 0 && (g.ldc & 3) == 0;
  const bool rows_in = m0 + BM <= g.M;
  if (EPI == EPI_SWIGLU) {
    // gate fragment f (< DFBH) and up fragment f + DFBH: tile channel 16 DFBH wn + 16 f,
    // in sub-block (16 DFBH wn + 16 f) / 32 of each half
    bool live[DFBH];
    bool all_live = true;
#pragma unroll
    for (int f = 0; f < DFBH; ++f) {
      const int sb = (16 * DFBH * wn + 16 * f) / SUB;
      live[f] = bval[sb] && bval[4 + sb];
      all_live = all_live && live[f];
    }
    const int ch0 = ccol[0] + 16 * DFBH * wn + cq;
    auto interior = [&](auto rnd) {
      constexpr int R = decltype(rnd)::value;
#pragma unroll
      for (int f = 0; f < DFBH; ++f)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          float h[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) h[j] = swiglu_epi<R>(acc[i][f][j], acc[i][f + DFBH][j]);
          store4_fast(g.C, static_cast<int64_t>(crow + 16 * i) * g.ldc + ch0 + 16 * f, h);
        }
    };
    if (vec && rows_in && all_live && ccol[0] + 128 <= g.N) {
      if (g.rounding == FSI_ROUND_FP32) interior(std::integral_constant<int, FSI_ROUND_FP32>{});
      else if (g.rounding == FSI_ROUND_FUSED) interior(std::integral_constant<int, FSI_ROUND_FUSED>{});
      else interior(std::integral_constant<int, FSI_ROUND_EAGER>{});
    } else {
#pragma unroll
      for (int f = 0; f < DFBH; ++f) {
        const int ch = ch0 + 16 * f;
        if (ch >= g.N) continue;
        const int n = g.N - ch;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int m = crow + 16 * i;
          if (m >= g.M) continue;
          float h[4];
#pragma unroll
          for (int j = 0; j < 4; ++j)
            h[j] = live[f] ? pattention_act<ACT_SWIGLU>(acc[i][f][j], acc[i][f + DFBH][j], g.rounding) : 0.f;
          store4_bf16(g.C, static_cast<int64_t>(m) * g.ldc + ch, h, n, vec);
        }
      }
    }
  } else if (EPI == EPI_ENERGY) {
    // wave wn holds the tile's channels 16 DFBH wn .. + 16 DFBH, DFBH / 2 groups of 32
    // (gate fragments f = 2 gi, 2 gi + 1): each lane sums its 8 channels of row
    // 16 i + r, then the four lanes r, r + 16, r + 32, r + 48 of the row are added
#pragma unroll
    for (int gi = 0; gi < DFBH / 2; ++gi) {
      const int grp_ch = ccol[0] + 16 * DFBH * wn + 32 * gi;
      if (grp_ch < g.N) {
        const int sb = (16 * DFBH * wn + 32 * gi) / SUB;
        const bool live = bval[sb] && bval[4 + sb];
        auto sums = [&](auto rnd) {
          constexpr int R = decltype(rnd)::value;
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            float e = 0.f;
            if (live) {
#pragma unroll
              for (int j = 0; j < 4; ++j)
                e += energy_term(acc[i][2 * gi][j], acc[i][2 * gi + DFBH][j], R) +
                     energy_term(acc[i][2 * gi + 1][j], acc[i][2 * gi + 1 + DFBH][j], R);
            }
            e = sum_rows4(e);
            const int m = crow + 16 * i;
            if (fchunk == 0 && m < g.M) g.E[static_cast<int64_t>(m) * g.ldc + grp_ch / SUB] = e;
          }
        };
        if (g.rounding == FSI_ROUND_FP32) sums(std::integral_constant<int, FSI_ROUND_FP32>{});
        else if (g.rounding == FSI_ROUND_FUSED) sums(std::integral_constant<int, FSI_ROUND_FUSED>{});
        else sums(std::integral_constant<int, FSI_ROUND_EAGER>{});
      }
    }
  } else {
    bool all = vec && rows_in;
#pragma unroll
    for (int sb = 0; sb < 8; ++sb) all = all && (NM == N_DIRECT ? ccol[sb] + SUB <= g.N : bval[sb]);
    if (all) {
#pragma unroll
      for (int f = 0; f < DFB; ++f) {
        const int tc = bcol(f);
        const int s = tc / SUB;
        const int col = ccol[s] + (tc % SUB) + cq;
        float bv[4] = {0.f, 0.f, 0.f, 0.f};
        if (g.bias) {
#pragma unroll
          for (int j = 0; j < 4; ++j)
            bv[j] = bf16_to_f32(g.bias[NM == N_GATHER ? brow[s] + (tc % SUB) + cq + j : col + j]);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          float o[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) o[j] = acc[i][f][j] + bv[j];
          store4_fast(g.C, static_cast<int64_t>(crow + 16 * i) * g.ldc + col, o);
        }
      }
    } else {
#pragma unroll
      for (int f = 0; f < DFB; ++f) {
        const int tc = bcol(f);
        const int s = tc / SUB;
        if (NM != N_DIRECT && !bval[s]) continue;
        const int col = ccol[s] + (tc % SUB) + cq;
        if (NM == N_DIRECT && col >= g.N) continue;
        const int n = NM == N_DIRECT ? g.N - col : 4;
        float bv[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
          bv[j] = g.bias && j < n ? bf16_to_f32(g.bias[NM == N_GATHER ? brow[s] + (tc % SUB) + cq + j : col + j]) : 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int m = crow + 16 * i;
          if (m >= g.M) continue;
          float o[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) o[j] = acc[i][f][j] + bv[j];
          store4_bf16(g.C, static_cast<int64_t>(m) * g.ldc + col, o, n, vec);
        }
      }
    }
  }
}

// Zero the columns of C whose column block is inactive (BlockSparseLinear's
// torch.zeros + scatter); mask[b] != 0 marks active block b.
__global__ __launch_bounds__(256) void zero_inactive_kernel(bf16_t* __restrict__ C, int64_t ldc, int M, int N,
                                                            int block, const uint8_t* __restrict__ mask) {
  const int64_t total = static_cast<int64_t>(M) * (N / 8);
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * 256) {
    const int m = static_cast<int>(i / (N / 8));
    const int c = static_cast<int>(i % (N / 8)) * 8;
    if (!mask[c / block]) *reinterpret_cast<u32x4_t*>(C + m * ldc + c) = u32x4_t{0u, 0u, 0u, 0u};
  }
}

__global__ __launch_bounds__(256) void block_mask_kernel(const int32_t* __restrict__ blocks, int n, int n_blocks,
                                                         uint8_t* __restrict__ mask, int* __restrict__ err) {
  // mask was cleared by a fill kernel before this launch
  for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) {
    const int b = blocks[i];
    if (b >= 0 && b < n_blocks) mask[b] = 1;
    else if (err) set_error(err, FSI_ERR_INDEX_RANGE);
  }
}

__global__ __launch_bounds__(256) void fill_u8_kernel(uint8_t* __restrict__ p, int64_t n) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += static_cast<int64_t>(gridDim.x) * 256)
    p[i] = 0;
}

template <int NM, int KM, int EPI>
hipError_t launch(const GemmArgs& a, unsigned grid, hipStream_t st) {
  bsgemm_kernel<NM, KM, EPI><<<grid, GT, 0, st>>>(a);
  return hipGetLastError();
}

// Rows from which the 256 x 256 kernel replaces the 128 x 128 one.
#ifndef FSI_GEMM_BIG_MIN_M
#define FSI_GEMM_BIG_MIN_M 256
#endif
constexpr int BIG_MIN_M = FSI_GEMM_BIG_MIN_M;

// Sets the tile grid for the kernel `big` selects and launches it.
template <int NM, int KM, int EPI>
hipError_t launch_tiled(GemmArgs& a, bool big, hipStream_t st) {
  const int tm = big ? BM : TM;
  const int tn = NM == N_DUAL ? (big ? BN / 2 : TN / 2) : (big ? BN : TN);
  a.m_tiles = (a.M + tm - 1) / tm;
  a.n_tiles = (a.N + tn - 1) / tn;
  const unsigned grid = static_cast<unsigned>(a.m_tiles) * a.n_tiles;
  // Direct-to-LDS for dense K; the K-gathered down projection reads half lines
  // per 32-wide step and runs better on the 64-wide-step kernel.
  if (big && FSI_GEMM_DMA && (KM == K_GATHER_B ? FSI_GEMM_DMA_KGATHER != 0 : a.K % DK == 0)) {
    bsgemm_dma_kernel<NM, KM, EPI><<<grid, DTHREADS, 0, st>>>(a);
    return hipGetLastError();
  }
  if constexpr (EPI != EPI_ENERGY) {
    if (big) {
      bsgemm_big_kernel<NM, KM, EPI><<<grid, BT, 0, st>>>(a);
      return hipGetLastError();
    }
  }
  return launch<NM, KM, EPI>(a, grid, st);
}

}  // namespace

namespace fsi_gemm {

// Pattention prefill building blocks, used by fsi_pattention_fwd.
// H[M, 64 n_active] = act(x K_gate[S]^T, x K_up[S]^T), S = active blocks of block_n (multiple of 32)
int gateup_swiglu(const bf16_t* x, int64_t ldx, const bf16_t* kg, const bf16_t* ku, int64_t ldk, int N_p,
                  const int32_t* blocks, int n_active, int block_n, int M, int K, int rounding, bf16_t* H,
                  int64_t ldh, int* err, hipStream_t st) {
  GemmArgs a{};
  a.A = x;
  a.B0 = kg;
  a.B1 = ku;
  a.C = H;
  a.lda = ldx;
  a.ldb = ldk;
  a.ldc = ldh;
  a.M = M;
  a.N = n_active * block_n;
  a.K = K;
  a.blocks = blocks;
  a.n_blocks = n_active;
  a.block = block_n;
  a.n_rows_total = N_p;
  a.act = ACT_SWIGLU;
  a.rounding = rounding;
  a.err = err;
  return launch_tiled<N_DUAL, K_DENSE, EPI_SWIGLU>(a, M >= BIG_MIN_M, st) == hipSuccess ? 0 : -1;
}

// E[M, N / 32] = per-row sums over 32-channel groups of |act(x K_gate^T, x K_up^T)| for all N
// channels (dense; N % 32 == 0).  The 256 x 256 direct-to-LDS kernel needs K % 32 == 0;
// otherwise the 128 x 128 kernel runs.
int gateup_energy(const bf16_t* x, int64_t ldx, const bf16_t* kg, const bf16_t* ku, int64_t ldk, int N, int M, int K,
                  int rounding, float* E, int64_t lde, int* err, hipStream_t st) {
  GemmArgs a{};
  a.A = x;
  a.B0 = kg;
  a.B1 = ku;
  a.E = E;
  a.lda = ldx;
  a.ldb = ldk;
  a.ldc = lde;
  a.M = M;
  a.N = N;
  a.K = K;
  a.blocks = nullptr;
  a.n_blocks = N / SUB;
  a.block = SUB;
  a.n_rows_total = N;
  a.act = ACT_SWIGLU;
  a.rounding = rounding;
  a.err = err;
  const bool big = M >= BIG_MIN_M && K % DK == 0;
  return launch_tiled<N_DUAL, K_DENSE, EPI_ENERGY>(a, big, st) == hipSuccess ? 0 : -1;
}

// Prefill GEMMs over the packed decode weights (B operands as contiguous 1 KiB MFMA
// tiles).  Need M >= 256 rows' worth of work to pay for the 256 x 256 tiles, K % 32 == 0.
int gateup_swiglu_packed(const bf16_t* x, int64_t ldx, const bf16_t* kgp, const bf16_t* kup, int S, int N_p,
                         const int32_t* blocks, int n_active, int block_n, int M, int K, int rounding, bf16_t* H,
                         int64_t ldh, int* err, hipStream_t st) {
  GemmArgs a{};
  a.A = x;
  a.Bp0 = kgp;
  a.Bp1 = kup;
  a.pk_S = S;
  a.C = H;
  a.lda = ldx;
  a.ldc = ldh;
  a.M = M;
  a.N = n_active * block_n;
  a.K = K;
  a.blocks = blocks;
  a.n_blocks = n_active;
  a.block = block_n;
  a.n_rows_total = N_p;
  a.act = ACT_SWIGLU;
  a.rounding = rounding;
  a.err = err;
  a.m_tiles = (M + BM - 1) / BM;
  a.n_tiles = (a.N + BN / 2 - 1) / (BN / 2);
  const unsigned grid = static_cast<unsigned>(a.m_tiles) * a.n_tiles;
  bsgemm_dma_kernel<N_DUAL, K_DENSE, EPI_SWIGLU, true><<<grid, DTHREADS, 0, st>>>(a);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

int down_gather_packed(const bf16_t* H, int64_t ldh, const bf16_t* vp, int DT, int CB, int N_p,
                       const int32_t* blocks, int n_active, int block_n, int M, int D, bf16_t* out, int64_t ldo,
                       int* err, hipStream_t st) {
  if (n_active > KTAB_MAX) return 1;
  GemmArgs a{};
  a.A = H;
  a.Bp0 = vp;
  a.pk_DT = DT;
  a.pk_CB = CB;
  a.C = out;
  a.lda = ldh;
  a.ldc = ldo;
  a.M = M;
  a.N = D;
  a.K = n_active * block_n;
  a.blocks = blocks;
  a.n_blocks = n_active;
  a.block = block_n;
  a.n_rows_total = N_p;
  a.err = err;
  a.m_tiles = (M + BM - 1) / BM;
  a.n_tiles = (D + BN - 1) / BN;
  const unsigned grid = static_cast<unsigned>(a.m_tiles) * a.n_tiles;
  bsgemm_dma_kernel<N_DIRECT, K_GATHER_B, EPI_STORE, true><<<grid, DTHREADS, 0, st>>>(a);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

// out[M, D] = H[M, 64 n_active] W_down[:, S]^T with W_down [D, N_p] (row stride ldw)
int down_gather(const bf16_t* H, int64_t ldh, const bf16_t* wd, int64_t ldw, int N_p, const int32_t* blocks,
                int n_active, int block_n, int M, int D, bf16_t* out, int64_t ldo, int* err, hipStream_t st) {
  if (n_active > KTAB_MAX) return 1;  // more active blocks than the LDS table holds
  GemmArgs a{};
  a.A = H;
  a.B0 = a.B1 = wd;
  a.C = out;
  a.lda = ldh;
  a.ldb = ldw;
  a.ldc = ldo;
  a.M = M;
  a.N = D;
  a.K = n_active * block_n;
  a.blocks = blocks;
  a.n_blocks = n_active;
  a.block = block_n;
  a.n_rows_total = N_p;
  a.err = err;
  return launch_tiled<N_DIRECT, K_GATHER_B, EPI_STORE>(a, M >= BIG_MIN_M, st) == hipSuccess ? 0 : -1;
}

}  // namespace fsi_gemm

extern "C" {

FSI_API size_t fsi_block_sparse_linear_workspace_size(int64_t N, int64_t block_size) {
  if (block_size <= 0) return FSI_WORKSPACE_COUNTER_BYTES;
  return FSI_WORKSPACE_COUNTER_BYTES + static_cast<size_t>((N / block_size + 255) / 256 * 256);
}

FSI_API int fsi_block_sparse_linear(const void* x, int64_t ldx, const void* w, int64_t ldw, const void* bias,
                                    const int32_t* active_blocks, int64_t n_active, int64_t block_size, int64_t M,
                                    int64_t N, int64_t K, int dtype, void* out, int64_t ldo, void* workspace,
                                    size_t workspace_bytes, int* err, void* stream) {
  using namespace fsi_host;
  FSI_CHECK_ARG(dtype == FSI_DTYPE_BF16 || dtype == FSI_DTYPE_F32, FSI_ERR_DTYPE, "block_sparse_linear: dtype %d",
                dtype);
  FSI_CHECK_ARG(M >= 0 && N >= 0 && K > 0 && n_active >= 0, FSI_ERR_SHAPE, "block_sparse_linear: bad sizes");
  if (dtype == FSI_DTYPE_F32 || block_size % SUB != 0 || K % 8 || ldx % 8 || ldw % 8 || ldo % 8 || N % 8 ||
      reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(w) % 16 ||
      reinterpret_cast<uintptr_t>(out) % 16) {
    // fp32, and bf16 shapes the MFMA engine does not tile: the generic kernel
    if (M == 0 || N == 0) return FSI_OK;
    FSI_CHECK_ARG(x && w && out && (active_blocks || n_active == 0), FSI_ERR_INVALID_ARG,
                  "block_sparse_linear: null pointer");
    FSI_CHECK_ARG(block_size > 0 && N % block_size == 0, FSI_ERR_SHAPE,
                  "block_sparse_linear: block_size %lld must divide N %lld", (long long)block_size, (long long)N);
    const size_t need = fsi_block_sparse_linear_workspace_size(N, block_size);
    FSI_CHECK_ARG(workspace && workspace_bytes >= need, FSI_ERR_WORKSPACE,
                  "block_sparse_linear: workspace %zu < %zu bytes", workspace_bytes, need);
    return fsi_bs_generic::column_gemm(x, ldx, w, ldw, bias, active_blocks, n_active, block_size, M, N, K, dtype, out,
                                       ldo, static_cast<uint8_t*>(workspace) + FSI_WORKSPACE_COUNTER_BYTES, err,
                                       reinterpret_cast<hipStream_t>(stream));
  }
  FSI_CHECK_ARG(block_size > 0 && block_size % SUB == 0 && N % block_size == 0, FSI_ERR_SHAPE,
                "block_sparse_linear: block_size %lld must be a multiple of %d dividing N %lld", (long long)block_size,
                SUB, (long long)N);
  FSI_CHECK_ARG(K % 8 == 0 && ldx % 8 == 0 && ldw % 8 == 0 && ldo % 8 == 0 && N % 8 == 0, FSI_ERR_ALIGN,
                "block_sparse_linear: K, N and leading dimensions must be multiples of 8");
  FSI_CHECK_ARG(ldx >= K && ldw >= K && ldo >= N, FSI_ERR_SHAPE, "block_sparse_linear: leading dimension too small");
  FSI_CHECK_ARG(M <= 0x7fffffff && N <= 0x7fffffff && K <= 0x7fffffff, FSI_ERR_SHAPE,
                "block_sparse_linear: sizes beyond int32");
  if (M == 0 || N == 0) return FSI_OK;
  FSI_CHECK_ARG(x && w && out && (active_blocks || n_active == 0), FSI_ERR_INVALID_ARG,
                "block_sparse_linear: null pointer");
  FSI_CHECK_ARG(reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(w) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(out) % 16 == 0,
                FSI_ERR_ALIGN, "block_sparse_linear: x, w and out must be 16-byte aligned");
  const int64_t nb = N / block_size;
  const size_t need = fsi_block_sparse_linear_workspace_size(N, block_size);
  FSI_CHECK_ARG(workspace && workspace_bytes >= need, FSI_ERR_WORKSPACE,
                "block_sparse_linear: workspace %zu < %zu bytes", workspace_bytes, need);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  uint8_t* mask = static_cast<uint8_t*>(workspace) + FSI_WORKSPACE_COUNTER_BYTES;
  fill_u8_kernel<<<1, 256, 0, st>>>(mask, nb);
  if (n_active > 0)
    block_mask_kernel<<<static_cast<unsigned>((n_active + 255) / 256), 256, 0, st>>>(active_blocks, (int)n_active,
                                                                                    (int)nb, mask, err);
  const int64_t zero_items = M * (N / 8);
  zero_inactive_kernel<<<static_cast<unsigned>(std::min<int64_t>((zero_items + 255) / 256, 1 << 16)), 256, 0, st>>>(
      static_cast<bf16_t*>(out), ldo, (int)M, (int)N, (int)block_size, mask);
  FSI_HIP_LAUNCH_CHECK("block_sparse_linear zero");
  if (n_active == 0) return FSI_OK;
  GemmArgs a{};
  a.A = static_cast<const bf16_t*>(x);
  a.B0 = a.B1 = static_cast<const bf16_t*>(w);
  a.bias = static_cast<const bf16_t*>(bias);
  a.C = static_cast<bf16_t*>(out);
  a.lda = ldx;
  a.ldb = ldw;
  a.ldc = ldo;
  a.M = (int)M;
  a.N = (int)(n_active * block_size);
  a.K = (int)K;
  a.blocks = active_blocks;
  a.n_blocks = (int)n_active;
  a.block = (int)block_size;
  a.n_rows_total = (int)N;
  a.scatter_c = 1;
  a.err = err;
  const hipError_t e = launch_tiled<N_GATHER, K_DENSE, EPI_STORE>(a, M >= BIG_MIN_M, st);
  FSI_CHECK_ARG(e == hipSuccess, FSI_ERR_HIP, "block_sparse_linear: launch failed: %s", hipGetErrorString(e));
  return FSI_OK;
}

}  // extern "C"
