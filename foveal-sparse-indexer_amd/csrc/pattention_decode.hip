// Decode-shaped block-sparse Pattention (up to 64 tokens) for MI355X (gfx950).
//
//   out[M, D] = act(x K_gate[S]^T, x K_up[S]^T) V[S]      (foveal_pattention.py:328-335)
//
// The step is bandwidth-bound on the active weight rows (3 x 32 MiB for 64
// blocks of 64 rows at d_model 4096), so the kernels are built around one
// stream of weight bytes per wave with several k-steps of loads in flight:
//   1. gate/up partials.  A workgroup of 8 waves owns 64 channels x one K
//      range: 4 channel tiles of 16 x 2 halves of the range.  The x tile of
//      the range (tokens x K range) is staged once into LDS, so x costs one
//      L2 read per workgroup instead of one per wave; each wave streams the
//      16 B-per-lane gate and up rows of its tile from HBM through a
//      register ring of 8 k-steps and feeds the 16x16x32 bf16 MFMA with x
//      from LDS.  The two halves are summed through LDS and one fp32 partial
//      per K range goes to a workspace slab.
//   2. activation: H = act(sum of gate partials, sum of up partials) with the
//      requested bf16 rounding points, summed in range order (deterministic).
//   3. down partials, the same structure with H as the staged operand: a
//      workgroup owns 128 output dims x one channel range; the weight operand
//      is the down_proj-layout V^T [D, N_p] row, 8 consecutive channels of one
//      active block per lane.
//   4. reduction of the down partials, rounded once to bf16.
// Weights are read exactly once.  All loops are fully unrolled: a loop back
// edge makes the compiler wait for every load in flight.
#include "fsi_common.h"

using namespace fsi;

namespace {

constexpr int KSTEP = 32;  // MFMA k per step
#ifndef FSI_DEC_RING
#define FSI_DEC_RING 8
#endif
constexpr int RING = FSI_DEC_RING;
// Fewest workgroups (one per CU) the split choice below aims for.
#ifndef FSI_DEC_MIN_WGS1
#define FSI_DEC_MIN_WGS1 256
#endif
#ifndef FSI_DEC_MIN_WGS2
#define FSI_DEC_MIN_WGS2 256
#endif  // k-steps of weight loads in flight per wave (at most)
constexpr int NKH = 2;     // waves along the k range of a workgroup (summed through LDS)
constexpr int NCT = 4;     // 16-channel tiles per gate/up workgroup
constexpr int DT = 2;      // 16-dim tiles per down wave
constexpr int NDG = 4;     // 32-dim groups per down workgroup
constexpr int GU_THREADS = 64 * NCT * NKH;
constexpr int DN_THREADS = 64 * NDG * NKH;
constexpr int CH_ALIGN = 256;  // channel padding: every range size below divides it

// Keeps the scheduler from hoisting the next step's MFMAs above the refill loads.
#define DEC_SCHED_FENCE() __builtin_amdgcn_sched_barrier(0)

__device__ __forceinline__ u32x4_t ld16g(const bf16_t* p) { return *reinterpret_cast<const u32x4_t*>(p); }

struct DecArgs {
  const bf16_t* x;
  int64_t ldx;
  const bf16_t* kg;
  const bf16_t* ku;
  int64_t ldk;
  const bf16_t* vt;  // [D, N_p] row stride ldv
  int64_t ldv;
  const int32_t* active;
  int n_blocks_valid;  // ceil(N_p / bn)
  int log2bn;
  int64_t N_p;
  int M, K, n_ch, n_ch_pad, D;
  int S, S2;    // gate/up K ranges and down channel ranges
  int rounding;
  float* pg;    // [S][64][n_ch_pad]
  float* pu;
  bf16_t* h;    // [64][n_ch_pad]
  float* py;    // [S2][64][D_pad]
  int D_pad;
  bf16_t* out;
  int64_t ldo;
  int* err;
};

// Weight rows of NG channel groups c[0..NG) (16 or 32 channels each, inside
// one block since bn >= 32): row of the group's first channel, or -1 when the
// group is past n_ch or its block id is out of range (*bad is set then).  The
// c[] are wave-uniform, so the block ids are scalar loads, all issued before
// the first wait and independent of the vector loads already in flight.
// A dense call (no block list) runs on an identity list the host writes first.
template <int NG>
__device__ __forceinline__ void group_rows(const DecArgs& a, const int* c, int64_t* row, bool* bad) {
  int32_t blk[NG];
#pragma unroll
  for (int j = 0; j < NG; ++j) blk[j] = a.active[(c[j] < a.n_ch ? c[j] : 0) >> a.log2bn];
#pragma unroll
  for (int j = 0; j < NG; ++j) {
    const bool in = c[j] < a.n_ch;
    const bool ok = blk[j] >= 0 && blk[j] < a.n_blocks_valid;
    *bad |= in && !ok;
    row[j] = in && ok ? (static_cast<int64_t>(blk[j]) << a.log2bn) | (c[j] & ((1 << a.log2bn) - 1)) : -1;
  }
}

// A [ROWS][COLS] bf16 tile (rows >= valid read row 0) staged from global memory
// into LDS with a row pitch of 2 COLS + 16 bytes: the 16 lanes of one ds_read_b128
// quarter read 16 different rows at the same column and land on 16 different
// 16-byte bank groups.  Consecutive threads take consecutive 16 bytes of a row.
template <int ROWS, int COLS, int NT>
struct LdsTile {
  static constexpr int PITCH = 2 * COLS + 16;
  static constexpr int BYTES = ROWS * PITCH;
  static constexpr int CPR = COLS / 8;
  static constexpr int PER = ROWS * CPR / NT;
  static_assert(ROWS * CPR % NT == 0, "tile must split evenly over the workgroup");
  u32x4_t v[PER];
  __device__ __forceinline__ void load(const bf16_t* src, int64_t ld, int valid, int c0) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int idx = static_cast<int>(threadIdx.x) + i * NT;
      const int row = idx / CPR, c = idx % CPR;
      v[i] = ld16g(src + static_cast<int64_t>(row < valid ? row : 0) * ld + c0 + 8 * c);
    }
  }
  __device__ __forceinline__ void store(char* lds) const {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int idx = static_cast<int>(threadIdx.x) + i * NT;
      const int row = idx / CPR, c = idx % CPR;
      *reinterpret_cast<u32x4_t*>(lds + row * PITCH + 16 * c) = v[i];
    }
  }
};

// Sums the NACC accumulators of the NKH waves that share one output tile: waves
// with kh > 0 park theirs in LDS (lane-contiguous, conflict-free), wave kh == 0
// adds them.  Every thread of the workgroup must call it (it holds barriers).
template <int NACC, int NGROUP>
__device__ __forceinline__ void reduce_k_halves(char* lds, f32x4_t* acc, int group, int kh, int lane) {
  __syncthreads();  // every wave is done with the staged tile
  float* red = reinterpret_cast<float*>(lds);
  if (kh > 0) {
    float* w = red + static_cast<int64_t>((kh - 1) * NGROUP + group) * NACC * 4 * 64 + lane;
#pragma unroll
    for (int i = 0; i < NACC; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) w[(i * 4 + j) * 64] = acc[i][j];
  }
  __syncthreads();
  if (kh == 0) {
#pragma unroll
    for (int o = 1; o < NKH; ++o) {
      const float* w = red + static_cast<int64_t>((o - 1) * NGROUP + group) * NACC * 4 * 64 + lane;
#pragma unroll
      for (int i = 0; i < NACC; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] += w[(i * 4 + j) * 64];
    }
  }
}

// ---------------------------------------------------------------------------
// 1. gate/up partials: workgroup = 4 channel tiles x 2 k halves, K range s
// ---------------------------------------------------------------------------
template <int TT, bool HAS_UP, int NS>
__global__ __launch_bounds__(GU_THREADS) void dec_gateup_kernel(DecArgs a) {
  constexpr int KR = NS * NKH * KSTEP;  // k of one workgroup
  constexpr int NACC = TT * (HAS_UP ? 2 : 1);
  using XTile = LdsTile<TT * 16, KR, GU_THREADS>;
  constexpr int RED_BYTES = (NKH - 1) * NCT * NACC * 4 * 64 * 4;
  __shared__ __attribute__((aligned(16))) char lds[XTile::BYTES > RED_BYTES ? XTile::BYTES : RED_BYTES];
  constexpr int RG = NS < RING ? NS : RING;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
  const int ctl = wave % NCT, kh = wave / NCT;
  const int ct = blockIdx.x * NCT + ctl;  // < n_ch_pad / 16 by the grid
  const int s = blockIdx.y;
  const int kw0 = s * KR;
  const int kk0 = kh * NS * KSTEP;  // this wave's first k inside the range
  const int r = lane & 15, q = lane >> 4;

  XTile xt;
  xt.load(a.x, a.ldx, a.M, kw0);
  DEC_SCHED_FENCE();
  bool bad = false;
  const int cg = ct * 16;
  int64_t row0;
  group_rows<1>(a, &cg, &row0, &bad);
  const int64_t row = row0 + r;
  const bool rv = row0 >= 0 && cg + r < a.n_ch && row < a.N_p;
  // Loaded data is never masked (a select right after a load would wait for
  // it): rows of invalid channels read row 0 and their outputs are zeroed.
  const bf16_t* gp = a.kg + (rv ? row : 0) * a.ldk + kw0 + kk0 + 8 * q;
  const bf16_t* up = HAS_UP ? a.ku + (rv ? row : 0) * a.ldk + kw0 + kk0 + 8 * q : gp;
  u32x4_t rg[RG], ru[RG];
  auto load = [&](int slot, int step) {
    rg[slot] = ld16g(gp + step * KSTEP);
    if (HAS_UP) ru[slot] = ld16g(up + step * KSTEP);
  };
#pragma unroll
  for (int d = 0; d < RG; ++d) load(d, d);
  DEC_SCHED_FENCE();
  xt.store(lds);
  __syncthreads();

  // lane (r, q) feeds token 16 t + r, k = 8 q .. 8 q + 7 of each step
  const char* xl = lds + r * XTile::PITCH + (kk0 + 8 * q) * 2;
  u32x4_t xr[2][TT];
  auto rdx = [&](int buf, int step) {
#pragma unroll
    for (int t = 0; t < TT; ++t)
      xr[buf][t] = *reinterpret_cast<const u32x4_t*>(xl + t * 16 * XTile::PITCH + step * KSTEP * 2);
  };
  f32x4_t acc[NACC];
#pragma unroll
  for (int i = 0; i < NACC; ++i) acc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  rdx(0, 0);
#pragma unroll
  for (int j = 0; j < NS; ++j) {
    if (j + 1 < NS) rdx((j + 1) & 1, j + 1);
#pragma unroll
    for (int t = 0; t < TT; ++t) {
      acc[t] = mfma16x16x32(xr[j & 1][t], rg[j % RG], acc[t]);
      if (HAS_UP) acc[TT + t] = mfma16x16x32(xr[j & 1][t], ru[j % RG], acc[TT + t]);
    }
    if (j + RG < NS) load(j % RG, j + RG);  // resolved at compile time
    DEC_SCHED_FENCE();
  }
  reduce_k_halves<NACC, NCT>(lds, acc, ctl, kh, lane);
  if (kh > 0) return;
  if (bad && lane == 0 && a.err) set_error(a.err, FSI_ERR_INDEX_RANGE);

  const float keep = rv ? 1.f : 0.f;
  // lane holds C[token 4 q + j][channel r] of each tile
  float* og = a.pg + static_cast<int64_t>(s) * 64 * a.n_ch_pad + ct * 16 + r;
  float* ou = a.pu + static_cast<int64_t>(s) * 64 * a.n_ch_pad + ct * 16 + r;
#pragma unroll
  for (int t = 0; t < TT; ++t)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t tok = 16 * t + 4 * q + j;
      og[tok * a.n_ch_pad] = acc[t][j] * keep;
      if (HAS_UP) ou[tok * a.n_ch_pad] = acc[TT + t][j] * keep;
    }
}

// ---------------------------------------------------------------------------
// 2. H = act(sum_s G_s, sum_s U_s).  Workgroup = one 64-channel group x 16
//    tokens, four channels per thread.  Its linear id is congruent mod 8 with
//    the ids of the gate/up workgroups that wrote the group's partials
//    (n_ch_pad / 64 is a multiple of 8 at the sizes that matter), so on
//    MI355X's round-robin XCD dispatch it reads them from its own XCD's L2.
// ---------------------------------------------------------------------------
template <int ACT, bool HAS_UP>
__global__ __launch_bounds__(256) void dec_act_kernel(DecArgs a) {
  const int ncg = a.n_ch_pad / 64;
  const int cg = blockIdx.x % ncg, tg = blockIdx.x / ncg;
  const int tok = tg * 16 + (threadIdx.x >> 4);
  if (tok >= a.M) return;
  const int c = cg * 64 + (threadIdx.x & 15) * 4;
  float4 g = make_float4(0.f, 0.f, 0.f, 0.f), u = g;
#pragma unroll 4
  for (int s = 0; s < a.S; ++s) {
    const int64_t off = (static_cast<int64_t>(s) * 64 + tok) * a.n_ch_pad + c;
    const float4 gs = *reinterpret_cast<const float4*>(a.pg + off);
    g.x += gs.x;
    g.y += gs.y;
    g.z += gs.z;
    g.w += gs.w;
    if (HAS_UP) {
      const float4 us = *reinterpret_cast<const float4*>(a.pu + off);
      u.x += us.x;
      u.y += us.y;
      u.z += us.z;
      u.w += us.w;
    }
  }
  const float h0 = pattention_act<ACT>(g.x, u.x, a.rounding);
  const float h1 = pattention_act<ACT>(g.y, u.y, a.rounding);
  const float h2 = pattention_act<ACT>(g.z, u.z, a.rounding);
  const float h3 = pattention_act<ACT>(g.w, u.w, a.rounding);
  *reinterpret_cast<u32x2_t*>(a.h + static_cast<int64_t>(tok) * a.n_ch_pad + c) =
      u32x2_t{pack_bf16x2(h0, h1), pack_bf16x2(h2, h3)};
}

// ---------------------------------------------------------------------------
// 3. down partials: workgroup = 4 groups of 32 dims x 2 k halves, channel range s2
// ---------------------------------------------------------------------------
template <int TT, int NS>
__global__ __launch_bounds__(DN_THREADS) void dec_down_kernel(DecArgs a) {
  constexpr int CR = NS * NKH * KSTEP;  // channels of one workgroup
  constexpr int NACC = DT * TT;
  using HTile = LdsTile<TT * 16, CR, DN_THREADS>;
  constexpr int RED_BYTES = (NKH - 1) * NDG * NACC * 4 * 64 * 4;
  __shared__ __attribute__((aligned(16))) char lds[HTile::BYTES > RED_BYTES ? HTile::BYTES : RED_BYTES];
  constexpr int RG = NS < RING ? NS : RING;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
  const int dgl = wave % NDG, kh = wave / NDG;
  const int dt0 = (blockIdx.x * NDG + dgl) * DT;  // first 16-dim tile of the wave
  const bool dims_live = dt0 * 16 < a.D;          // waves past D compute on row 0, store nothing
  const int s2 = blockIdx.y;
  const int c0 = s2 * CR;
  const int cc0 = kh * NS * KSTEP;
  const int r = lane & 15, q = lane >> 4;
  const bf16_t* vp[DT];
#pragma unroll
  for (int d = 0; d < DT; ++d) {
    const int dim = (dt0 + d) * 16 + r;
    vp[d] = a.vt + static_cast<int64_t>(dim < a.D ? dim : 0) * a.ldv + 8 * q;
  }
  HTile ht;
  ht.load(a.h, a.n_ch_pad, a.M, c0);
  DEC_SCHED_FENCE();
  // Row base of each 32-channel step.  Channels of invalid blocks have H == 0
  // (their gate/up partials were zeroed), so they read row 0 of V and add nothing.
  int cs[NS];
  int64_t rbs[NS];
  bool bad = false;
#pragma unroll
  for (int j = 0; j < NS; ++j) cs[j] = c0 + cc0 + j * KSTEP;
  group_rows<NS>(a, cs, rbs, &bad);
#pragma unroll
  for (int j = 0; j < NS; ++j) rbs[j] = rbs[j] >= 0 && rbs[j] + KSTEP <= a.N_p ? rbs[j] : 0;
  u32x4_t rv[RG][DT];
  auto load = [&](int slot, int step) {
#pragma unroll
    for (int d = 0; d < DT; ++d) rv[slot][d] = ld16g(vp[d] + rbs[step]);
  };
#pragma unroll
  for (int d = 0; d < RG; ++d) load(d, d);
  DEC_SCHED_FENCE();
  ht.store(lds);
  __syncthreads();

  const char* hl = lds + r * HTile::PITCH + (cc0 + 8 * q) * 2;
  u32x4_t hr[2][TT];
  auto rdh = [&](int buf, int step) {
#pragma unroll
    for (int t = 0; t < TT; ++t)
      hr[buf][t] = *reinterpret_cast<const u32x4_t*>(hl + t * 16 * HTile::PITCH + step * KSTEP * 2);
  };
  f32x4_t acc[NACC];
#pragma unroll
  for (int i = 0; i < NACC; ++i) acc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  rdh(0, 0);
#pragma unroll
  for (int j = 0; j < NS; ++j) {
    if (j + 1 < NS) rdh((j + 1) & 1, j + 1);
#pragma unroll
    for (int t = 0; t < TT; ++t)
#pragma unroll
      for (int d = 0; d < DT; ++d) acc[d * TT + t] = mfma16x16x32(hr[j & 1][t], rv[j % RG][d], acc[d * TT + t]);
    if (j + RG < NS) load(j % RG, j + RG);
    DEC_SCHED_FENCE();
  }
  reduce_k_halves<NACC, NDG>(lds, acc, dgl, kh, lane);
  if (kh > 0 || !dims_live) return;

  // lane holds C[token 4 q + j][dim r] of each tile; D_pad covers whole 32-dim groups
#pragma unroll
  for (int d = 0; d < DT; ++d) {
    float* o = a.py + static_cast<int64_t>(s2) * 64 * a.D_pad + (dt0 + d) * 16 + r;
#pragma unroll
    for (int t = 0; t < TT; ++t)
#pragma unroll
      for (int j = 0; j < 4; ++j) o[static_cast<int64_t>(16 * t + 4 * q + j) * a.D_pad] = acc[d * TT + t][j];
  }
}

// ---------------------------------------------------------------------------
// 4. out = bf16(sum_s2 Y_s2).  Workgroup = one 128-dim group x 8 tokens, four
//    dims per thread, on the XCD of the down workgroups of that dim group
//    (as for the activation kernel).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void dec_reduce_kernel(DecArgs a) {
  const int ndg = (a.D + 127) / 128;
  const int dg = blockIdx.x % ndg, tg = blockIdx.x / ndg;
  const int tok = tg * 8 + (threadIdx.x >> 5);
  const int d = dg * 128 + (threadIdx.x & 31) * 4;
  if (tok >= a.M || d >= a.D) return;
  float4 y = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll 8
  for (int s = 0; s < a.S2; ++s) {
    const float4 v = *reinterpret_cast<const float4*>(a.py + (static_cast<int64_t>(s) * 64 + tok) * a.D_pad + d);
    y.x += v.x;
    y.y += v.y;
    y.z += v.z;
    y.w += v.w;
  }
  bf16_t* o = a.out + static_cast<int64_t>(tok) * a.ldo + d;
  const float vals[4] = {y.x, y.y, y.z, y.w};
#pragma unroll
  for (int e = 0; e < 4; ++e)
    if (d + e < a.D) o[e] = f32_to_bf16(vals[e]);
}

__global__ __launch_bounds__(256) void dec_iota_kernel(int32_t* p, int n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = i;
}

}  // namespace

namespace fsi_dec {

// Ranges and workspace layout of the decode path.
struct Layout {
  int S, S2, n_ch_pad, D_pad;
  int NS1, NS2;  // k-steps per wave of the gate/up and down kernels
  size_t off_pg, off_pu, off_h, off_py, off_ids, total;
};

bool layout(int64_t M, int64_t K, int64_t D, int64_t n_ch, int log2bn, Layout* L) {
  if (M < 1 || M > 64 || log2bn < 5 || n_ch < 1 || K % 256 != 0 || D < 1) return false;
  Layout l{};
  l.n_ch_pad = static_cast<int>((n_ch + CH_ALIGN - 1) / CH_ALIGN * CH_ALIGN);
  l.D_pad = static_cast<int>((D + 16 * DT - 1) / (16 * DT) * (16 * DT));  // whole 32-dim groups
  const int64_t wgs_per_range1 = l.n_ch_pad / (16 * NCT);
  const int64_t wgs_per_range2 = (D + 16 * DT * NDG - 1) / (16 * DT * NDG);
  // The longest k range per workgroup (fewest partials) that still gives one
  // workgroup per CU; the shortest when none does.
  l.NS1 = 4;
  for (int ns : {16, 8}) {
    const int64_t kr = int64_t(ns) * NKH * KSTEP;
    if (K % kr == 0 && wgs_per_range1 * (K / kr) >= FSI_DEC_MIN_WGS1) {
      l.NS1 = ns;
      break;
    }
  }
  l.NS2 = 4;
  {
    const int64_t cr = 8 * NKH * KSTEP;
    if (l.n_ch_pad % cr == 0 && wgs_per_range2 * (l.n_ch_pad / cr) >= FSI_DEC_MIN_WGS2) l.NS2 = 8;
  }
  const int64_t S = K / (int64_t(l.NS1) * NKH * KSTEP);
  const int64_t S2 = l.n_ch_pad / (int64_t(l.NS2) * NKH * KSTEP);
  if (S > 65535 || S2 > 65535 || wgs_per_range1 > (1 << 30) || wgs_per_range2 > (1 << 30)) return false;
  l.S = static_cast<int>(S);
  l.S2 = static_cast<int>(S2);
  size_t o = FSI_WORKSPACE_COUNTER_BYTES;
  auto take = [&](size_t bytes) {
    const size_t at = o;
    o += (bytes + 255) / 256 * 256;
    return at;
  };
  l.off_pg = take(sizeof(float) * static_cast<size_t>(S) * 64 * l.n_ch_pad);
  l.off_pu = take(sizeof(float) * static_cast<size_t>(S) * 64 * l.n_ch_pad);
  l.off_h = take(sizeof(bf16_t) * 64 * static_cast<size_t>(l.n_ch_pad));
  l.off_py = take(sizeof(float) * static_cast<size_t>(S2) * 64 * l.D_pad);
  l.off_ids = take(sizeof(int32_t) * static_cast<size_t>((n_ch >> log2bn) + 1));  // identity block list
  l.total = o;
  *L = l;
  return true;
}

size_t workspace_bytes(int64_t M, int64_t K, int64_t D, int64_t n_ch, int log2bn) {
  Layout l;
  return layout(M, K, D, n_ch, log2bn, &l) ? l.total : 0;
}

// Returns 0 when launched, 1 when this path does not apply, -1 on a launch error.
int run(const bf16_t* x, int64_t ldx, const bf16_t* kg, const bf16_t* ku, int64_t ldk, const bf16_t* vt, int64_t ldv,
        const int32_t* active, int64_t n_blocks_valid, int log2bn, int64_t N_p, int M, int K, int64_t n_ch, int D,
        int activation, int rounding, bf16_t* out, int64_t ldo, void* workspace, size_t ws_bytes, int* err,
        hipStream_t st) {
  Layout l;
  if (!layout(M, K, D, n_ch, log2bn, &l) || ws_bytes < l.total) return 1;
  if (ldx % 8 || ldk % 8 || ldv % 8 || reinterpret_cast<uintptr_t>(vt) % 16 || reinterpret_cast<uintptr_t>(x) % 16 ||
      reinterpret_cast<uintptr_t>(kg) % 16 || (ku && reinterpret_cast<uintptr_t>(ku) % 16))
    return 1;
  // the down kernel reads 32 channels of V^T per step from one block
  if (N_p % KSTEP != 0) return 1;
  const bool up = activation == FSI_ACT_SWIGLU;
  if (up && ku == nullptr) return 1;
  char* ws = static_cast<char*>(workspace);
  DecArgs a{};
  a.x = x;
  a.ldx = ldx;
  a.kg = kg;
  a.ku = ku;
  a.ldk = ldk;
  a.vt = vt;
  a.ldv = ldv;
  if (active == nullptr) {
    const int nb = static_cast<int>((n_ch + (1 << log2bn) - 1) >> log2bn);
    int32_t* ids = reinterpret_cast<int32_t*>(ws + l.off_ids);
    dec_iota_kernel<<<static_cast<unsigned>((nb + 255) / 256), 256, 0, st>>>(ids, nb);
    active = ids;
  }
  a.active = active;
  a.n_blocks_valid = static_cast<int>(n_blocks_valid);
  a.log2bn = log2bn;
  a.N_p = N_p;
  a.M = M;
  a.K = K;
  a.n_ch = static_cast<int>(n_ch);
  a.n_ch_pad = l.n_ch_pad;
  a.D = D;
  a.D_pad = l.D_pad;
  a.S = l.S;
  a.S2 = l.S2;
  a.rounding = rounding;
  a.pg = reinterpret_cast<float*>(ws + l.off_pg);
  a.pu = reinterpret_cast<float*>(ws + l.off_pu);
  a.h = reinterpret_cast<bf16_t*>(ws + l.off_h);
  a.py = reinterpret_cast<float*>(ws + l.off_py);
  a.out = out;
  a.ldo = ldo;
  a.err = err;
  const int tt = (M + 15) / 16;
  const dim3 g1(static_cast<unsigned>(l.n_ch_pad / (16 * NCT)), static_cast<unsigned>(l.S));
#define GU_NS(TTV, NSV)                                                        \
  do {                                                                         \
    if (up) dec_gateup_kernel<TTV, true, NSV><<<g1, GU_THREADS, 0, st>>>(a);   \
    else dec_gateup_kernel<TTV, false, NSV><<<g1, GU_THREADS, 0, st>>>(a);     \
  } while (0)
#define GU(TTV)                          \
  do {                                   \
    if (l.NS1 == 16) GU_NS(TTV, 16);     \
    else if (l.NS1 == 8) GU_NS(TTV, 8);  \
    else GU_NS(TTV, 4);                  \
  } while (0)
  switch (tt) {
    case 1: GU(1); break;
    case 2: GU(2); break;
    case 3: GU(3); break;
    default: GU(4); break;
  }
#undef GU
#undef GU_NS
  const unsigned g2 = static_cast<unsigned>((l.n_ch_pad / 64) * ((M + 15) / 16));
  switch (activation) {
    case FSI_ACT_SWIGLU: dec_act_kernel<ACT_SWIGLU, true><<<g2, 256, 0, st>>>(a); break;
    case FSI_ACT_SILU: dec_act_kernel<ACT_SILU, false><<<g2, 256, 0, st>>>(a); break;
    case FSI_ACT_GELU: dec_act_kernel<ACT_GELU, false><<<g2, 256, 0, st>>>(a); break;
    case FSI_ACT_RELU: dec_act_kernel<ACT_RELU, false><<<g2, 256, 0, st>>>(a); break;
    default: dec_act_kernel<ACT_RELU2, false><<<g2, 256, 0, st>>>(a); break;
  }
  const dim3 g3(static_cast<unsigned>((D + 16 * DT * NDG - 1) / (16 * DT * NDG)), static_cast<unsigned>(l.S2));
#define DN(TTV)                                                                   \
  do {                                                                            \
    if (l.NS2 == 8) dec_down_kernel<TTV, 8><<<g3, DN_THREADS, 0, st>>>(a);        \
    else dec_down_kernel<TTV, 4><<<g3, DN_THREADS, 0, st>>>(a);                   \
  } while (0)
  switch (tt) {
    case 1: DN(1); break;
    case 2: DN(2); break;
    case 3: DN(3); break;
    default: DN(4); break;
  }
#undef DN
  const unsigned g4 = static_cast<unsigned>(((D + 127) / 128) * ((M + 7) / 8));
  dec_reduce_kernel<<<g4, 256, 0, st>>>(a);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace fsi_dec
