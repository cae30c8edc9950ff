// Packed-weight decode path of the bf16 SwiGLU Pattention MLP (up to 64 tokens)
// for MI355X (gfx950).
//
//   out[M, D] = (silu(x K_gate[S]^T) * (x K_up[S]^T)) V[S]   (foveal_pattention.py:328-335)
//
// The weights are repacked once (fsi_pattention_pack) into the MFMA operand
// layout: every 16 x 32 bf16 operand tile of v_mfma_f32_16x16x32_bf16 is 1 KiB
// contiguous in lane order (lane l = 16 q + r holds row r, k = 8 q .. 8 q + 7),
// so each 16-byte-per-lane wave load is one contiguous KiB of HBM instead of 16
// row fragments of 64 B, 8 KiB apart.
//   gate / up : tile (ct, s) = rows 16 ct .. +16, k 32 s .. +32, at (ct S + s) KiB
//               (S = K / 32): a 16-channel tile's whole K is contiguous;
//   down      : tile (b, dt, cl) = channels b bn + 32 cl .. +32 of block b,
//               dims 16 dt .. +16, at ((b DT + dt) CB + cl) KiB (DT = D / 16,
//               CB = bn / 32): an active block's channels of one dim tile are
//               contiguous.
//
// Two kernels per step, no split-K partials (cross-workgroup sums in a kernel
// need device-scope stores and loads whose round trips cost as much as the
// launch boundary they would save):
//   1. ws_gateup_kernel: one workgroup per 16 active channels (256 at the 8B
//      shape, one per CU) over the full K.  Eight consumer waves take one
//      32-wide MFMA step each of every 256-wide K chunk, streaming their gate
//      and up tiles from HBM through a register ring; eight producer waves
//      stage the x chunks into LDS.  The consumers' partial sums are added
//      through LDS in wave order, SwiGLU is applied with the requested rounding
//      points and H goes out in the packed operand layout (tile (cs, t) =
//      channels 32 cs .., tokens 16 t .., at (cs TT + t) KiB).
//   2. ws_down_kernel: one workgroup per 16 output dims over all channels;
//      consumer w owns channel steps [w NS, (w + 1) NS) and streams their V
//      tiles, the producers stage the matching H tiles; partial sums are added
//      in wave order and rounded once to bf16.
// Every workgroup reads all of x (resp. H) once, 128 MiB of L2 reads per kernel
// at the 8B shape next to 64 (resp. 32) MiB of weights from HBM.
#include <algorithm>

#include "fsi_common.h"

using namespace fsi;

namespace fsi_gemm {
int gateup_swiglu_packed(const bf16_t* x, int64_t ldx, const bf16_t* kgp, const bf16_t* kup, int S, int N_p,
                         const int32_t* blocks, int n_active, int block_n, int M, int K, int rounding, bf16_t* H,
                         int64_t ldh, int* err, hipStream_t st);
int down_gather_packed(const bf16_t* H, int64_t ldh, const bf16_t* vp, int DT, int CB, int N_p,
                       const int32_t* blocks, int n_active, int block_n, int M, int D, bf16_t* out, int64_t ldo,
                       int* err, hipStream_t st);
}  // namespace fsi_gemm

namespace {

constexpr int PK_TILE = 512;  // bf16 elements of one 16 x 32 operand tile
constexpr int PK_WAVES = 8;   // consumer waves: K chunks and channel ranges split eight ways
constexpr int KC = PK_WAVES * 32;  // k of one gate/up chunk: one MFMA step per consumer

#define PK_SCHED_FENCE() __builtin_amdgcn_sched_barrier(0)

__device__ __forceinline__ u32x4_t ldg16(const bf16_t* p) { return *reinterpret_cast<const u32x4_t*>(p); }
// Weight tiles are read once per step: non-temporal loads keep them from displacing
// the shared x / H operand in L2 (a 64 MiB tile stream runs ~13% faster this way).
__device__ __forceinline__ u32x4_t ldnt16(const bf16_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
}

// ---------------------------------------------------------------------------
// Packing (once per weight version)
// ---------------------------------------------------------------------------
// W [rows, K] (row stride ld) -> tiles (ct, s); one thread per 16 bytes.
__global__ __launch_bounds__(256) void pack_rows_kernel(const bf16_t* __restrict__ w, int64_t ld, int64_t n_tiles,
                                                        int S, bf16_t* __restrict__ out) {
  const int64_t total = n_tiles * S * 64;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * 256) {
    const int l = static_cast<int>(i & 63);
    const int64_t ts = i >> 6;
    const int s = static_cast<int>(ts % S);
    const int64_t ct = ts / S;
    const int r = l & 15, q = l >> 4;
    *reinterpret_cast<u32x4_t*>(out + i * 8) = ldg16(w + (16 * ct + r) * ld + 32 * s + 8 * q);
  }
}

// V -> tiles (b, dt, cl).  VT: V stored as V^T [D, N_p] (row stride ldv, 8
// consecutive channels of one dim are one 16-byte load); otherwise V [N_p, D].
template <bool VT>
__global__ __launch_bounds__(256) void pack_down_kernel(const bf16_t* __restrict__ v, int64_t ldv, int n_blocks,
                                                        int DT, int CB, int bn, bf16_t* __restrict__ out) {
  const int64_t total = static_cast<int64_t>(n_blocks) * DT * CB * 64;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * 256) {
    const int l = static_cast<int>(i & 63);
    int64_t rest = i >> 6;
    const int cl = static_cast<int>(rest % CB);
    rest /= CB;
    const int dt = static_cast<int>(rest % DT);
    const int64_t b = rest / DT;
    const int r = l & 15, q = l >> 4;
    const int64_t c0 = b * bn + 32 * cl + 8 * q;
    const int64_t d = 16 * dt + r;
    u32x4_t val;
    if (VT) {
      val = ldg16(v + d * ldv + c0);
    } else {
      uint32_t w[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        w[e] = static_cast<uint32_t>(v[(c0 + 2 * e) * ldv + d]) |
               (static_cast<uint32_t>(v[(c0 + 2 * e + 1) * ldv + d]) << 16);
      val = u32x4_t{w[0], w[1], w[2], w[3]};
    }
    *reinterpret_cast<u32x4_t*>(out + i * 8) = val;
  }
}

struct PkArgs {
  const bf16_t* x;
  int64_t ldx;
  const bf16_t* pg;  // packed gate tiles
  const bf16_t* pu;  // packed up tiles
  const bf16_t* pd;  // packed down tiles
  const int32_t* active;
  int n_blocks;  // valid block ids are [0, n_blocks)
  int log2bn;
  int M, n_ch, S, DT, CB;
  int rounding;
  bf16_t* hp;  // packed H, n_ch_pad / 32 x TT tiles
  bf16_t* out;
  int64_t ldo;
  int* err;
};

// ---------------------------------------------------------------------------
// Warp-specialised kernels.  A wave's vector loads complete in issue order, so
// a wave that streams weights from HBM and also loads the shared operand (x or
// H, L2 hits) makes every L2 hit wait behind the HBM loads issued before it,
// and its register ring then holds both: the weight stream runs with fewer
// bytes in flight than it needs.  Here eight producer waves move the shared
// operand into a ring of LDS stages with direct-to-LDS loads
// (global_load_lds_dwordx4: lane l's 16 bytes land at M0 + 16 l) three steps
// ahead, and eight consumer waves hold only the weight ring in registers and
// read their MFMA fragments from LDS.  Producers wait with explicit vmcnt
// counts and every wave meets at a bare s_barrier per step.
// ---------------------------------------------------------------------------
constexpr int WS_CONS = PK_WAVES;
// Eight producers (16 waves, four per SIMD, at most 128 VGPRs each) measured ~0.7 %
// faster per decode step than four at the 8B shape; two were no slower than four.
constexpr int WS_PROD = 8;
constexpr int WS_THREADS = 64 * (WS_CONS + WS_PROD);
// Gate/up weight chunks each consumer keeps in flight.  At the 8B decode shape 4-6
// measured 1.5 % faster per step than 10: a deeper weight ring only crowds the x
// stream the producers need.
#ifndef FSI_WS_GU_RING
#define FSI_WS_GU_RING 5
#endif
#ifndef FSI_WS_DN_RING
#define FSI_WS_DN_RING 16
#endif
typedef __attribute__((address_space(3))) void ws_lds_t;
typedef __attribute__((address_space(1))) void ws_glb_t;

template <int N>
__device__ __forceinline__ void ws_wait_vmcnt() {
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}
// Wait until at most n direct loads of this wave are in flight (n is a
// compile-time constant after unrolling; a smaller threshold is always safe).
__device__ __forceinline__ void ws_wait_at_most(int n) {
  if (n >= 32) ws_wait_vmcnt<32>();
  else if (n >= 24) ws_wait_vmcnt<24>();
  else if (n >= 16) ws_wait_vmcnt<16>();
  else if (n >= 12) ws_wait_vmcnt<12>();
  else if (n >= 8) ws_wait_vmcnt<8>();
  else if (n >= 6) ws_wait_vmcnt<6>();
  else if (n >= 4) ws_wait_vmcnt<4>();
  else if (n >= 2) ws_wait_vmcnt<2>();
  else ws_wait_vmcnt<0>();
}
// Barrier without the fence of __syncthreads(), which would wait for every
// direct load in flight; the clobber keeps LDS accesses on their side of it.
__device__ __forceinline__ void ws_barrier() { asm volatile("s_barrier" ::: "memory"); }
__device__ __forceinline__ void ws_load_lds(const bf16_t* src, char* lds_wave_base) {
  __builtin_amdgcn_global_load_lds((ws_glb_t*)src, (ws_lds_t*)lds_wave_base, 16, 0, 0);
}

// 1''. gate/up + SwiGLU for one 16-channel tile, full K.  The x chunk of 256 k
//      is staged row-contiguously with the 16-byte columns of row r
//      XOR-swizzled by r % 16, so the 16 rows of a fragment read land on 16
//      different bank groups.
template <int TT, int NC>
__global__ __launch_bounds__(WS_THREADS) void ws_gateup_kernel(PkArgs a) {
  constexpr int ROWS = 16 * TT;
  constexpr int XST = ROWS * 512;  // bytes of one x chunk (ROWS rows x 256 k)
  constexpr int XI = ROWS / 2;     // 1 KiB loads per chunk (two rows each)
  constexpr int XIW = (XI + WS_PROD - 1) / WS_PROD;
  constexpr int AHEAD = NC < 3 ? NC : 3;
  constexpr int STAGES = AHEAD + 1;
  constexpr int P = NC < FSI_WS_GU_RING ? NC : FSI_WS_GU_RING;
  constexpr int RED = WS_CONS * 2 * TT * 1024;
  constexpr int LDS = STAGES * XST > RED + ROWS * 32 ? STAGES * XST : RED + ROWS * 32;
  __shared__ __attribute__((aligned(1024))) char lds[LDS];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int cta = blockIdx.x;
  const int c0 = 16 * cta;
  bf16_t* hdst = a.hp + static_cast<int64_t>(cta >> 1) * TT * PK_TILE;

  if (c0 >= a.n_ch) {  // padding tile: H = 0
    if (tid < ROWS * 2) {
      const int tok = tid >> 1, g8 = tid & 1;
      *reinterpret_cast<u32x4_t*>(hdst + (tok >> 4) * PK_TILE + (16 * (2 * (cta & 1) + g8) + (tok & 15)) * 8) =
          u32x4_t{0u, 0u, 0u, 0u};
    }
    return;
  }
  const int blk = a.active[c0 >> a.log2bn];
  const bool ok = blk >= 0 && blk < a.n_blocks;
  f32x4_t ag[TT], au[TT];
#pragma unroll
  for (int t = 0; t < TT; ++t) ag[t] = au[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  if (wave >= WS_CONS) {
    // ---- producers: x chunks into the LDS ring ----
    const int pw = wave - WS_CONS;
    const bf16_t* src[XIW];
    int dst[XIW];
#pragma unroll
    for (int i = 0; i < XIW; ++i) {
      const int inst = pw * XIW + i < XI ? pw * XIW + i : XI - 1;  // rows 2 inst, 2 inst + 1
      const int row = 2 * inst + (lane >> 5), slot = lane & 31;
      const int rr = row < a.M ? row : a.M - 1;
      src[i] = a.x + static_cast<int64_t>(rr) * a.ldx + 8 * (slot ^ (row & 15));
      dst[i] = inst * 1024;
    }
    auto issue = [&](int c) {
#pragma unroll
      for (int i = 0; i < XIW; ++i)
        if (pw * XIW + i < XI) ws_load_lds(src[i] + c * 256, lds + (c % STAGES) * XST + dst[i]);
    };
#pragma unroll
    for (int c = 0; c < AHEAD; ++c) issue(c);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int later = (c + AHEAD - 1 < NC - 1 ? c + AHEAD - 1 : NC - 1) - c;  // chunks issued after c
      ws_wait_at_most(later * XIW);
      ws_barrier();  // chunk c is in LDS
      if (c + AHEAD < NC) issue(c + AHEAD);
    }
  } else {
    // ---- consumers: gate/up tiles from HBM, x fragments from LDS ----
    const int64_t ct = ok ? (static_cast<int64_t>(blk) << (a.log2bn - 4)) + ((c0 & ((1 << a.log2bn) - 1)) >> 4) : 0;
    const bf16_t* gp = a.pg + (ct * a.S + wave) * PK_TILE + lane * 8;
    const bf16_t* up = a.pu + (ct * a.S + wave) * PK_TILE + lane * 8;
    u32x4_t rg[P], ru[P];
    auto issue = [&](int slot, int c) {
      rg[slot] = ldnt16(gp + c * PK_WAVES * PK_TILE);
      ru[slot] = ldnt16(up + c * PK_WAVES * PK_TILE);
    };
#pragma unroll
    for (int d = 0; d < P; ++d) issue(d, d);
    const int r = lane & 15, q = lane >> 4;
    const int xoff = r * 512 + (((4 * wave + q) ^ r) * 16);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      ws_barrier();
      const char* st = lds + (c % STAGES) * XST + xoff;
      u32x4_t xf[TT];
#pragma unroll
      for (int t = 0; t < TT; ++t) xf[t] = *reinterpret_cast<const u32x4_t*>(st + t * 16 * 512);
#pragma unroll
      for (int t = 0; t < TT; ++t) {
        ag[t] = mfma16x16x32(xf[t], rg[c % P], ag[t]);
        au[t] = mfma16x16x32(xf[t], ru[c % P], au[t]);
      }
      if (c + P < NC) issue(c % P, c + P);
      PK_SCHED_FENCE();
    }
  }

  // ---- sum the consumers' partials in wave order, SwiGLU, packed H store ----
  __syncthreads();
  float* red = reinterpret_cast<float*>(lds);  // [wave][g/u][t][j][lane]
  if (wave < WS_CONS) {
#pragma unroll
    for (int t = 0; t < TT; ++t)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        red[((wave * 2 + 0) * TT + t) * 256 + j * 64 + lane] = ag[t][j];
        red[((wave * 2 + 1) * TT + t) * 256 + j * 64 + lane] = au[t][j];
      }
  }
  __syncthreads();
  bf16_t* hb = reinterpret_cast<bf16_t*>(lds + RED);
  // element (t, j, ln) of the accumulators: token 16 t + 4 (ln / 16) + j, channel ln % 16;
  // consecutive threads take consecutive ln, so each of the 16 partial reads is one
  // conflict-free 256-byte row (an element order by token put 4 lanes on each bank)
  for (int e = tid; e < ROWS * 16; e += WS_THREADS) {
    const int ln = e & 63, tj = e >> 6, t = tj >> 2, j = tj & 3;
    const int tok = 16 * t + 4 * (ln >> 4) + j, ch = ln & 15;
    float g = 0.f, u = 0.f;
#pragma unroll
    for (int w = 0; w < WS_CONS; ++w) {
      g += red[((w * 2 + 0) * TT + t) * 256 + j * 64 + ln];
      u += red[((w * 2 + 1) * TT + t) * 256 + j * 64 + ln];
    }
    hb[tok * 16 + ch] = f32_to_bf16(ok && tok < a.M ? pattention_act<ACT_SWIGLU>(g, u, a.rounding) : 0.f);
  }
  if (!ok && tid == 0) set_error(a.err, FSI_ERR_INDEX_RANGE);
  __syncthreads();
  if (tid < ROWS * 2) {
    const int tok = tid >> 1, g8 = tid & 1;
    *reinterpret_cast<u32x4_t*>(hdst + (tok >> 4) * PK_TILE + (16 * (2 * (cta & 1) + g8) + (tok & 15)) * 8) =
        *reinterpret_cast<const u32x4_t*>(hb + tok * 16 + g8 * 8);
  }
}

// 2''. down projection for 16 output dims, full channel range: consumer w owns
//      channel steps [w NS, (w + 1) NS); per step the producers move the eight
//      consumers' H tiles (TT KiB each) into an LDS stage.
template <int TT, int NS>
__global__ __launch_bounds__(WS_THREADS) void ws_down_kernel(PkArgs a) {
  constexpr int ROWS = 16 * TT;
  constexpr int HST = WS_CONS * TT * 1024;  // bytes of one stage
  constexpr int HI = WS_CONS * TT;          // 1 KiB loads per step
  constexpr int HIW = HI / WS_PROD;
  static_assert(HI % WS_PROD == 0, "H loads must split over the producers");
  constexpr int AHEAD = NS < 3 ? NS : 3;
  constexpr int STAGES = AHEAD + 1;
  constexpr int R = NS < FSI_WS_DN_RING ? NS : FSI_WS_DN_RING;
  constexpr int RED = WS_CONS * TT * 1024;
  constexpr int LDS = STAGES * HST > RED ? STAGES * HST : RED;
  __shared__ __attribute__((aligned(1024))) char lds[LDS];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int dt = blockIdx.x;
  f32x4_t acc[TT];
#pragma unroll
  for (int t = 0; t < TT; ++t) acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  bool bad = false;

  if (wave >= WS_CONS) {
    // ---- producers: H tiles (cs = w NS + j, t) of step j into stage j % STAGES ----
    const int pw = wave - WS_CONS;
    const bf16_t* src[HIW];
    int dst[HIW];
#pragma unroll
    for (int i = 0; i < HIW; ++i) {
      const int inst = pw * HIW + i;  // (consumer w, token tile t)
      const int w = inst / TT, t = inst % TT;
      src[i] = a.hp + (static_cast<int64_t>(w * NS) * TT + t) * PK_TILE + lane * 8;
      dst[i] = inst * 1024;
    }
    auto issue = [&](int j) {
#pragma unroll
      for (int i = 0; i < HIW; ++i) ws_load_lds(src[i] + j * TT * PK_TILE, lds + (j % STAGES) * HST + dst[i]);
    };
#pragma unroll
    for (int j = 0; j < AHEAD; ++j) issue(j);
#pragma unroll
    for (int j = 0; j < NS; ++j) {
      const int later = (j + AHEAD - 1 < NS - 1 ? j + AHEAD - 1 : NS - 1) - j;
      ws_wait_at_most(later * HIW);
      ws_barrier();
      if (j + AHEAD < NS) issue(j + AHEAD);
    }
  } else {
    // ---- consumers: V tiles from HBM, H fragments from LDS ----
    const int cs0 = wave * NS;
    int tile[NS];
#pragma unroll
    for (int j = 0; j < NS; ++j) {
      const int c = 32 * (cs0 + j);
      const int cc = c < a.n_ch ? c : 32 * cs0 < a.n_ch ? 32 * cs0 : 0;
      const int blk = a.active[cc >> a.log2bn];
      const bool ok = blk >= 0 && blk < a.n_blocks;
      bad |= c < a.n_ch && !ok;
      tile[j] = ok ? (blk * a.DT + dt) * a.CB + ((cc & ((1 << a.log2bn) - 1)) >> 5) : dt * a.CB;
    }
    const bf16_t* vbase = a.pd + lane * 8;
    u32x4_t rv[R];
    auto issue = [&](int slot, int j) { rv[slot] = ldnt16(vbase + static_cast<int64_t>(tile[j]) * PK_TILE); };
#pragma unroll
    for (int d = 0; d < R; ++d) issue(d, d);
    const int hoff = wave * TT * 1024 + lane * 16;
#pragma unroll
    for (int j = 0; j < NS; ++j) {
      ws_barrier();
      const char* st = lds + (j % STAGES) * HST + hoff;
      u32x4_t hf[TT];
#pragma unroll
      for (int t = 0; t < TT; ++t) hf[t] = *reinterpret_cast<const u32x4_t*>(st + t * 1024);
#pragma unroll
      for (int t = 0; t < TT; ++t) acc[t] = mfma16x16x32(hf[t], rv[j % R], acc[t]);
      if (j + R < NS) issue(j % R, j + R);
      PK_SCHED_FENCE();
    }
  }
  if (bad && lane == 0) set_error(a.err, FSI_ERR_INDEX_RANGE);

  __syncthreads();
  float* red = reinterpret_cast<float*>(lds);
  if (wave < WS_CONS) {
#pragma unroll
    for (int t = 0; t < TT; ++t)
#pragma unroll
      for (int j = 0; j < 4; ++j) red[(wave * TT + t) * 256 + j * 64 + lane] = acc[t][j];
  }
  __syncthreads();
  for (int e = tid; e < ROWS * 16; e += WS_THREADS) {  // element order as in ws_gateup_kernel
    const int ln = e & 63, tj = e >> 6, t = tj >> 2, j = tj & 3;
    const int tok = 16 * t + 4 * (ln >> 4) + j, d = ln & 15;
    float y = 0.f;
#pragma unroll
    for (int w = 0; w < WS_CONS; ++w) y += red[(w * TT + t) * 256 + j * 64 + ln];
    if (tok < a.M) a.out[static_cast<int64_t>(tok) * a.ldo + 16 * dt + d] = f32_to_bf16(y);
  }
}

__global__ __launch_bounds__(256) void pk_iota_kernel(int32_t* p, int n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = i;
}

// Steps per down wave: the fewest of {4, 8, 16, 32} covering n_ch channels
// with 8 waves of 32-channel steps; 0 when n_ch is too large.
int down_steps(int64_t n_ch) {
  for (int ns : {4, 8, 16, 32})
    if (n_ch <= int64_t(PK_WAVES) * 32 * ns) return ns;
  return 0;
}

struct PkLayout {
  size_t gate, up, down, total;
};

PkLayout pk_layout(int64_t N_p, int64_t K, int64_t D) {
  PkLayout l{};
  const size_t mat = fsi_host::align_up(sizeof(bf16_t) * static_cast<size_t>(N_p) * static_cast<size_t>(K), 256);
  l.gate = 0;
  l.up = mat;
  l.down = 2 * mat;
  l.total = 2 * mat + fsi_host::align_up(sizeof(bf16_t) * static_cast<size_t>(N_p) * static_cast<size_t>(D), 256);
  return l;
}

// Prefill (M >= PK_PREFILL_MIN_M tokens) runs the two 256 x 256 direct-to-LDS GEMMs
// over the packed tiles with a row-major H [M, n_ch] in the workspace.
constexpr int64_t PK_PREFILL_MIN_M = 256;
constexpr int64_t PK_PREFILL_MAX_BLOCKS = 2048;

size_t pk_prefill_workspace(int64_t M, int64_t n_ch, int64_t n_blocks) {
  return FSI_WORKSPACE_COUNTER_BYTES + fsi_host::align_up(sizeof(bf16_t) * static_cast<size_t>(M) * n_ch, 256) +
         fsi_host::align_up(sizeof(int32_t) * static_cast<size_t>(n_blocks + 1), 256);
}

size_t pk_workspace(int64_t n_ch, int64_t n_blocks) {
  const int ns = down_steps(n_ch);
  const int64_t n_ch_pad = int64_t(PK_WAVES) * 32 * (ns ? ns : 32);
  return FSI_WORKSPACE_COUNTER_BYTES + fsi_host::align_up(sizeof(bf16_t) * 64 * static_cast<size_t>(n_ch_pad), 256) +
         fsi_host::align_up(sizeof(int32_t) * static_cast<size_t>(n_blocks + 1), 256);
}

}  // namespace

extern "C" {

size_t fsi_pattention_packed_size(int64_t N_p, int64_t K, int64_t D_out) {
  if (N_p <= 0 || K <= 0 || D_out <= 0) return 0;
  return pk_layout(N_p, K, D_out).total;
}

int fsi_pattention_pack(const void* k_gate, const void* k_up, int64_t ldk, const void* v, int64_t ldv,
                        int v_transposed, int64_t N_p, int64_t K, int64_t D_out, int64_t block_n, int dtype,
                        void* packed, size_t packed_bytes, void* stream) {
  using namespace fsi_host;
  FSI_CHECK_ARG(dtype == FSI_DTYPE_BF16, FSI_ERR_DTYPE, "pattention_pack: dtype %d (bf16 only)", dtype);
  FSI_CHECK_ARG(k_gate && k_up && v && packed, FSI_ERR_INVALID_ARG, "pattention_pack: null pointer");
  FSI_CHECK_ARG(is_pow2(block_n) && block_n >= 32 && N_p > 0 && N_p % block_n == 0 && K > 0 && K % 32 == 0 &&
                    D_out > 0 && D_out % 16 == 0,
                FSI_ERR_SHAPE,
                "pattention_pack: N_p=%lld K=%lld D_out=%lld block_n=%lld (block_n a power of two >= 32 dividing "
                "N_p, K %% 32 == 0, D_out %% 16 == 0)",
                (long long)N_p, (long long)K, (long long)D_out, (long long)block_n);
  FSI_CHECK_ARG(ldk >= K && ldk % 8 == 0 && (v_transposed ? ldv >= N_p && ldv % 8 == 0 : ldv >= D_out),
                FSI_ERR_ALIGN, "pattention_pack: leading dimensions");
  FSI_CHECK_ARG(reinterpret_cast<uintptr_t>(k_gate) % 16 == 0 && reinterpret_cast<uintptr_t>(k_up) % 16 == 0 &&
                    (!v_transposed || reinterpret_cast<uintptr_t>(v) % 16 == 0) &&
                    reinterpret_cast<uintptr_t>(packed) % 256 == 0,
                FSI_ERR_ALIGN, "pattention_pack: misaligned pointer");
  const PkLayout l = pk_layout(N_p, K, D_out);
  FSI_CHECK_ARG(packed_bytes >= l.total, FSI_ERR_WORKSPACE, "pattention_pack: buffer %zu < %zu", packed_bytes,
                l.total);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  char* base = static_cast<char*>(packed);
  const int S = static_cast<int>(K / 32);
  const int64_t n16 = N_p / 16;
  const unsigned g1 = static_cast<unsigned>(std::min<int64_t>((n16 * S * 64 + 255) / 256, 1 << 20));
  pack_rows_kernel<<<g1, 256, 0, st>>>(static_cast<const bf16_t*>(k_gate), ldk, n16, S,
                                       reinterpret_cast<bf16_t*>(base + l.gate));
  pack_rows_kernel<<<g1, 256, 0, st>>>(static_cast<const bf16_t*>(k_up), ldk, n16, S,
                                       reinterpret_cast<bf16_t*>(base + l.up));
  const int nb = static_cast<int>(N_p / block_n), DT = static_cast<int>(D_out / 16), CB = static_cast<int>(block_n / 32);
  const unsigned g2 = static_cast<unsigned>(std::min<int64_t>((int64_t(nb) * DT * CB * 64 + 255) / 256, 1 << 20));
  if (v_transposed)
    pack_down_kernel<true><<<g2, 256, 0, st>>>(static_cast<const bf16_t*>(v), ldv, nb, DT, CB, (int)block_n,
                                               reinterpret_cast<bf16_t*>(base + l.down));
  else
    pack_down_kernel<false><<<g2, 256, 0, st>>>(static_cast<const bf16_t*>(v), ldv, nb, DT, CB, (int)block_n,
                                                reinterpret_cast<bf16_t*>(base + l.down));
  FSI_HIP_LAUNCH_CHECK("pattention_pack");
  return FSI_OK;
}

size_t fsi_pattention_packed_workspace_size(int64_t M, int64_t K, int64_t D_out, int64_t n_channels,
                                            int64_t block_n) {
  if (M <= 0 || K <= 0 || D_out <= 0 || n_channels <= 0 || block_n <= 0) return FSI_WORKSPACE_COUNTER_BYTES;
  const int64_t nb = (n_channels + block_n - 1) / block_n;
  if (M >= PK_PREFILL_MIN_M) return pk_prefill_workspace(M, n_channels, nb);
  return pk_workspace(n_channels, nb);
}

int fsi_pattention_fwd_packed(const void* x, int64_t ldx, const void* packed, const int32_t* active_blocks,
                              int64_t n_active, int64_t block_n, int64_t M, int64_t K, int64_t N_p, int64_t D_out,
                              int dtype, int rounding, void* out, int64_t ldo, void* workspace,
                              size_t workspace_bytes, int* err, void* stream) {
  using namespace fsi_host;
  FSI_CHECK_ARG(dtype == FSI_DTYPE_BF16, FSI_ERR_DTYPE, "pattention_packed: dtype %d (bf16 only)", dtype);
  FSI_CHECK_ARG(rounding >= FSI_ROUND_EAGER && rounding <= FSI_ROUND_FP32, FSI_ERR_INVALID_ARG,
                "pattention_packed: rounding mode %d", rounding);
  FSI_CHECK_ARG(x && packed && out, FSI_ERR_INVALID_ARG, "pattention_packed: null pointer");
  FSI_CHECK_ARG(active_blocks != nullptr || n_active == 0, FSI_ERR_INVALID_ARG,
                "pattention_packed: n_active > 0 with null active_blocks");
  FSI_CHECK_ARG((M >= 1 && M <= 64) || M >= PK_PREFILL_MIN_M, FSI_ERR_SHAPE,
                "pattention_packed: M=%lld (1..64 tokens, or >= %lld)", (long long)M, (long long)PK_PREFILL_MIN_M);
  FSI_CHECK_ARG(M <= 0x7fffffff, FSI_ERR_SHAPE, "pattention_packed: M beyond int32");
  const int64_t nc = K / KC;
  FSI_CHECK_ARG(K % KC == 0 && (nc == 1 || nc == 2 || nc == 4 || nc == 8 || nc == 16 || nc == 32), FSI_ERR_SHAPE,
                "pattention_packed: K=%lld (256 x 1, 2, 4, ..., 32)", (long long)K);
  FSI_CHECK_ARG(is_pow2(block_n) && block_n >= 32 && N_p > 0 && N_p % block_n == 0 && D_out > 0 &&
                    D_out % 16 == 0 && D_out / 16 <= (1 << 30),
                FSI_ERR_SHAPE, "pattention_packed: N_p=%lld D_out=%lld block_n=%lld", (long long)N_p,
                (long long)D_out, (long long)block_n);
  const int64_t n_ch = active_blocks ? n_active * block_n : N_p;
  FSI_CHECK_ARG(n_active >= 0 && n_ch >= 1, FSI_ERR_SHAPE, "pattention_packed: no active channel");
  const bool prefill = M >= PK_PREFILL_MIN_M;
  const int ns = down_steps(n_ch);
  FSI_CHECK_ARG(prefill || ns > 0, FSI_ERR_SHAPE, "pattention_packed: %lld active channels (at most %d)",
                (long long)n_ch, PK_WAVES * 32 * 32);
  FSI_CHECK_ARG(ldx >= K && ldx % 8 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0 && ldo >= D_out,
                FSI_ERR_ALIGN, "pattention_packed: x must be 16-byte aligned with ldx %% 8 == 0");
  FSI_CHECK_ARG(reinterpret_cast<uintptr_t>(packed) % 256 == 0 && reinterpret_cast<uintptr_t>(out) % 2 == 0,
                FSI_ERR_ALIGN, "pattention_packed: misaligned pointer");
  FSI_CHECK_ARG(static_cast<uint64_t>(N_p) * static_cast<uint64_t>(D_out) / PK_TILE < (uint64_t(1) << 31),
                FSI_ERR_SHAPE, "pattention_packed: V too large");
  const int64_t n_blocks = N_p / block_n;
  const int64_t n_list = active_blocks ? n_active : n_blocks;
  FSI_CHECK_ARG(!prefill || n_list <= PK_PREFILL_MAX_BLOCKS, FSI_ERR_CAPACITY,
                "pattention_packed: %lld blocks (prefill: at most %lld)", (long long)n_list,
                (long long)PK_PREFILL_MAX_BLOCKS);
  const size_t need = prefill ? pk_prefill_workspace(M, n_ch, n_list) : pk_workspace(n_ch, n_list);
  FSI_CHECK_ARG(workspace && workspace_bytes >= need && reinterpret_cast<uintptr_t>(workspace) % 256 == 0,
                FSI_ERR_WORKSPACE, "pattention_packed: workspace %zu < %zu (or misaligned)", workspace_bytes, need);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const PkLayout l = pk_layout(N_p, K, D_out);
  if (prefill) {
    char* ws = static_cast<char*>(workspace);
    bf16_t* h = reinterpret_cast<bf16_t*>(ws + FSI_WORKSPACE_COUNTER_BYTES);
    int32_t* ids = reinterpret_cast<int32_t*>(ws + FSI_WORKSPACE_COUNTER_BYTES +
                                              align_up(sizeof(bf16_t) * static_cast<size_t>(M) * n_ch, 256));
    if (active_blocks == nullptr) {
      pk_iota_kernel<<<static_cast<unsigned>((n_blocks + 255) / 256), 256, 0, st>>>(ids, static_cast<int>(n_blocks));
      active_blocks = ids;
    }
    const char* pbase = static_cast<const char*>(packed);
    const bf16_t* pg = reinterpret_cast<const bf16_t*>(pbase + l.gate);
    const bf16_t* pu = reinterpret_cast<const bf16_t*>(pbase + l.up);
    const bf16_t* pd = reinterpret_cast<const bf16_t*>(pbase + l.down);
    if (fsi_gemm::gateup_swiglu_packed(static_cast<const bf16_t*>(x), ldx, pg, pu, static_cast<int>(K / 32),
                                       static_cast<int>(N_p), active_blocks, static_cast<int>(n_list),
                                       static_cast<int>(block_n), static_cast<int>(M), static_cast<int>(K), rounding,
                                       h, n_ch, err, st) != 0 ||
        fsi_gemm::down_gather_packed(h, n_ch, pd, static_cast<int>(D_out / 16), static_cast<int>(block_n / 32),
                                     static_cast<int>(N_p), active_blocks, static_cast<int>(n_list),
                                     static_cast<int>(block_n), static_cast<int>(M), static_cast<int>(D_out),
                                     static_cast<bf16_t*>(out), ldo, err, st) != 0) {
      set_last_error("pattention_packed: prefill GEMM launch failed: %s", hipGetErrorString(hipGetLastError()));
      return FSI_ERR_HIP;
    }
    return FSI_OK;
  }
  const int64_t n_ch_pad = int64_t(PK_WAVES) * 32 * ns;
  char* ws = static_cast<char*>(workspace);
  bf16_t* hp = reinterpret_cast<bf16_t*>(ws + FSI_WORKSPACE_COUNTER_BYTES);
  int32_t* ids = reinterpret_cast<int32_t*>(ws + FSI_WORKSPACE_COUNTER_BYTES +
                                            align_up(sizeof(bf16_t) * 64 * static_cast<size_t>(n_ch_pad), 256));
  const char* pbase = static_cast<const char*>(packed);
  PkArgs a{};
  a.x = static_cast<const bf16_t*>(x);
  a.ldx = ldx;
  a.pg = reinterpret_cast<const bf16_t*>(pbase + l.gate);
  a.pu = reinterpret_cast<const bf16_t*>(pbase + l.up);
  a.pd = reinterpret_cast<const bf16_t*>(pbase + l.down);
  if (active_blocks == nullptr) {
    pk_iota_kernel<<<static_cast<unsigned>((n_blocks + 255) / 256), 256, 0, st>>>(ids, static_cast<int>(n_blocks));
    active_blocks = ids;
  }
  a.active = active_blocks;
  a.n_blocks = static_cast<int>(n_blocks);
  a.log2bn = ilog2(block_n);
  a.M = static_cast<int>(M);
  a.n_ch = static_cast<int>(n_ch);
  a.S = static_cast<int>(K / 32);
  a.DT = static_cast<int>(D_out / 16);
  a.CB = static_cast<int>(block_n / 32);
  a.rounding = rounding;
  a.hp = hp;
  a.out = static_cast<bf16_t*>(out);
  a.ldo = ldo;
  a.err = err;
  const int tt = static_cast<int>((M + 15) / 16);
  const unsigned g1 = static_cast<unsigned>(n_ch_pad / 16);
  const unsigned g2 = static_cast<unsigned>(D_out / 16);
  {
    auto launch_ws = [&](auto tt_tag) {
      constexpr int TT = decltype(tt_tag)::value;
      switch (nc) {
        case 1: ws_gateup_kernel<TT, 1><<<g1, WS_THREADS, 0, st>>>(a); break;
        case 2: ws_gateup_kernel<TT, 2><<<g1, WS_THREADS, 0, st>>>(a); break;
        case 4: ws_gateup_kernel<TT, 4><<<g1, WS_THREADS, 0, st>>>(a); break;
        case 8: ws_gateup_kernel<TT, 8><<<g1, WS_THREADS, 0, st>>>(a); break;
        case 16: ws_gateup_kernel<TT, 16><<<g1, WS_THREADS, 0, st>>>(a); break;
        default: ws_gateup_kernel<TT, 32><<<g1, WS_THREADS, 0, st>>>(a); break;
      }
      switch (ns) {
        case 4: ws_down_kernel<TT, 4><<<g2, WS_THREADS, 0, st>>>(a); break;
        case 8: ws_down_kernel<TT, 8><<<g2, WS_THREADS, 0, st>>>(a); break;
        case 16: ws_down_kernel<TT, 16><<<g2, WS_THREADS, 0, st>>>(a); break;
        default: ws_down_kernel<TT, 32><<<g2, WS_THREADS, 0, st>>>(a); break;
      }
    };
    switch (tt) {
      case 1: launch_ws(std::integral_constant<int, 1>{}); break;
      case 2: launch_ws(std::integral_constant<int, 2>{}); break;
      case 3: launch_ws(std::integral_constant<int, 3>{}); break;
      default: launch_ws(std::integral_constant<int, 4>{}); break;
    }
    FSI_HIP_LAUNCH_CHECK("pattention_packed");
    return FSI_OK;
  }
}

}  // extern "C"
