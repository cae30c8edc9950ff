// 2-D tile-sparse bf16 GEMM for MI355X (gfx950): fsi_blockwise_matmul
// (BlockwiseMatMul2D, foveal_indexer/block_matmul.py:335-392).
//
// C[M, N] = A[M, K] (B o T)^T with B [N, K] K-contiguous (the F.linear layout)
// and T the expansion of a (block_k x block_n) tile mask, one mask per group of
// rows_per_group rows.  One workgroup (4 waves, 2 x 2 of 64 x 64) owns one
// 128 x 128 output tile, which lies in one row group:
//   * prologue: the workgroup reads its group's mask column(s) for its n
//     block(s) and compacts the active k blocks, in ascending order, into an
//     LDS list (ballot + prefix over 64-block chunks) -- no list-building
//     launches;
//   * main loop: 32-wide K-steps over the active blocks only, operands going
//     global -> LDS with global_load_lds_dwordx4 into a ring of STAGES stages
//     (16 KiB each), so STAGES - 1 steps are in flight without staging
//     registers; the fragments of step s + 1 are read while step s's MFMAs run;
//   * tile order: the hardware deals workgroup b to XCD b % 8, so consecutive
//     logical tiles are given to one XCD, and logical tiles walk bands of
//     GROUP_M m tiles across N (GROUP_M = 1: all n tiles of one m tile, i.e.
//     of one row group, before the next).  The tiles an XCD runs at once then
//     share their group's X tiles in that XCD's L2, and the eight XCDs walk the
//     n tiles in step, so a W tile several groups use is fetched while the
//     other XCDs' copies are still in the last-level cache.  Bands of several m
//     tiles (W shared in L2 as well) measured slower: tiles with different
//     k-block lists drift apart and the shared W tiles are evicted between uses.
//   * load balance: a tile's time grows with its number of active k blocks,
//     and the hardware hands tiles to free workgroup slots in dispatch order,
//     so a grid of several rounds ends with the slots that drew the heaviest
//     late tiles.  Given a workspace, a pre-pass (tile_order_kernel, one
//     workgroup per band) counts the active k blocks of the band's tiles and
//     writes them heaviest first (a counting sort); each band's positions keep
//     their place in the walk above, so the last tiles an XCD runs are the
//     lightest of its last band.  A global heaviest-first order mixed all
//     groups on every XCD and ran 1.6x slower: X tiles stop being shared.
// When block_n < 128 a tile spans several n blocks whose masks differ; the list
// then holds every k block at which any of them is active, with the per-n-block
// bits beside it, and a B fragment (16 columns, inside one n block) of an
// inactive n block is zeroed in registers before its MFMAs.
#include "fsi_common.h"

using namespace fsi;

namespace fsi_bs_generic {  // csrc/bsgemm_generic.hip: fp32 and the tilings this kernel does not take
int tile_gemm(const void* x, int64_t ldx, const void* w, int64_t ldw, const void* bias, const uint8_t* mask,
              int64_t groups, int64_t rows_per_group, int64_t block_k, int64_t block_n, int64_t M, int64_t N,
              int64_t K, int dtype, void* out, int64_t ldo, hipStream_t st);
}  // namespace fsi_bs_generic

namespace {

constexpr int TT = 128;       // output tile edge
constexpr int KS = 32;        // K-step
#ifndef FSI_TG_WAVES
#define FSI_TG_WAVES 4
#endif
constexpr int NW = FSI_TG_WAVES;  // waves per workgroup: 2 along M x NW / 2 along N
static_assert(NW == 4 || NW == 8, "wave layouts");
constexpr int NTHREADS = 64 * NW;
constexpr int AF = 8 / NW;         // A (and B) 16-row fragments each wave loads per K-step
constexpr int WNW = NW / 2;        // waves along N
constexpr int WCOLS = TT / WNW;    // output columns of a wave
constexpr int FB = WCOLS / 16;     // B fragments a wave multiplies (A: 4)
#ifndef FSI_TG_STAGES
#define FSI_TG_STAGES 4
#endif
constexpr int STAGES = FSI_TG_STAGES;
static_assert(STAGES >= 3 && STAGES <= 8, "pipeline depth");
#ifndef FSI_TG_WG_PER_CU
#define FSI_TG_WG_PER_CU (FSI_TG_STAGES <= 4 ? 2 : 1)
#endif
constexpr int WG_PER_CU = FSI_TG_WG_PER_CU;
#ifndef FSI_TG_GROUP_M
#define FSI_TG_GROUP_M 1
#endif
constexpr int GROUP_M = FSI_TG_GROUP_M;
#ifndef FSI_TG_PREFETCH
#define FSI_TG_PREFETCH 1
#endif
#ifndef FSI_TG_LIST_MAX
#define FSI_TG_LIST_MAX 2048
#endif
constexpr int LIST_MAX = FSI_TG_LIST_MAX;  // k blocks per tile (K / block_k)
constexpr int LOADS = 2 * AF;       // global_load_lds per wave and step: AF A + AF B fragments of 1 KiB
constexpr int FRAG_ELEMS = 16 * KS;  // one 16-row fragment of a stage

struct TileArgs {
  const void* A;  // bf16 or fp32 (the kernel's element type)
  const void* B;
  void* C;
  const void* bias;  // optional, block_k == K only: added on the columns of active n blocks
  int64_t lda, ldb, ldc;
  int M, N, K;
  const uint8_t* mask;  // [groups][nkb * nnb], tile id k_b * nnb + n_b
  int groups, rows_per_group, nkb, nnb, block_k, block_n;
  int m_tiles, n_tiles;
  const int32_t* order;  // tile ids heaviest first (tile_order_kernel), or null: dispatch order
};

typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void glb_void_t;

// 16-byte chunk slot of row r in a 64-byte LDS row: rows r and r + 1 differ in
// their 64-byte half, and row bits 1-2 spread the eight rows a 128-bit fragment
// read serves at once over the four slots (no bank conflicts).
__device__ __forceinline__ int chunk_swz(int r) { return (r >> 1) & 3; }

// s_waitcnt vmcnt(N) leaving expcnt and lgkmcnt alone (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Waits until at most `steps` K-steps of direct-to-LDS loads are in flight.
__device__ __forceinline__ void wait_steps(int steps) {
  switch (steps) {
    case 0: wait_vmcnt<0>(); break;
    case 1: wait_vmcnt<LOADS>(); break;
    case 2: wait_vmcnt<2 * LOADS>(); break;
    case 3: wait_vmcnt<3 * LOADS>(); break;
    case 4: wait_vmcnt<4 * LOADS>(); break;
    default: wait_vmcnt<5 * LOADS>(); break;
  }
}

// Workgroup barrier without the release fence of __syncthreads(), which would
// wait for every direct-to-LDS load in flight; the caller has waited for the
// loads the next step reads.
__device__ __forceinline__ void stage_barrier() { asm volatile("s_barrier" ::: "memory"); }

__device__ __forceinline__ uint32_t cvt_pk_bf16(float a, float b) {
  typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2_t;
  const bf16x2_t v = {static_cast<__bf16>(a), static_cast<__bf16>(b)};
  return __builtin_bit_cast(uint32_t, v);
}

// Workgroup b runs on XCD b % 8: logical ids [x q', (x + 1) q') go to XCD x in
// dispatch order (q' = the number of workgroups that XCD receives).
__device__ __forceinline__ int xcd_contiguous(int b, int n) {
  const int x = b & 7, q = n >> 3, r = n & 7;
  return (x < r ? x * (q + 1) : r * (q + 1) + (x - r) * q) + (b >> 3);
}

// Logical tile lid -> (m tile, n tile): bands of GROUP_M m tiles walked across N.
__device__ __forceinline__ void tile_coords(const TileArgs& g, int lid, int& mt, int& nt) {
  const int per_band = GROUP_M * g.n_tiles;
  const int band = lid / per_band, within = lid - band * per_band;
  const int mfirst = band * GROUP_M;
  const int bh = g.m_tiles - mfirst < GROUP_M ? g.m_tiles - mfirst : GROUP_M;
  mt = mfirst + within % bh;
  nt = within / bh;
}

// Active k blocks in [kb0, kb0 + ORDER_KB_CHUNK) of tile (mt, nt): those at which
// any of its n blocks is active (the tile's share of the list the GEMM prologue
// builds).  The chunk's loads are independent and issued together.
constexpr int ORDER_KB_CHUNK = 16;
__device__ int tile_kcount_chunk(const TileArgs& g, int mt, int nt, int kb0) {
  int grp = mt * TT / g.rows_per_group;
  grp = grp < g.groups ? grp : g.groups - 1;
  const int nsub = g.block_n < TT ? TT / g.block_n : 1;
  const int nb0 = nt * TT / g.block_n;
  const int cnt = (nb0 + nsub < g.nnb ? nb0 + nsub : g.nnb) - nb0;  // 1 .. TT / 16 (block_n >= 16)
  const uint8_t* col = g.mask + static_cast<int64_t>(grp) * g.nkb * g.nnb + nb0;
  // branch-free: rows past nkb re-read the last row and are not counted, so the
  // chunk's loads issue together
  uint32_t any[ORDER_KB_CHUNK];
#pragma unroll
  for (int k = 0; k < ORDER_KB_CHUNK; ++k) {
    const int kb = kb0 + k < g.nkb ? kb0 + k : g.nkb - 1;
    any[k] = col[static_cast<int64_t>(kb) * g.nnb];
  }
  if (cnt > 1) {
#pragma unroll
    for (int k = 0; k < ORDER_KB_CHUNK; ++k) {
      const int kb = kb0 + k < g.nkb ? kb0 + k : g.nkb - 1;
      const uint8_t* row = col + static_cast<int64_t>(kb) * g.nnb;
      for (int j = 1; j < cnt; ++j) any[k] |= row[j];
    }
  }
  int n = 0;
#pragma unroll
  for (int k = 0; k < ORDER_KB_CHUNK; ++k) n += (kb0 + k < g.nkb) & (any[k] != 0u);
  return n;
}

constexpr int ORDER_THREADS = 256;
constexpr int64_t ORDER_MIN_TILES = 512;           // at most one round of workgroup slots: nothing to balance
constexpr int64_t ORDER_MAX_MASK_READS = 1 << 22;  // mask bytes one pre-pass workgroup may read
constexpr int ORDER_MAX_BAND = 4096;               // tiles of one band (counts held in LDS)
constexpr int ORDER_OWN = (LIST_MAX + 1 + ORDER_THREADS - 1) / ORDER_THREADS;

// Workgroup b sorts band b (GROUP_M m tiles x all n tiles, logical positions
// [b GROUP_M n_tiles, ...)) by active k-block count, largest first: order[p] is
// the logical tile run at position p.  Positions keep their band, so the
// tiles an XCD runs at once still share their group's X tiles in its L2; only
// the order inside a band changes.  Counting sort; ties in any order (every
// tile's result is independent of the workgroup that computes it).
__global__ __launch_bounds__(ORDER_THREADS) void tile_order_kernel(TileArgs g, int32_t* __restrict__ order) {
  __shared__ int32_t start[LIST_MAX + 1];  // tiles per bin, then the next position of each bin
  __shared__ int32_t kcs[ORDER_MAX_BAND];  // active k blocks per tile of the band
  __shared__ int32_t wave_sum[ORDER_THREADS / 64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int per_band = GROUP_M * g.n_tiles;
  const int first = blockIdx.x * per_band;
  const int mfirst = blockIdx.x * GROUP_M;
  const int count = (g.m_tiles - mfirst < GROUP_M ? g.m_tiles - mfirst : GROUP_M) * g.n_tiles;
  const int nbins = g.nkb + 1;  // bin p holds count nkb - p (descending)
  for (int i = tid; i < nbins; i += ORDER_THREADS) start[i] = 0;
  for (int i = tid; i < count; i += ORDER_THREADS) kcs[i] = 0;
  __syncthreads();
  // (tile, 16-k-block chunk) items; neighbouring threads take neighbouring tiles,
  // i.e. neighbouring mask bytes of one row
  const int chunks = (g.nkb + ORDER_KB_CHUNK - 1) / ORDER_KB_CHUNK;
  for (int it = tid; it < count * chunks; it += ORDER_THREADS) {
    const int i = it % count, c = it / count;
    int mt, nt;
    tile_coords(g, first + i, mt, nt);
    const int n = tile_kcount_chunk(g, mt, nt, c * ORDER_KB_CHUNK);
    if (n) atomicAdd(&kcs[i], n);
  }
  __syncthreads();
  for (int i = tid; i < count; i += ORDER_THREADS) atomicAdd(&start[g.nkb - kcs[i]], 1);
  __syncthreads();
  // exclusive scan of the bins: thread t owns bins [t per, (t + 1) per)
  const int per = (nbins + ORDER_THREADS - 1) / ORDER_THREADS;
  int own[ORDER_OWN];
  int sum = 0;
#pragma unroll
  for (int i = 0; i < ORDER_OWN; ++i) {
    const int b = tid * per + i;
    own[i] = i < per && b < nbins ? start[b] : 0;
    sum += own[i];
  }
  int incl = sum;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int v = __shfl_up(incl, d);
    if (lane >= d) incl += v;
  }
  if (lane == 63) wave_sum[wave] = incl;
  __syncthreads();
  int base = first + incl - sum;
  for (int w = 0; w < wave; ++w) base += wave_sum[w];
#pragma unroll
  for (int i = 0; i < ORDER_OWN; ++i) {
    const int b = tid * per + i;
    if (i < per && b < nbins) start[b] = base;
    base += own[i];
  }
  __syncthreads();
  for (int i = tid; i < count; i += ORDER_THREADS) {
    const int pos = atomicAdd(&start[g.nkb - kcs[i]], 1);
    if (pos < first + count) order[pos] = first + i;
  }
}

// fp32 runs the same byte layout: a 64-byte LDS row holds 32 bf16 or 16 fp32 k
// values, a fragment read 8 bf16 (one v_mfma_f32_16x16x32_bf16) or 4 fp32 (four
// v_mfma_f32_16x16x4_f32, k-step kk taking k = 4 (lane / 16) + kk: A and B use the
// same k order, so the four steps together cover the 16 k of the row).
template <typename T, bool MASKED>
__global__ __launch_bounds__(NTHREADS, WG_PER_CU) void tile_list_gemm_kernel(TileArgs g) {
  constexpr bool F32 = sizeof(T) == 4;
  constexpr int KSE = 64 / static_cast<int>(sizeof(T));  // K-step in elements (64 bytes of a row)
  constexpr int CE = 16 / static_cast<int>(sizeof(T));   // elements per 16-byte chunk
  __shared__ __attribute__((aligned(1024))) bf16_t lds[STAGES][2][TT * KS];  // [stage][A/B][row * 32 + k]
  __shared__ int32_t klist[LIST_MAX];  // k block | active n-block bits << 16 (MASKED)
  __shared__ int32_t chunk_count[LIST_MAX / 64];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WNW, wn = wave % WNW;

  // ---- which tile ---------------------------------------------------------------
  const int pos = xcd_contiguous(blockIdx.x, gridDim.x);
  const int lid = g.order ? g.order[pos] : pos;
  int mt, nt;
  tile_coords(g, lid, mt, nt);
  const int m0 = mt * TT, n0 = nt * TT;

  // ---- active k blocks of this tile -> klist -----------------------------------
  int grp = m0 / g.rows_per_group;
  grp = grp < g.groups ? grp : g.groups - 1;
  const uint8_t* gmask = g.mask + static_cast<int64_t>(grp) * g.nkb * g.nnb;
  const int nsub = MASKED ? TT / g.block_n : 1;
  const int nb0 = n0 / g.block_n;
  const int rounds = (g.nkb + NTHREADS - 1) / NTHREADS;  // <= LIST_MAX / NTHREADS
  constexpr int MAX_ROUNDS = LIST_MAX / NTHREADS;
  uint32_t bits[MAX_ROUNDS];
  uint64_t bal[MAX_ROUNDS];
#pragma unroll
  for (int i = 0; i < MAX_ROUNDS; ++i) {
    bits[i] = 0;
    if (i < rounds) {
      const int kb = i * NTHREADS + tid;
      if (kb < g.nkb) {
        const uint8_t* row = gmask + static_cast<int64_t>(kb) * g.nnb + nb0;
        for (int j = 0; j < nsub; ++j)
          if (nb0 + j < g.nnb && row[j]) bits[i] |= 1u << j;
      }
    }
  }
#pragma unroll
  for (int i = 0; i < MAX_ROUNDS; ++i) {
    if (i < rounds) {
      bal[i] = __ballot(bits[i] != 0);
      if (lane == 0) chunk_count[i * NW + wave] = __popcll(bal[i]);
    }
  }
  __syncthreads();
  int nact = 0;
  for (int c = 0; c < rounds * NW; ++c) nact += chunk_count[c];
#pragma unroll
  for (int i = 0; i < MAX_ROUNDS; ++i) {
    if (i < rounds && bits[i]) {
      int base = 0;
      for (int c = 0; c < i * NW + wave; ++c) base += chunk_count[c];
      const int pos = base + __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(bal[i] >> 32),
                                                       __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(bal[i]), 0));
      klist[pos] = (i * NTHREADS + tid) | (MASKED ? static_cast<int>(bits[i] << 16) : 0);
    }
  }
  __syncthreads();
  nact = __builtin_amdgcn_readfirstlane(nact);
  const int per = g.block_k / KSE;
  const int kcount = nact * per;

  // ---- this lane's source rows: wave w loads fragments AF w .. AF w + AF - 1 of A
  // and B; lane l lands at fragment row l / 4, slot l % 4, holding logical chunk
  // (l % 4) ^ chunk_swz(row) --------------------------------------------------
  const T* asrc[AF];
  const T* bsrc[AF];
#pragma unroll
  for (int j = 0; j < AF; ++j) {
    const int r = 16 * (AF * wave + j) + (lane >> 2);
    const int lc = (lane & 3) ^ chunk_swz(r);
    const int m = m0 + r < g.M ? m0 + r : g.M - 1;  // rows past M read row M - 1, never stored
    const int n = n0 + r < g.N ? n0 + r : g.N - 1;
    asrc[j] = static_cast<const T*>(g.A) + static_cast<int64_t>(m) * g.lda + lc * CE;
    bsrc[j] = static_cast<const T*>(g.B) + static_cast<int64_t>(n) * g.ldb + lc * CE;
  }
  // list entries in registers, 64 at a time (lane i holds entry 64 c + i): an LDS
  // read in the issue path would wait for the direct-to-LDS loads in flight
  auto list_chunk = [&](int c) { return 64 * c + lane < nact ? klist[64 * c + lane] : 0; };
  int iss_blk = 0, iss_sub = 0;
  int iss_cur = list_chunk(0), iss_next = list_chunk(1);
  int rd_blk = 0, rd_sub = 0, rd_cur = iss_cur, rd_next = iss_next;
  auto issue = [&](int stage) {
    const int e = __builtin_amdgcn_readlane(iss_cur, iss_blk & 63);
    const int64_t k = static_cast<int64_t>(e & 0xffff) * g.block_k + iss_sub * KSE;
    if (++iss_sub == per) {
      iss_sub = 0;
      if ((++iss_blk & 63) == 0) {
        iss_cur = iss_next;
        iss_next = list_chunk((iss_blk >> 6) + 1);
      }
    }
#pragma unroll
    for (int j = 0; j < AF; ++j) {
      __builtin_amdgcn_global_load_lds((glb_void_t*)(asrc[j] + k),
                                       (lds_void_t*)&lds[stage][0][(AF * wave + j) * FRAG_ELEMS], 16, 0, 0);
      __builtin_amdgcn_global_load_lds((glb_void_t*)(bsrc[j] + k),
                                       (lds_void_t*)&lds[stage][1][(AF * wave + j) * FRAG_ELEMS], 16, 0, 0);
    }
  };

  f32x4_t acc[4][FB];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int f = 0; f < FB; ++f) acc[i][f] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // wave (wm, wn): rows 64 wm + 16 i, columns WCOLS wn + 16 f of the tile
  const int frow = lane & 15, fchunk = lane >> 4;
  int fsub[FB];  // n block (within the tile) of each B fragment
#pragma unroll
  for (int f = 0; f < FB; ++f) fsub[f] = MASKED ? (WCOLS * wn + 16 * f) / g.block_n : 0;
  auto read_frags = [&](int stage, u32x4_t (&fa)[4], u32x4_t (&fb)[FB]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 64 * wm + 16 * i + frow;
      fa[i] = *reinterpret_cast<const u32x4_t*>(&lds[stage][0][r * KS + (fchunk ^ chunk_swz(r)) * 8]);
    }
#pragma unroll
    for (int f = 0; f < FB; ++f) {
      const int c = WCOLS * wn + 16 * f + frow;
      fb[f] = *reinterpret_cast<const u32x4_t*>(&lds[stage][1][c * KS + (fchunk ^ chunk_swz(c)) * 8]);
    }
    if (MASKED) {  // zero the B fragments of n blocks inactive at this k block
      const uint32_t on = static_cast<uint32_t>(__builtin_amdgcn_readlane(rd_cur, rd_blk & 63)) >> 16;
      if (++rd_sub == per) {
        rd_sub = 0;
        if ((++rd_blk & 63) == 0) {
          rd_cur = rd_next;
          rd_next = list_chunk((rd_blk >> 6) + 1);
        }
      }
#pragma unroll
      for (int f = 0; f < FB; ++f)
        if (!((on >> fsub[f]) & 1u)) fb[f] = u32x4_t{0u, 0u, 0u, 0u};
    }
  };
  auto mfmas = [&](const u32x4_t (&fa)[4], const u32x4_t (&fb)[FB]) {
    if constexpr (F32) {
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int f = 0; f < FB; ++f)  // C^T fragment
            // (element by value: this clang's __builtin_bit_cast of a vector element
            // reads element 0 whatever the index)
            acc[i][f] = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(fb[f][kk]), __uint_as_float(fa[i][kk]),
                                                              acc[i][f], 0, 0, 0);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int f = 0; f < FB; ++f) acc[i][f] = mfma16x16x32(fb[f], fa[i], acc[i][f]);  // C^T fragment
    }
  };
#if FSI_TG_PREFETCH
  // step s + 2 must have landed at the end of iteration s (its fragments are read
  // during iteration s + 1); later steps may stay in flight
  auto wait_through = [&](int s) {
    const int last = kcount - 1 < s + STAGES - 1 ? kcount - 1 : s + STAGES - 1;  // last step issued
    const int after = last - (s + 2);
    wait_steps(after > 0 ? after : 0);
  };
  auto iteration = [&](int step, const u32x4_t (&ca)[4], const u32x4_t (&cb)[FB], u32x4_t (&na)[4],
                       u32x4_t (&nb)[FB]) {
    // the stage of step + STAGES - 1 was last read during iteration step - 2
    if (step + STAGES - 1 < kcount) issue((step + STAGES - 1) % STAGES);
    // unconditional: past the last step it reads a stage that is never used
    read_frags((step + 1) % STAGES, na, nb);
    mfmas(ca, cb);
    // MFMAs per fragment read of the next step (4 + FB reads, 4 FB MFMAs, x 4 in fp32)
    constexpr int MF = (F32 ? 4 : 1) * FB / 2;
    __builtin_amdgcn_sched_group_barrier(0x008, MF, 0);
#pragma unroll
    for (int r = 0; r < 4 + FB; ++r) {
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, MF, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, F32 ? 0 : MF, 0);
    wait_through(step);
    stage_barrier();
  };

  // prologue: steps 0 .. STAGES - 2 into their stages; steps 0 and 1 land first
  const int pre = kcount < STAGES - 1 ? kcount : STAGES - 1;
  for (int p = 0; p < pre; ++p) issue(p);
  wait_steps(pre - 2 > 0 ? pre - 2 : 0);
  stage_barrier();
  u32x4_t fa0[4], fb0[FB], fa1[4], fb1[FB];
  if (kcount > 0) read_frags(0, fa0, fb0);
  int step = 0;
  for (; step + 1 < kcount; step += 2) {
    iteration(step, fa0, fb0, fa1, fb1);
    iteration(step + 1, fa1, fb1, fa0, fb0);
  }
  if (step < kcount) mfmas(fa0, fb0);  // odd step count: the last step's fragments are in set 0
#else
  // Each iteration reads its own step's fragments, so only step s + 1 must have
  // landed at the end of iteration s: STAGES - 2 steps stay in flight across the
  // barrier (the global-load latency, not the MFMA work, sets the step time when
  // operands come from beyond L2).
  const int pre = kcount < STAGES - 1 ? kcount : STAGES - 1;
  for (int p = 0; p < pre; ++p) issue(p);
  wait_steps(pre - 1 > 0 ? pre - 1 : 0);
  stage_barrier();
  for (int step = 0; step < kcount; ++step) {
    // the stage of step + STAGES - 1 was last read during iteration step - 1
    if (step + STAGES - 1 < kcount) issue((step + STAGES - 1) % STAGES);
    u32x4_t fa[4], fb[FB];
    read_frags(step % STAGES, fa, fb);
    mfmas(fa, fb);
    const int last = kcount - 1 < step + STAGES - 1 ? kcount - 1 : step + STAGES - 1;
    const int after = last - (step + 1);
    wait_steps(after > 0 ? after : 0);
    stage_barrier();
  }
#endif

  // ---- epilogue: lane (q = lane / 16, r = lane % 16) of fragment (i, f) holds row
  // 16 i + r of the wave's rows and columns 4 q .. 4 q + 3 of the fragment ----------
  const int crow = m0 + 64 * wm + frow;
  const int ccol = n0 + WCOLS * wn + 4 * fchunk;
  T* C = static_cast<T*>(g.C);
  if (g.bias) {  // block_k == K: the bias of the columns whose n block is active
    const T* bias = static_cast<const T*>(g.bias);
    const uint8_t* row0 = g.mask + static_cast<int64_t>(grp) * g.nkb * g.nnb;
#pragma unroll
    for (int f = 0; f < FB; ++f)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int n = ccol + 16 * f + j;
        float bv = 0.f;
        if (n < g.N && row0[n / g.block_n]) {
          if constexpr (F32) bv = bias[n];
          else bv = bf16_to_f32(bias[n]);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i][f][j] += bv;
      }
  }
  const bool vec = (reinterpret_cast<uintptr_t>(g.C) & (F32 ? 15 : 7)) == 0 && (g.ldc & 3) == 0;
  if (vec && m0 + TT <= g.M && n0 + TT <= g.N) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int f = 0; f < FB; ++f) {
        T* dst = C + static_cast<int64_t>(crow + 16 * i) * g.ldc + ccol + 16 * f;
        if constexpr (F32) {
          *reinterpret_cast<f32x4_t*>(dst) = acc[i][f];
        } else {
          uint2 w;
          w.x = cvt_pk_bf16(acc[i][f][0], acc[i][f][1]);
          w.y = cvt_pk_bf16(acc[i][f][2], acc[i][f][3]);
          *reinterpret_cast<uint2*>(dst) = w;
        }
      }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = crow + 16 * i;
      if (m >= g.M) continue;
#pragma unroll
      for (int f = 0; f < FB; ++f)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int n = ccol + 16 * f + j;
          if (n < g.N) {
            if constexpr (F32) C[static_cast<int64_t>(m) * g.ldc + n] = acc[i][f][j];
            else C[static_cast<int64_t>(m) * g.ldc + n] = f32_to_bf16(acc[i][f][j]);
          }
        }
    }
  }
}

}  // namespace

namespace fsi_tile {

// The list-driven tile GEMM (bf16 or fp32) when the tiling fits it: block_k a
// multiple of the 64-byte K-step, block_n a multiple or a divisor (>= 16) of 128,
// row groups of whole 128-row tiles, 16-byte aligned rows.  Returns 1 when the
// shape does not fit (the caller runs the generic kernel), else an FSI status.
// `order_ws` (tiles int32, may be null) takes the heaviest-first tile order.
int tile_gemm(const void* x, int64_t ldx, const void* w, int64_t ldw, const void* bias, const uint8_t* mask,
              int64_t groups, int64_t rows_per_group, int64_t block_k, int64_t block_n, int64_t M, int64_t N,
              int64_t K, int dtype, void* out, int64_t ldo, int32_t* order_ws, hipStream_t st) {
  using namespace fsi_host;
  const int64_t esz = dtype == FSI_DTYPE_F32 ? 4 : 2;
  const int64_t kse = 64 / esz, ce = 16 / esz;
  const int64_t nkb = K / block_k, nnb = N / block_n;
  const bool tiles_ok = block_k % kse == 0 && (block_n % TT == 0 || (TT % block_n == 0 && block_n >= 16)) &&
                        nkb <= LIST_MAX && (rows_per_group % TT == 0 || groups == 1) &&
                        (bias == nullptr || nkb == 1);
  const bool aligned = ldx % ce == 0 && ldw % ce == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0 &&
                       (reinterpret_cast<uintptr_t>(w) & 15) == 0;  // 16-byte direct-to-LDS loads
  if (!tiles_ok || !aligned) return 1;
  TileArgs a{};
  a.A = x;
  a.B = w;
  a.C = out;
  a.bias = bias;
  a.lda = ldx;
  a.ldb = ldw;
  a.ldc = ldo;
  a.M = (int)M;
  a.N = (int)N;
  a.K = (int)K;
  a.mask = mask;
  a.groups = (int)groups;
  a.rows_per_group = (int)(rows_per_group < 0x7fffffff ? rows_per_group : 0x7fffffff);
  a.nkb = (int)nkb;
  a.nnb = (int)nnb;
  a.block_k = (int)block_k;
  a.block_n = (int)block_n;
  a.m_tiles = (int)((M + TT - 1) / TT);
  a.n_tiles = (int)((N + TT - 1) / TT);
  const int64_t tiles = static_cast<int64_t>(a.m_tiles) * a.n_tiles;
  FSI_CHECK_ARG(tiles <= 0x7fffffff, FSI_ERR_SHAPE, "blockwise_matmul: too many tiles");
  const unsigned grid = static_cast<unsigned>(tiles);
  // Heaviest-first order inside each band when the grid takes several rounds of
  // workgroup slots and a band's counting pass (nkb x its n blocks' mask bytes per
  // tile) is small.
  const int64_t nsub = block_n < TT ? TT / block_n : 1;
  const int64_t bands = (a.m_tiles + GROUP_M - 1) / GROUP_M;
  if (order_ws != nullptr && tiles > ORDER_MIN_TILES && int64_t{GROUP_M} * a.n_tiles <= ORDER_MAX_BAND &&
      int64_t{GROUP_M} * a.n_tiles * nkb * nsub <= ORDER_MAX_MASK_READS) {
    tile_order_kernel<<<static_cast<unsigned>(bands), ORDER_THREADS, 0, st>>>(a, order_ws);
    a.order = order_ws;
  }
  if (dtype == FSI_DTYPE_F32) {
    if (block_n < TT) tile_list_gemm_kernel<float, true><<<grid, NTHREADS, 0, st>>>(a);
    else tile_list_gemm_kernel<float, false><<<grid, NTHREADS, 0, st>>>(a);
  } else {
    if (block_n < TT) tile_list_gemm_kernel<bf16_t, true><<<grid, NTHREADS, 0, st>>>(a);
    else tile_list_gemm_kernel<bf16_t, false><<<grid, NTHREADS, 0, st>>>(a);
  }
  const hipError_t e = hipGetLastError();
  FSI_CHECK_ARG(e == hipSuccess, FSI_ERR_HIP, "blockwise_matmul: launch failed: %s", hipGetErrorString(e));
  return FSI_OK;
}

}  // namespace fsi_tile

extern "C" {

FSI_API size_t fsi_blockwise_matmul_workspace_size(int64_t M, int64_t N, int64_t K, int64_t block_k) {
  (void)K;
  (void)block_k;
  // Every tile builds its k-block list in LDS; the workspace holds the tile order
  // (one int32 per 128 x 128 output tile) after the counter area.
  if (M <= 0 || N <= 0) return FSI_WORKSPACE_COUNTER_BYTES;
  const int64_t tiles = ((M + TT - 1) / TT) * ((N + TT - 1) / TT);
  return FSI_WORKSPACE_COUNTER_BYTES + static_cast<size_t>(tiles) * sizeof(int32_t);
}

FSI_API int fsi_blockwise_matmul(const void* x, int64_t ldx, const void* w, int64_t ldw,
                                 const uint8_t* tile_mask, int64_t groups, int64_t rows_per_group, int64_t block_k,
                                 int64_t block_n, int64_t M, int64_t N, int64_t K, int dtype, void* out, int64_t ldo,
                                 void* workspace, size_t workspace_bytes, void* stream) {
  using namespace fsi_host;
  FSI_CHECK_ARG(dtype == FSI_DTYPE_BF16 || dtype == FSI_DTYPE_F32, FSI_ERR_DTYPE, "blockwise_matmul: dtype %d",
                dtype);
  FSI_CHECK_ARG(M >= 0 && N > 0 && K > 0 && groups > 0 && rows_per_group > 0 && block_k > 0 && block_n > 0,
                FSI_ERR_SHAPE, "blockwise_matmul: bad sizes");
  FSI_CHECK_ARG(K % block_k == 0 && N % block_n == 0, FSI_ERR_SHAPE,
                "blockwise_matmul: tiles %lldx%lld must divide K = %lld and N = %lld", (long long)block_k,
                (long long)block_n, (long long)K, (long long)N);
  FSI_CHECK_ARG(M <= 0x7fffffff && N <= 0x7fffffff && K <= 0x7fffffff, FSI_ERR_SHAPE,
                "blockwise_matmul: sizes beyond int32");
  FSI_CHECK_ARG(groups == 1 || groups * rows_per_group >= M, FSI_ERR_SHAPE,
                "blockwise_matmul: %lld row groups of %lld rows do not cover %lld rows", (long long)groups,
                (long long)rows_per_group, (long long)M);
  if (M == 0) return FSI_OK;
  FSI_CHECK_ARG(x && w && tile_mask && out, FSI_ERR_INVALID_ARG, "blockwise_matmul: null pointer");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  FSI_CHECK_ARG(ldx >= K && ldw >= K && ldo >= N, FSI_ERR_SHAPE, "blockwise_matmul: leading dimensions");
  FSI_CHECK_ARG(workspace == nullptr || workspace_bytes >= FSI_WORKSPACE_COUNTER_BYTES, FSI_ERR_WORKSPACE,
                "blockwise_matmul: workspace %zu < %d", workspace_bytes, FSI_WORKSPACE_COUNTER_BYTES);
  const int64_t tiles = ((M + TT - 1) / TT) * ((N + TT - 1) / TT);
  int32_t* order = workspace != nullptr && workspace_bytes >= FSI_WORKSPACE_COUNTER_BYTES + tiles * sizeof(int32_t)
                       ? reinterpret_cast<int32_t*>(static_cast<char*>(workspace) + FSI_WORKSPACE_COUNTER_BYTES)
                       : nullptr;
  const int rc = fsi_tile::tile_gemm(x, ldx, w, ldw, nullptr, tile_mask, groups, rows_per_group, block_k, block_n, M,
                                     N, K, dtype, out, ldo, order, st);
  if (rc != 1) return rc;
  // tilings the list kernel does not take: the generic kernel
  return fsi_bs_generic::tile_gemm(x, ldx, w, ldw, nullptr, tile_mask, groups, rows_per_group, block_k, block_n, M,
                                   N, K, dtype, out, ldo, st);
}

}  // extern "C"
