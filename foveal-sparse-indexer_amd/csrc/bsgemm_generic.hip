// Tile-masked GEMM for the shapes outside the MFMA engines of bsgemm.hip and
// tile_gemm.hip (which also runs fp32, the reference modules' default dtype):
// block sizes those engines do not tile (block_k not a multiple of 16 fp32 /
// 32 bf16, column blocks neither a divisor >= 16 nor a multiple of 128,
// unaligned rows).
//
//   out[m, n] = sum_k x[m, k] w[n, k] [tile (k / block_k, n / block_n) active for
//               the row group of m]  (+ bias[n] where n's column block is active)
//
// which is BlockwiseMatMul2D's X (W o M)^T (block_matmul.py:381-392) with a mask
// per row group, and triton_block_sparse_linear / BlockSparseLinear's column-
// block product (triton_ops.py:95-140) when block_k = K.  Math in fp32 on
// v_mfma_f32_16x16x4f32: a workgroup of four waves owns a 64 x 64 output tile,
// each wave 32 x 32 (2 x 2 MFMA tiles); operands go through LDS 16 k at a time,
// weight elements of inactive tiles are stored as zero, and k-steps whose 64
// columns have no active tile for the group are skipped.
#include "fsi_common.h"

namespace {

using namespace fsi;

constexpr int GT = 64;   // output tile
constexpr int GK = 16;   // k per step
constexpr int GPAD = 1;  // LDS row padding (floats)

typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f4_t;

template <typename T>
__device__ __forceinline__ float ldf(const T* p);
template <>
__device__ __forceinline__ float ldf<float>(const float* p) { return *p; }
template <>
__device__ __forceinline__ float ldf<bf16_t>(const bf16_t* p) { return bf16_to_f32(*p); }

template <typename T>
__device__ __forceinline__ void stf(T* p, float v);
template <>
__device__ __forceinline__ void stf<float>(float* p, float v) { *p = v; }
template <>
__device__ __forceinline__ void stf<bf16_t>(bf16_t* p, float v) { *p = f32_to_bf16(v); }

struct GenGemmParams {
  const void* x;
  int64_t ldx;
  const void* w;
  int64_t ldw;
  const void* bias;      // optional, length N
  const uint8_t* mask;   // (groups, nkb * nnb), tile id k_b * nnb + n_b
  int rows_per_group;
  int block_k, block_n, nkb, nnb;
  int M, N, K;
  void* out;
  int64_t ldo;
};

template <typename T>
__global__ __launch_bounds__(256) void bs_generic_kernel(GenGemmParams P) {
  __shared__ float As[GT][GK + GPAD];
  __shared__ float Bs[GT][GK + GPAD];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int m0 = blockIdx.y * GT, n0 = blockIdx.x * GT;
  const int g = m0 / P.rows_per_group;  // the host guarantees one row group per 64-row tile
  const uint8_t* gmask = P.mask + static_cast<int64_t>(g) * P.nkb * P.nnb;
  const T* x = static_cast<const T*>(P.x);
  const T* w = static_cast<const T*>(P.w);
  const int wr = (wave >> 1) * 32, wc = (wave & 1) * 32;
  f32x4_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // each thread stages one row x 4 k of A and of B per step
  const int lr = tid >> 2, lk = (tid & 3) * 4;
  const int am = m0 + lr, bn = n0 + lr;
  for (int k0 = 0; k0 < P.K; k0 += GK) {
    // activity of this thread's four weight elements
    bool act[4];
    bool any = false;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int k = k0 + lk + e;
      act[e] = bn < P.N && k < P.K && gmask[(k / P.block_k) * P.nnb + bn / P.block_n] != 0;
      any |= act[e];
    }
    if (!__syncthreads_or(any)) continue;  // no active tile in these 64 columns and 16 k
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int k = k0 + lk + e;
      As[lr][lk + e] = (am < P.M && k < P.K) ? ldf<T>(x + am * P.ldx + k) : 0.f;
      Bs[lr][lk + e] = act[e] ? ldf<T>(w + bn * P.ldw + k) : 0.f;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < GK / 4; ++kk) {
      const int kc = 4 * kk + (lane >> 4);
      float a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) a[i] = As[wr + 16 * i + (lane & 15)][kc];
#pragma unroll
      for (int j = 0; j < 2; ++j) b[j] = Bs[wc + 16 * j + (lane & 15)][kc];
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    __syncthreads();
  }
  T* out = static_cast<T*>(P.out);
  const T* bias = static_cast<const T*>(P.bias);
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int n = n0 + wc + 16 * j + (lane & 15);
    if (n >= P.N) continue;
    float bv = 0.f;
    if (bias && P.nkb == 1 && gmask[n / P.block_n]) bv = ldf<T>(bias + n);
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + wr + 16 * i + 4 * (lane >> 4) + r;
        if (m < P.M) stf<T>(out + m * P.ldo + n, acc[i][j][r] + bv);
      }
  }
}

__global__ __launch_bounds__(256) void col_mask_kernel(const int32_t* __restrict__ blocks, int n_active, int nnb,
                                                       uint8_t* __restrict__ mask, int* __restrict__ err) {
  // mask[b] = 1 for listed column blocks (one block of 256 threads clears, then marks)
  for (int i = threadIdx.x; i < nnb; i += 256) mask[i] = 0;
  __syncthreads();
  for (int i = threadIdx.x; i < n_active; i += 256) {
    const int b = blocks[i];
    if (b >= 0 && b < nnb) mask[b] = 1;
    else set_error(err, FSI_ERR_INDEX_RANGE);
  }
}

}  // namespace

namespace fsi_tile {  // csrc/tile_gemm.hip: 1 when the tiling does not fit the list kernel
int tile_gemm(const void* x, int64_t ldx, const void* w, int64_t ldw, const void* bias, const uint8_t* mask,
              int64_t groups, int64_t rows_per_group, int64_t block_k, int64_t block_n, int64_t M, int64_t N,
              int64_t K, int dtype, void* out, int64_t ldo, int32_t* order_ws, hipStream_t st);
}  // namespace fsi_tile

namespace fsi_bs_generic {

// 2-D tile mask form.  rows_per_group must be a multiple of 64 unless groups == 1.
int tile_gemm(const void* x, int64_t ldx, const void* w, int64_t ldw, const void* bias, const uint8_t* mask,
              int64_t groups, int64_t rows_per_group, int64_t block_k, int64_t block_n, int64_t M, int64_t N,
              int64_t K, int dtype, void* out, int64_t ldo, hipStream_t st) {
  FSI_CHECK_ARG(dtype == FSI_DTYPE_F32 || dtype == FSI_DTYPE_BF16, FSI_ERR_DTYPE, "block-sparse gemm: dtype %d",
                dtype);
  FSI_CHECK_ARG(M >= 0 && N > 0 && K > 0 && block_k > 0 && block_n > 0 && K % block_k == 0 && N % block_n == 0,
                FSI_ERR_SHAPE, "block-sparse gemm: M %lld N %lld K %lld block_k %lld block_n %lld", (long long)M,
                (long long)N, (long long)K, (long long)block_k, (long long)block_n);
  FSI_CHECK_ARG(groups == 1 || rows_per_group % GT == 0, FSI_ERR_SHAPE,
                "block-sparse gemm: rows_per_group %lld must be a multiple of %d with several groups",
                (long long)rows_per_group, GT);
  FSI_CHECK_ARG(ldx >= K && ldw >= K && ldo >= N && M <= 0x7fffffff && N <= 0x7fffffff && K <= 0x7fffffff,
                FSI_ERR_SHAPE, "block-sparse gemm: leading dimensions");
  if (M == 0) return FSI_OK;
  GenGemmParams P{};
  P.x = x;
  P.ldx = ldx;
  P.w = w;
  P.ldw = ldw;
  P.bias = bias;
  P.mask = mask;
  P.rows_per_group = groups == 1 ? static_cast<int>(M + GT) : static_cast<int>(rows_per_group);
  P.block_k = static_cast<int>(block_k);
  P.block_n = static_cast<int>(block_n);
  P.nkb = static_cast<int>(K / block_k);
  P.nnb = static_cast<int>(N / block_n);
  P.M = static_cast<int>(M);
  P.N = static_cast<int>(N);
  P.K = static_cast<int>(K);
  P.out = out;
  P.ldo = ldo;
  const dim3 grid(static_cast<unsigned>((N + GT - 1) / GT), static_cast<unsigned>((M + GT - 1) / GT));
  if (dtype == FSI_DTYPE_F32)
    bs_generic_kernel<float><<<grid, 256, 0, st>>>(P);
  else
    bs_generic_kernel<bf16_t><<<grid, 256, 0, st>>>(P);
  FSI_HIP_LAUNCH_CHECK("block-sparse gemm (generic)");
  return FSI_OK;
}

// Column-block form: the active block list becomes a one-k-block tile mask in
// `mask_ws` (N / block_size bytes), then tile_gemm with block_k = K.
int column_gemm(const void* x, int64_t ldx, const void* w, int64_t ldw, const void* bias,
                const int32_t* active_blocks, int64_t n_active, int64_t block_size, int64_t M, int64_t N, int64_t K,
                int dtype, void* out, int64_t ldo, uint8_t* mask_ws, int* err, hipStream_t st) {
  FSI_CHECK_ARG(block_size > 0 && N % block_size == 0, FSI_ERR_SHAPE, "block_sparse_linear: block_size %lld",
                (long long)block_size);
  const int nnb = static_cast<int>(N / block_size);
  col_mask_kernel<<<1, 256, 0, st>>>(active_blocks, static_cast<int>(n_active), nnb, mask_ws, err);
  FSI_HIP_LAUNCH_CHECK("block_sparse_linear mask");
  // the list-driven MFMA tile kernel when the tiling fits it (csrc/tile_gemm.hip)
  const int rc = fsi_tile::tile_gemm(x, ldx, w, ldw, bias, mask_ws, 1, M, K, block_size, M, N, K, dtype, out, ldo,
                                     nullptr, st);
  if (rc != 1) return rc;
  return tile_gemm(x, ldx, w, ldw, bias, mask_ws, 1, M, K, block_size, M, N, K, dtype, out, ldo, st);
}

}  // namespace fsi_bs_generic
