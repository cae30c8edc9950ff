// Dense teacher block targets on MI355X (gfx950): the block-energy distillation
// targets of the Pattention speedrun trainer
// (archive/hy_mt2/llm_pattention/train_foveal_pattention_speedrun.py:176-185):
//   act          = silu(h W_gate^T) * (h W_up^T)                    (all I channels)
//   dw_norm[b]   = mean over block b of ||W_down[:, i]||_2
//   energy[m, b] = mean over block b of |act[m, i]| * dw_norm[b]
//   P[m, :]      = softmax(energy[m, :] / T)                        (fp32)
// The gate/up GEMM runs on the block-sparse GEMM engine with an epilogue that
// reduces |act| over 32-channel groups in registers, so the (M, I) activation is
// never written.  bf16 rounding points follow the reference's tensors: g, u,
// silu(g) and the product rounded (eager SwiGLU), the column norms, their block
// means, the block means of |act| and the energy product rounded to bf16.
#include <cmath>

#include "fsi_common.h"

using namespace fsi;

namespace fsi_gemm {
int gateup_energy(const bf16_t* x, int64_t ldx, const bf16_t* kg, const bf16_t* ku, int64_t ldk, int N, int M, int K,
                  int rounding, float* E, int64_t lde, int* err, hipStream_t st);
}  // namespace fsi_gemm

namespace {

// ||W[:, i]||_2 for W [D, I] (row stride ldw) in two passes.  Pass 1: workgroup
// (column tile of 512, row slice of CN_ROWS); each lane owns 8 consecutive
// columns (one 16-byte load per row), the four waves take every fourth row of
// the slice, and the slice's sums of squares go to ss[slice][i].  Pass 2 adds
// the slices in order, takes the root and rounds it to bf16 (torch's bf16 norm).
constexpr int CN_ROWS = 128;

__global__ __launch_bounds__(256) void column_sumsq_kernel(const bf16_t* __restrict__ w, int64_t ldw, int D, int I,
                                                           float* __restrict__ ss) {
  __shared__ float part[4][512];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int c0 = blockIdx.x * 512 + lane * 8;
  const int r0 = blockIdx.y * CN_ROWS;
  const int r1 = r0 + CN_ROWS < D ? r0 + CN_ROWS : D;
  float acc[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) acc[k] = 0.f;
  if (c0 < I) {
    for (int r = r0 + wave; r < r1; r += 4) {
      const uint4 v = *reinterpret_cast<const uint4*>(w + static_cast<int64_t>(r) * ldw + c0);
      const uint32_t q[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float lo = lo_bf16(q[k]), hi = hi_bf16(q[k]);
        acc[2 * k] = fmaf(lo, lo, acc[2 * k]);
        acc[2 * k + 1] = fmaf(hi, hi, acc[2 * k + 1]);
      }
    }
  }
#pragma unroll
  for (int k = 0; k < 8; ++k) part[wave][lane * 8 + k] = acc[k];
  __syncthreads();
  for (int c = threadIdx.x; c < 512; c += 256) {
    const int col = blockIdx.x * 512 + c;
    if (col < I) ss[static_cast<int64_t>(blockIdx.y) * I + col] = (part[0][c] + part[1][c]) + (part[2][c] + part[3][c]);
  }
}

__global__ __launch_bounds__(256) void column_norms_kernel(const float* __restrict__ ss, int slices, int I,
                                                           float* __restrict__ norms) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= I) return;
  float t = 0.f;
  for (int s = 0; s < slices; ++s) t += ss[static_cast<int64_t>(s) * I + i];
  norms[i] = round_bf16(sqrtf(t));
}

// Block means of the column norms: dwn[b] = bf16(mean(norms[b bs .. b bs + bs))).
__global__ __launch_bounds__(256) void block_mean_kernel(const float* __restrict__ norms, int bs, int nb,
                                                         float* __restrict__ dwn) {
  const int b = blockIdx.x * 256 + threadIdx.x;
  if (b >= nb) return;
  float s = 0.f;
  for (int c = 0; c < bs; ++c) s += norms[static_cast<int64_t>(b) * bs + c];
  dwn[b] = round_bf16(s / static_cast<float>(bs));
}

// One workgroup per row: energy from the 32-channel partial sums, then softmax.
constexpr int TS_THREADS = 256;

__global__ __launch_bounds__(TS_THREADS) void block_softmax_kernel(const float* __restrict__ partial, int64_t ldp,
                                                                   const float* __restrict__ dwn, int bs, int nb,
                                                                   float inv_t, float* __restrict__ out,
                                                                   int64_t ldo) {
  __shared__ float red[TS_THREADS / 64];
  const int64_t m = blockIdx.x;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int gpb = bs / 32;  // 32-channel groups per block
  auto energy = [&](int b) {
    float s = 0.f;
    for (int q = 0; q < gpb; ++q) s += partial[m * ldp + static_cast<int64_t>(b) * gpb + q];
    const float a = round_bf16(s / static_cast<float>(bs));  // act_blocks (bf16)
    return round_bf16(a * dwn[b]) * inv_t;                     // block_energy (bf16) / T
  };
  auto reduce = [&](float x, bool is_max) {
    x = is_max ? wave_max(x) : wave_sum(x);
    if (lane == 0) red[wave] = x;
    __syncthreads();
    float r = red[0];
#pragma unroll
    for (int w = 1; w < TS_THREADS / 64; ++w) r = is_max ? fmaxf(r, red[w]) : r + red[w];
    __syncthreads();
    return r;
  };
  float mx = -INFINITY;
  for (int b = threadIdx.x; b < nb; b += TS_THREADS) mx = fmaxf(mx, energy(b));
  mx = reduce(mx, true);
  float z = 0.f;
  for (int b = threadIdx.x; b < nb; b += TS_THREADS) z += expf(energy(b) - mx);
  z = reduce(z, false);
  for (int b = threadIdx.x; b < nb; b += TS_THREADS) out[m * ldo + b] = expf(energy(b) - mx) / z;
}

size_t align256(size_t v) { return (v + 255) / 256 * 256; }

}  // namespace

extern "C" {

// Workspace: [M, I / 32] partial |act| sums, [I] column norms, [I / block_size] block
// means, [ceil(D / CN_ROWS), I] column sums of squares.
FSI_API size_t fsi_dense_block_targets_workspace_size(int64_t M, int64_t D, int64_t I, int64_t block_size) {
  if (M <= 0 || D <= 0 || I <= 0 || block_size <= 0) return 0;
  const int64_t slices = (D + CN_ROWS - 1) / CN_ROWS;
  return align256(static_cast<size_t>(M) * (I / 32) * sizeof(float)) + align256(static_cast<size_t>(I) * sizeof(float)) +
         align256(static_cast<size_t>(I / block_size) * sizeof(float)) +
         align256(static_cast<size_t>(slices) * I * sizeof(float));
}

FSI_API int fsi_dense_block_targets(const void* h, int64_t ldh, const void* w_gate, const void* w_up, int64_t ld_gu,
                                    const void* w_down, int64_t ld_down, int64_t M, int64_t D, int64_t I,
                                    int64_t block_size, float temperature, float* out, int64_t ldo, void* workspace,
                                    size_t workspace_bytes, void* stream) {
  using namespace fsi_host;
  FSI_CHECK_ARG(M >= 0 && D > 0 && I > 0, FSI_ERR_SHAPE, "dense_block_targets: bad sizes M %lld D %lld I %lld",
                (long long)M, (long long)D, (long long)I);
  FSI_CHECK_ARG(block_size >= 32 && block_size % 32 == 0 && I % block_size == 0, FSI_ERR_SHAPE,
                "dense_block_targets: block_size %lld must be a multiple of 32 dividing I %lld", (long long)block_size,
                (long long)I);
  FSI_CHECK_ARG(temperature > 0.0f && std::isfinite(temperature), FSI_ERR_INVALID_ARG,
                "dense_block_targets: temperature %g", (double)temperature);
  FSI_CHECK_ARG(M <= 0x7fffffff && D <= 0x7fffffff && I <= 0x7fffffff, FSI_ERR_SHAPE,
                "dense_block_targets: sizes beyond int32");
  if (M == 0) return FSI_OK;
  FSI_CHECK_ARG(h && w_gate && w_up && w_down && out, FSI_ERR_INVALID_ARG, "dense_block_targets: null pointer");
  FSI_CHECK_ARG(ldh >= D && ld_gu >= D && ld_down >= I && ldo >= I / block_size, FSI_ERR_SHAPE,
                "dense_block_targets: leading dimension too small");
  FSI_CHECK_ARG(ldh % 8 == 0 && ld_gu % 8 == 0 && D % 8 == 0, FSI_ERR_ALIGN,
                "dense_block_targets: rows of h and the gate/up weights must be 16-byte aligned (D, ld % 8)");
  FSI_CHECK_ARG(reinterpret_cast<uintptr_t>(h) % 16 == 0 && reinterpret_cast<uintptr_t>(w_gate) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(w_up) % 16 == 0,
                FSI_ERR_ALIGN, "dense_block_targets: h and gate/up weights must be 16-byte aligned");
  const size_t need = fsi_dense_block_targets_workspace_size(M, D, I, block_size);
  FSI_CHECK_ARG(workspace && workspace_bytes >= need, FSI_ERR_WORKSPACE,
                "dense_block_targets: workspace %zu < %zu bytes", workspace_bytes, need);
  FSI_CHECK_ARG(reinterpret_cast<uintptr_t>(workspace) % 256 == 0, FSI_ERR_ALIGN,
                "dense_block_targets: workspace must be 256-byte aligned");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  float* partial = reinterpret_cast<float*>(ws);
  float* norms = reinterpret_cast<float*>(ws + align256(static_cast<size_t>(M) * (I / 32) * sizeof(float)));
  float* dwn = reinterpret_cast<float*>(reinterpret_cast<char*>(norms) + align256(static_cast<size_t>(I) * sizeof(float)));
  const int nb = static_cast<int>(I / block_size);
  float* ss = reinterpret_cast<float*>(reinterpret_cast<char*>(dwn) + align256(static_cast<size_t>(nb) * sizeof(float)));
  const int slices = static_cast<int>((D + CN_ROWS - 1) / CN_ROWS);

  FSI_CHECK_ARG(I % 8 == 0 && ld_down % 8 == 0 && reinterpret_cast<uintptr_t>(w_down) % 16 == 0, FSI_ERR_ALIGN,
                "dense_block_targets: W_down rows must be 16-byte aligned");
  FSI_CHECK_ARG(slices <= 65535, FSI_ERR_SHAPE, "dense_block_targets: D too large");
  column_sumsq_kernel<<<dim3(static_cast<unsigned>((I + 511) / 512), static_cast<unsigned>(slices)), 256, 0, st>>>(
      static_cast<const bf16_t*>(w_down), ld_down, (int)D, (int)I, ss);
  FSI_HIP_LAUNCH_CHECK("dense_block_targets (column sums of squares)");
  column_norms_kernel<<<static_cast<unsigned>((I + 255) / 256), 256, 0, st>>>(ss, slices, (int)I, norms);
  FSI_HIP_LAUNCH_CHECK("dense_block_targets (column norms)");
  block_mean_kernel<<<static_cast<unsigned>((nb + 255) / 256), 256, 0, st>>>(norms, (int)block_size, nb, dwn);
  FSI_HIP_LAUNCH_CHECK("dense_block_targets (block means)");
  if (fsi_gemm::gateup_energy(static_cast<const bf16_t*>(h), ldh, static_cast<const bf16_t*>(w_gate),
                              static_cast<const bf16_t*>(w_up), ld_gu, (int)I, (int)M, (int)D, FSI_ROUND_EAGER,
                              partial, I / 32, nullptr, st) != 0) {
    fsi_host::set_last_error("dense_block_targets: GEMM launch failed: %s", hipGetErrorString(hipGetLastError()));
    return FSI_ERR_HIP;
  }
  block_softmax_kernel<<<static_cast<unsigned>(M), TS_THREADS, 0, st>>>(partial, I / 32, dwn, (int)block_size, nb,
                                                                        1.0f / temperature, out, ldo);
  FSI_HIP_LAUNCH_CHECK("dense_block_targets (softmax)");
  return FSI_OK;
}

}  // extern "C"
