// Block-level KL distillation loss of the 16-D indexer, forward and backward.
//
// FovealIndexer.distillation_loss (foveal_indexer/core.py:315-353) trains the
// student block scores s against a teacher block mass t.  Per routed row
// r = (b, q) with valid set V (all entries, the causal set p < q, or a caller
// mask):
//   z_i      = s_i / T                              (fp32, i in V)
//   target_i = max(t_i, 0) / sum_V max(t, 0)        if that sum > 1e-12
//            = 1 / |V|                              otherwise
//   loss_r   = -sum_V target_i * log_softmax_V(z)_i
// and the loss is the mean of loss_r over the rows with |V| > 0 (0 if none).
// The gradient is d loss / d s_i = g / n_rows * (p_i * sum_V target - target_i) / T
// on valid entries of valid rows (p = softmax_V(z)), 0 elsewhere; the teacher
// takes no gradient.
//
// Layout: one wave per row; a row is read in 64-lane strips, three passes
// (max / teacher mass / count, exp-sum, weighted log-probabilities), all of it
// from L1/L2 after the first pass.  The mean over rows is a second one-workgroup
// kernel, so the loss never leaves the device and the backward reads the row
// count from there too (no host synchronisation).
#include "fsi_common.h"

namespace {

using namespace fsi;

constexpr int DK_WAVES = 4;  // rows per 256-thread workgroup

enum MaskMode : int { MASK_ALL = 0, MASK_CAUSAL = 1, MASK_EXPLICIT = 2 };

template <bool BF16>
__device__ __forceinline__ float ld(const void* p, int64_t i) {
  if (BF16) return bf16_to_f32(static_cast<const bf16_t*>(p)[i]);
  return static_cast<const float*>(p)[i];
}

struct RowMask {
  int mode;
  int q;
  const uint8_t* m;  // row base of an explicit mask
  int64_t sn;
  __device__ __forceinline__ bool valid(int i) const {
    if (mode == MASK_ALL) return true;
    if (mode == MASK_CAUSAL) return i < q;
    return m[i * sn] != 0;
  }
};

// Row statistics shared by the forward and the backward.
struct RowStats {
  float zmax;     // max of z over V
  float lse;      // log sum_V exp(z - zmax)
  float denom;    // sum_V max(t, 0)
  int count;      // |V|
};

template <bool SB, bool TB>
__device__ RowStats row_stats(const void* s, const void* t, int64_t base, int N, const RowMask& rm,
                              float temperature, int lane) {
  float zmax = -INFINITY, tsum = 0.f;
  int cnt = 0;
  for (int i = lane; i < N; i += 64) {
    if (!rm.valid(i)) continue;
    const float z = ld<SB>(s, base + i) / temperature;
    zmax = fmaxf(zmax, z);
    tsum += fmaxf(ld<TB>(t, base + i), 0.0f);
    ++cnt;
  }
  zmax = wave_max(zmax);
  tsum = wave_sum(tsum);
  cnt = wave_sum_i(cnt);
  float esum = 0.f;
  if (cnt > 0) {
    for (int i = lane; i < N; i += 64) {
      if (!rm.valid(i)) continue;
      esum += expf(ld<SB>(s, base + i) / temperature - zmax);
    }
  }
  esum = wave_sum(esum);
  RowStats r;
  r.zmax = zmax;
  r.lse = cnt > 0 ? logf(esum) : 0.f;
  r.denom = tsum;
  r.count = cnt;
  return r;
}

__device__ __forceinline__ float target_of(float t, const RowStats& r) {
  // torch.where(denom > 1e-12, t / denom.clamp_min(1e-12), uniform)
  return r.denom > 1e-12f ? fmaxf(t, 0.0f) / r.denom : 1.0f / static_cast<float>(r.count);
}

template <bool SB, bool TB>
__global__ __launch_bounds__(64 * DK_WAVES) void distill_rows_kernel(
    const void* __restrict__ s, const void* __restrict__ t, int B, int Q, int N, int mode,
    const uint8_t* __restrict__ mask, int64_t msb, int64_t msq, int64_t msn, float temperature,
    float* __restrict__ row_loss, int* __restrict__ row_valid) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * DK_WAVES + (threadIdx.x >> 6);
  if (row >= static_cast<int64_t>(B) * Q) return;
  const int b = static_cast<int>(row / Q), q = static_cast<int>(row % Q);
  RowMask rm{mode, q, mode == MASK_EXPLICIT ? mask + b * msb + q * msq : nullptr, msn};
  const int64_t base = row * N;
  const RowStats r = row_stats<SB, TB>(s, t, base, N, rm, temperature, lane);
  float acc = 0.f;
  if (r.count > 0) {
    for (int i = lane; i < N; i += 64) {
      if (!rm.valid(i)) continue;
      const float logp = (ld<SB>(s, base + i) / temperature - r.zmax) - r.lse;
      acc += target_of(ld<TB>(t, base + i), r) * logp;
    }
  }
  acc = wave_sum(acc);
  if (lane == 0) {
    row_loss[row] = r.count > 0 ? -acc : 0.f;
    row_valid[row] = r.count > 0 ? 1 : 0;
  }
}

// loss[0] = mean of row_loss over valid rows (0 if none); n_rows[0] = their count.
__global__ __launch_bounds__(256) void distill_mean_kernel(const float* __restrict__ row_loss,
                                                           const int* __restrict__ row_valid, int64_t rows,
                                                           float* __restrict__ loss, int* __restrict__ n_rows) {
  __shared__ float ps[4];
  __shared__ int pc[4];
  float acc = 0.f;
  int cnt = 0;
  for (int64_t i = threadIdx.x; i < rows; i += 256) {
    if (row_valid[i]) {
      acc += row_loss[i];
      ++cnt;
    }
  }
  acc = wave_sum(acc);
  cnt = wave_sum_i(cnt);
  if ((threadIdx.x & 63) == 0) {
    ps[threadIdx.x >> 6] = acc;
    pc[threadIdx.x >> 6] = cnt;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    const float tot = (ps[0] + ps[1]) + (ps[2] + ps[3]);
    const int c = (pc[0] + pc[1]) + (pc[2] + pc[3]);
    loss[0] = c > 0 ? tot / static_cast<float>(c) : 0.f;
    n_rows[0] = c;
  }
}

template <bool SB, bool TB>
__global__ __launch_bounds__(64 * DK_WAVES) void distill_bwd_kernel(
    const void* __restrict__ s, const void* __restrict__ t, int B, int Q, int N, int mode,
    const uint8_t* __restrict__ mask, int64_t msb, int64_t msq, int64_t msn, float temperature,
    const float* __restrict__ dloss, const int* __restrict__ n_rows, void* __restrict__ ds) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * DK_WAVES + (threadIdx.x >> 6);
  if (row >= static_cast<int64_t>(B) * Q) return;
  const int b = static_cast<int>(row / Q), q = static_cast<int>(row % Q);
  RowMask rm{mode, q, mode == MASK_EXPLICIT ? mask + b * msb + q * msq : nullptr, msn};
  const int64_t base = row * N;
  const RowStats r = row_stats<SB, TB>(s, t, base, N, rm, temperature, lane);
  const int nr = n_rows[0];
  float tsum = 0.f;
  if (r.count > 0) {
    for (int i = lane; i < N; i += 64)
      if (rm.valid(i)) tsum += target_of(ld<TB>(t, base + i), r);
  }
  tsum = wave_sum(tsum);
  const float g = (r.count > 0 && nr > 0) ? dloss[0] / static_cast<float>(nr) : 0.f;
  for (int i = lane; i < N; i += 64) {
    float d = 0.f;
    if (g != 0.f && rm.valid(i)) {
      const float p = expf(ld<SB>(s, base + i) / temperature - r.zmax - r.lse);
      d = g * (p * tsum - target_of(ld<TB>(t, base + i), r)) / temperature;
    }
    if (SB)
      static_cast<bf16_t*>(ds)[base + i] = f32_to_bf16(d);
    else
      static_cast<float*>(ds)[base + i] = d;
  }
}

int check_common(const void* s, int s_dtype, const void* t, int t_dtype, int64_t B, int64_t Q, int64_t N, int mode,
                 const uint8_t* mask, float temperature, const char* what) {
  FSI_CHECK_ARG(s && t, FSI_ERR_INVALID_ARG, "%s: null pointer", what);
  FSI_CHECK_ARG((s_dtype == FSI_DTYPE_F32 || s_dtype == FSI_DTYPE_BF16) &&
                    (t_dtype == FSI_DTYPE_F32 || t_dtype == FSI_DTYPE_BF16),
                FSI_ERR_DTYPE, "%s: dtypes %d / %d", what, s_dtype, t_dtype);
  FSI_CHECK_ARG(B > 0 && Q > 0 && N > 0 && B * Q < (int64_t(1) << 31) && N < (int64_t(1) << 31), FSI_ERR_SHAPE,
                "%s: B=%lld Q=%lld N=%lld", what, (long long)B, (long long)Q, (long long)N);
  FSI_CHECK_ARG(mode >= MASK_ALL && mode <= MASK_EXPLICIT, FSI_ERR_INVALID_ARG, "%s: mask mode %d", what, mode);
  FSI_CHECK_ARG(mode != MASK_EXPLICIT || mask, FSI_ERR_INVALID_ARG, "%s: explicit mask missing", what);
  FSI_CHECK_ARG(temperature > 0.f, FSI_ERR_INVALID_ARG, "%s: temperature %g", what, (double)temperature);
  return FSI_OK;
}

}  // namespace

extern "C" {

FSI_API size_t fsi_distill_kl_workspace_size(int64_t B, int64_t Q) {
  const size_t rows = static_cast<size_t>(B * Q);
  return FSI_WORKSPACE_COUNTER_BYTES + fsi_host::align_up(rows * sizeof(float), 256) +
         fsi_host::align_up(rows * sizeof(int), 256);
}

FSI_API int fsi_distill_kl_fwd(const void* scores, int s_dtype, const void* teacher, int t_dtype, int64_t B,
                               int64_t Q, int64_t N, int mask_mode, const uint8_t* mask, int64_t mask_stride_b,
                               int64_t mask_stride_q, int64_t mask_stride_n, float temperature, float* loss,
                               int32_t* n_rows, void* workspace, size_t workspace_bytes, void* stream) {
  const int c = check_common(scores, s_dtype, teacher, t_dtype, B, Q, N, mask_mode, mask, temperature,
                             "distill_kl_fwd");
  if (c != FSI_OK) return c;
  FSI_CHECK_ARG(loss && n_rows, FSI_ERR_INVALID_ARG, "distill_kl_fwd: null output");
  const size_t need = fsi_distill_kl_workspace_size(B, Q);
  FSI_CHECK_ARG(workspace && workspace_bytes >= need, FSI_ERR_WORKSPACE, "distill_kl_fwd: workspace %zu < %zu",
                workspace_bytes, need);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int64_t rows = B * Q;
  float* row_loss = reinterpret_cast<float*>(static_cast<char*>(workspace) + FSI_WORKSPACE_COUNTER_BYTES);
  int* row_valid = reinterpret_cast<int*>(reinterpret_cast<char*>(row_loss) +
                                          fsi_host::align_up(rows * sizeof(float), 256));
  const dim3 grid(static_cast<unsigned>((rows + DK_WAVES - 1) / DK_WAVES));
  const bool sb = s_dtype == FSI_DTYPE_BF16, tb = t_dtype == FSI_DTYPE_BF16;
#define FSI_DK_LAUNCH(SB, TB)                                                                                     \
  distill_rows_kernel<SB, TB><<<grid, 64 * DK_WAVES, 0, st>>>(scores, teacher, (int)B, (int)Q, (int)N, mask_mode, \
                                                              mask, mask_stride_b, mask_stride_q, mask_stride_n,  \
                                                              temperature, row_loss, row_valid)
  if (sb && tb) FSI_DK_LAUNCH(true, true);
  else if (sb) FSI_DK_LAUNCH(true, false);
  else if (tb) FSI_DK_LAUNCH(false, true);
  else FSI_DK_LAUNCH(false, false);
#undef FSI_DK_LAUNCH
  FSI_HIP_LAUNCH_CHECK("distill_kl_fwd rows");
  distill_mean_kernel<<<1, 256, 0, st>>>(row_loss, row_valid, rows, loss, n_rows);
  FSI_HIP_LAUNCH_CHECK("distill_kl_fwd mean");
  return FSI_OK;
}

FSI_API int fsi_distill_kl_bwd(const void* scores, int s_dtype, const void* teacher, int t_dtype, int64_t B,
                               int64_t Q, int64_t N, int mask_mode, const uint8_t* mask, int64_t mask_stride_b,
                               int64_t mask_stride_q, int64_t mask_stride_n, float temperature, const float* dloss,
                               const int32_t* n_rows, void* dscores, void* stream) {
  const int c = check_common(scores, s_dtype, teacher, t_dtype, B, Q, N, mask_mode, mask, temperature,
                             "distill_kl_bwd");
  if (c != FSI_OK) return c;
  FSI_CHECK_ARG(dloss && n_rows && dscores, FSI_ERR_INVALID_ARG, "distill_kl_bwd: null pointer");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int64_t rows = B * Q;
  const dim3 grid(static_cast<unsigned>((rows + DK_WAVES - 1) / DK_WAVES));
  const bool sb = s_dtype == FSI_DTYPE_BF16, tb = t_dtype == FSI_DTYPE_BF16;
#define FSI_DK_LAUNCH(SB, TB)                                                                                    \
  distill_bwd_kernel<SB, TB><<<grid, 64 * DK_WAVES, 0, st>>>(scores, teacher, (int)B, (int)Q, (int)N, mask_mode, \
                                                             mask, mask_stride_b, mask_stride_q, mask_stride_n,  \
                                                             temperature, dloss, n_rows, dscores)
  if (sb && tb) FSI_DK_LAUNCH(true, true);
  else if (sb) FSI_DK_LAUNCH(true, false);
  else if (tb) FSI_DK_LAUNCH(false, true);
  else FSI_DK_LAUNCH(false, false);
#undef FSI_DK_LAUNCH
  FSI_HIP_LAUNCH_CHECK("distill_kl_bwd");
  return FSI_OK;
}

}  // extern "C"
