// Attention for the shapes and dtypes outside the MFMA kernels' layouts:
// fp32 (the reference's default dtype), bf16 with page / block sizes that are
// not multiples of 16, and any head_dim up to 256.  Plain fp32 VALU math, one
// wave per query row, keys taken 64 at a time (one per lane):
//   1. lane j scores key j of the chunk against the query held in LDS;
//   2. online softmax over the chunk (wave max / sum);
//   3. the chunk's probabilities and key ids go to LDS and every lane
//      accumulates its own head dims over the 64 keys (V rows read coalesced).
//
//   decode_attn_dense_kernel: FovealSparseAttention.decode_step's attention
//     over the contiguous reference-layout cache (attention.py:339-367):
//     tokens [max(0, pos + 1 - W), pos] then every token of each selected page,
//     concatenated as the reference does (no de-duplication).
//   sparse_attn_generic_kernel: the prefill patterns of fsi_sparse_attn
//     (attention.py:148-218 union mask; triton_ops.py:26-93 block lists).
#include "fsi_common.h"

namespace {

using namespace fsi;

constexpr int GA_WAVES = 4;
constexpr int GA_MAX_HD = 256;
constexpr int GA_DPL = GA_MAX_HD / 64;  // head dims per lane at most

template <typename T>
__device__ __forceinline__ float ld(const T* p, int64_t i);
template <>
__device__ __forceinline__ float ld<float>(const float* p, int64_t i) { return p[i]; }
template <>
__device__ __forceinline__ float ld<bf16_t>(const bf16_t* p, int64_t i) { return bf16_to_f32(p[i]); }

template <typename T>
__device__ __forceinline__ void st(T* p, int64_t i, float v);
template <>
__device__ __forceinline__ void st<float>(float* p, int64_t i, float v) { p[i] = v; }
template <>
__device__ __forceinline__ void st<bf16_t>(bf16_t* p, int64_t i, float v) { p[i] = f32_to_bf16(v); }

// Per-wave online-softmax state over chunks of up to 64 keys.
struct Acc {
  float m = -INFINITY;
  float l = 0.f;
  float o[GA_DPL] = {0.f, 0.f, 0.f, 0.f};
};

template <typename T>
__device__ __forceinline__ void write_out(const Acc& a, T* out, int hd, int lane) {
  const float inv = a.l > 0.f ? 1.0f / a.l : 0.f;
#pragma unroll
  for (int e = 0; e < GA_DPL; ++e) {
    const int d = lane + 64 * e;
    if (d < hd) st<T>(out, d, a.o[e] * inv);
  }
}

// ---------------------------------------------------------------------------
// Decode over the contiguous cache (B, Hkv, S, hd).
// ---------------------------------------------------------------------------
struct DenseDecodeParams {
  const void* q;  // (B, Hq, hd) contiguous
  const void* k;
  const void* v;
  int64_t ks_b, ks_h, ks_t, vs_b, vs_h, vs_t;
  int S;  // cache length (tokens)
  const int32_t* pos_rows;
  int pos, window, page;
  const int32_t* remote;  // (B, cap)
  const int32_t* counts;  // (B)
  int cap;
  int B, Hq, Hkv, hd;
  float scale;
  void* out;  // (B, Hq, hd) contiguous
  int* err;
};

template <typename T>
__global__ __launch_bounds__(64 * GA_WAVES) void decode_attn_dense_kernel(DenseDecodeParams P) {
  __shared__ float qs_all[GA_WAVES][GA_MAX_HD];
  __shared__ float ps_all[GA_WAVES][64];
  __shared__ int64_t ks_all[GA_WAVES][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * GA_WAVES + w;  // (b, h)
  if (row >= static_cast<int64_t>(P.B) * P.Hq) return;
  const int b = static_cast<int>(row / P.Hq), h = static_cast<int>(row % P.Hq);
  const int g = h / (P.Hq / P.Hkv);
  const T* q = static_cast<const T*>(P.q) + row * P.hd;
  for (int d = lane; d < P.hd; d += 64) qs_all[w][d] = ld<T>(q, d);
  __builtin_amdgcn_wave_barrier();
  const int pos = P.pos_rows ? P.pos_rows[b] : P.pos;
  const int ls = max(0, pos + 1 - P.window);
  const int n_local = pos >= 0 ? pos - ls + 1 : 0;
  int cnt = P.cap > 0 ? P.counts[b] : 0;
  cnt = cnt < 0 ? 0 : (cnt > P.cap ? P.cap : cnt);
  const int total = n_local + cnt * P.page;
  const T* k = static_cast<const T*>(P.k) + b * P.ks_b + g * P.ks_h;
  const T* v = static_cast<const T*>(P.v) + b * P.vs_b + g * P.vs_h;
  Acc a;
  bool bad = false;
  for (int base = 0; base < total; base += 64) {
    const int i = base + lane;
    int tok = -1;
    if (i < n_local) {
      tok = ls + i;
    } else if (i < total) {
      const int j = (i - n_local) / P.page;
      const int pg = P.remote[static_cast<int64_t>(b) * P.cap + j];
      const int t = pg * P.page + (i - n_local) % P.page;
      if (pg >= 0 && t < P.S) tok = t;
      else bad = true;
    }
    if (tok >= P.S) tok = -1;
    // K rows by ks_t, V rows by vs_t: score with K, then accumulate with V
    const int64_t krow = tok >= 0 ? static_cast<int64_t>(tok) * P.ks_t : -1;
    float s = -INFINITY;
    if (krow >= 0) {
      float acc = 0.f;
      for (int d = 0; d < P.hd; ++d) acc = fmaf(qs_all[w][d], ld<T>(k + krow, d), acc);
      s = acc * P.scale;
    }
    const float cm = wave_max(s);
    if (cm == -INFINITY) continue;
    const float m_new = fmaxf(a.m, cm);
    const float alpha = a.m == -INFINITY ? 0.f : expf(a.m - m_new);
    const float p = krow >= 0 ? expf(s - m_new) : 0.f;
    a.l = a.l * alpha + wave_sum(p);
    a.m = m_new;
    ps_all[w][lane] = p;
    ks_all[w][lane] = tok >= 0 ? static_cast<int64_t>(tok) * P.vs_t : -1;
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int e = 0; e < GA_DPL; ++e) {
      const int d = lane + 64 * e;
      if (d >= P.hd) break;
      float o = a.o[e] * alpha;
      for (int j = 0; j < 64; ++j) {
        const int64_t r = ks_all[w][j];
        if (r >= 0) o = fmaf(ps_all[w][j], ld<T>(v + r, d), o);
      }
      a.o[e] = o;
    }
    __builtin_amdgcn_wave_barrier();
  }
  if (bad) set_error(P.err, FSI_ERR_INDEX_RANGE);
  write_out<T>(a, static_cast<T*>(P.out) + row * P.hd, P.hd, lane);
}

// ---------------------------------------------------------------------------
// Prefill over (B, H, T, hd) tensors given by element strides.
// ---------------------------------------------------------------------------
struct GenSparseParams {
  const void* q;
  int64_t qs_b, qs_h, qs_t;
  const void* k;
  int64_t ks_b, ks_h, ks_t;
  const void* v;
  int64_t vs_b, vs_h, vs_t;
  int B, Hq, Hkv, T, hd, block, mode, window;
  const int32_t* lists;
  int64_t ls_b, ls_q;
  int cap;
  const int32_t* counts;
  int64_t cs_b, cs_q;
  float scale;
  void* out;
  int64_t os_b, os_h, os_t;
  int* err;
};

template <typename T>
__global__ __launch_bounds__(64 * GA_WAVES) void sparse_attn_generic_kernel(GenSparseParams P) {
  __shared__ float qs_all[GA_WAVES][GA_MAX_HD];
  __shared__ float ps_all[GA_WAVES][64];
  __shared__ int64_t ks_all[GA_WAVES][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int t = blockIdx.x * GA_WAVES + w;
  const int bh = blockIdx.y;
  if (t >= P.T) return;
  const int b = bh / P.Hq, h = bh % P.Hq;
  const int g = h / (P.Hq / P.Hkv);
  const T* q = static_cast<const T*>(P.q) + b * P.qs_b + h * P.qs_h + static_cast<int64_t>(t) * P.qs_t;
  for (int d = lane; d < P.hd; d += 64) qs_all[w][d] = ld<T>(q, d);
  __builtin_amdgcn_wave_barrier();
  const T* k = static_cast<const T*>(P.k) + b * P.ks_b + g * P.ks_h;
  const T* v = static_cast<const T*>(P.v) + b * P.vs_b + g * P.vs_h;
  const int qb = t / P.block;
  const int n_blocks = (P.T + P.block - 1) / P.block;
  int cnt = P.counts[b * P.cs_b + qb * P.cs_q];
  cnt = cnt < 0 ? 0 : (cnt > P.cap ? P.cap : cnt);
  const int32_t* list = P.lists ? P.lists + b * P.ls_b + qb * P.ls_q : nullptr;
  const bool local = P.mode == FSI_SATTN_LOCAL_REMOTE;
  const int w0 = local ? max(0, t - P.window + 1) : 0;
  const int n_local = local ? t - w0 + 1 : 0;
  const int total = n_local + cnt * P.block;
  Acc a;
  bool bad = false;
  for (int base = 0; base < total; base += 64) {
    const int i = base + lane;
    int key = -1;
    if (i < n_local) {
      key = w0 + i;
    } else if (i < total) {
      const int j = (i - n_local) / P.block;
      const int pg = list[j];
      if (pg < 0 || pg >= n_blocks) {
        bad = true;
      } else {
        const int s = pg * P.block + (i - n_local) % P.block;
        bool keep = s < P.T;
        if (local) {
          // union semantics: skip keys the window already covers and pages listed earlier
          keep = keep && !(s > t - P.window && s <= t);
          for (int jj = 0; keep && jj < j; ++jj) keep = list[jj] != pg;
        }
        if (keep) key = s;
      }
    }
    const int64_t krow = key >= 0 ? static_cast<int64_t>(key) * P.ks_t : -1;
    float s = -INFINITY;
    if (krow >= 0) {
      float acc = 0.f;
      for (int d = 0; d < P.hd; ++d) acc = fmaf(qs_all[w][d], ld<T>(k + krow, d), acc);
      s = acc * P.scale;
    }
    const float cm = wave_max(s);
    if (cm == -INFINITY) continue;
    const float m_new = fmaxf(a.m, cm);
    const float alpha = a.m == -INFINITY ? 0.f : expf(a.m - m_new);
    const float p = krow >= 0 ? expf(s - m_new) : 0.f;
    a.l = a.l * alpha + wave_sum(p);
    a.m = m_new;
    ps_all[w][lane] = p;
    ks_all[w][lane] = key >= 0 ? static_cast<int64_t>(key) * P.vs_t : -1;
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int e = 0; e < GA_DPL; ++e) {
      const int d = lane + 64 * e;
      if (d >= P.hd) break;
      float o = a.o[e] * alpha;
      for (int j = 0; j < 64; ++j) {
        const int64_t r = ks_all[w][j];
        if (r >= 0) o = fmaf(ps_all[w][j], ld<T>(v + r, d), o);
      }
      a.o[e] = o;
    }
    __builtin_amdgcn_wave_barrier();
  }
  if (bad) set_error(P.err, FSI_ERR_INDEX_RANGE);
  T* out = static_cast<T*>(P.out) + b * P.os_b + h * P.os_h + static_cast<int64_t>(t) * P.os_t;
  write_out<T>(a, out, P.hd, lane);
}

}  // namespace

namespace fsi_dec32 {  // csrc/decode_attn_f32.hip: run() returns 1 when the call does not fit its kernels
size_t workspace_bytes(int64_t B, int64_t Hq, int64_t head_dim, int64_t window, int64_t capacity, int64_t page_size,
                       int64_t max_seq);
int run(const float* q, const float* k, const float* v, int64_t ks_b, int64_t ks_h, int64_t ks_t, int64_t vs_b,
        int64_t vs_h, int64_t vs_t, int64_t max_seq, const int32_t* pos_rows, int64_t pos, int64_t window,
        int64_t page_size, const int32_t* remote_pages, const int32_t* remote_counts, int64_t capacity, int64_t B,
        int64_t Hq, int64_t Hkv, int64_t head_dim, float scale, float* out, float* part, size_t part_bytes, int* err,
        hipStream_t st);
}  // namespace fsi_dec32

// Generic prefill launch used by fsi_sparse_attn for the cases its MFMA kernels
// do not take (fp32, block % 16 != 0, head_dim outside {16, 32, 64, 128}).
namespace fsi_attn_generic {

int sparse_attn(const void* q, int64_t qs_b, int64_t qs_h, int64_t qs_t, const void* k, int64_t ks_b, int64_t ks_h,
                int64_t ks_t, const void* v, int64_t vs_b, int64_t vs_h, int64_t vs_t, int64_t B, int64_t Hq,
                int64_t Hkv, int64_t T, int64_t head_dim, int64_t block, int mode, int64_t window,
                const int32_t* lists, int64_t ls_b, int64_t ls_q, int64_t capacity, const int32_t* counts,
                int64_t cs_b, int64_t cs_q, float scale, int dtype, void* out, int64_t os_b, int64_t os_h,
                int64_t os_t, int* err, void* stream) {
  FSI_CHECK_ARG(dtype == FSI_DTYPE_F32 || dtype == FSI_DTYPE_BF16, FSI_ERR_DTYPE, "sparse_attn: dtype %d", dtype);
  FSI_CHECK_ARG(head_dim > 0 && head_dim <= GA_MAX_HD, FSI_ERR_SHAPE, "sparse_attn: head_dim %lld (1..%d)",
                (long long)head_dim, GA_MAX_HD);
  FSI_CHECK_ARG(block > 0 && T > 0 && T <= (int64_t(1) << 30) && B * Hq <= 65535, FSI_ERR_SHAPE,
                "sparse_attn: block %lld T %lld B*Hq %lld", (long long)block, (long long)T, (long long)(B * Hq));
  GenSparseParams P{};
  P.q = q;
  P.qs_b = qs_b;
  P.qs_h = qs_h;
  P.qs_t = qs_t;
  P.k = k;
  P.ks_b = ks_b;
  P.ks_h = ks_h;
  P.ks_t = ks_t;
  P.v = v;
  P.vs_b = vs_b;
  P.vs_h = vs_h;
  P.vs_t = vs_t;
  P.B = (int)B;
  P.Hq = (int)Hq;
  P.Hkv = (int)Hkv;
  P.T = (int)T;
  P.hd = (int)head_dim;
  P.block = (int)block;
  P.mode = mode;
  P.window = (int)window;
  P.lists = lists;
  P.ls_b = ls_b;
  P.ls_q = ls_q;
  P.cap = (int)capacity;
  P.counts = counts;
  P.cs_b = cs_b;
  P.cs_q = cs_q;
  P.scale = scale;
  P.out = out;
  P.os_b = os_b;
  P.os_h = os_h;
  P.os_t = os_t;
  P.err = err;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>((T + GA_WAVES - 1) / GA_WAVES), static_cast<unsigned>(B * Hq));
  if (dtype == FSI_DTYPE_F32)
    sparse_attn_generic_kernel<float><<<grid, 64 * GA_WAVES, 0, s>>>(P);
  else
    sparse_attn_generic_kernel<bf16_t><<<grid, 64 * GA_WAVES, 0, s>>>(P);
  FSI_HIP_LAUNCH_CHECK("sparse_attn generic");
  return FSI_OK;
}

}  // namespace fsi_attn_generic

extern "C" {

FSI_API size_t fsi_decode_attn_dense_workspace_size(int64_t B, int64_t Hq, int64_t head_dim, int64_t window,
                                                    int64_t capacity, int64_t page_size, int64_t max_seq) {
  // the counter area every workspace starts with, then the split partials
  if (B <= 0 || Hq <= 0 || head_dim <= 0) return FSI_WORKSPACE_COUNTER_BYTES;
  return FSI_WORKSPACE_COUNTER_BYTES +
         fsi_dec32::workspace_bytes(B, Hq, head_dim, window < 0 ? 0 : window, capacity < 0 ? 0 : capacity,
                                    page_size < 1 ? 1 : page_size, max_seq < 1 ? 1 : max_seq);
}

FSI_API int fsi_decode_attn_dense(const void* q, const void* k_cache, const void* v_cache, int64_t ks_b, int64_t ks_h,
                                  int64_t ks_t, int64_t vs_b, int64_t vs_h, int64_t vs_t, int64_t max_seq,
                                  const int32_t* pos_rows, int64_t pos, int64_t window, int64_t page_size,
                                  const int32_t* remote_pages, const int32_t* remote_counts, int64_t capacity,
                                  int64_t B, int64_t Hq, int64_t Hkv, int64_t head_dim, float scale, int dtype,
                                  void* out, void* workspace, size_t workspace_bytes, int* err, void* stream) {
  FSI_CHECK_ARG(dtype == FSI_DTYPE_F32 || dtype == FSI_DTYPE_BF16, FSI_ERR_DTYPE, "decode_attn_dense: dtype %d",
                dtype);
  FSI_CHECK_ARG(head_dim > 0 && head_dim <= GA_MAX_HD, FSI_ERR_SHAPE, "decode_attn_dense: head_dim %lld (1..%d)",
                (long long)head_dim, GA_MAX_HD);
  FSI_CHECK_ARG(B >= 0 && Hkv > 0 && Hq > 0 && Hq % Hkv == 0 && page_size > 0 && window >= 0 && capacity >= 0 &&
                    max_seq > 0 && max_seq <= 0x7fffffff,
                FSI_ERR_SHAPE, "decode_attn_dense: bad sizes");
  FSI_CHECK_ARG(pos_rows || (pos >= 0 && pos < max_seq), FSI_ERR_INDEX_RANGE,
                "decode_attn_dense: position %lld outside the cache (%lld tokens)", (long long)pos,
                (long long)max_seq);
  if (B == 0) return FSI_OK;
  FSI_CHECK_ARG(q && k_cache && v_cache && out, FSI_ERR_INVALID_ARG, "decode_attn_dense: null pointer");
  FSI_CHECK_ARG(capacity == 0 || (remote_pages && remote_counts), FSI_ERR_INVALID_ARG,
                "decode_attn_dense: remote page list or counts missing");
  if (dtype == FSI_DTYPE_F32 && workspace != nullptr && workspace_bytes > FSI_WORKSPACE_COUNTER_BYTES) {
    // fp32 over the keys split across waves, on MFMA (csrc/decode_attn_f32.hip)
    const int rc = fsi_dec32::run(static_cast<const float*>(q), static_cast<const float*>(k_cache),
                                  static_cast<const float*>(v_cache), ks_b, ks_h, ks_t, vs_b, vs_h, vs_t, max_seq,
                                  pos_rows, pos, window, page_size, remote_pages, remote_counts, capacity, B, Hq, Hkv,
                                  head_dim, scale, static_cast<float*>(out),
                                  reinterpret_cast<float*>(static_cast<char*>(workspace) + FSI_WORKSPACE_COUNTER_BYTES),
                                  workspace_bytes - FSI_WORKSPACE_COUNTER_BYTES, err,
                                  reinterpret_cast<hipStream_t>(stream));
    if (rc != 1) return rc;
  }
  DenseDecodeParams P{};
  P.q = q;
  P.k = k_cache;
  P.v = v_cache;
  P.ks_b = ks_b;
  P.ks_h = ks_h;
  P.ks_t = ks_t;
  P.vs_b = vs_b;
  P.vs_h = vs_h;
  P.vs_t = vs_t;
  P.S = (int)max_seq;
  P.pos_rows = pos_rows;
  P.pos = (int)pos;
  P.window = (int)window;
  P.page = (int)page_size;
  P.remote = remote_pages;
  P.counts = remote_counts;
  P.cap = (int)capacity;
  P.B = (int)B;
  P.Hq = (int)Hq;
  P.Hkv = (int)Hkv;
  P.hd = (int)head_dim;
  P.scale = scale;
  P.out = out;
  P.err = err;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>((B * Hq + GA_WAVES - 1) / GA_WAVES));
  if (dtype == FSI_DTYPE_F32)
    decode_attn_dense_kernel<float><<<grid, 64 * GA_WAVES, 0, s>>>(P);
  else
    decode_attn_dense_kernel<bf16_t><<<grid, 64 * GA_WAVES, 0, s>>>(P);
  FSI_HIP_LAUNCH_CHECK("decode_attn_dense");
  return FSI_OK;
}

}  // extern "C"
