// Paged KV cache writer / reader and the C ABI of foveal decode attention
// (foveal_indexer/attention.py:339-367); the attention kernels themselves are
// in decode_attn_body.h, shared with the fused decode step of routing.hip.
#include <algorithm>
#include <atomic>
#include <mutex>

#include "decode_attn_body.h"

using namespace fsi;

namespace {

// ---------------------------------------------------------------------------
// Writer: scatter n_tok tokens per sequence from (B, Hkv, n_tok, HD) K and V
// (any strides in elements) into the paged pools at positions start .. start+n_tok-1
// (start per sequence or shared).  One thread per (b, g, token, 8 dims).
// ---------------------------------------------------------------------------
template <int HD>
__global__ __launch_bounds__(256) void kv_write_kernel(const bf16_t* __restrict__ k, const bf16_t* __restrict__ v,
                                                      int64_t ks_b, int64_t ks_g, int64_t ks_t, int64_t vs_b,
                                                      int64_t vs_g, int64_t vs_t, int B, int Hkv, int n_tok,
                                                      const int32_t* __restrict__ start_rows, int start,
                                                      const int32_t* __restrict__ page_table, int max_pages,
                                                      int64_t n_phys, bf16_t* __restrict__ k_pool,
                                                      bf16_t* __restrict__ v_pool, int* __restrict__ err) {
  constexpr int PIECES = HD / 8;
  const int64_t total = static_cast<int64_t>(B) * Hkv * n_tok * PIECES;
  for (int64_t gid = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; gid < total;
       gid += static_cast<int64_t>(gridDim.x) * 256) {
  const int piece = static_cast<int>(gid % PIECES);
  int64_t r = gid / PIECES;
  const int t = static_cast<int>(r % n_tok);
  r /= n_tok;
  const int g = static_cast<int>(r % Hkv);
  const int b = static_cast<int>(r / Hkv);
  const int p = (start_rows ? start_rows[b] : start) + t;
  const int lp = p / PAGE, off = p % PAGE;
  if (p < 0 || lp >= max_pages) {
    if (err) set_error(err, FSI_ERR_INDEX_RANGE);
    continue;
  }
  const int64_t phys = page_table[static_cast<int64_t>(b) * max_pages + lp];
  if (phys < 0 || phys >= n_phys) {
    if (err) set_error(err, FSI_ERR_INDEX_RANGE);
    continue;
  }
  const int64_t page_base = (phys * Hkv + g) * PAGE * HD;
  const int d0 = piece * 8;
  // K: chunk d0/32, token off, dims d0%32 .. +8 (16 contiguous bytes)
  const u32x4_t kv = *reinterpret_cast<const u32x4_t*>(k + b * ks_b + g * ks_g + t * ks_t + d0);
  *reinterpret_cast<u32x4_t*>(k_pool + page_base + (d0 / 32) * PAGE * 32 + off * 32 + (d0 % 32)) = kv;
  // V: half off/32, dim rows d0..d0+7, slot v_slot(off%32)
  const u32x4_t vv = *reinterpret_cast<const u32x4_t*>(v + b * vs_b + g * vs_g + t * vs_t + d0);
  bf16_t* vb = v_pool + page_base + (off / CHUNK) * HD * CHUNK + v_slot(off % CHUNK);
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    vb[(d0 + 2 * w) * CHUNK] = static_cast<bf16_t>(vv[w] & 0xffffu);
    vb[(d0 + 2 * w + 1) * CHUNK] = static_cast<bf16_t>(vv[w] >> 16);
  }
  }
}

// Reader for tests and cache export: pooled tokens [0, n_tok) of every
// sequence back to (B, Hkv, n_tok, HD).
template <int HD>
__global__ __launch_bounds__(256) void kv_read_kernel(const bf16_t* __restrict__ k_pool,
                                                     const bf16_t* __restrict__ v_pool, int B, int Hkv, int n_tok,
                                                     const int32_t* __restrict__ page_table, int max_pages,
                                                     int64_t n_phys, bf16_t* __restrict__ k_out,
                                                     bf16_t* __restrict__ v_out) {
  const int64_t total = static_cast<int64_t>(B) * Hkv * n_tok * HD;
  for (int64_t gid = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; gid < total;
       gid += static_cast<int64_t>(gridDim.x) * 256) {
  const int d = static_cast<int>(gid % HD);
  int64_t r = gid / HD;
  const int t = static_cast<int>(r % n_tok);
  r /= n_tok;
  const int g = static_cast<int>(r % Hkv);
  const int b = static_cast<int>(r / Hkv);
  const int lp = t / PAGE, off = t % PAGE;
  const int64_t phys = lp < max_pages ? page_table[static_cast<int64_t>(b) * max_pages + lp] : -1;
  bf16_t kk = 0, vv = 0;
  if (phys >= 0 && phys < n_phys) {
    const int64_t base = (phys * Hkv + g) * PAGE * HD;
    kk = k_pool[base + (d / 32) * PAGE * 32 + off * 32 + (d % 32)];
    vv = v_pool[base + (off / CHUNK) * HD * CHUNK + d * CHUNK + v_slot(off % CHUNK)];
  }
  k_out[gid] = kk;
  v_out[gid] = vv;
  }
}

}  // namespace

extern "C" {

FSI_API int fsi_kv_write(const void* k, const void* v, int64_t k_stride_b, int64_t k_stride_h, int64_t k_stride_t,
                         int64_t v_stride_b, int64_t v_stride_h, int64_t v_stride_t, int64_t B, int64_t Hkv,
                         int64_t n_tok, int64_t head_dim, const int32_t* start_rows, int64_t start,
                         const int32_t* page_table, int64_t max_pages, int64_t n_phys_pages, void* k_pool,
                         void* v_pool, int* err, void* stream) {
  using namespace fsi_host;
  FSI_CHECK_ARG(head_dim == 64 || head_dim == 128, FSI_ERR_SHAPE, "kv_write: head_dim %lld not 64 or 128",
                (long long)head_dim);
  FSI_CHECK_ARG(B >= 0 && Hkv > 0 && n_tok >= 0 && max_pages > 0 && n_phys_pages > 0 && start >= 0, FSI_ERR_SHAPE,
                "kv_write: bad sizes");
  FSI_CHECK_ARG(max_pages * PAGE <= 0x7fffffff && B <= 0x7fffffff && n_tok <= 0x7fffffff, FSI_ERR_SHAPE,
                "kv_write: sizes beyond int32");
  if (B == 0 || n_tok == 0) return FSI_OK;
  FSI_CHECK_ARG(k && v && page_table && k_pool && v_pool, FSI_ERR_INVALID_ARG, "kv_write: null pointer");
  FSI_CHECK_ARG(reinterpret_cast<uintptr_t>(k) % 16 == 0 && reinterpret_cast<uintptr_t>(v) % 16 == 0 &&
                    (k_stride_b | k_stride_h | k_stride_t | v_stride_b | v_stride_h | v_stride_t) % 8 == 0,
                FSI_ERR_ALIGN, "kv_write: K/V rows must be 16-byte aligned");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int64_t total = B * Hkv * n_tok * (head_dim / 8);
  const unsigned grid = static_cast<unsigned>(std::min<int64_t>((total + 255) / 256, 1 << 20));
#define KVW(HDV)                                                                                                   \
  kv_write_kernel<HDV><<<grid, 256, 0, st>>>(                                                                      \
      static_cast<const bf16_t*>(k), static_cast<const bf16_t*>(v), k_stride_b, k_stride_h, k_stride_t,             \
      v_stride_b, v_stride_h, v_stride_t, (int)B, (int)Hkv, (int)n_tok, start_rows, (int)start, page_table,         \
      (int)max_pages, n_phys_pages, static_cast<bf16_t*>(k_pool), static_cast<bf16_t*>(v_pool), err)
  if (head_dim == 128) KVW(128);
  else KVW(64);
#undef KVW
  FSI_HIP_LAUNCH_CHECK("kv_write");
  return FSI_OK;
}

FSI_API int fsi_kv_read(const void* k_pool, const void* v_pool, int64_t B, int64_t Hkv, int64_t n_tok,
                        int64_t head_dim, const int32_t* page_table, int64_t max_pages, int64_t n_phys_pages,
                        void* k_out, void* v_out, void* stream) {
  using namespace fsi_host;
  FSI_CHECK_ARG(head_dim == 64 || head_dim == 128, FSI_ERR_SHAPE, "kv_read: head_dim %lld not 64 or 128",
                (long long)head_dim);
  FSI_CHECK_ARG(B >= 0 && Hkv > 0 && n_tok >= 0 && max_pages > 0 && n_phys_pages > 0, FSI_ERR_SHAPE,
                "kv_read: bad sizes");
  if (B == 0 || n_tok == 0) return FSI_OK;
  FSI_CHECK_ARG(k_pool && v_pool && page_table && k_out && v_out, FSI_ERR_INVALID_ARG, "kv_read: null pointer");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int64_t total = B * Hkv * n_tok * head_dim;
  const unsigned grid = static_cast<unsigned>(std::min<int64_t>((total + 255) / 256, 1 << 20));
#define KVR(HDV)                                                                                                  \
  kv_read_kernel<HDV><<<grid, 256, 0, st>>>(static_cast<const bf16_t*>(k_pool), static_cast<const bf16_t*>(v_pool), \
                                            (int)B, (int)Hkv, (int)n_tok, page_table, (int)max_pages,              \
                                            n_phys_pages, static_cast<bf16_t*>(k_out), static_cast<bf16_t*>(v_out))
  if (head_dim == 128) KVR(128);
  else KVR(64);
#undef KVR
  FSI_HIP_LAUNCH_CHECK("kv_read");
  return FSI_OK;
}

}  // extern "C"

namespace {

// Scratch of fsi_decode_attn_noalloc: the per-wave partials live in this
// file-scope device array, one copy per GPU, held until the process ends.  Host
// code never passes the symbol itself to a kernel: the array's device address
// is looked up once per device with hipGetSymbolAddress.
constexpr size_t NOALLOC_SCRATCH_BYTES = FSI_DECODE_ATTN_NOALLOC_MAX_BYTES;
__device__ __align__(256) char scratch[NOALLOC_SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;
std::atomic<char*> g_scratch_ptr[MAX_DEVICES];
std::mutex g_scratch_mu;

// Device address of `scratch` on the current device (looked up on the first call
// there, with that device current), or null with the last-error message set.
char* scratch_on_current_device() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) {
    fsi_host::set_last_error("decode_attn_noalloc: no current HIP device (or index >= %d)", MAX_DEVICES);
    return nullptr;
  }
  char* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (p) return p;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
  if (p) return p;
  void* addr = nullptr;
  const hipError_t e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
  if (e != hipSuccess || addr == nullptr) {
    fsi_host::set_last_error("decode_attn_noalloc: hipGetSymbolAddress(scratch) on device %d: %s", dev,
                             hipGetErrorString(e));
    return nullptr;
  }
  p = static_cast<char*>(addr);
  g_scratch_ptr[dev].store(p, std::memory_order_release);
  return p;
}

}  // namespace

extern "C" {

FSI_API size_t fsi_decode_attn_workspace_size(int64_t B, int64_t Hq, int64_t Hkv, int64_t head_dim, int64_t window,
                                              int64_t capacity, int64_t max_pages) {
  if (B <= 0 || Hkv <= 0 || Hq <= 0 || head_dim <= 0 || max_pages <= 0 || window < 0 || capacity < 0)
    return FSI_WORKSPACE_COUNTER_BYTES;
  return FSI_WORKSPACE_COUNTER_BYTES + decode_attn_partials_bytes(B, Hq, Hkv, head_dim, window, capacity, max_pages) +
         256;
}

FSI_API int fsi_decode_attn(const void* q, const void* k_pool, const void* v_pool, const int32_t* page_table,
                            int64_t max_pages, int64_t n_phys_pages, const int32_t* pos_rows, int64_t pos,
                            int64_t window, const int32_t* remote_pages, const int32_t* remote_counts,
                            int64_t capacity, int64_t B, int64_t Hq, int64_t Hkv, int64_t head_dim, float scale,
                            void* out, void* workspace, size_t workspace_bytes, int* err, void* stream) {
  const int c = decode_attn_check(q, k_pool, v_pool, page_table, max_pages, n_phys_pages, pos_rows, pos, window,
                                  remote_pages, remote_counts, capacity, B, Hq, Hkv, head_dim, out);
  if (c != FSI_OK || B == 0) return c;
  const size_t need = fsi_decode_attn_workspace_size(B, Hq, Hkv, head_dim, window, capacity, max_pages);
  FSI_CHECK_ARG(workspace && workspace_bytes >= need, FSI_ERR_WORKSPACE, "decode_attn: workspace %zu < %zu bytes",
                workspace_bytes, need);
  FSI_CHECK_ARG(reinterpret_cast<uintptr_t>(workspace) % 16 == 0, FSI_ERR_ALIGN,
                "decode_attn: workspace must be 16-byte aligned");
  return decode_attn_launch(q, k_pool, v_pool, page_table, max_pages, n_phys_pages, pos_rows, pos, window,
                            remote_pages, remote_counts, capacity, B, Hq, Hkv, head_dim, scale, out,
                            static_cast<char*>(workspace) + FSI_WORKSPACE_COUNTER_BYTES, err, stream);
}

FSI_API int fsi_decode_attn_noalloc(const void* q, const void* k_pool, const void* v_pool, const int32_t* page_table,
                                    int64_t max_pages, int64_t n_phys_pages, const int32_t* pos_rows, int64_t pos,
                                    int64_t window, const int32_t* remote_pages, const int32_t* remote_counts,
                                    int64_t capacity, int64_t B, int64_t Hq, int64_t Hkv, int64_t head_dim,
                                    float scale, void* out, int* err, void* stream) {
  const int c = decode_attn_check(q, k_pool, v_pool, page_table, max_pages, n_phys_pages, pos_rows, pos, window,
                                  remote_pages, remote_counts, capacity, B, Hq, Hkv, head_dim, out);
  if (c != FSI_OK || B == 0) return c;
  const size_t need = decode_attn_partials_bytes(B, Hq, Hkv, head_dim, window, capacity, max_pages);
  FSI_CHECK_ARG(need <= NOALLOC_SCRATCH_BYTES, FSI_ERR_CAPACITY,
                "decode_attn_noalloc: %zu bytes of partials exceed the %zu-byte device scratch "
                "(use fsi_decode_attn with a workspace)",
                need, NOALLOC_SCRATCH_BYTES);
  char* ws = scratch_on_current_device();
  if (!ws) return FSI_ERR_HIP;
  return decode_attn_launch(q, k_pool, v_pool, page_table, max_pages, n_phys_pages, pos_rows, pos, window,
                            remote_pages, remote_counts, capacity, B, Hq, Hkv, head_dim, scale, out, ws, err, stream);
}

}  // extern "C"

namespace {

// ---------------------------------------------------------------------------
// Query gradient of decode attention (the cache is inference state, a
// constant): dq_h = scale sum_t p_t (dout_h . v_t - dout_h . o_h) k_t over
// each sequence's support (window tokens, then every token of each selected
// page, as the forward attends it).  One wave per (sequence, query head), two
// passes over the support in chunks of 64 tokens: the softmax statistics and
// o, then dq.  Paged pools (bf16, page 64) are read through the page table in
// their MFMA layouts; the contiguous reference-layout cache by its strides.
// ---------------------------------------------------------------------------
struct DecodeBwdParams {
  const void* q;     // (B, Hq, hd) contiguous
  const void* dout;  // (B, Hq, hd) contiguous
  const void* k;
  const void* v;
  int64_t ks_b, ks_h, ks_t, vs_b, vs_h, vs_t;  // contiguous cache strides
  const int32_t* page_table;                   // paged pools
  int max_pages;
  int64_t n_phys;
  int S;  // tokens the contiguous cache holds
  const int32_t* pos_rows;
  int pos, window, page;
  const int32_t* remote;
  const int32_t* counts;
  int cap;
  int B, Hq, Hkv, hd;
  float scale;
  float* dq;  // (B, Hq, hd) fp32
  int* err;
};

constexpr int DB_WAVES = 4;
constexpr int DB_MAX_HD = 256;
constexpr int DB_DPL = DB_MAX_HD / 64;

template <typename T>
__device__ __forceinline__ float db_ld(const T* p, int64_t i);
template <>
__device__ __forceinline__ float db_ld<float>(const float* p, int64_t i) { return p[i]; }
template <>
__device__ __forceinline__ float db_ld<bf16_t>(const bf16_t* p, int64_t i) { return bf16_to_f32(p[i]); }

// Element d of key / value token `tok` (offsets per token computed once):
// paged K: kb + (d / 32) * 64 * 32 + d % 32, V: vb + d * 32; contiguous: kb + d, vb + d.
template <bool PAGED>
__device__ __forceinline__ int64_t db_koff(int64_t kb, int d) {
  return PAGED ? kb + (d >> 5) * (PAGE * CHUNK) + (d & 31) : kb + d;
}
template <bool PAGED>
__device__ __forceinline__ int64_t db_voff(int64_t vb, int d) {
  return PAGED ? vb + static_cast<int64_t>(d) * CHUNK : vb + d;
}

template <typename T, bool PAGED>
__global__ __launch_bounds__(64 * DB_WAVES) void decode_bwd_q_kernel(DecodeBwdParams P) {
  __shared__ float qs_all[DB_WAVES][DB_MAX_HD], gs_all[DB_WAVES][DB_MAX_HD];
  __shared__ float ps_all[DB_WAVES][64];
  __shared__ int64_t kb_all[DB_WAVES][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * DB_WAVES + w;  // (b, h)
  if (row >= static_cast<int64_t>(P.B) * P.Hq) return;  // whole wave; no workgroup barrier follows
  const int b = static_cast<int>(row / P.Hq), h = static_cast<int>(row % P.Hq);
  const int g = h / (P.Hq / P.Hkv);
  const T* q = static_cast<const T*>(P.q) + row * P.hd;
  const T* go = static_cast<const T*>(P.dout) + row * P.hd;
  for (int d = lane; d < P.hd; d += 64) {
    qs_all[w][d] = db_ld<T>(q, d);
    gs_all[w][d] = db_ld<T>(go, d);
  }
  __builtin_amdgcn_wave_barrier();
  const T* kp = static_cast<const T*>(P.k);
  const T* vp = static_cast<const T*>(P.v);
  const int pos = P.pos_rows ? P.pos_rows[b] : P.pos;
  const int ls = max(0, pos + 1 - P.window);
  const int n_local = pos >= 0 ? pos - ls + 1 : 0;
  int cnt = P.cap > 0 ? P.counts[b] : 0;
  cnt = cnt < 0 ? 0 : (cnt > P.cap ? P.cap : cnt);
  const int total = n_local + cnt * P.page;
  bool bad = false;
  // token i of the support -> (key offset, value offset), or -1 when skipped
  auto locate = [&](int i, int64_t& kb, int64_t& vb) {
    int tok = -1;
    if (i < n_local) {
      tok = ls + i;
    } else if (i < total) {
      const int j = (i - n_local) / P.page;
      const int pg = P.remote[static_cast<int64_t>(b) * P.cap + j];
      if (pg >= 0) tok = pg * P.page + (i - n_local) % P.page;
    }
    kb = vb = -1;
    if (tok < 0) {
      if (i < total) bad = true;
      return;
    }
    if (PAGED) {
      const int lp = tok / PAGE, off = tok % PAGE;
      if (lp >= P.max_pages) {
        bad = true;
        return;
      }
      const int64_t phys = P.page_table[static_cast<int64_t>(b) * P.max_pages + lp];
      if (phys < 0 || phys >= P.n_phys) {
        bad = true;
        return;
      }
      const int64_t base = (phys * P.Hkv + g) * PAGE * P.hd;
      kb = base + off * CHUNK;
      vb = base + (off / CHUNK) * P.hd * CHUNK + v_slot(off % CHUNK);
    } else {
      if (tok >= P.S) {
        bad = true;
        return;
      }
      kb = b * P.ks_b + g * P.ks_h + static_cast<int64_t>(tok) * P.ks_t;
      vb = b * P.vs_b + g * P.vs_h + static_cast<int64_t>(tok) * P.vs_t;
    }
  };
  auto score = [&](int64_t kb) {
    float acc = 0.f;
    for (int d = 0; d < P.hd; ++d) acc = fmaf(qs_all[w][d], db_ld<T>(kp, db_koff<PAGED>(kb, d)), acc);
    return acc * P.scale;
  };

  // pass 1: m, l and o = sum p v (lanes over head dims for o)
  float m = -INFINITY, l = 0.f;
  float o[DB_DPL] = {0.f, 0.f, 0.f, 0.f};
  for (int base = 0; base < total; base += 64) {
    int64_t kb, vb;
    locate(base + lane, kb, vb);
    const float s = kb >= 0 ? score(kb) : -INFINITY;
    const float cm = wave_max(s);
    if (cm == -INFINITY) continue;
    const float mn = fmaxf(m, cm);
    const float alpha = m == -INFINITY ? 0.f : expf(m - mn);
    const float p = kb >= 0 ? expf(s - mn) : 0.f;
    l = l * alpha + wave_sum(p);
    m = mn;
    ps_all[w][lane] = p;
    kb_all[w][lane] = vb;
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int e = 0; e < DB_DPL; ++e) {
      const int d = lane + 64 * e;
      if (d >= P.hd) break;
      float acc = o[e] * alpha;
      for (int j = 0; j < 64; ++j) {
        const int64_t r = kb_all[w][j];
        if (r >= 0) acc = fmaf(ps_all[w][j], db_ld<T>(vp, db_voff<PAGED>(r, d)), acc);
      }
      o[e] = acc;
    }
    __builtin_amdgcn_wave_barrier();
  }
  float dd = 0.f;  // D = dout . o
#pragma unroll
  for (int e = 0; e < DB_DPL; ++e) {
    const int d = lane + 64 * e;
    if (d < P.hd) dd = fmaf(gs_all[w][d], l > 0.f ? o[e] / l : 0.f, dd);
  }
  dd = wave_sum(dd);

  // pass 2: dq = scale sum_t p_t (dout . v_t - D) k_t (lanes over head dims)
  float gq[DB_DPL] = {0.f, 0.f, 0.f, 0.f};
  if (l > 0.f) {
    for (int base = 0; base < total; base += 64) {
      int64_t kb, vb;
      locate(base + lane, kb, vb);
      float ds = 0.f;
      if (kb >= 0) {
        const float p = expf(score(kb) - m) / l;
        float dp = 0.f;
        for (int d = 0; d < P.hd; ++d) dp = fmaf(gs_all[w][d], db_ld<T>(vp, db_voff<PAGED>(vb, d)), dp);
        ds = p * (dp - dd);
      }
      ps_all[w][lane] = ds;
      kb_all[w][lane] = kb;
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int e = 0; e < DB_DPL; ++e) {
        const int d = lane + 64 * e;
        if (d >= P.hd) break;
        float acc = gq[e];
        for (int j = 0; j < 64; ++j) {
          const int64_t r = kb_all[w][j];
          if (r >= 0) acc = fmaf(ps_all[w][j], db_ld<T>(kp, db_koff<PAGED>(r, d)), acc);
        }
        gq[e] = acc;
      }
      __builtin_amdgcn_wave_barrier();
    }
  }
  if (bad && P.err) set_error(P.err, FSI_ERR_INDEX_RANGE);
#pragma unroll
  for (int e = 0; e < DB_DPL; ++e) {
    const int d = lane + 64 * e;
    if (d < P.hd) P.dq[row * P.hd + d] = gq[e] * P.scale;
  }
}

}  // namespace

extern "C" {

FSI_API int fsi_decode_attn_bwd_q(const void* q, const void* dout, const void* k_cache, const void* v_cache,
                                  int64_t ks_b, int64_t ks_h, int64_t ks_t, int64_t vs_b, int64_t vs_h, int64_t vs_t,
                                  int64_t max_seq, const int32_t* page_table, int64_t max_pages, int64_t n_phys_pages,
                                  const int32_t* pos_rows, int64_t pos, int64_t window, int64_t page_size,
                                  const int32_t* remote_pages, const int32_t* remote_counts, int64_t capacity,
                                  int64_t B, int64_t Hq, int64_t Hkv, int64_t head_dim, float scale, int dtype,
                                  float* dq, int* err, void* stream) {
  using namespace fsi_host;
  FSI_CHECK_ARG(dtype == FSI_DTYPE_F32 || dtype == FSI_DTYPE_BF16, FSI_ERR_DTYPE, "decode_attn_bwd_q: dtype %d",
                dtype);
  FSI_CHECK_ARG(head_dim > 0 && head_dim <= DB_MAX_HD, FSI_ERR_SHAPE, "decode_attn_bwd_q: head_dim %lld (1..%d)",
                (long long)head_dim, DB_MAX_HD);
  FSI_CHECK_ARG(B >= 0 && Hkv > 0 && Hq > 0 && Hq % Hkv == 0 && window >= 0 && capacity >= 0 && page_size > 0,
                FSI_ERR_SHAPE, "decode_attn_bwd_q: bad sizes");
  const bool paged = page_table != nullptr;
  FSI_CHECK_ARG(!paged || (dtype == FSI_DTYPE_BF16 && page_size == PAGE && (head_dim == 64 || head_dim == 128) &&
                           max_pages > 0 && n_phys_pages > 0),
                FSI_ERR_SHAPE, "decode_attn_bwd_q: paged pools hold bf16 pages of 64 tokens, head_dim 64 or 128");
  FSI_CHECK_ARG(paged || (max_seq > 0 && max_seq <= 0x7fffffff), FSI_ERR_SHAPE, "decode_attn_bwd_q: max_seq");
  FSI_CHECK_ARG(B * Hq <= (int64_t)0x7fffffff && (paged ? max_pages * PAGE : max_seq) <= 0x7fffffff, FSI_ERR_SHAPE,
                "decode_attn_bwd_q: sizes beyond int32");
  if (B == 0) return FSI_OK;
  FSI_CHECK_ARG(q && dout && k_cache && v_cache && dq, FSI_ERR_INVALID_ARG, "decode_attn_bwd_q: null pointer");
  FSI_CHECK_ARG(capacity == 0 || (remote_pages && remote_counts), FSI_ERR_INVALID_ARG,
                "decode_attn_bwd_q: remote page list or counts missing");
  DecodeBwdParams P{};
  P.q = q;
  P.dout = dout;
  P.k = k_cache;
  P.v = v_cache;
  P.ks_b = ks_b;
  P.ks_h = ks_h;
  P.ks_t = ks_t;
  P.vs_b = vs_b;
  P.vs_h = vs_h;
  P.vs_t = vs_t;
  P.page_table = page_table;
  P.max_pages = (int)max_pages;
  P.n_phys = n_phys_pages;
  P.S = (int)max_seq;
  P.pos_rows = pos_rows;
  P.pos = (int)pos;
  P.window = (int)(window < 0x7fffffff ? window : 0x7fffffff);
  P.page = (int)page_size;
  P.remote = remote_pages;
  P.counts = remote_counts;
  P.cap = (int)capacity;
  P.B = (int)B;
  P.Hq = (int)Hq;
  P.Hkv = (int)Hkv;
  P.hd = (int)head_dim;
  P.scale = scale;
  P.dq = dq;
  P.err = err;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const unsigned grid = static_cast<unsigned>((B * Hq + DB_WAVES - 1) / DB_WAVES);
  if (paged) decode_bwd_q_kernel<bf16_t, true><<<grid, 64 * DB_WAVES, 0, st>>>(P);
  else if (dtype == FSI_DTYPE_F32) decode_bwd_q_kernel<float, false><<<grid, 64 * DB_WAVES, 0, st>>>(P);
  else decode_bwd_q_kernel<bf16_t, false><<<grid, 64 * DB_WAVES, 0, st>>>(P);
  FSI_HIP_LAUNCH_CHECK("decode_attn_bwd_q");
  return FSI_OK;
}

}  // extern "C"
