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
