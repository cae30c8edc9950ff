// HBM read-bandwidth probe: the practical ceiling the HBM-bound kernels of this
// library are measured against (a plain device copy through torch reaches less
// than this library's own paged-KV stream, so it cannot serve as the ceiling).
//
// Every lane streams 16-byte loads over a grid-strided range with UNROLL loads in
// flight, XOR-folds them into one register and writes one dword per lane, so the
// loads cannot be removed and the writes are negligible (4 bytes per 64 KiB+).
#include "fsi_common.h"

namespace {

template <int UNROLL>
__global__ __launch_bounds__(256) void stream_read_kernel(const fsi::u32x4_t* __restrict__ src, int64_t n16,
                                                          uint32_t* __restrict__ sink) {
  const int64_t tid = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  uint32_t acc = 0;
  int64_t i = tid;
  for (; i + (UNROLL - 1) * stride < n16; i += UNROLL * stride) {
    fsi::u32x4_t v[UNROLL];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) v[u] = __builtin_nontemporal_load(src + i + u * stride);
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
  }
  for (; i < n16; i += stride) {
    const fsi::u32x4_t v = src[i];
    acc ^= v[0] ^ v[1] ^ v[2] ^ v[3];
  }
  sink[tid] = acc;
}

}  // namespace

extern "C" {

/* Read `bytes` (a multiple of 16, 16-byte aligned) from src once with a grid of
 * `workgroups` x 256 lanes; sink receives workgroups * 256 dwords.  unroll: loads
 * in flight per lane (1, 4, 8 or 16).  For measurement only. */
FSI_API int fsi_stream_read(const void* src, int64_t bytes, int64_t workgroups, int unroll, uint32_t* sink,
                            void* stream) {
  FSI_CHECK_ARG(src && sink, FSI_ERR_INVALID_ARG, "stream_read: null pointer");
  FSI_CHECK_ARG(bytes > 0 && bytes % 16 == 0 && workgroups > 0 && workgroups <= (1 << 20), FSI_ERR_SHAPE,
                "stream_read: bytes %lld workgroups %lld", (long long)bytes, (long long)workgroups);
  FSI_CHECK_ARG(reinterpret_cast<uintptr_t>(src) % 16 == 0, FSI_ERR_ALIGN, "stream_read: src not 16-byte aligned");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const auto* s16 = static_cast<const fsi::u32x4_t*>(src);
  const dim3 grid(static_cast<unsigned>(workgroups));
  switch (unroll) {
    case 1: stream_read_kernel<1><<<grid, 256, 0, st>>>(s16, bytes / 16, sink); break;
    case 4: stream_read_kernel<4><<<grid, 256, 0, st>>>(s16, bytes / 16, sink); break;
    case 8: stream_read_kernel<8><<<grid, 256, 0, st>>>(s16, bytes / 16, sink); break;
    case 16: stream_read_kernel<16><<<grid, 256, 0, st>>>(s16, bytes / 16, sink); break;
    default: FSI_CHECK_ARG(false, FSI_ERR_INVALID_ARG, "stream_read: unroll %d (1, 4, 8 or 16)", unroll);
  }
  FSI_HIP_LAUNCH_CHECK("stream_read");
  return FSI_OK;
}

}  // extern "C"
