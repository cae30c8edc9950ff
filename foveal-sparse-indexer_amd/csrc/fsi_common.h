// Shared device/host helpers for the foveal sparse-indexer HIP kernels (gfx950 / CDNA4).
//
// Everything here is written for 64-lane wavefronts and the gfx950 bf16 MFMA
// instructions (v_mfma_f32_16x16x32_bf16).  No other target is supported.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "fsi.h"

namespace fsi {

// ---------------------------------------------------------------------------
// bf16 storage type: raw 16-bit pattern.  Conversions are explicit and use
// round-to-nearest-even, which is what torch's CPU bf16 casts do.
// ---------------------------------------------------------------------------
typedef uint16_t bf16_t;

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;
typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4_t;
typedef __attribute__((__vector_size__(2 * sizeof(uint32_t)))) uint32_t u32x2_t;

__device__ __forceinline__ float bf16_to_f32(bf16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

__device__ __forceinline__ bf16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<bf16_t>((u >> 16) | 0x40u);  // quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<bf16_t>(u >> 16);
}

// Round an fp32 value to the nearest bf16 and return it widened back to fp32.
__device__ __forceinline__ float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// Low / high bf16 of a packed dword, widened to fp32.
__device__ __forceinline__ float lo_bf16(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_bf16(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return static_cast<uint32_t>(f32_to_bf16(lo)) | (static_cast<uint32_t>(f32_to_bf16(hi)) << 16);
}

// ---------------------------------------------------------------------------
// MFMA wrapper.  16x16x32 bf16: lane l supplies A[l%16][8*(l/16)+e] and
// B[8*(l/16)+e][l%16] for e = 0..7; it receives C[4*(l/16)+j][l%16], j = 0..3.
// ---------------------------------------------------------------------------
__device__ __forceinline__ f32x4_t mfma16x16x32(const u32x4_t& a, const u32x4_t& b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                  __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// ---------------------------------------------------------------------------
// Activation codes (foveal_indexer/pattention_triton.py:245) and rounding modes.
// ---------------------------------------------------------------------------
enum Act : int { ACT_SWIGLU = 0, ACT_SILU = 1, ACT_GELU = 2, ACT_RELU = 3, ACT_RELU2 = 4 };

__device__ __forceinline__ float silu_f32(float g) { return g / (1.0f + expf(-g)); }
__device__ __forceinline__ float gelu_f32(float g) {
  return 0.5f * g * (1.0f + erff(g * 0.70710678118654752440f));
}

// Activation epilogue for bf16 Pattention.
//   FSI_ROUND_EAGER : g,u -> bf16; f(g) -> bf16; [product -> bf16]          (torch eager)
//   FSI_ROUND_FUSED : g,u -> bf16; one rounding of f(g)[*u] computed in fp32 (fused SwiGLU)
//   FSI_ROUND_FP32  : f(g)[*u] from the fp32 accumulators, one rounding      (fused Pattention)
template <int ACT>
__device__ __forceinline__ float pattention_act(float g, float u, int rounding) {
  if (rounding != FSI_ROUND_FP32) {
    g = round_bf16(g);
    u = round_bf16(u);
  }
  float a;
  if (ACT == ACT_SWIGLU) {
    float s = silu_f32(g);
    if (rounding == FSI_ROUND_EAGER) s = round_bf16(s);
    a = s * u;
  } else if (ACT == ACT_SILU) {
    a = silu_f32(g);
  } else if (ACT == ACT_GELU) {
    a = gelu_f32(g);
  } else if (ACT == ACT_RELU) {
    a = fmaxf(g, 0.0f);
  } else {  // ACT_RELU2
    float r = fmaxf(g, 0.0f);
    if (rounding == FSI_ROUND_EAGER) r = round_bf16(r);
    a = r * r;
  }
  return a;
}

// ---------------------------------------------------------------------------
// Sum / max over the lanes l, l ^ 16, l ^ 32, l ^ 48 (the four row groups of a
// 16 x 16 MFMA result column) with gfx950's v_permlane16_swap / v_permlane32_swap.
// Each swap leaves a lane's own value in one output and its partner's in the
// other, so combining the two outputs reduces a pair.  VALU only: a shuffle that
// compiles to ds_bpermute is an LDS instruction, and in a kernel with
// direct-to-LDS loads in flight the compiler waits for all of them before it.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float sum_rows4(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}
__device__ __forceinline__ float max_rows4(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

// v_max3_f32 as written.  fmaxf's IEEE semantics make the compiler quiet every
// operand it cannot prove canonical (a v_max_f32 x, x, x each); for scores that are
// finite or -inf (softmax maxima) that doubles the instructions of a max tree.
__device__ __forceinline__ float max3_raw(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

// ---------------------------------------------------------------------------
// Wave-level reductions (64 lanes).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}
__device__ __forceinline__ int wave_sum_i(int v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// ---------------------------------------------------------------------------
// Device-side error word.  Kernels never read out of bounds; when an input
// index is out of range they skip it and record the first error code here.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void set_error(int* err, int code) {
  if (err) atomicCAS(err, 0, code);
}

}  // namespace fsi

// ---------------------------------------------------------------------------
// Host-side helpers shared by the C-ABI entry points.
// ---------------------------------------------------------------------------
namespace fsi_host {

void set_last_error(const char* fmt, ...);

#define FSI_CHECK_ARG(cond, code, ...)        \
  do {                                        \
    if (!(cond)) {                            \
      ::fsi_host::set_last_error(__VA_ARGS__); \
      return (code);                          \
    }                                         \
  } while (0)

#define FSI_HIP_LAUNCH_CHECK(what)                                              \
  do {                                                                          \
    hipError_t e_ = hipGetLastError();                                          \
    if (e_ != hipSuccess) {                                                     \
      ::fsi_host::set_last_error("%s: %s", (what), hipGetErrorString(e_));      \
      return FSI_ERR_HIP;                                                       \
    }                                                                           \
  } while (0)

inline bool is_pow2(int64_t v) { return v > 0 && (v & (v - 1)) == 0; }
inline int ilog2(int64_t v) {
  int r = 0;
  while ((int64_t(1) << r) < v) ++r;
  return r;
}
inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

}  // namespace fsi_host
