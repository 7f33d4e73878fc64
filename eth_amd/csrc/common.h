// Shared helpers for the eth_amd HIP kernels (gfx950 / CDNA4 only).
//
// Every exported entry point returns an int status (ETH_OK on success) and
// records a message retrievable through eth_last_error().  Kernels are
// launched on the caller's stream; nothing here allocates device memory on a
// hot path.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <string>

#include "../../include/eth_amd.h"

namespace eth {

void set_error(const char* fmt, ...);

#define ETH_CHECK_ARG(cond, ...)              \
  do {                                        \
    if (!(cond)) {                            \
      ::eth::set_error(__VA_ARGS__);          \
      return ETH_ERR_INVALID;                 \
    }                                         \
  } while (0)

#define ETH_CHECK_LAUNCH(what)                                              \
  do {                                                                      \
    hipError_t _e = hipGetLastError();                                      \
    if (_e != hipSuccess) {                                                 \
      ::eth::set_error("%s: launch failed: %s", what, hipGetErrorString(_e)); \
      return ETH_ERR_HIP;                                                   \
    }                                                                       \
  } while (0)

typedef uint16_t bf16_t;
typedef _Float16 f16_t;

// float -> bfloat16, round to nearest even (v_cvt_pk_bf16_f32; denormals are
// kept, NaN stays NaN).
__device__ __forceinline__ bf16_t f2bf(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}
// two floats -> packed bf16 pair (lo in bits 0-15), one conversion instruction
typedef float eth_f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 eth_bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t f2bf_pair(float lo, float hi) {
  const eth_f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, eth_bf16x2_t));
}
// two floats -> packed fp16 pair (lo in bits 0-15), each rounded to nearest
// even from its fp32 value.  The empty asm pins the fp32 values in
// registers: otherwise the compiler may fold the multiply that produced them
// into a mixed-precision fma with a +0 addend (v_fma_mixlo_f16), which
// rounds the exact product once and turns a -0 product into +0.
typedef _Float16 eth_f16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t f2h_pair(float lo, float hi) {
  eth_f32x2_t v = {lo, hi};
  asm volatile("" : "+v"(v));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, eth_f16x2_t));
}
// the same rounding for one value, returned as fp32
__device__ __forceinline__ float round_to_f16(float f) {
  asm volatile("" : "+v"(f));
  return (float)(_Float16)f;
}
__device__ __forceinline__ float bf2f(bf16_t h) {
  return __uint_as_float(((uint32_t)h) << 16);
}
// float -> fp16 bits, rounded to nearest even from the fp32 value (pinned
// in a register for the reason given at f2h_pair)
__device__ __forceinline__ uint16_t f2h_bits(float f) {
  asm volatile("" : "+v"(f));
  return __builtin_bit_cast(uint16_t, (f16_t)f);
}
__device__ __forceinline__ float h2f_bits(uint16_t b) {
  f16_t h = *reinterpret_cast<f16_t*>(&b);
  return (float)h;
}

// Load/store one element of a tensor whose dtype is chosen at run time.
__device__ __forceinline__ float load_elem(const void* p, int64_t i, int dtype) {
  if (dtype == ETH_F32) return reinterpret_cast<const float*>(p)[i];
  uint16_t b = reinterpret_cast<const uint16_t*>(p)[i];
  return dtype == ETH_BF16 ? bf2f(b) : h2f_bits(b);
}
__device__ __forceinline__ void store_elem(void* p, int64_t i, int dtype, float v) {
  if (dtype == ETH_F32) {
    reinterpret_cast<float*>(p)[i] = v;
  } else {
    reinterpret_cast<uint16_t*>(p)[i] = dtype == ETH_BF16 ? f2bf(v) : f2h_bits(v);
  }
}

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

// Block-wide sum for blockDim.x == NT (multiple of 64).  `red` must hold
// NT/64 floats of shared memory.  Every thread receives the total.
template <int NT>
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  if (lane == 0) red[wid] = v;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int w = 0; w < NT / 64; ++w) t += red[w];
  __syncthreads();
  return t;
}

// out[c] (+)= sum_g part[g*ld + c] for c < cols (cols % 4 == 0, part and ld
// 16-byte aligned): 64 columns per workgroup, one round trip of float4 loads
// per lane, fixed summation order (deterministic).  With gridDim.y == 2 the
// second slab (columns [cols, 2 cols) of each partial row) goes to out1.
__global__ void reduce_partials_kernel(const float* __restrict__ part, int groups, int cols, int64_t ld,
                                       float* __restrict__ out0, float* __restrict__ out1, int accumulate);
inline dim3 reduce_partials_grid(int cols, int slabs = 1) { return dim3((cols + 63) / 64, slabs); }
constexpr int kReducePartialsThreads = 256;

// 32-bit mix of (seed, index): the dropout keep decision of element `idx`
// (kept when >= p * 2^32).  Shared by every kernel that applies or replays a
// dropout mask, so they all draw the same one.
__device__ __forceinline__ uint32_t hash_u32(uint64_t seed, uint64_t idx) {
  uint64_t z = seed + 0x9E3779B97F4A7C15ull * (idx + 1);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  z ^= z >> 31;
  return (uint32_t)(z >> 32);
}

// Host side of the dropout mask: keep threshold (0 when p == 0, no mask) and
// the 1/(1-p) scale of kept elements.
inline void dropout_params(float p, uint32_t& thresh, float& scale) {
  thresh = p <= 0.f ? 0u : (uint32_t)fmin(4294967295.0, (double)p * 4294967296.0);
  scale = p <= 0.f ? 1.f : (float)(1.0 / (1.0 - (double)p));
}

inline int dtype_size(int dtype) { return dtype == ETH_F32 ? 4 : 2; }
inline bool valid_dtype(int dtype) {
  return dtype == ETH_F32 || dtype == ETH_F16 || dtype == ETH_BF16;
}

}  // namespace eth
