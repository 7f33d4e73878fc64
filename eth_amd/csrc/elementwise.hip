// Elementwise layer ops of the GPT block and the bias-gradient reduction.
//
//   bias-GELU   y = gelu_tanh(bf16(x + b))        (flex_ops.py:60-63,1897:
//               F.gelu(x + b, approximate="tanh"); the add is rounded to the
//               activation dtype first, as the separate torch add does)
//   dGELU       dx = dy * gelu_tanh'(bf16(x + b))  (closed form of
//               model/fused_bias_gelu.py:39-45 with torch's exact sqrt(2/pi))
//   bias-dropout-add  out = residual + dropout(bf16(x + b), p)
//               (flex_ops.py:104-134); dropout keeps an element when a
//               counter-based hash of (seed, element index) is >= p*2^32 and
//               scales kept elements by 1/(1-p); p == 0 is the identity, as in
//               torch
//   column sum  out[c] (+)= sum_r x[r, c] in fp32 (bias gradients), two
//               deterministic passes
//
// All kernels stream 16-byte vectors (8 x 16-bit) and compute in fp32.
#include "common.h"

namespace eth {

template <bool FP16>
__device__ __forceinline__ float cin(uint16_t v) {
  return FP16 ? h2f_bits(v) : bf2f(v);
}
template <bool FP16>
__device__ __forceinline__ uint16_t cout(float v) {
  return FP16 ? f2h_bits(v) : f2bf(v);
}

constexpr float kBeta = 0.7978845608028654f;  // sqrt(2/pi)
constexpr float kKappa = 0.044715f;

// tanh(u) = 1 - 2 / (1 + e^{2u}) with the hardware exp2 and reciprocal: a
// few ulp in fp32, far below the 16-bit output rounding, and exact at the
// saturated ends (e^{2u} = inf -> 1, 0 -> -1).  libm tanhf made these
// kernels VALU-bound.
__device__ __forceinline__ float fast_tanh(float u) {
  const float e = __builtin_amdgcn_exp2f(u * 2.8853900817779268f);  // 2 / ln 2
  return 1.0f - 2.0f * __builtin_amdgcn_rcpf(1.0f + e);
}
__device__ __forceinline__ float gelu_tanh(float x) {
  const float x3 = x * x * x;
  const float inner = kBeta * (x + kKappa * x3);
  return 0.5f * x * (1.0f + fast_tanh(inner));
}
__device__ __forceinline__ float gelu_tanh_grad(float x) {
  const float x2 = x * x;
  const float t = fast_tanh(kBeta * (x + kKappa * (x2 * x)));
  const float left = 0.5f * x, right = 1.0f + t;
  return 0.5f * right + left * (1.0f - t * t) * kBeta * (1.0f + 3.0f * kKappa * x2);
}

// 32-bit mix of (seed, index): keep decision for dropout.
__device__ __forceinline__ uint32_t hash_u32(uint64_t seed, uint64_t idx) {
  uint64_t z = seed + 0x9E3779B97F4A7C15ull * (idx + 1);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  z ^= z >> 31;
  return (uint32_t)(z >> 32);
}

constexpr int kEwThreads = 256;

template <bool FP16>
__global__ void __launch_bounds__(kEwThreads) bias_gelu_fwd_kernel(const uint16_t* __restrict__ x,
                                                                   const uint16_t* __restrict__ b,
                                                                   uint16_t* __restrict__ y,
                                                                   int64_t nvec, int cols) {
  for (int64_t v = blockIdx.x * (int64_t)kEwThreads + threadIdx.x; v < nvec;
       v += (int64_t)gridDim.x * kEwThreads) {
    const int c = (int)((v * 8) % cols);
    uint4 xr = reinterpret_cast<const uint4*>(x)[v];
    uint4 br = *reinterpret_cast<const uint4*>(b + c);
    const uint16_t* xe = reinterpret_cast<const uint16_t*>(&xr);
    const uint16_t* be = reinterpret_cast<const uint16_t*>(&br);
    uint4 out;
    uint16_t* oe = reinterpret_cast<uint16_t*>(&out);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float t = cin<FP16>(cout<FP16>(cin<FP16>(xe[j]) + cin<FP16>(be[j])));
      oe[j] = cout<FP16>(gelu_tanh(t));
    }
    reinterpret_cast<uint4*>(y)[v] = out;
  }
}

template <bool FP16>
__global__ void __launch_bounds__(kEwThreads) bias_gelu_bwd_kernel(const uint16_t* __restrict__ dy,
                                                                   const uint16_t* __restrict__ x,
                                                                   const uint16_t* __restrict__ b,
                                                                   uint16_t* __restrict__ dx,
                                                                   int64_t nvec, int cols) {
  for (int64_t v = blockIdx.x * (int64_t)kEwThreads + threadIdx.x; v < nvec;
       v += (int64_t)gridDim.x * kEwThreads) {
    const int c = (int)((v * 8) % cols);
    uint4 xr = reinterpret_cast<const uint4*>(x)[v];
    uint4 dr = reinterpret_cast<const uint4*>(dy)[v];
    uint4 br = *reinterpret_cast<const uint4*>(b + c);
    const uint16_t* xe = reinterpret_cast<const uint16_t*>(&xr);
    const uint16_t* de = reinterpret_cast<const uint16_t*>(&dr);
    const uint16_t* be = reinterpret_cast<const uint16_t*>(&br);
    uint4 out;
    uint16_t* oe = reinterpret_cast<uint16_t*>(&out);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float t = cin<FP16>(cout<FP16>(cin<FP16>(xe[j]) + cin<FP16>(be[j])));
      oe[j] = cout<FP16>(cin<FP16>(de[j]) * gelu_tanh_grad(t));
    }
    reinterpret_cast<uint4*>(dx)[v] = out;
  }
}

template <bool FP16>
__global__ void __launch_bounds__(kEwThreads) bda_fwd_kernel(const uint16_t* __restrict__ x,
                                                             const uint16_t* __restrict__ b,
                                                             const uint16_t* __restrict__ res,
                                                             uint16_t* __restrict__ out,
                                                             int64_t nvec, int cols, uint32_t thresh,
                                                             float keep_scale, uint64_t seed) {
  for (int64_t v = blockIdx.x * (int64_t)kEwThreads + threadIdx.x; v < nvec;
       v += (int64_t)gridDim.x * kEwThreads) {
    const int c = (int)((v * 8) % cols);
    uint4 xr = reinterpret_cast<const uint4*>(x)[v];
    uint4 rr = reinterpret_cast<const uint4*>(res)[v];
    uint4 br = *reinterpret_cast<const uint4*>(b + c);
    const uint16_t* xe = reinterpret_cast<const uint16_t*>(&xr);
    const uint16_t* re = reinterpret_cast<const uint16_t*>(&rr);
    const uint16_t* be = reinterpret_cast<const uint16_t*>(&br);
    uint4 o;
    uint16_t* oe = reinterpret_cast<uint16_t*>(&o);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float t = cin<FP16>(cout<FP16>(cin<FP16>(xe[j]) + cin<FP16>(be[j])));
      if (thresh) {
        const bool keep = hash_u32(seed, (uint64_t)v * 8 + j) >= thresh;
        t = cin<FP16>(cout<FP16>(keep ? t * keep_scale : 0.f));
      }
      oe[j] = cout<FP16>(cin<FP16>(re[j]) + t);
    }
    reinterpret_cast<uint4*>(out)[v] = o;
  }
}

template <bool FP16>
__global__ void __launch_bounds__(kEwThreads) dropout_bwd_kernel(const uint16_t* __restrict__ dy,
                                                                 uint16_t* __restrict__ dx, int64_t nvec,
                                                                 uint32_t thresh, float keep_scale,
                                                                 uint64_t seed) {
  for (int64_t v = blockIdx.x * (int64_t)kEwThreads + threadIdx.x; v < nvec;
       v += (int64_t)gridDim.x * kEwThreads) {
    uint4 dr = reinterpret_cast<const uint4*>(dy)[v];
    const uint16_t* de = reinterpret_cast<const uint16_t*>(&dr);
    uint4 o;
    uint16_t* oe = reinterpret_cast<uint16_t*>(&o);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const bool keep = hash_u32(seed, (uint64_t)v * 8 + j) >= thresh;
      oe[j] = cout<FP16>(keep ? cin<FP16>(de[j]) * keep_scale : 0.f);
    }
    reinterpret_cast<uint4*>(dx)[v] = o;
  }
}

// Column sums: workgroup g handles rows [g*rpg, (g+1)*rpg) for a 2048-column
// slab (256 threads x 8 columns); partials to part[g][cols].
template <bool FP16>
__global__ void __launch_bounds__(kEwThreads) col_sum_part_kernel(const uint16_t* __restrict__ x,
                                                                  int64_t ld, int rows, int cols,
                                                                  int rpg, float* __restrict__ part) {
  const int c = (blockIdx.y * kEwThreads + threadIdx.x) * 8;
  if (c >= cols) return;
  float acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = 0.f;
  const int r0 = blockIdx.x * rpg, r1 = min(rows, r0 + rpg);
  for (int r = r0; r < r1; ++r) {
    uint4 xr = *reinterpret_cast<const uint4*>(x + (int64_t)r * ld + c);
    const uint16_t* xe = reinterpret_cast<const uint16_t*>(&xr);
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] += cin<FP16>(xe[j]);
  }
  float* p = part + (int64_t)blockIdx.x * cols + c;
#pragma unroll
  for (int j = 0; j < 8; ++j) p[j] = acc[j];
}

inline int ew_grid(int64_t nvec) {
  int64_t g = (nvec + kEwThreads - 1) / kEwThreads;
  return (int)(g > 8192 ? 8192 : (g < 1 ? 1 : g));
}

}  // namespace eth

using namespace eth;

#define ETH_EW_COMMON(name)                                                                       \
  ETH_CHECK_ARG(dtype == ETH_BF16 || dtype == ETH_F16, name ": dtype must be bf16/fp16");         \
  ETH_CHECK_ARG(rows >= 0 && cols > 0 && cols % 8 == 0, name ": cols must be a multiple of 8"); \
  if (rows == 0) return ETH_OK;

extern "C" int eth_bias_gelu_fwd(const void* x, const void* bias, void* y, int64_t rows,
                                 int64_t cols, int dtype, void* stream) {
  ETH_EW_COMMON("eth_bias_gelu_fwd");
  ETH_CHECK_ARG(x && bias && y, "eth_bias_gelu_fwd: null pointer");
  const int64_t nvec = rows * cols / 8;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == ETH_BF16)
    bias_gelu_fwd_kernel<false><<<ew_grid(nvec), kEwThreads, 0, s>>>((const uint16_t*)x, (const uint16_t*)bias,
                                                                     (uint16_t*)y, nvec, (int)cols);
  else
    bias_gelu_fwd_kernel<true><<<ew_grid(nvec), kEwThreads, 0, s>>>((const uint16_t*)x, (const uint16_t*)bias,
                                                                    (uint16_t*)y, nvec, (int)cols);
  ETH_CHECK_LAUNCH("eth_bias_gelu_fwd");
  return ETH_OK;
}

extern "C" int eth_bias_gelu_bwd(const void* dy, const void* x, const void* bias, void* dx,
                                 int64_t rows, int64_t cols, int dtype, void* stream) {
  ETH_EW_COMMON("eth_bias_gelu_bwd");
  ETH_CHECK_ARG(dy && x && bias && dx, "eth_bias_gelu_bwd: null pointer");
  const int64_t nvec = rows * cols / 8;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == ETH_BF16)
    bias_gelu_bwd_kernel<false><<<ew_grid(nvec), kEwThreads, 0, s>>>(
        (const uint16_t*)dy, (const uint16_t*)x, (const uint16_t*)bias, (uint16_t*)dx, nvec, (int)cols);
  else
    bias_gelu_bwd_kernel<true><<<ew_grid(nvec), kEwThreads, 0, s>>>(
        (const uint16_t*)dy, (const uint16_t*)x, (const uint16_t*)bias, (uint16_t*)dx, nvec, (int)cols);
  ETH_CHECK_LAUNCH("eth_bias_gelu_bwd");
  return ETH_OK;
}

static void dropout_params(float p, uint32_t& thresh, float& scale) {
  thresh = p <= 0.f ? 0u : (uint32_t)fmin(4294967295.0, (double)p * 4294967296.0);
  scale = p <= 0.f ? 1.f : (float)(1.0 / (1.0 - (double)p));
}

extern "C" int eth_bias_dropout_add_fwd(const void* x, const void* bias, const void* residual,
                                        void* out, int64_t rows, int64_t cols, float p,
                                        uint64_t seed, int dtype, void* stream) {
  ETH_EW_COMMON("eth_bias_dropout_add_fwd");
  ETH_CHECK_ARG(x && bias && residual && out, "eth_bias_dropout_add_fwd: null pointer");
  ETH_CHECK_ARG(p >= 0.f && p < 1.f, "eth_bias_dropout_add_fwd: p must be in [0, 1)");
  uint32_t thresh;
  float scale;
  dropout_params(p, thresh, scale);
  const int64_t nvec = rows * cols / 8;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == ETH_BF16)
    bda_fwd_kernel<false><<<ew_grid(nvec), kEwThreads, 0, s>>>((const uint16_t*)x, (const uint16_t*)bias,
                                                               (const uint16_t*)residual, (uint16_t*)out, nvec,
                                                               (int)cols, thresh, scale, seed);
  else
    bda_fwd_kernel<true><<<ew_grid(nvec), kEwThreads, 0, s>>>((const uint16_t*)x, (const uint16_t*)bias,
                                                              (const uint16_t*)residual, (uint16_t*)out, nvec,
                                                              (int)cols, thresh, scale, seed);
  ETH_CHECK_LAUNCH("eth_bias_dropout_add_fwd");
  return ETH_OK;
}

extern "C" int eth_dropout_bwd(const void* dy, void* dx, int64_t rows, int64_t cols, float p,
                               uint64_t seed, int dtype, void* stream) {
  ETH_EW_COMMON("eth_dropout_bwd");
  ETH_CHECK_ARG(dy && dx, "eth_dropout_bwd: null pointer");
  ETH_CHECK_ARG(p > 0.f && p < 1.f, "eth_dropout_bwd: p must be in (0, 1)");
  uint32_t thresh;
  float scale;
  dropout_params(p, thresh, scale);
  const int64_t nvec = rows * cols / 8;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == ETH_BF16)
    dropout_bwd_kernel<false><<<ew_grid(nvec), kEwThreads, 0, s>>>((const uint16_t*)dy, (uint16_t*)dx, nvec,
                                                                   thresh, scale, seed);
  else
    dropout_bwd_kernel<true><<<ew_grid(nvec), kEwThreads, 0, s>>>((const uint16_t*)dy, (uint16_t*)dx, nvec,
                                                                  thresh, scale, seed);
  ETH_CHECK_LAUNCH("eth_dropout_bwd");
  return ETH_OK;
}

extern "C" int64_t eth_col_sum_workspace(int64_t rows, int64_t cols) {
  const int64_t groups = rows < 512 ? (rows + 15) / 16 : 512;
  return (groups < 1 ? 1 : groups) * cols;
}

extern "C" int eth_col_sum(const void* x, int64_t ld, int64_t rows, int64_t cols, float* out,
                           float* workspace, int accumulate, int dtype, void* stream) {
  ETH_EW_COMMON("eth_col_sum");
  ETH_CHECK_ARG(x && out && workspace && ld >= cols && ld % 8 == 0, "eth_col_sum: bad arguments");
  const int groups = (int)(rows < 512 ? (rows + 15) / 16 : 512);
  const int rpg = (int)((rows + groups - 1) / groups);
  dim3 grid(groups, (unsigned)((cols + 8 * kEwThreads - 1) / (8 * kEwThreads)));
  hipStream_t s = (hipStream_t)stream;
  if (dtype == ETH_BF16)
    col_sum_part_kernel<false><<<grid, kEwThreads, 0, s>>>((const uint16_t*)x, ld, (int)rows, (int)cols, rpg,
                                                           workspace);
  else
    col_sum_part_kernel<true><<<grid, kEwThreads, 0, s>>>((const uint16_t*)x, ld, (int)rows, (int)cols, rpg,
                                                          workspace);
  ETH_CHECK_LAUNCH("eth_col_sum");
  reduce_partials_kernel<<<reduce_partials_grid((int)cols), kReducePartialsThreads, 0, s>>>(
      workspace, groups, (int)cols, cols, out, accumulate);
  ETH_CHECK_LAUNCH("eth_col_sum reduce");
  return ETH_OK;
}
