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

// Only fused multiply-adds written as __builtin_fmaf are fused, so that every
// kernel computing the same element (bias_gelu_bwd_kernel and the fused
// bias-gradient variant) rounds it alike.
#pragma clang fp contract(off)

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
  return __builtin_fmaf(-2.0f, __builtin_amdgcn_rcpf(1.0f + e), 1.0f);
}
__device__ __forceinline__ float gelu_tanh(float x) {
  const float x3 = x * x * x;
  const float inner = kBeta * __builtin_fmaf(kKappa, x3, x);
  return 0.5f * x * (1.0f + fast_tanh(inner));
}
__device__ __forceinline__ float gelu_tanh_grad(float x) {
  const float x2 = x * x;
  const float t = fast_tanh(kBeta * __builtin_fmaf(kKappa, x2 * x, x));
  const float left = 0.5f * x, right = 1.0f + t;
  return __builtin_fmaf(0.5f, right, left * __builtin_fmaf(-t, t, 1.0f) * kBeta * __builtin_fmaf(3.0f * kKappa, x2, 1.0f));
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

// Column-strip kernel (column sums): workgroup (g, s) owns the 512 columns [s*512, s*512 + 512) of
// rows [g*rpg, min(rows, (g+1)*rpg)); wave w takes rows r0+w, r0+w+4, ...,
// kStripBatch rows per trip with every load issued first.  Each lane keeps
// fp32 sums of its 8 columns; the 4 waves' sums are added through LDS in
// fixed order and stored to part[g][cols], which reduce_partials_kernel
// folds (deterministic end to end).
constexpr int kStripWaves = 4, kStripBatch = 4;
typedef uint32_t ew_u32x4 __attribute__((ext_vector_type(4)));
typedef float ew_f32x4 __attribute__((ext_vector_type(4)));

template <bool FP16>
__device__ __forceinline__ float ew_half(const ew_u32x4& v, int j) {
  const uint32_t w = v[j >> 1];
  return cin<FP16>((uint16_t)((j & 1) ? (w >> 16) : (w & 0xffffu)));
}

__device__ __forceinline__ void strip_store(const float (&acc)[8], float* __restrict__ part_row, int cols) {
  __shared__ float red[kStripWaves][512];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  ew_f32x4* rw = reinterpret_cast<ew_f32x4*>(&red[w][lane * 8]);
  rw[0] = ew_f32x4{acc[0], acc[1], acc[2], acc[3]};
  rw[1] = ew_f32x4{acc[4], acc[5], acc[6], acc[7]};
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 512 / (64 * kStripWaves); ++k) {
    const int e = threadIdx.x + k * 64 * kStripWaves;
    const int c = blockIdx.y * 512 + e;
    if (c < cols) {
      float a = 0.f;
#pragma unroll
      for (int t = 0; t < kStripWaves; ++t) a += red[t][e];
      part_row[c] = a;
    }
  }
}

template <bool FP16>
__global__ void __launch_bounds__(64 * kStripWaves) col_sum_part_kernel(const uint16_t* __restrict__ x,
                                                                        int64_t ld, int rows, int cols,
                                                                        int rpg, float* __restrict__ part) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int c = blockIdx.y * 512 + lane * 8;
  float acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = 0.f;
  const int r0 = blockIdx.x * rpg, r1 = min(rows, r0 + rpg);
  if (c < cols) {
    const uint16_t* base = x + c;
    int r = r0 + w;
    for (; r + (kStripBatch - 1) * kStripWaves < r1; r += kStripBatch * kStripWaves) {
      ew_u32x4 v[kStripBatch];
#pragma unroll
      for (int b = 0; b < kStripBatch; ++b)
        v[b] = *reinterpret_cast<const ew_u32x4*>(base + (int64_t)(r + b * kStripWaves) * ld);
#pragma unroll
      for (int b = 0; b < kStripBatch; ++b)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] += ew_half<FP16>(v[b], j);
    }
    for (; r < r1; r += kStripWaves) {
      const ew_u32x4 v = *reinterpret_cast<const ew_u32x4*>(base + (int64_t)r * ld);
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] += ew_half<FP16>(v, j);
    }
  }
  strip_store(acc, part + (int64_t)blockIdx.x * cols, cols);
}

// dx = dy * gelu_tanh'(bf16(x + b)) as bias_gelu_bwd_kernel, plus the column
// sums of the stored (rounded) dx: the bias gradient.
template <bool FP16>
__device__ __forceinline__ ew_u32x4 gelu_bwd_vec(const ew_u32x4& d, const ew_u32x4& xv, const float (&bias)[8],
                                                 float (&acc)[8]) {
  ew_u32x4 o;
#pragma unroll
  for (int j = 0; j < 8; j += 2) {
    float v[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const float t = cin<FP16>(cout<FP16>(ew_half<FP16>(xv, j + h) + bias[j + h]));
      v[h] = ew_half<FP16>(d, j + h) * gelu_tanh_grad(t);
    }
    const uint32_t w = FP16 ? f2h_pair(v[0], v[1]) : f2bf_pair(v[0], v[1]);
    o[j >> 1] = w;
    acc[j] += cin<FP16>((uint16_t)(w & 0xffffu));
    acc[j + 1] += cin<FP16>((uint16_t)(w >> 16));
  }
  return o;
}

// Sweep mapping for the fused bias gradient: workgroup b covers the 2048
// columns of column block b % CB (CB = ceil(cols / 2048), 8 per lane) on rows
// g, g + G, g + 2G, ... of row lane g = b / CB, kGeluBatch rows per trip with
// every load issued first.  The G row lanes together walk the tensor from
// top to bottom, so the whole GPU streams through one band of rows at a
// time; each lane's column sums go to part[g][cols].
constexpr int kGeluBatch = 8;

template <bool FP16>
__global__ void __launch_bounds__(256) bias_gelu_bwd_dbias_kernel(
    const uint16_t* __restrict__ dy, const uint16_t* __restrict__ x, const uint16_t* __restrict__ b,
    uint16_t* __restrict__ dx, int rows, int cols, int lanes, float* __restrict__ part) {
  const int cblocks = (cols + 2047) / 2048;
  const int cb = blockIdx.x % cblocks, g = blockIdx.x / cblocks;
  const int c = cb * 2048 + threadIdx.x * 8;
  if (c >= cols) return;
  float acc[8], bias[8];
  const ew_u32x4 bv = *reinterpret_cast<const ew_u32x4*>(b + c);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    acc[j] = 0.f;
    bias[j] = ew_half<FP16>(bv, j);
  }
  int r = g;
  for (; r + (kGeluBatch - 1) * lanes < rows; r += kGeluBatch * lanes) {
    ew_u32x4 dv[kGeluBatch], xv[kGeluBatch];
#pragma unroll
    for (int k = 0; k < kGeluBatch; ++k) {
      const int64_t o = (int64_t)(r + k * lanes) * cols + c;
      dv[k] = *reinterpret_cast<const ew_u32x4*>(dy + o);
      xv[k] = *reinterpret_cast<const ew_u32x4*>(x + o);
    }
#pragma unroll
    for (int k = 0; k < kGeluBatch; ++k) {
      const int64_t o = (int64_t)(r + k * lanes) * cols + c;
      *reinterpret_cast<ew_u32x4*>(dx + o) = gelu_bwd_vec<FP16>(dv[k], xv[k], bias, acc);
    }
  }
  for (; r < rows; r += lanes) {
    const int64_t o = (int64_t)r * cols + c;
    const ew_u32x4 dv = *reinterpret_cast<const ew_u32x4*>(dy + o);
    const ew_u32x4 xv = *reinterpret_cast<const ew_u32x4*>(x + o);
    *reinterpret_cast<ew_u32x4*>(dx + o) = gelu_bwd_vec<FP16>(dv, xv, bias, acc);
  }
  ew_f32x4* p = reinterpret_cast<ew_f32x4*>(part + (int64_t)g * cols + c);
  p[0] = ew_f32x4{acc[0], acc[1], acc[2], acc[3]};
  p[1] = ew_f32x4{acc[4], acc[5], acc[6], acc[7]};
}

// Row lanes of the sweep: one workgroup per CU in all (measured best for the
// [8192, 8192] MLP activation), at least kGeluBatch rows per lane.
inline int gelu_lanes(int64_t rows, int64_t cols) {
  const int64_t cblocks = (cols + 2047) / 2048;
  int64_t g = 256 / cblocks;
  const int64_t by_rows = rows / kGeluBatch;
  if (g > by_rows) g = by_rows;
  if (g < 1) g = 1;
  return (int)g;
}

// Row groups of the strip kernels: about 1024 workgroups in all, at most
// 256 groups (partials stay a few MB), at least 16 rows per group.
inline int strip_groups(int64_t rows, int64_t cols) {
  const int64_t slabs = (cols + 511) / 512;
  int64_t g = 1024 / slabs;
  if (g > 256) g = 256;
  if (g < 64) g = 64;
  const int64_t by_rows = (rows + 15) / 16;
  if (g > by_rows) g = by_rows;
  if (g < 1) g = 1;
  const int64_t rpg = (rows + g - 1) / g;
  return (int)((rows + rpg - 1) / rpg);
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
  if (rows <= 0 || cols <= 0) return 1;
  return (int64_t)strip_groups(rows, cols) * cols;
}

extern "C" int eth_col_sum(const void* x, int64_t ld, int64_t rows, int64_t cols, float* out,
                           float* workspace, int accumulate, int dtype, void* stream) {
  ETH_EW_COMMON("eth_col_sum");
  ETH_CHECK_ARG(x && out && workspace && ld >= cols && ld % 8 == 0, "eth_col_sum: bad arguments");
  ETH_CHECK_ARG(rows < (1LL << 31) && cols < (1LL << 31), "eth_col_sum: shape too large");
  ETH_CHECK_ARG((((uintptr_t)x | (uintptr_t)workspace) & 15u) == 0, "eth_col_sum: operands must be 16-byte aligned");
  const int groups = strip_groups(rows, cols);
  const int rpg = (int)((rows + groups - 1) / groups);
  dim3 grid(groups, (unsigned)((cols + 511) / 512));
  hipStream_t s = (hipStream_t)stream;
  if (dtype == ETH_BF16)
    col_sum_part_kernel<false><<<grid, 64 * kStripWaves, 0, s>>>((const uint16_t*)x, ld, (int)rows, (int)cols, rpg,
                                                                 workspace);
  else
    col_sum_part_kernel<true><<<grid, 64 * kStripWaves, 0, s>>>((const uint16_t*)x, ld, (int)rows, (int)cols, rpg,
                                                                workspace);
  ETH_CHECK_LAUNCH("eth_col_sum");
  reduce_partials_kernel<<<reduce_partials_grid((int)cols), kReducePartialsThreads, 0, s>>>(
      workspace, groups, (int)cols, cols, out, nullptr, accumulate);
  ETH_CHECK_LAUNCH("eth_col_sum reduce");
  return ETH_OK;
}

extern "C" int64_t eth_bias_gelu_bwd_workspace(int64_t rows, int64_t cols) {
  if (rows <= 0 || cols <= 0) return 1;
  return (int64_t)gelu_lanes(rows, cols) * cols;
}

extern "C" int eth_bias_gelu_bwd_dbias(const void* dy, const void* x, const void* bias, void* dx, float* dbias,
                                       float* workspace, int64_t rows, int64_t cols, int accumulate, int dtype,
                                       void* stream) {
  ETH_EW_COMMON("eth_bias_gelu_bwd_dbias");
  ETH_CHECK_ARG(dy && x && bias && dx && dbias && workspace, "eth_bias_gelu_bwd_dbias: null pointer");
  ETH_CHECK_ARG(rows < (1LL << 31) && cols < (1LL << 31), "eth_bias_gelu_bwd_dbias: shape too large");
  ETH_CHECK_ARG((((uintptr_t)dy | (uintptr_t)x | (uintptr_t)bias | (uintptr_t)dx | (uintptr_t)workspace) & 15u) == 0,
                "eth_bias_gelu_bwd_dbias: operands must be 16-byte aligned");
  const int lanes = gelu_lanes(rows, cols);
  const dim3 grid((unsigned)(lanes * ((cols + 2047) / 2048)));
  hipStream_t s = (hipStream_t)stream;
  if (dtype == ETH_BF16)
    bias_gelu_bwd_dbias_kernel<false><<<grid, 256, 0, s>>>((const uint16_t*)dy, (const uint16_t*)x,
                                                           (const uint16_t*)bias, (uint16_t*)dx, (int)rows,
                                                           (int)cols, lanes, workspace);
  else
    bias_gelu_bwd_dbias_kernel<true><<<grid, 256, 0, s>>>((const uint16_t*)dy, (const uint16_t*)x,
                                                          (const uint16_t*)bias, (uint16_t*)dx, (int)rows,
                                                          (int)cols, lanes, workspace);
  ETH_CHECK_LAUNCH("eth_bias_gelu_bwd_dbias");
  reduce_partials_kernel<<<reduce_partials_grid((int)cols), kReducePartialsThreads, 0, s>>>(
      workspace, lanes, (int)cols, cols, dbias, nullptr, accumulate);
  ETH_CHECK_LAUNCH("eth_bias_gelu_bwd_dbias reduce");
  return ETH_OK;
}
