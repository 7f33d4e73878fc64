// Mixed-precision LayerNorm (bf16/fp16 activations, 16-bit gamma/beta, fp32
// statistics), forward and backward.
//
// Forward: one 64-lane wavefront per row; the row is read once with 16-byte
// loads, mean and variance are computed in fp32 (two-pass over registers, so
// no Welford merge is needed), y = (x - mu) * rstd * gamma + beta, and the
// fp32 mean / inverse std are saved for backward.
// Backward: one wavefront per row computes
//   dx = rstd/H * (H*dy*g - sum(dy*g) - xhat*sum(dy*g*xhat))
// and accumulates per-column partial dgamma = sum(dy*xhat), dbeta = sum(dy)
// for its group of rows; a second pass reduces the partials in a fixed
// order (deterministic) and either stores or adds them into fp32 gradients.
//
// Restates fused_mix_prec_layer_norm_cuda.forward_affine / backward_affine
// (eth/runtime/megatron/fused_kernels/layer_norm_cuda.cpp:121-201,
// layer_norm_cuda_kernel.cu:290-334,415-655) with eps = 1e-5 as in
// model/fused_layer_norm.py:62-89.
#include "common.h"

namespace eth {

constexpr int kLnWaves = 4;  // rows per workgroup in the row kernels
constexpr int kMaxCols = 8192;

template <bool FP16>
__device__ __forceinline__ float cvt_in(uint16_t v) {
  return FP16 ? h2f_bits(v) : bf2f(v);
}
template <bool FP16>
__device__ __forceinline__ uint16_t cvt_out(float v) {
  return FP16 ? f2h_bits(v) : f2bf(v);
}

// Each lane handles VPL vectors of 8 elements: cols == VPL * 8 * 64 * ... we
// loop in strides of 512 elements (64 lanes x 8).
template <int NV, bool FP16>
__global__ void __launch_bounds__(64 * kLnWaves) ln_fwd_kernel(const uint16_t* __restrict__ x,
                                                               const uint16_t* __restrict__ gamma,
                                                               const uint16_t* __restrict__ beta,
                                                               uint16_t* __restrict__ y,
                                                               float* __restrict__ mean,
                                                               float* __restrict__ rstd, int rows,
                                                               int cols, float eps) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * kLnWaves + (threadIdx.x >> 6);
  if (row >= rows) return;
  const uint16_t* xr = x + (int64_t)row * cols;
  float v[NV][8];
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = (i * 64 + lane) * 8;
    if (c < cols) {
      uint4 raw = *reinterpret_cast<const uint4*>(xr + c);
      const uint16_t* e = reinterpret_cast<const uint16_t*>(&raw);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        v[i][j] = cvt_in<FP16>(e[j]);
        s += v[i][j];
      }
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) v[i][j] = 0.f;
    }
  }
  const float mu = wave_sum(s) / cols;
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = (i * 64 + lane) * 8;
    if (c < cols) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float d = v[i][j] - mu;
        q += d * d;
      }
    }
  }
  const float var = wave_sum(q) / cols;
  const float r = rsqrtf(var + eps);
  uint16_t* yr = y + (int64_t)row * cols;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = (i * 64 + lane) * 8;
    if (c < cols) {
      uint4 gr = *reinterpret_cast<const uint4*>(gamma + c);
      uint4 br = *reinterpret_cast<const uint4*>(beta + c);
      const uint16_t* ge = reinterpret_cast<const uint16_t*>(&gr);
      const uint16_t* be = reinterpret_cast<const uint16_t*>(&br);
      uint4 out;
      uint16_t* oe = reinterpret_cast<uint16_t*>(&out);
#pragma unroll
      for (int j = 0; j < 8; ++j)
        oe[j] = cvt_out<FP16>((v[i][j] - mu) * r * cvt_in<FP16>(ge[j]) + cvt_in<FP16>(be[j]));
      *reinterpret_cast<uint4*>(yr + c) = out;
    }
  }
  if (lane == 0) {
    mean[row] = mu;
    rstd[row] = r;
  }
}

// Backward, row part.  Workgroup = kLnWaves waves; rows are assigned in
// contiguous groups of `rows_per_group` to each workgroup, whose per-column
// dgamma/dbeta partials (fp32) go to part[blockIdx.x][2][cols].
template <int NV, bool FP16>
__global__ void __launch_bounds__(64 * kLnWaves) ln_bwd_kernel(
    const uint16_t* __restrict__ dy, const uint16_t* __restrict__ x, const float* __restrict__ mean,
    const float* __restrict__ rstd, const uint16_t* __restrict__ gamma, uint16_t* __restrict__ dx,
    float* __restrict__ part, int rows, int cols, int rows_per_group) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  float dg[NV][8], db[NV][8], g[NV][8];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = (i * 64 + lane) * 8;
#pragma unroll
    for (int j = 0; j < 8; ++j) dg[i][j] = db[i][j] = 0.f;
    if (c < cols) {
      uint4 gr = *reinterpret_cast<const uint4*>(gamma + c);
      const uint16_t* ge = reinterpret_cast<const uint16_t*>(&gr);
#pragma unroll
      for (int j = 0; j < 8; ++j) g[i][j] = cvt_in<FP16>(ge[j]);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) g[i][j] = 0.f;
    }
  }
  const int r_begin = blockIdx.x * rows_per_group;
  const int r_end = min(rows, r_begin + rows_per_group);
  for (int row = r_begin + wid; row < r_end; row += kLnWaves) {
    const float mu = mean[row], rs = rstd[row];
    float xh[NV][8], d[NV][8];
    float s1 = 0.f, s2 = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = (i * 64 + lane) * 8;
      if (c < cols) {
        uint4 xr = *reinterpret_cast<const uint4*>(x + (int64_t)row * cols + c);
        uint4 dr = *reinterpret_cast<const uint4*>(dy + (int64_t)row * cols + c);
        const uint16_t* xe = reinterpret_cast<const uint16_t*>(&xr);
        const uint16_t* de = reinterpret_cast<const uint16_t*>(&dr);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          xh[i][j] = (cvt_in<FP16>(xe[j]) - mu) * rs;
          d[i][j] = cvt_in<FP16>(de[j]);
          const float dyg = d[i][j] * g[i][j];
          s1 += dyg;
          s2 += dyg * xh[i][j];
          dg[i][j] += d[i][j] * xh[i][j];
          db[i][j] += d[i][j];
        }
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) xh[i][j] = d[i][j] = 0.f;
      }
    }
    s1 = wave_sum(s1);
    s2 = wave_sum(s2);
    const float inv_n = 1.0f / cols;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = (i * 64 + lane) * 8;
      if (c < cols) {
        uint4 out;
        uint16_t* oe = reinterpret_cast<uint16_t*>(&out);
#pragma unroll
        for (int j = 0; j < 8; ++j)
          oe[j] = cvt_out<FP16>(rs * (d[i][j] * g[i][j] - inv_n * (s1 + xh[i][j] * s2)));
        *reinterpret_cast<uint4*>(dx + (int64_t)row * cols + c) = out;
      }
    }
  }
  // reduce the 4 waves' column partials through LDS, then one store per column
  __shared__ float red[kLnWaves][2][512];
  float* out = part + (int64_t)blockIdx.x * 2 * cols;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = (i * 64 + lane) * 8;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      red[wid][0][lane * 8 + j] = dg[i][j];
      red[wid][1][lane * 8 + j] = db[i][j];
    }
    __syncthreads();
    for (int t = threadIdx.x; t < 1024; t += 64 * kLnWaves) {
      const int which = t >> 9, e = t & 511;
      const int col = i * 512 + e;
      if (col < cols) {
        float a = 0.f;
#pragma unroll
        for (int w = 0; w < kLnWaves; ++w) a += red[w][which][e];
        out[which * cols + col] = a;
      }
    }
    __syncthreads();
    (void)c;
  }
}

template <bool FP16>
static void launch_fwd(const uint16_t* x, const uint16_t* g, const uint16_t* b, uint16_t* y, float* mean,
                       float* rstd, int rows, int cols, float eps, hipStream_t s) {
  const int grid = (rows + kLnWaves - 1) / kLnWaves;
  const int nv = (cols + 511) / 512;
  switch (nv) {
#define ETH_LN_CASE(N) \
  case N: ln_fwd_kernel<N, FP16><<<grid, 64 * kLnWaves, 0, s>>>(x, g, b, y, mean, rstd, rows, cols, eps); break;
    ETH_LN_CASE(1) ETH_LN_CASE(2) ETH_LN_CASE(3) ETH_LN_CASE(4) ETH_LN_CASE(5) ETH_LN_CASE(6)
    ETH_LN_CASE(7) ETH_LN_CASE(8) ETH_LN_CASE(9) ETH_LN_CASE(10) ETH_LN_CASE(11) ETH_LN_CASE(12)
    ETH_LN_CASE(13) ETH_LN_CASE(14) ETH_LN_CASE(15) ETH_LN_CASE(16)
#undef ETH_LN_CASE
  }
}

template <bool FP16>
static void launch_bwd(const uint16_t* dy, const uint16_t* x, const float* mean, const float* rstd,
                       const uint16_t* g, uint16_t* dx, float* part, int groups, int rpg, int rows,
                       int cols, hipStream_t s) {
  const int nv = (cols + 511) / 512;
  switch (nv) {
#define ETH_LN_CASE(N)                                                                                 \
  case N:                                                                                              \
    ln_bwd_kernel<N, FP16><<<groups, 64 * kLnWaves, 0, s>>>(dy, x, mean, rstd, g, dx, part, rows, cols, \
                                                             rpg);                                     \
    break;
    ETH_LN_CASE(1) ETH_LN_CASE(2) ETH_LN_CASE(3) ETH_LN_CASE(4) ETH_LN_CASE(5) ETH_LN_CASE(6)
    ETH_LN_CASE(7) ETH_LN_CASE(8) ETH_LN_CASE(9) ETH_LN_CASE(10) ETH_LN_CASE(11) ETH_LN_CASE(12)
    ETH_LN_CASE(13) ETH_LN_CASE(14) ETH_LN_CASE(15) ETH_LN_CASE(16)
#undef ETH_LN_CASE
  }
}

}  // namespace eth

using namespace eth;

extern "C" int eth_ln_fwd(const void* x, const void* gamma, const void* beta, void* y, float* mean,
                          float* rstd, int64_t rows, int64_t cols, float eps, int dtype,
                          void* stream) {
  ETH_CHECK_ARG(dtype == ETH_BF16 || dtype == ETH_F16, "eth_ln_fwd: dtype must be bf16/fp16");
  ETH_CHECK_ARG(rows >= 0 && rows < (1LL << 31) && cols > 0 && cols <= kMaxCols && cols % 8 == 0,
                "eth_ln_fwd: cols must be a positive multiple of 8 up to %d (got %lld)", kMaxCols,
                (long long)cols);
  if (rows == 0) return ETH_OK;
  ETH_CHECK_ARG(x && gamma && beta && y && mean && rstd, "eth_ln_fwd: null pointer");
  hipStream_t s = (hipStream_t)stream;
  if (dtype == ETH_BF16)
    launch_fwd<false>((const uint16_t*)x, (const uint16_t*)gamma, (const uint16_t*)beta, (uint16_t*)y,
                      mean, rstd, (int)rows, (int)cols, eps, s);
  else
    launch_fwd<true>((const uint16_t*)x, (const uint16_t*)gamma, (const uint16_t*)beta, (uint16_t*)y,
                     mean, rstd, (int)rows, (int)cols, eps, s);
  ETH_CHECK_LAUNCH("eth_ln_fwd");
  return ETH_OK;
}

extern "C" int64_t eth_ln_bwd_workspace(int64_t rows, int64_t cols) {
  const int64_t groups = rows < 1024 ? (rows + 31) / 32 : 1024;
  return groups * 2 * cols;
}

extern "C" int eth_ln_bwd(const void* dy, const void* x, const float* mean, const float* rstd,
                          const void* gamma, void* dx, float* dgamma, float* dbeta,
                          float* workspace, int64_t rows, int64_t cols, int accumulate, int dtype,
                          void* stream) {
  ETH_CHECK_ARG(dtype == ETH_BF16 || dtype == ETH_F16, "eth_ln_bwd: dtype must be bf16/fp16");
  ETH_CHECK_ARG(rows >= 0 && rows < (1LL << 31) && cols > 0 && cols <= kMaxCols && cols % 8 == 0,
                "eth_ln_bwd: bad shape");
  if (rows == 0) return ETH_OK;
  ETH_CHECK_ARG(dy && x && mean && rstd && gamma && dx && dgamma && dbeta && workspace,
                "eth_ln_bwd: null pointer");
  const int groups = (int)(rows < 1024 ? (rows + 31) / 32 : 1024);
  const int rpg = (int)((rows + groups - 1) / groups);
  hipStream_t s = (hipStream_t)stream;
  if (dtype == ETH_BF16)
    launch_bwd<false>((const uint16_t*)dy, (const uint16_t*)x, mean, rstd, (const uint16_t*)gamma,
                      (uint16_t*)dx, workspace, groups, rpg, (int)rows, (int)cols, s);
  else
    launch_bwd<true>((const uint16_t*)dy, (const uint16_t*)x, mean, rstd, (const uint16_t*)gamma,
                     (uint16_t*)dx, workspace, groups, rpg, (int)rows, (int)cols, s);
  ETH_CHECK_LAUNCH("eth_ln_bwd");
  // partials are [groups][2][cols]: dgamma rows at offset 0, dbeta at +cols
  reduce_partials_kernel<<<reduce_partials_grid((int)cols), kReducePartialsThreads, 0, s>>>(
      workspace, groups, (int)cols, 2 * cols, dgamma, accumulate);
  reduce_partials_kernel<<<reduce_partials_grid((int)cols), kReducePartialsThreads, 0, s>>>(
      workspace + cols, groups, (int)cols, 2 * cols, dbeta, accumulate);
  ETH_CHECK_LAUNCH("eth_ln_bwd reduce");
  return ETH_OK;
}
