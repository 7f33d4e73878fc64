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

// Only the fused multiply-adds written as __builtin_fmaf are fused: with
// contraction left to the compiler, a product followed by the 16-bit output
// rounding can become one single-rounding mixed-precision instruction in one
// template instantiation and not in another, and the instantiations (plain,
// residual, residual + column sums) must round alike.
#pragma clang fp contract(off)

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

// Row r of a [batch, seq] view of an x stored [seq, batch] (trb = batch;
// 0 leaves rows as they are): the transposed LayerNorm reads and writes x
// there while y, mean, rstd and dy stay in [batch, seq] row order.
__device__ __forceinline__ int sb_row(int r, int rows, int trb) {
  if (!trb) return r;
  const int seq = rows / trb;
  return (r % seq) * trb + r / seq;
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
                                                               int cols, float eps, int trb) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * kLnWaves + (threadIdx.x >> 6);
  if (row >= rows) return;
  const uint16_t* xr = x + (int64_t)sb_row(row, rows, trb) * cols;
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
        q = __builtin_fmaf(d, d, q);
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
        oe[j] = cvt_out<FP16>(__builtin_fmaf((v[i][j] - mu) * r, cvt_in<FP16>(ge[j]), cvt_in<FP16>(be[j])));
      *reinterpret_cast<uint4*>(yr + c) = out;
    }
  }
  if (lane == 0) {
    mean[row] = mu;
    rstd[row] = r;
  }
}

// Bias-dropout-add and the LayerNorm that follows it, one wave per row:
// h = residual + dropout(16-bit(x + b)) is rounded and stored exactly as
// bda_fwd_kernel does (same mask: the hash of the element's flat index), and
// the stored 16-bit h values are then normalized with ln_fwd_kernel's
// arithmetic, so h, y, mean and rstd are bit-identical to the two kernels in
// sequence while h is read from HBM once less.
template <int NV, bool FP16>
__global__ void __launch_bounds__(64 * kLnWaves) bda_ln_fwd_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ bias, const uint16_t* __restrict__ res,
    uint16_t* __restrict__ h, const uint16_t* __restrict__ gamma, const uint16_t* __restrict__ beta,
    uint16_t* __restrict__ y, float* __restrict__ mean, float* __restrict__ rstd, int rows, int cols, float eps,
    uint32_t thresh, float keep_scale, uint64_t seed) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * kLnWaves + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t base = (int64_t)row * cols;
  float v[NV][8];
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = (i * 64 + lane) * 8;
    if (c < cols) {
      const uint4 xr = *reinterpret_cast<const uint4*>(x + base + c);
      const uint4 rr = *reinterpret_cast<const uint4*>(res + base + c);
      const uint4 br = *reinterpret_cast<const uint4*>(bias + c);
      const uint16_t* xe = reinterpret_cast<const uint16_t*>(&xr);
      const uint16_t* re = reinterpret_cast<const uint16_t*>(&rr);
      const uint16_t* be = reinterpret_cast<const uint16_t*>(&br);
      uint4 hr;
      uint16_t* he = reinterpret_cast<uint16_t*>(&hr);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        float t = cvt_in<FP16>(cvt_out<FP16>(cvt_in<FP16>(xe[j]) + cvt_in<FP16>(be[j])));
        if (thresh) {
          const bool keep = hash_u32(seed, (uint64_t)(base + c + j)) >= thresh;
          t = cvt_in<FP16>(cvt_out<FP16>(keep ? t * keep_scale : 0.f));
        }
        he[j] = cvt_out<FP16>(cvt_in<FP16>(re[j]) + t);
        v[i][j] = cvt_in<FP16>(he[j]);
        s += v[i][j];
      }
      *reinterpret_cast<uint4*>(h + base + c) = hr;
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
        q = __builtin_fmaf(d, d, q);
      }
    }
  }
  const float var = wave_sum(q) / cols;
  const float r = rsqrtf(var + eps);
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = (i * 64 + lane) * 8;
    if (c < cols) {
      const uint4 gr = *reinterpret_cast<const uint4*>(gamma + c);
      const uint4 br = *reinterpret_cast<const uint4*>(beta + c);
      const uint16_t* ge = reinterpret_cast<const uint16_t*>(&gr);
      const uint16_t* be = reinterpret_cast<const uint16_t*>(&br);
      uint4 out;
      uint16_t* oe = reinterpret_cast<uint16_t*>(&out);
#pragma unroll
      for (int j = 0; j < 8; ++j)
        oe[j] = cvt_out<FP16>(__builtin_fmaf((v[i][j] - mu) * r, cvt_in<FP16>(ge[j]), cvt_in<FP16>(be[j])));
      *reinterpret_cast<uint4*>(y + base + c) = out;
    }
  }
  if (lane == 0) {
    mean[row] = mu;
    rstd[row] = r;
  }
}

// Backward.  A workgroup of kLnBwdWaves waves owns rows g, g + G, g + 2G, ...;
// T waves share a row (T = 1 up to 1024 columns, 2 up to 2048, 4 up to
// 4096, 8 up to 8192), each covering NVW <= 2 vectors of 512 columns (the
// per-lane state then fits the 256 registers of two waves per SIMD without
// spilling), so a group of T waves
// ("team") handles one row per iteration and the workgroup kLnBwdWaves / T
// rows.  The next row's x / dy / dresid are loaded while the current one is
// computed.  Per lane fp32 column sums of dy * xhat (dgamma), dy (dbeta) and,
// with CSUM, of the stored dx (the bias gradient of the bias-dropout-add whose
// output this LayerNorm normalised) stay in registers for all of the group's
// rows; the teams' sums are added through LDS in fixed order and stored to
// part[g][2][cols] / cpart[g][cols].  With RESID the stored gradient is
// dx = bf16(bf16(dx_ln) + dresid): the LayerNorm input gradient plus the
// residual branch's gradient, rounded as the two separate 16-bit tensors and
// their add would be.
constexpr int kLnBwdWaves = 8;
typedef uint32_t ln_u32x4 __attribute__((ext_vector_type(4)));
typedef float ln_f32x4 __attribute__((ext_vector_type(4)));

template <bool FP16>
__device__ __forceinline__ float half_at(const ln_u32x4& v, int j) {
  const uint32_t w = v[j >> 1];
  return cvt_in<FP16>((uint16_t)((j & 1) ? (w >> 16) : (w & 0xffffu)));
}

// A buffer descriptor over one row (cols 16-bit elements): lanes whose
// vector lies past the row end read zeros and their stores are dropped; a
// row that is not `live` reads as zeros throughout.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_rsrc(const uint16_t* base, int64_t row, int cols,
                                                           bool live = true) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(base + row * cols), (short)0,
                                           live ? cols * 2 : 0, 0x00020000);
}

template <int T, int NVW, bool FP16, bool RESID, bool CSUM>
__global__ void __launch_bounds__(64 * kLnBwdWaves) ln_bwd_kernel(
    const uint16_t* __restrict__ dy, const uint16_t* __restrict__ x, const float* __restrict__ mean,
    const float* __restrict__ rstd, const uint16_t* __restrict__ gamma, const uint16_t* __restrict__ dres,
    uint16_t* __restrict__ dx, float* __restrict__ part, float* __restrict__ cpart, int rows, int cols,
    int trb) {
  constexpr int TEAMS = kLnBwdWaves / T;
  constexpr int NQ = CSUM ? 3 : 2;
  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int team = wid / T, sub = wid - team * T;
  // vector i of this lane: columns (sub*NVW + i)*512 + lane*8 .. +7, byte
  // offset voff + i*1024 within the row
  const int voff = ((sub * NVW) * 64 + lane) * 16;
  ln_u32x4 g16[NVW];
  float acc[NQ][NVW][8];
  {
    const __amdgpu_buffer_rsrc_t gr = row_rsrc(gamma, 0, cols);
#pragma unroll
    for (int i = 0; i < NVW; ++i) {
      g16[i] = __builtin_amdgcn_raw_buffer_load_b128(gr, voff + i * 1024, 0, 0);
#pragma unroll
      for (int q = 0; q < NQ; ++q)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[q][i][j] = 0.f;
    }
  }
  // group g owns rows g, g + G, g + 2G, ... (G = gridDim.x): the groups
  // together sweep the tensor one band of G rows at a time
  const int G = gridDim.x, g = blockIdx.x;
  const int nrows = (rows - g + G - 1) / G;           // rows of this group
  const int iters = (nrows + TEAMS - 1) / TEAMS;      // equal for every wave of the group
  const float inv_n = 1.0f / cols;
  __shared__ float rsum[2][kLnBwdWaves][2];

  ln_u32x4 nx[NVW], nd[NVW], nr[NVW];
  auto load_row = [&](int k) __attribute__((always_inline)) {
    const bool live = k < nrows;
    const int r = g + k * G;
    const __amdgpu_buffer_rsrc_t xr = row_rsrc(x, live ? sb_row(r, rows, trb) : r, cols, live);
    const __amdgpu_buffer_rsrc_t dr = row_rsrc(dy, r, cols, live);
#pragma unroll
    for (int i = 0; i < NVW; ++i) {
      nx[i] = __builtin_amdgcn_raw_buffer_load_b128(xr, voff + i * 1024, 0, 0);
      nd[i] = __builtin_amdgcn_raw_buffer_load_b128(dr, voff + i * 1024, 0, 0);
    }
    if (RESID) {
      const __amdgpu_buffer_rsrc_t rr = row_rsrc(dres, r, cols, live);
#pragma unroll
      for (int i = 0; i < NVW; ++i) nr[i] = __builtin_amdgcn_raw_buffer_load_b128(rr, voff + i * 1024, 0, 0);
    }
  };
  load_row(team);
  for (int it = 0; it < iters; ++it) {
    const int k = it * TEAMS + team;
    const int r = g + k * G;
    const bool valid = k < nrows;
    ln_u32x4 cx[NVW], cd[NVW], cr[NVW];
#pragma unroll
    for (int i = 0; i < NVW; ++i) {
      cx[i] = nx[i];
      cd[i] = nd[i];
      if (RESID) cr[i] = nr[i];
    }
    const float mu = valid ? mean[r] : 0.f;
    const float rs = valid ? rstd[r] : 0.f;
    if (it + 1 < iters) load_row(k + TEAMS);
    float s1 = 0.f, s2 = 0.f;
#pragma unroll
    for (int i = 0; i < NVW; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float dv = half_at<FP16>(cd[i], j);
        const float xh = (half_at<FP16>(cx[i], j) - mu) * rs;
        const float dyg = dv * half_at<FP16>(g16[i], j);
        s1 += dyg;
        s2 = __builtin_fmaf(dyg, xh, s2);
        acc[0][i][j] = __builtin_fmaf(dv, xh, acc[0][i][j]);
        acc[1][i][j] += dv;
      }
    s1 = wave_sum(s1);
    s2 = wave_sum(s2);
    if (T > 1) {
      if (lane == 0) {
        rsum[it & 1][wid][0] = s1;
        rsum[it & 1][wid][1] = s2;
      }
      __syncthreads();
      s1 = s2 = 0.f;
#pragma unroll
      for (int t = 0; t < T; ++t) {
        s1 += rsum[it & 1][team * T + t][0];
        s2 += rsum[it & 1][team * T + t][1];
      }
    }
    // pass 2 converts the packed 16-bit values again: without this the
    // compiler keeps pass 1's 2 x 8 x NVW fp32 values live and spills
#pragma unroll
    for (int i = 0; i < NVW; ++i) {
      asm volatile("" : "+v"(cx[i]), "+v"(cd[i]));
      asm volatile("" : "+v"(g16[i]));
    }
    if (valid) {
      const __amdgpu_buffer_rsrc_t orow = row_rsrc(dx, sb_row(r, rows, trb), cols);
#pragma unroll
      for (int i = 0; i < NVW; ++i) {
        ln_u32x4 o;
#pragma unroll
        for (int j = 0; j < 8; j += 2) {
          float v[2];
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const float dv = half_at<FP16>(cd[i], j + h);
            const float xh = (half_at<FP16>(cx[i], j + h) - mu) * rs;
            v[h] = rs * __builtin_fmaf(-inv_n, __builtin_fmaf(xh, s2, s1), dv * half_at<FP16>(g16[i], j + h));
            if (RESID) v[h] = cvt_in<FP16>(cvt_out<FP16>(v[h])) + half_at<FP16>(cr[i], j + h);
          }
          const uint32_t w = FP16 ? f2h_pair(v[0], v[1]) : f2bf_pair(v[0], v[1]);
          o[j >> 1] = w;
          if (CSUM) {
            acc[NQ - 1][i][j] += cvt_in<FP16>((uint16_t)(w & 0xffffu));
            acc[NQ - 1][i][j + 1] += cvt_in<FP16>((uint16_t)(w >> 16));
          }
        }
        __builtin_amdgcn_raw_buffer_store_b128(o, orow, voff + i * 1024, 0, 0);
      }
    }
  }
  // teams' column sums -> one partial row per quantity, fixed order
  __shared__ float red[kLnBwdWaves][512];
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    float* dst = q < 2 ? part + ((int64_t)blockIdx.x * 2 + q) * cols : cpart + (int64_t)blockIdx.x * cols;
#pragma unroll
    for (int i = 0; i < NVW; ++i) {
      __syncthreads();
      ln_f32x4* rw = reinterpret_cast<ln_f32x4*>(&red[wid][lane * 8]);
      rw[0] = ln_f32x4{acc[q][i][0], acc[q][i][1], acc[q][i][2], acc[q][i][3]};
      rw[1] = ln_f32x4{acc[q][i][4], acc[q][i][5], acc[q][i][6], acc[q][i][7]};
      __syncthreads();
#pragma unroll
      for (int k = 0; k < T; ++k) {
        const int e = threadIdx.x;  // 512 threads: one column of sub k's chunk each
        const int c = (k * NVW + i) * 512 + e;
        if (c < cols) {
          float a = 0.f;
#pragma unroll
          for (int t = 0; t < TEAMS; ++t) a += red[t * T + k][e];
          dst[c] = a;
        }
      }
    }
  }
}

// Row groups of the backward: at most 256 workgroups (one per CU), each with
// at least one row per team.
inline int ln_bwd_team_waves(int64_t cols) {
  return cols <= 1024 ? 1 : (cols <= 2048 ? 2 : (cols <= 4096 ? 4 : 8));
}
inline int ln_bwd_groups(int64_t rows, int64_t cols) {
  const int64_t teams = kLnBwdWaves / ln_bwd_team_waves(cols);
  int64_t g = (rows + teams - 1) / teams;
  if (g > 256) g = 256;
  if (g < 1) g = 1;
  return (int)g;
}

template <bool FP16>
static void launch_fwd(const uint16_t* x, const uint16_t* g, const uint16_t* b, uint16_t* y, float* mean,
                       float* rstd, int rows, int cols, float eps, hipStream_t s, int trb = 0) {
  const int grid = (rows + kLnWaves - 1) / kLnWaves;
  const int nv = (cols + 511) / 512;
  switch (nv) {
#define ETH_LN_CASE(N) \
  case N: ln_fwd_kernel<N, FP16><<<grid, 64 * kLnWaves, 0, s>>>(x, g, b, y, mean, rstd, rows, cols, eps, trb); break;
    ETH_LN_CASE(1) ETH_LN_CASE(2) ETH_LN_CASE(3) ETH_LN_CASE(4) ETH_LN_CASE(5) ETH_LN_CASE(6)
    ETH_LN_CASE(7) ETH_LN_CASE(8) ETH_LN_CASE(9) ETH_LN_CASE(10) ETH_LN_CASE(11) ETH_LN_CASE(12)
    ETH_LN_CASE(13) ETH_LN_CASE(14) ETH_LN_CASE(15) ETH_LN_CASE(16)
#undef ETH_LN_CASE
  }
}

template <bool FP16>
static void launch_bda_ln(const uint16_t* x, const uint16_t* bias, const uint16_t* res, uint16_t* h,
                          const uint16_t* g, const uint16_t* b, uint16_t* y, float* mean, float* rstd, int rows,
                          int cols, float eps, uint32_t thresh, float keep_scale, uint64_t seed, hipStream_t s) {
  const int grid = (rows + kLnWaves - 1) / kLnWaves;
  const int nv = (cols + 511) / 512;
  switch (nv) {
#define ETH_BDA_LN_CASE(N)                                                                                  \
  case N:                                                                                                   \
    bda_ln_fwd_kernel<N, FP16><<<grid, 64 * kLnWaves, 0, s>>>(x, bias, res, h, g, b, y, mean, rstd, rows, cols, \
                                                               eps, thresh, keep_scale, seed);              \
    break;
    ETH_BDA_LN_CASE(1) ETH_BDA_LN_CASE(2) ETH_BDA_LN_CASE(3) ETH_BDA_LN_CASE(4) ETH_BDA_LN_CASE(5)
    ETH_BDA_LN_CASE(6) ETH_BDA_LN_CASE(7) ETH_BDA_LN_CASE(8) ETH_BDA_LN_CASE(9) ETH_BDA_LN_CASE(10)
    ETH_BDA_LN_CASE(11) ETH_BDA_LN_CASE(12) ETH_BDA_LN_CASE(13) ETH_BDA_LN_CASE(14) ETH_BDA_LN_CASE(15)
    ETH_BDA_LN_CASE(16)
#undef ETH_BDA_LN_CASE
  }
}

template <bool FP16, bool RESID, bool CSUM>
static void launch_bwd(const uint16_t* dy, const uint16_t* x, const float* mean, const float* rstd,
                       const uint16_t* g, const uint16_t* dres, uint16_t* dx, float* part, float* cpart,
                       int groups, int rows, int cols, hipStream_t s, int trb) {
  const int nv = (cols + 511) / 512;
  const dim3 block(64 * kLnBwdWaves);
#define ETH_LN_BWD(T, N)                                                                              \
  ln_bwd_kernel<T, N, FP16, RESID, CSUM><<<groups, block, 0, s>>>(dy, x, mean, rstd, g, dres, dx, part, \
                                                                  cpart, rows, cols, trb)
  if (nv == 1) ETH_LN_BWD(1, 1);
  else if (nv == 2) ETH_LN_BWD(1, 2);
  else if (nv <= 4) ETH_LN_BWD(2, 2);
  else if (nv <= 8) ETH_LN_BWD(4, 2);
  else ETH_LN_BWD(8, 2);
#undef ETH_LN_BWD
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

extern "C" int eth_bda_ln_fwd(const void* x, const void* bias, const void* residual, void* h,
                              const void* gamma, const void* beta, void* y, float* mean, float* rstd,
                              int64_t rows, int64_t cols, float p, uint64_t seed, float eps, int dtype,
                              void* stream) {
  ETH_CHECK_ARG(dtype == ETH_BF16 || dtype == ETH_F16, "eth_bda_ln_fwd: dtype must be bf16/fp16");
  ETH_CHECK_ARG(rows >= 0 && rows < (1LL << 31) && cols > 0 && cols <= kMaxCols && cols % 8 == 0,
                "eth_bda_ln_fwd: cols must be a positive multiple of 8 up to %d (got %lld)", kMaxCols,
                (long long)cols);
  ETH_CHECK_ARG(p >= 0.f && p < 1.f, "eth_bda_ln_fwd: p must be in [0, 1)");
  if (rows == 0) return ETH_OK;
  ETH_CHECK_ARG(x && bias && residual && h && gamma && beta && y && mean && rstd, "eth_bda_ln_fwd: null pointer");
  uint32_t thresh;
  float scale;
  dropout_params(p, thresh, scale);
  hipStream_t s = (hipStream_t)stream;
  if (dtype == ETH_BF16)
    launch_bda_ln<false>((const uint16_t*)x, (const uint16_t*)bias, (const uint16_t*)residual, (uint16_t*)h,
                         (const uint16_t*)gamma, (const uint16_t*)beta, (uint16_t*)y, mean, rstd, (int)rows,
                         (int)cols, eps, thresh, scale, seed, s);
  else
    launch_bda_ln<true>((const uint16_t*)x, (const uint16_t*)bias, (const uint16_t*)residual, (uint16_t*)h,
                        (const uint16_t*)gamma, (const uint16_t*)beta, (uint16_t*)y, mean, rstd, (int)rows,
                        (int)cols, eps, thresh, scale, seed, s);
  ETH_CHECK_LAUNCH("eth_bda_ln_fwd");
  return ETH_OK;
}

extern "C" int64_t eth_ln_bwd_groups(int64_t rows, int64_t cols) {
  if (rows <= 0 || cols <= 0) return 1;
  return ln_bwd_groups(rows, cols);
}

extern "C" int64_t eth_ln_bwd_workspace(int64_t rows, int64_t cols) {
  return eth_ln_bwd_groups(rows, cols) * 2 * cols;
}

template <bool RESID, bool CSUM>
static void ln_bwd_dispatch(const void* dy, const void* x, const float* mean, const float* rstd,
                            const void* gamma, const void* dresid, void* dx, float* part, float* cpart,
                            int groups, int rows, int cols, int dtype, hipStream_t s, int trb = 0) {
  if (dtype == ETH_BF16)
    launch_bwd<false, RESID, CSUM>((const uint16_t*)dy, (const uint16_t*)x, mean, rstd, (const uint16_t*)gamma,
                                   (const uint16_t*)dresid, (uint16_t*)dx, part, cpart, groups, rows, cols, s, trb);
  else
    launch_bwd<true, RESID, CSUM>((const uint16_t*)dy, (const uint16_t*)x, mean, rstd, (const uint16_t*)gamma,
                                  (const uint16_t*)dresid, (uint16_t*)dx, part, cpart, groups, rows, cols, s, trb);
}

extern "C" int eth_ln_bwd_residual(const void* dy, const void* x, const float* mean, const float* rstd,
                                   const void* gamma, const void* dresid, void* dx, float* dgamma,
                                   float* dbeta, float* colsum_part, float* workspace, int64_t rows,
                                   int64_t cols, int accumulate, int dtype, void* stream) {
  ETH_CHECK_ARG(dtype == ETH_BF16 || dtype == ETH_F16, "eth_ln_bwd: dtype must be bf16/fp16");
  ETH_CHECK_ARG(rows >= 0 && rows < (1LL << 31) && cols > 0 && cols <= kMaxCols && cols % 8 == 0,
                "eth_ln_bwd: cols must be a positive multiple of 8 up to %d (got %lld)", kMaxCols,
                (long long)cols);
  if (rows == 0) return ETH_OK;
  ETH_CHECK_ARG(dy && x && mean && rstd && gamma && dx && dgamma && dbeta && workspace,
                "eth_ln_bwd: null pointer");
  ETH_CHECK_ARG(dresid || !colsum_part, "eth_ln_bwd_residual: colsum_part needs dresid");
  ETH_CHECK_ARG((((uintptr_t)workspace | (uintptr_t)dy | (uintptr_t)x | (uintptr_t)dx | (uintptr_t)gamma |
                  (uintptr_t)dresid | (uintptr_t)colsum_part) & 15u) == 0,
                "eth_ln_bwd: operands must be 16-byte aligned");
  const int groups = (int)eth_ln_bwd_groups(rows, cols);
  hipStream_t s = (hipStream_t)stream;
  if (!dresid)
    ln_bwd_dispatch<false, false>(dy, x, mean, rstd, gamma, nullptr, dx, workspace, nullptr, groups, (int)rows,
                                  (int)cols, dtype, s);
  else if (!colsum_part)
    ln_bwd_dispatch<true, false>(dy, x, mean, rstd, gamma, dresid, dx, workspace, nullptr, groups, (int)rows,
                                 (int)cols, dtype, s);
  else
    ln_bwd_dispatch<true, true>(dy, x, mean, rstd, gamma, dresid, dx, workspace, colsum_part, groups,
                                (int)rows, (int)cols, dtype, s);
  ETH_CHECK_LAUNCH("eth_ln_bwd");
  // partials are [groups][2][cols]: dgamma at offset 0, dbeta at +cols; one
  // launch reduces both
  reduce_partials_kernel<<<reduce_partials_grid((int)cols, 2), kReducePartialsThreads, 0, s>>>(
      workspace, groups, (int)cols, 2 * cols, dgamma, dbeta, accumulate);
  ETH_CHECK_LAUNCH("eth_ln_bwd reduce");
  return ETH_OK;
}

extern "C" int eth_ln_bwd(const void* dy, const void* x, const float* mean, const float* rstd,
                          const void* gamma, void* dx, float* dgamma, float* dbeta,
                          float* workspace, int64_t rows, int64_t cols, int accumulate, int dtype,
                          void* stream) {
  return eth_ln_bwd_residual(dy, x, mean, rstd, gamma, nullptr, dx, dgamma, dbeta, nullptr, workspace, rows, cols,
                             accumulate, dtype, stream);
}

// The LayerNorm of a [seq, batch, cols] input written as [batch, seq, cols]
// (and its backward, taking dy in [batch, seq] order and writing dx as
// [seq, batch]): the same kernels, reading and writing x through the row
// permutation, so the results are those of the transposed copy followed by
// eth_ln_fwd / eth_ln_bwd bit for bit.
extern "C" int eth_ln_fwd_sb(const void* x, const void* gamma, const void* beta, void* y, float* mean,
                             float* rstd, int64_t seq, int64_t batch, int64_t cols, float eps, int dtype,
                             void* stream) {
  ETH_CHECK_ARG(dtype == ETH_BF16 || dtype == ETH_F16, "eth_ln_fwd_sb: dtype must be bf16/fp16");
  ETH_CHECK_ARG(seq >= 0 && batch >= 0 && seq * batch < (1LL << 31) && cols > 0 && cols <= kMaxCols &&
                    cols % 8 == 0,
                "eth_ln_fwd_sb: bad sizes (seq %lld, batch %lld, cols %lld)", (long long)seq, (long long)batch,
                (long long)cols);
  if (seq * batch == 0) return ETH_OK;
  ETH_CHECK_ARG(x && gamma && beta && y && mean && rstd, "eth_ln_fwd_sb: null pointer");
  hipStream_t s = (hipStream_t)stream;
  const int rows = (int)(seq * batch);
  if (dtype == ETH_BF16)
    launch_fwd<false>((const uint16_t*)x, (const uint16_t*)gamma, (const uint16_t*)beta, (uint16_t*)y,
                      mean, rstd, rows, (int)cols, eps, s, (int)batch);
  else
    launch_fwd<true>((const uint16_t*)x, (const uint16_t*)gamma, (const uint16_t*)beta, (uint16_t*)y,
                     mean, rstd, rows, (int)cols, eps, s, (int)batch);
  ETH_CHECK_LAUNCH("eth_ln_fwd_sb");
  return ETH_OK;
}

extern "C" int eth_ln_bwd_sb(const void* dy, const void* x, const float* mean, const float* rstd,
                             const void* gamma, void* dx, float* dgamma, float* dbeta, float* workspace,
                             int64_t seq, int64_t batch, int64_t cols, int accumulate, int dtype,
                             void* stream) {
  ETH_CHECK_ARG(dtype == ETH_BF16 || dtype == ETH_F16, "eth_ln_bwd_sb: dtype must be bf16/fp16");
  ETH_CHECK_ARG(seq >= 0 && batch >= 0 && seq * batch < (1LL << 31) && cols > 0 && cols <= kMaxCols &&
                    cols % 8 == 0,
                "eth_ln_bwd_sb: bad sizes (seq %lld, batch %lld, cols %lld)", (long long)seq, (long long)batch,
                (long long)cols);
  const int64_t rows = seq * batch;
  if (rows == 0) return ETH_OK;
  ETH_CHECK_ARG(dy && x && mean && rstd && gamma && dx && dgamma && dbeta && workspace,
                "eth_ln_bwd_sb: null pointer");
  ETH_CHECK_ARG((((uintptr_t)workspace | (uintptr_t)dy | (uintptr_t)x | (uintptr_t)dx | (uintptr_t)gamma) & 15u) == 0,
                "eth_ln_bwd_sb: operands must be 16-byte aligned");
  const int groups = (int)eth_ln_bwd_groups(rows, cols);
  hipStream_t s = (hipStream_t)stream;
  ln_bwd_dispatch<false, false>(dy, x, mean, rstd, gamma, nullptr, dx, workspace, nullptr, groups, (int)rows,
                                (int)cols, dtype, s, (int)batch);
  ETH_CHECK_LAUNCH("eth_ln_bwd_sb");
  reduce_partials_kernel<<<reduce_partials_grid((int)cols, 2), kReducePartialsThreads, 0, s>>>(
      workspace, groups, (int)cols, 2 * cols, dgamma, dbeta, accumulate);
  ETH_CHECK_LAUNCH("eth_ln_bwd_sb reduce");
  return ETH_OK;
}
