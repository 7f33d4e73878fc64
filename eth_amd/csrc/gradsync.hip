// Block-wise gradient synchronization, local half: bucket pack, fused
// unpack / normalization / unscale / inf-nan flag / L2 partials, and the
// norm finalize.  One workgroup per chunk (<= ETH_CHUNK_ELEMS elements); a
// chunk is a strided 2-D block of one main_grad tensor.  The payload side is
// always contiguous, so contiguous chunks stream with 16-byte accesses.
//
// Semantics follow eth/runtime/megatron/grad_sync/executor.py:199-261 (pack,
// mul_, unpack), optimizer/optimizer.py:436-461 (unscale + found_inf) and
// grad_sync/optimizer_semantics.py:563-595 (L2 statistic + coefficient).
#include <stdarg.h>

#include "common.h"

namespace eth {

static thread_local std::string g_last_error;

void set_error(const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
}

constexpr int kThreads = 256;
constexpr int kPipe = 8;  // 16-byte vectors in flight per thread in the contiguous paths
typedef uint32_t gs_v4 __attribute__((ext_vector_type(4)));

template <typename T>
struct Elem;
template <>
struct Elem<float> {
  static constexpr int kVec = 4;
  typedef float4 V;
  __device__ static float get(float x, int) { return x; }
  __device__ static float put(float v, int) { return v; }
};
template <>
struct Elem<uint16_t> {
  static constexpr int kVec = 8;
  typedef uint4 V;
  __device__ static float get(uint16_t x, int dt) { return dt == ETH_BF16 ? bf2f(x) : h2f_bits(x); }
  __device__ static uint16_t put(float v, int dt) { return dt == ETH_BF16 ? f2bf(v) : f2h_bits(v); }
};

template <typename T>
__device__ __forceinline__ bool aligned16(const T* p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

// ---------------------------------------------------------------- pack ---
// payload[c.dst + i] = src[i] * c.scale for one chunk (the whole workgroup)
template <typename T>
__device__ __forceinline__ void pack_chunk(const eth_chunk_t& c, T* __restrict__ payload, int dtype) {
  const T* src = reinterpret_cast<const T*>(c.src);
  T* dst = payload + c.dst;
  const float scale = c.scale;
  const bool scaled = scale != 1.0f;
  const int64_t n = (int64_t)c.rows * c.row_len;
  constexpr int VW = Elem<T>::kVec;
  typedef typename Elem<T>::V V;
  if (c.rows == 1 && aligned16(src) && aligned16(dst)) {
    // kPipe 16-byte loads in flight per thread; main_grad is read once
    // (nontemporal), the payload stays cacheable for the collective and the
    // unpack that follow
    const int nv = (int)(n / VW);
    const gs_v4* s = reinterpret_cast<const gs_v4*>(src);
    gs_v4* d = reinterpret_cast<gs_v4*>(dst);
    auto scale_vec = [&](gs_v4& x) __attribute__((always_inline)) {
      if (scaled) {
        V y = __builtin_bit_cast(V, x);
        T* e = reinterpret_cast<T*>(&y);
#pragma unroll
        for (int j = 0; j < VW; ++j) e[j] = Elem<T>::put(Elem<T>::get(e[j], dtype) * scale, dtype);
        x = __builtin_bit_cast(gs_v4, y);
      }
    };
    int i = threadIdx.x;
    for (; i + (kPipe - 1) * kThreads < nv; i += kPipe * kThreads) {
      gs_v4 x[kPipe];
#pragma unroll
      for (int u = 0; u < kPipe; ++u) x[u] = __builtin_nontemporal_load(s + i + u * kThreads);
#pragma unroll
      for (int u = 0; u < kPipe; ++u) {
        scale_vec(x[u]);
        d[i + u * kThreads] = x[u];
      }
    }
    for (; i < nv; i += kThreads) {
      gs_v4 x = __builtin_nontemporal_load(s + i);
      scale_vec(x);
      d[i] = x;
    }
    for (int64_t i = (int64_t)nv * VW + threadIdx.x; i < n; i += kThreads) {
      T x = src[i];
      dst[i] = scaled ? Elem<T>::put(Elem<T>::get(x, dtype) * scale, dtype) : x;
    }
  } else {
    for (int64_t i = threadIdx.x; i < n; i += kThreads) {
      const int64_t r = i / c.row_len, col = i - r * c.row_len;
      T x = src[r * c.src_stride + col];
      dst[i] = scaled ? Elem<T>::put(Elem<T>::get(x, dtype) * scale, dtype) : x;
    }
  }
}

template <typename T>
__global__ void __launch_bounds__(kThreads) pack_kernel(const eth_chunk_t* __restrict__ chunks,
                                                        T* __restrict__ payload, int dtype) {
  pack_chunk<T>(chunks[blockIdx.x], payload, dtype);
}

// -------------------------------------------------------------- unpack ---
// One element of the fused unpack: v = payload * norm (rounded to T when
// norm != 1), stored to *keep when keep is given; the gradient g = v (times
// inv with ETH_UNPACK_UNSCALE) to out.  Returns g*g for the norm statistic.
template <typename T>
__device__ __forceinline__ float unpack_one(T pay, T* keep, T& out, float norm, float inv, int flags, int dtype,
                                            bool& bad) {
  float v = Elem<T>::get(pay, dtype);
  T vb = pay;
  if (norm != 1.0f) {
    vb = Elem<T>::put(v * norm, dtype);
    v = Elem<T>::get(vb, dtype);
  }
  if (keep) *keep = vb;
  float g = v;
  if (flags & ETH_UNPACK_UNSCALE) g = v * inv;  // fp32 only (checked on host)
  bad |= !isfinite(v);
  out = Elem<T>::put(g, dtype);
  return g * g;
}

// One chunk of the unpack: payload values from `src` (the chunk's payload
// range), the normalized payload values to `keep` (the same range of a
// payload buffer, possibly `src` itself; nullptr: not kept), gradients to the
// chunk's main_grad block.
template <typename T>
__device__ __forceinline__ void unpack_chunk(const eth_chunk_t& c, const T* src, T* keep, float norm, float inv,
                                             int flags, int dtype, float& sq, bool& bad) {
  T* dstp = reinterpret_cast<T*>(c.src);
  const int64_t n = (int64_t)c.rows * c.row_len;
  constexpr int VW = Elem<T>::kVec;
  typedef typename Elem<T>::V V;
  if (c.rows == 1 && aligned16(dstp) && aligned16(src) && (keep == nullptr || aligned16(keep))) {
    // kPipe 16-byte loads in flight per thread; main_grad is not read again
    // before the optimizer, after every bucket (nontemporal stores)
    const int nv = (int)(n / VW);
    const gs_v4* p = reinterpret_cast<const gs_v4*>(src);
    gs_v4* kp = reinterpret_cast<gs_v4*>(keep);
    gs_v4* d = reinterpret_cast<gs_v4*>(dstp);
    auto one_vec = [&](gs_v4 xv, int idx) __attribute__((always_inline)) {
      V x = __builtin_bit_cast(V, xv), k, y;
      T* xe = reinterpret_cast<T*>(&x);
      T* ke = reinterpret_cast<T*>(&k);
      T* ye = reinterpret_cast<T*>(&y);
#pragma unroll
      for (int j = 0; j < VW; ++j) sq += unpack_one<T>(xe[j], ke + j, ye[j], norm, inv, flags, dtype, bad);
      if (kp) kp[idx] = __builtin_bit_cast(gs_v4, k);
      __builtin_nontemporal_store(__builtin_bit_cast(gs_v4, y), d + idx);
    };
    int i = threadIdx.x;
    for (; i + (kPipe - 1) * kThreads < nv; i += kPipe * kThreads) {
      gs_v4 x[kPipe];
#pragma unroll
      for (int u = 0; u < kPipe; ++u) x[u] = p[i + u * kThreads];
#pragma unroll
      for (int u = 0; u < kPipe; ++u) one_vec(x[u], i + u * kThreads);
    }
    for (; i < nv; i += kThreads) one_vec(p[i], i);
    for (int64_t i = (int64_t)nv * VW + threadIdx.x; i < n; i += kThreads)
      sq += unpack_one<T>(src[i], keep ? keep + i : nullptr, dstp[i], norm, inv, flags, dtype, bad);
  } else {
    for (int64_t i = threadIdx.x; i < n; i += kThreads) {
      const int64_t r = i / c.row_len, col = i - r * c.row_len;
      sq += unpack_one<T>(src[i], keep ? keep + i : nullptr, dstp[r * c.src_stride + col], norm, inv, flags, dtype,
                          bad);
    }
  }
}

template <typename T>
__device__ __forceinline__ void unpack_stats(const eth_chunk_t& c, int flags, float sq, bool bad, float* found_inf,
                                             double* partials, int64_t slot, float* red) {
  if (flags & ETH_UNPACK_STATS) {
    if (bad) *found_inf = 1.0f;
    float tot = block_sum<kThreads>(sq, red);
    if (threadIdx.x == 0) partials[slot] = (c.flags & ETH_CHUNK_NORM) ? (double)tot : 0.0;
  }
}

template <typename T>
__global__ void __launch_bounds__(kThreads) unpack_kernel(const eth_chunk_t* __restrict__ chunks,
                                                          T* __restrict__ payload, int dtype,
                                                          float norm, float inv, int flags,
                                                          float* __restrict__ found_inf,
                                                          double* __restrict__ partials,
                                                          int64_t partial_base) {
  __shared__ float red[kThreads / 64];
  const eth_chunk_t c = chunks[blockIdx.x];
  // the normalized payload is written back in place (the reference's
  // payload.mul_), except where a later bucket of the pass packs over it
  const bool wb = (flags & ETH_UNPACK_WRITEBACK) && norm != 1.0f && !(c.flags & ETH_CHUNK_SHADOWED);
  T* pay = payload + c.dst;
  float sq = 0.f;
  bool bad = false;
  unpack_chunk<T>(c, pay, wb ? pay : nullptr, norm, inv, flags, dtype, sq, bad);
  unpack_stats<T>(c, flags, sq, bad, found_inf, partials, partial_base + blockIdx.x, red);
}

// ------------------------------------------------------ staged local pass ---
// One launch of the staged single-rank pass: workgroups [0, nu) unpack bucket
// k-1 from its staging half `ustage`, the rest pack bucket k into the other
// half `pstage`, so the two touch different memory.  A chunk that no later
// bucket packs over (not ETH_CHUNK_SHADOWED) also stores its payload values v
// into the bucket's own payload `upay` -- the values the per-bucket sequence
// leaves there -- so that buffer ends the pass as that sequence leaves it.
template <typename T>
__global__ void __launch_bounds__(kThreads) staged_step_kernel(const eth_chunk_t* __restrict__ uchunks, int nu,
                                                               const T* __restrict__ ustage, T* __restrict__ upay,
                                                               const eth_chunk_t* __restrict__ pchunks,
                                                               T* __restrict__ pstage, int dtype, float norm,
                                                               float inv, int flags, float* __restrict__ found_inf,
                                                               double* __restrict__ partials,
                                                               int64_t partial_base) {
  __shared__ float red[kThreads / 64];
  if ((int)blockIdx.x >= nu) {  // uniform per workgroup
    pack_chunk<T>(pchunks[blockIdx.x - nu], pstage, dtype);
    return;
  }
  const eth_chunk_t c = uchunks[blockIdx.x];
  float sq = 0.f;
  bool bad = false;
  unpack_chunk<T>(c, ustage + c.dst, (c.flags & ETH_CHUNK_SHADOWED) ? nullptr : upay + c.dst, norm, inv, flags,
                  dtype, sq, bad);
  unpack_stats<T>(c, flags, sq, bad, found_inf, partials, partial_base + blockIdx.x, red);
}

// ------------------------------------------------- standalone statistics ---
// TIED: the chunk's gradient g is first replaced by g + g[copy_off] -- the
// tied word-embedding sum, stored into both the root (g) and the copy --
// and the statistics are taken of that sum, element for element as the
// plain form takes them of a gradient holding it.
template <bool TIED>
__global__ void __launch_bounds__(kThreads) stats_kernel(const eth_chunk_t* __restrict__ chunks,
                                                         float inv, int flags,
                                                         float* __restrict__ found_inf,
                                                         double* __restrict__ partials,
                                                         int64_t partial_base, int64_t copy_off) {
  // every product and sum rounded on its own, so both forms of the kernel
  // form the same partials from the same values
#pragma clang fp contract(off)
  __shared__ float red[kThreads / 64];
  const eth_chunk_t c = chunks[blockIdx.x];
  float* g = reinterpret_cast<float*>(c.src);
  const int64_t n = (int64_t)c.rows * c.row_len;
  const bool unscale = !TIED && (flags & ETH_UNPACK_UNSCALE);
  // the scaled-overflow check multiplies by the loss scale (passed in `inv`)
  // without storing; with unscaling it is meaningless and ignored
  const float chk = (!unscale && (flags & ETH_STATS_SCALED_OVERFLOW)) ? inv : 1.0f;
  float sq = 0.f;
  bool bad = false;
  if (c.rows == 1 && aligned16(g)) {
    // the walk over the gradient is the same in both forms; a copy that is
    // not 16-byte aligned is read and written element by element
    const bool cvec = !TIED || aligned16(g + copy_off);
    const int64_t nv = n / 4;
    float4* gv = reinterpret_cast<float4*>(g);
    // one vector of the walk: vector i of the gradient, x its value (y the
    // copy's, for the tied sum)
    auto step = [&](int64_t i, float4 x, float4 y) __attribute__((always_inline)) {
      if (TIED) {
        float* cp = g + copy_off + 4 * i;
        x.x = x.x + y.x; x.y = x.y + y.y; x.z = x.z + y.z; x.w = x.w + y.w;
        gv[i] = x;
        if (cvec) {
          *reinterpret_cast<float4*>(cp) = x;
        } else {
          cp[0] = x.x; cp[1] = x.y; cp[2] = x.z; cp[3] = x.w;
        }
      }
      bad |= !isfinite(x.x * chk) | !isfinite(x.y * chk) | !isfinite(x.z * chk) | !isfinite(x.w * chk);
      if (unscale) {
        x.x *= inv; x.y *= inv; x.z *= inv; x.w *= inv;
        gv[i] = x;
      }
      sq += x.x * x.x + x.y * x.y + x.z * x.z + x.w * x.w;
    };
    auto copy_at = [&](int64_t i) __attribute__((always_inline)) {
      const float* cp = g + copy_off + 4 * i;
      return cvec ? *reinterpret_cast<const float4*>(cp) : make_float4(cp[0], cp[1], cp[2], cp[3]);
    };
    int64_t i = threadIdx.x;
    // four vectors per operand in flight per trip, taken in the order of
    // the one-vector walk below (the same sums, rounded alike)
    for (; i + 3 * kThreads < nv; i += 4 * kThreads) {
      float4 x[4], y[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        x[u] = gv[i + u * kThreads];
        y[u] = TIED ? copy_at(i + u * kThreads) : x[u];
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) step(i + u * kThreads, x[u], y[u]);
    }
    for (; i < nv; i += kThreads) step(i, gv[i], TIED ? copy_at(i) : gv[i]);
    for (int64_t i = nv * 4 + threadIdx.x; i < n; i += kThreads) {
      float x = g[i];
      if (TIED) g[i] = g[i + copy_off] = x = x + g[i + copy_off];
      bad |= !isfinite(x * chk);
      if (unscale) g[i] = x = x * inv;
      sq += x * x;
    }
  } else {
    for (int64_t i = threadIdx.x; i < n; i += kThreads) {
      const int64_t r = i / c.row_len, col = i - r * c.row_len;
      float* e = g + r * c.src_stride + col;
      float x = *e;
      if (TIED) *e = e[copy_off] = x = x + e[copy_off];
      bad |= !isfinite(x * chk);
      if (unscale) *e = x = x * inv;
      sq += x * x;
    }
  }
  if (bad) *found_inf = 1.0f;
  float tot = block_sum<kThreads>(sq, red);
  if (threadIdx.x == 0)
    partials[partial_base + blockIdx.x] = (c.flags & ETH_CHUNK_NORM) ? (double)tot : 0.0;
}

// ------------------------------------- widening copy + statistics ---
// 16-bit main grads (chunk.src, strided rows) into contiguous fp32 gradients
// out[chunk.dst ...]: g = float(x) (exact), then the unscale / flag / sum of
// squares of stats_kernel on g, in the same pass (R 2 B + W 4 B per element
// instead of a copy and a separate read-modify-write).
__global__ void __launch_bounds__(kThreads) widen_stats_kernel(const eth_chunk_t* __restrict__ chunks,
                                                               float* __restrict__ out, int dtype, float inv,
                                                               int flags, float* __restrict__ found_inf,
                                                               double* __restrict__ partials,
                                                               int64_t partial_base) {
  __shared__ float red[kThreads / 64];
  const eth_chunk_t c = chunks[blockIdx.x];
  const uint16_t* src = reinterpret_cast<const uint16_t*>(c.src);
  float* g = out + c.dst;
  const int64_t n = (int64_t)c.rows * c.row_len;
  const bool unscale = flags & ETH_UNPACK_UNSCALE;
  float sq = 0.f;
  bool bad = false;
  if (c.rows == 1 && aligned16(src) && aligned16(g)) {
    const int64_t nv = n / 8;
    for (int64_t i = threadIdx.x; i < nv; i += kThreads) {
      const uint4 a = reinterpret_cast<const uint4*>(src)[i];
      const uint16_t* e = reinterpret_cast<const uint16_t*>(&a);
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        float x = Elem<uint16_t>::get(e[j], dtype);
        bad |= !isfinite(x);
        if (unscale) x *= inv;
        sq += x * x;
        v[j] = x;
      }
      reinterpret_cast<float4*>(g)[2 * i] = make_float4(v[0], v[1], v[2], v[3]);
      reinterpret_cast<float4*>(g)[2 * i + 1] = make_float4(v[4], v[5], v[6], v[7]);
    }
    for (int64_t i = nv * 8 + threadIdx.x; i < n; i += kThreads) {
      float x = Elem<uint16_t>::get(src[i], dtype);
      bad |= !isfinite(x);
      if (unscale) x *= inv;
      sq += x * x;
      g[i] = x;
    }
  } else {
    for (int64_t i = threadIdx.x; i < n; i += kThreads) {
      const int64_t r = i / c.row_len, col = i - r * c.row_len;
      float x = Elem<uint16_t>::get(src[r * c.src_stride + col], dtype);
      bad |= !isfinite(x);
      if (unscale) x *= inv;
      sq += x * x;
      g[i] = x;
    }
  }
  if (flags & ETH_UNPACK_STATS) {
    if (bad) *found_inf = 1.0f;
    float tot = block_sum<kThreads>(sq, red);
    if (threadIdx.x == 0)
      partials[partial_base + blockIdx.x] = (c.flags & ETH_CHUNK_NORM) ? (double)tot : 0.0;
  }
}

// ---------------------------------------------------------- finalize ---
__global__ void __launch_bounds__(1024) finalize_kernel(const double* __restrict__ partials,
                                                        int64_t n, double max_norm,
                                                        double* __restrict__ stats) {
  __shared__ double red[1024];
  double s = 0.0;
  for (int64_t i = threadIdx.x; i < n; i += 1024) s += partials[i];
  red[threadIdx.x] = s;
  __syncthreads();
  for (int w = 512; w > 0; w >>= 1) {
    if (threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    const double tot = red[0];
    const double norm = sqrt(tot);
    stats[0] = tot;
    stats[1] = norm;
    stats[2] = max_norm > 0.0 ? max_norm / (norm + 1.0e-6) : 1.0;
  }
}

__global__ void __launch_bounds__(kReducePartialsThreads)
    reduce_partials_kernel(const float* __restrict__ part, int groups, int cols, int64_t ld,
                           float* __restrict__ out0, float* __restrict__ out1, int accumulate) {
  // 64 columns x 16 group-lanes per workgroup: lane (q, gl) sums float4
  // column quad q over groups gl, gl + 16, ... with four loads in flight,
  // then the 16 group-lane sums are added in fixed order (deterministic).
  // blockIdx.y selects the slab: 1 reads columns [cols, 2 cols) of each
  // partial row and writes out1.
  typedef float f4 __attribute__((ext_vector_type(4)));
  __shared__ f4 red[16][17];
  const int q = threadIdx.x & 15, gl = threadIdx.x >> 4;
  const int c = blockIdx.x * 64 + q * 4;
  const float* src = part + (blockIdx.y ? cols : 0);
  float* out = blockIdx.y ? out1 : out0;
  f4 a = {0.f, 0.f, 0.f, 0.f};
  if (c < cols) {
    const f4* p = reinterpret_cast<const f4*>(src + c);
    const int64_t ld4 = ld / 4;
    int g = gl;
    for (; g + 48 < groups; g += 64) {
      const f4 v0 = p[g * ld4], v1 = p[(g + 16) * ld4], v2 = p[(g + 32) * ld4], v3 = p[(g + 48) * ld4];
      a += v0;
      a += v1;
      a += v2;
      a += v3;
    }
    for (; g < groups; g += 16) a += p[g * ld4];
  }
  red[gl][q] = a;
  __syncthreads();
  if (threadIdx.x < 64) {
    const int col = blockIdx.x * 64 + threadIdx.x;
    if (col < cols) {
      const int qq = threadIdx.x >> 2, e = threadIdx.x & 3;
      float t = 0.f;
#pragma unroll
      for (int w = 0; w < 16; ++w) t += red[w][qq][e];
      out[col] = accumulate ? out[col] + t : t;
    }
  }
}

// dst[0, n) = v: up to three scalars to the first 16-byte boundary, then
// kFillVec nontemporal 16-byte stores per thread in one trip (short
// workgroups keep HBM busy), then the scalar tail; workgroup 0 writes the
// scalars
constexpr int kFillThreads = 256, kFillVec = 4;
typedef float ff32x4_t __attribute__((ext_vector_type(4)));
__global__ void __launch_bounds__(kFillThreads) fill_kernel(float* dst, int64_t n, float v) {
  const int64_t head = min(n, (int64_t)(((16 - ((uintptr_t)dst & 15)) & 15) / 4));
  const int64_t nv = (n - head) / 4;
  ff32x4_t* dv = reinterpret_cast<ff32x4_t*>(dst + head);
  const ff32x4_t x = {v, v, v, v};
  const int64_t i0 = (int64_t)blockIdx.x * (kFillThreads * kFillVec) + threadIdx.x;
#pragma unroll
  for (int u = 0; u < kFillVec; ++u) {
    const int64_t i = i0 + u * kFillThreads;
    if (i < nv) __builtin_nontemporal_store(x, dv + i);
  }
  if (blockIdx.x == 0) {
    if (threadIdx.x < head) dst[threadIdx.x] = v;
    for (int64_t i = head + nv * 4 + threadIdx.x; i < n; i += kFillThreads) dst[i] = v;
  }
}

template <typename T>
static void staged_launch(const eth_bucket_t* u, const void* ustage, const eth_bucket_t* p, void* pstage,
                          float norm, float inv, int flags, float* found_inf, double* partials, hipStream_t s) {
  const int nu = u ? (int)u->n_chunks : 0, np = p ? (int)p->n_chunks : 0;
  staged_step_kernel<T><<<nu + np, kThreads, 0, s>>>(
      u ? u->chunks : nullptr, nu, (const T*)ustage, u ? (T*)u->payload : nullptr, p ? p->chunks : nullptr,
      (T*)pstage, u ? u->dtype : p->dtype, norm, inv, flags, found_inf, partials, u ? u->partial_base : 0);
}

static void staged_step(const eth_bucket_t* u, const void* ustage, const eth_bucket_t* p, void* pstage, float norm,
                        float inv, int flags, float* found_inf, double* partials, hipStream_t s) {
  if (u && u->n_chunks == 0) u = nullptr;
  if (p && p->n_chunks == 0) p = nullptr;
  if (!u && !p) return;
  if (u && p && u->dtype != p->dtype) {  // one dtype per launch
    staged_step(u, ustage, nullptr, nullptr, norm, inv, flags, found_inf, partials, s);
    staged_step(nullptr, nullptr, p, pstage, norm, inv, flags, found_inf, partials, s);
    return;
  }
  const int dtype = u ? u->dtype : p->dtype;
  const int f = dtype == ETH_F32 ? flags : flags & ~ETH_UNPACK_UNSCALE;
  if (dtype == ETH_F32)
    staged_launch<float>(u, ustage, p, pstage, norm, inv, f, found_inf, partials, s);
  else
    staged_launch<uint16_t>(u, ustage, p, pstage, norm, inv, f, found_inf, partials, s);
}

}  // namespace eth

using namespace eth;

extern "C" {

int eth_abi_version(void) { return 1; }

const char* eth_last_error(void) { return g_last_error.c_str(); }

int eth_reduce_partials(const float* part, int64_t groups, int64_t cols, int64_t ld, float* out, int accumulate,
                        void* stream) {
  ETH_CHECK_ARG(groups >= 1 && groups < (1LL << 31) && cols > 0 && cols < (1LL << 31) && cols % 4 == 0 &&
                    ld >= cols && ld % 4 == 0,
                "eth_reduce_partials: bad shape (groups %lld, cols %lld, ld %lld)", (long long)groups,
                (long long)cols, (long long)ld);
  ETH_CHECK_ARG(part && out && ((uintptr_t)part & 15u) == 0, "eth_reduce_partials: bad pointers");
  reduce_partials_kernel<<<reduce_partials_grid((int)cols), kReducePartialsThreads, 0, (hipStream_t)stream>>>(
      part, (int)groups, (int)cols, ld, out, nullptr, accumulate);
  ETH_CHECK_LAUNCH("eth_reduce_partials");
  return ETH_OK;
}

int eth_fill_f32(float* dst, int64_t n, float value, void* stream) {
  ETH_CHECK_ARG(n >= 0 && (n == 0 || dst), "eth_fill_f32: bad arguments");
  if (n == 0) return ETH_OK;
  int64_t blocks = (n / 4 + kFillThreads * kFillVec - 1) / (kFillThreads * kFillVec);
  if (blocks < 1) blocks = 1;  // the scalars alone
  ETH_CHECK_ARG(blocks < (1LL << 31), "eth_fill_f32: too many elements (%lld)", (long long)n);
  fill_kernel<<<(int)blocks, kFillThreads, 0, (hipStream_t)stream>>>(dst, n, value);
  ETH_CHECK_LAUNCH("eth_fill_f32");
  return ETH_OK;
}

int eth_bucket_pack(const eth_chunk_t* chunks, int64_t n_chunks, void* payload, int dtype,
                    void* stream) {
  ETH_CHECK_ARG(valid_dtype(dtype), "eth_bucket_pack: unsupported dtype %d", dtype);
  ETH_CHECK_ARG(n_chunks >= 0 && n_chunks < (1LL << 31), "eth_bucket_pack: bad chunk count %lld",
                (long long)n_chunks);
  if (n_chunks == 0) return ETH_OK;
  ETH_CHECK_ARG(chunks && payload, "eth_bucket_pack: null pointer");
  hipStream_t s = (hipStream_t)stream;
  if (dtype == ETH_F32)
    pack_kernel<float><<<(int)n_chunks, kThreads, 0, s>>>(chunks, (float*)payload, dtype);
  else
    pack_kernel<uint16_t><<<(int)n_chunks, kThreads, 0, s>>>(chunks, (uint16_t*)payload, dtype);
  ETH_CHECK_LAUNCH("eth_bucket_pack");
  return ETH_OK;
}

int eth_bucket_unpack(const eth_chunk_t* chunks, int64_t n_chunks, void* payload, int dtype,
                      float normalization_scale, float inv_loss_scale, int flags,
                      float* found_inf, double* partials, int64_t partial_base, void* stream) {
  ETH_CHECK_ARG(valid_dtype(dtype), "eth_bucket_unpack: unsupported dtype %d", dtype);
  ETH_CHECK_ARG(n_chunks >= 0 && n_chunks < (1LL << 31), "eth_bucket_unpack: bad chunk count");
  ETH_CHECK_ARG(!(flags & ETH_UNPACK_UNSCALE) || dtype == ETH_F32,
                "eth_bucket_unpack: unscale requires fp32 gradients");
  ETH_CHECK_ARG(!(flags & ETH_UNPACK_STATS) || (found_inf && partials && partial_base >= 0),
                "eth_bucket_unpack: statistics requested without buffers");
  if (n_chunks == 0) return ETH_OK;
  ETH_CHECK_ARG(chunks && payload, "eth_bucket_unpack: null pointer");
  hipStream_t s = (hipStream_t)stream;
  if (dtype == ETH_F32)
    unpack_kernel<float><<<(int)n_chunks, kThreads, 0, s>>>(chunks, (float*)payload, dtype,
                                                            normalization_scale, inv_loss_scale,
                                                            flags, found_inf, partials,
                                                            partial_base);
  else
    unpack_kernel<uint16_t><<<(int)n_chunks, kThreads, 0, s>>>(
        chunks, (uint16_t*)payload, dtype, normalization_scale, inv_loss_scale, flags, found_inf,
        partials, partial_base);
  ETH_CHECK_LAUNCH("eth_bucket_unpack");
  return ETH_OK;
}

int eth_bucket_sync_local(const eth_bucket_t* buckets, int64_t n_buckets, float normalization_scale,
                          float inv_loss_scale, int flags, float* found_inf, double* partials,
                          void* staging, int64_t staging_half_bytes, void* stream) {
  ETH_CHECK_ARG(!staging || (staging_half_bytes > 0 && staging_half_bytes % 16 == 0 && ((uintptr_t)staging & 15) == 0),
                "eth_bucket_sync_local: staging must be 16-byte aligned halves");
  ETH_CHECK_ARG(n_buckets >= 0 && (n_buckets == 0 || buckets), "eth_bucket_sync_local: bad bucket array");
  ETH_CHECK_ARG(!(flags & ETH_UNPACK_STATS) || (found_inf && partials),
                "eth_bucket_sync_local: statistics requested without buffers");
  // every entry is checked before anything is launched, so a bad entry
  // leaves no half-synced pass behind
  for (int64_t i = 0; i < n_buckets; ++i) {
    const eth_bucket_t& b = buckets[i];
    ETH_CHECK_ARG(valid_dtype(b.dtype), "eth_bucket_sync_local: bucket %lld has unsupported dtype %d",
                  (long long)i, b.dtype);
    ETH_CHECK_ARG(b.n_chunks >= 0 && b.n_chunks < (1LL << 31) && (b.n_chunks == 0 || (b.chunks && b.payload)),
                  "eth_bucket_sync_local: bucket %lld has a bad chunk table or payload", (long long)i);
    ETH_CHECK_ARG(b.partial_base >= 0, "eth_bucket_sync_local: bucket %lld has a negative partial base",
                  (long long)i);
  }
  if (staging) {
    // bucket i packs into staging half (i & 1) and unpacks from it; step k
    // unpacks bucket k-1 and packs bucket k in one launch
    char* half[2] = {(char*)staging, (char*)staging + staging_half_bytes};
    hipStream_t s = (hipStream_t)stream;
    for (int64_t k = 0; k <= n_buckets; ++k) {
      const eth_bucket_t* u = k > 0 ? &buckets[k - 1] : nullptr;
      const eth_bucket_t* p = k < n_buckets ? &buckets[k] : nullptr;
      staged_step(u, half[(k - 1) & 1], p, half[k & 1], normalization_scale, inv_loss_scale, flags, found_inf,
                  partials, s);
      ETH_CHECK_LAUNCH("eth_bucket_sync_local");
    }
    return ETH_OK;
  }
  for (int64_t i = 0; i < n_buckets; ++i) {
    const eth_bucket_t& b = buckets[i];
    int status = eth_bucket_pack(b.chunks, b.n_chunks, b.payload, b.dtype, stream);
    if (status != ETH_OK) return status;
    const int f = b.dtype == ETH_F32 ? flags : flags & ~ETH_UNPACK_UNSCALE;
    status = eth_bucket_unpack(b.chunks, b.n_chunks, b.payload, b.dtype, normalization_scale, inv_loss_scale, f,
                               found_inf, partials, b.partial_base, stream);
    if (status != ETH_OK) return status;
  }
  return ETH_OK;
}

int eth_grad_stats(const eth_chunk_t* chunks, int64_t n_chunks, float inv_loss_scale, int flags,
                   float* found_inf, double* partials, int64_t partial_base, void* stream) {
  ETH_CHECK_ARG(n_chunks >= 0 && n_chunks < (1LL << 31), "eth_grad_stats: bad chunk count");
  ETH_CHECK_ARG(found_inf && partials && partial_base >= 0, "eth_grad_stats: null buffers");
  if (n_chunks == 0) return ETH_OK;
  ETH_CHECK_ARG(chunks, "eth_grad_stats: null chunk table");
  stats_kernel<false><<<(int)n_chunks, kThreads, 0, (hipStream_t)stream>>>(
      chunks, inv_loss_scale, flags, found_inf, partials, partial_base, 0);
  ETH_CHECK_LAUNCH("eth_grad_stats");
  return ETH_OK;
}

int eth_tied_grad_sum_stats(const eth_chunk_t* chunks, int64_t n_chunks, float* root, float* copy,
                            float loss_scale, float* found_inf, double* partials, int64_t partial_base,
                            void* stream) {
  ETH_CHECK_ARG(n_chunks >= 0 && n_chunks < (1LL << 31), "eth_tied_grad_sum_stats: bad chunk count");
  ETH_CHECK_ARG(found_inf && partials && partial_base >= 0, "eth_tied_grad_sum_stats: null buffers");
  if (n_chunks == 0) return ETH_OK;
  ETH_CHECK_ARG(chunks && root && copy, "eth_tied_grad_sum_stats: null pointer");
  ETH_CHECK_ARG(((uintptr_t)copy - (uintptr_t)root) % sizeof(float) == 0,
                "eth_tied_grad_sum_stats: root and copy must be fp32-aligned alike");
  const int64_t off = ((intptr_t)copy - (intptr_t)root) / (int64_t)sizeof(float);
  stats_kernel<true><<<(int)n_chunks, kThreads, 0, (hipStream_t)stream>>>(
      chunks, loss_scale, ETH_STATS_SCALED_OVERFLOW, found_inf, partials, partial_base, off);
  ETH_CHECK_LAUNCH("eth_tied_grad_sum_stats");
  return ETH_OK;
}

int eth_widen_grad_stats(const eth_chunk_t* chunks, int64_t n_chunks, float* out, int dtype,
                         float inv_loss_scale, int flags, float* found_inf, double* partials,
                         int64_t partial_base, void* stream) {
  ETH_CHECK_ARG(dtype == ETH_BF16 || dtype == ETH_F16, "eth_widen_grad_stats: dtype must be bf16/fp16");
  ETH_CHECK_ARG(n_chunks >= 0 && n_chunks < (1LL << 31), "eth_widen_grad_stats: bad chunk count");
  if (n_chunks == 0) return ETH_OK;
  ETH_CHECK_ARG(chunks && out, "eth_widen_grad_stats: null table or output");
  ETH_CHECK_ARG(!(flags & ETH_UNPACK_STATS) || (found_inf && partials && partial_base >= 0),
                "eth_widen_grad_stats: statistics need found_inf and partials");
  widen_stats_kernel<<<(int)n_chunks, kThreads, 0, (hipStream_t)stream>>>(
      chunks, out, dtype, inv_loss_scale, flags, found_inf, partials, partial_base);
  ETH_CHECK_LAUNCH("eth_widen_grad_stats");
  return ETH_OK;
}

int eth_grad_norm_finalize(const double* partials, int64_t n, double max_norm, double* stats,
                           void* stream) {
  ETH_CHECK_ARG(n >= 0 && stats && (n == 0 || partials), "eth_grad_norm_finalize: bad arguments");
  finalize_kernel<<<1, 1024, 0, (hipStream_t)stream>>>(partials, n, max_norm, stats);
  ETH_CHECK_LAUNCH("eth_grad_norm_finalize");
  return ETH_OK;
}

}  // extern "C"
