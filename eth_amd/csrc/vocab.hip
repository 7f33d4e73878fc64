// Vocabulary-side kernels of the first / last pipeline stage.
//
//   embedding fwd   out[s, b, :] = word[tok[b, s]] + pos[pid[b, s]]   (16-bit,
//                   one rounding, written directly in the [s, b, h] layout the
//                   reference gets from .transpose(0, 1).contiguous())
//                   (Embedding_v1.forward, eth/runtime/megatron/model/flex_ops.py:450-485)
//   embedding bwd   dword[tok] += dout, dpos[pid] += dout in fp32 main grads
//                   (atomic adds; F.embedding's backward)
//   cross entropy   loss = logsumexp(z) - z[label] per row in fp32 from the
//                   16-bit logits (the `.float()` of flex_ops.py:1976-1981 is
//                   folded into the read); backward
//                   dz = (exp(z - lse) - onehot(label)) * dloss, written 16-bit
//                   (_VocabParallelCrossEntropy, mpu/cross_entropy.py:36-115, TP = 1)
//
// Token ids outside [0, V) are clamped for the memory access and reported in
// `bad_index` (set to 1), which the host checks; the reference's embedding
// would raise for them.
#include "common.h"

namespace eth {

template <bool FP16>
__device__ __forceinline__ float vin(uint16_t v) {
  return FP16 ? h2f_bits(v) : bf2f(v);
}
template <bool FP16>
__device__ __forceinline__ uint16_t vout(float v) {
  return FP16 ? f2h_bits(v) : f2bf(v);
}

// one wavefront per token row; lanes stride over h in 8-element vectors
template <bool FP16>
__global__ void __launch_bounds__(256) embedding_fwd_kernel(const int64_t* __restrict__ tok,
                                                            const int64_t* __restrict__ pid,
                                                            const uint16_t* __restrict__ word,
                                                            const uint16_t* __restrict__ pos,
                                                            uint16_t* __restrict__ out, int B, int S, int H,
                                                            int64_t V, int64_t P, int* __restrict__ bad) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);  // row = s * B + b
  if (row >= (int64_t)S * B) return;
  const int si = (int)(row / B), bi = (int)(row % B);
  int64_t t = tok[(int64_t)bi * S + si], p = pid[(int64_t)bi * S + si];
  if (t < 0 || t >= V || p < 0 || p >= P) {
    if (lane == 0) *bad = 1;
    t = t < 0 ? 0 : (t >= V ? V - 1 : t);
    p = p < 0 ? 0 : (p >= P ? P - 1 : p);
  }
  const uint16_t* w = word + t * H;
  const uint16_t* q = pos + p * H;
  uint16_t* o = out + row * H;
  for (int c = lane * 8; c < H; c += 512) {
    uint4 a = *reinterpret_cast<const uint4*>(w + c);
    uint4 bb = *reinterpret_cast<const uint4*>(q + c);
    const uint16_t* ae = reinterpret_cast<const uint16_t*>(&a);
    const uint16_t* be = reinterpret_cast<const uint16_t*>(&bb);
    uint4 r;
    uint16_t* re = reinterpret_cast<uint16_t*>(&r);
#pragma unroll
    for (int j = 0; j < 8; ++j) re[j] = vout<FP16>(vin<FP16>(ae[j]) + vin<FP16>(be[j]));
    *reinterpret_cast<uint4*>(o + c) = r;
  }
}

template <bool FP16>
__global__ void __launch_bounds__(256) embedding_bwd_kernel(const int64_t* __restrict__ tok,
                                                            const int64_t* __restrict__ pid,
                                                            const uint16_t* __restrict__ dout,
                                                            float* __restrict__ dword, float* __restrict__ dpos,
                                                            int B, int S, int H, int64_t V, int64_t P) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= (int64_t)S * B) return;
  const int si = (int)(row / B), bi = (int)(row % B);
  int64_t t = tok[(int64_t)bi * S + si], p = pid[(int64_t)bi * S + si];
  t = t < 0 ? 0 : (t >= V ? V - 1 : t);
  p = p < 0 ? 0 : (p >= P ? P - 1 : p);
  const uint16_t* g = dout + row * H;
  for (int c = lane * 8; c < H; c += 512) {
    uint4 a = *reinterpret_cast<const uint4*>(g + c);
    const uint16_t* ae = reinterpret_cast<const uint16_t*>(&a);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float v = vin<FP16>(ae[j]);
      if (dword) atomicAdd(dword + t * H + c + j, v);
      if (dpos) atomicAdd(dpos + p * H + c + j, v);
    }
  }
}

constexpr int kXentThreads = 256;

// one workgroup per row: online max / sum-exp over the vocabulary
template <bool FP16>
__global__ void __launch_bounds__(kXentThreads) xent_fwd_kernel(const uint16_t* __restrict__ logits, int64_t ld,
                                                                 const int64_t* __restrict__ labels,
                                                                 float* __restrict__ loss, float* __restrict__ lse,
                                                                 int64_t V, int* __restrict__ bad) {
  __shared__ float sm[kXentThreads / 64], ss[kXentThreads / 64];
  const int64_t row = blockIdx.x;
  const uint16_t* z = logits + row * ld;
  float m = -INFINITY, s = 0.f;
  const int64_t nv = V / 8;
  for (int64_t i = threadIdx.x; i < nv; i += kXentThreads) {
    uint4 a = *reinterpret_cast<const uint4*>(z + i * 8);
    const uint16_t* e = reinterpret_cast<const uint16_t*>(&a);
    float x[8], mx = m;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      x[j] = vin<FP16>(e[j]);
      mx = fmaxf(mx, x[j]);
    }
    s *= __expf(m - mx);
#pragma unroll
    for (int j = 0; j < 8; ++j) s += __expf(x[j] - mx);
    m = mx;
  }
  for (int64_t i = nv * 8 + threadIdx.x; i < V; i += kXentThreads) {
    const float x = vin<FP16>(z[i]);
    const float mx = fmaxf(m, x);
    s = s * __expf(m - mx) + __expf(x - mx);
    m = mx;
  }
  // combine (m, s) across the wavefront, then across waves
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float mo = __shfl_xor(m, off, 64), so = __shfl_xor(s, off, 64);
    const float mx = fmaxf(m, mo);
    s = (m == -INFINITY ? 0.f : s * __expf(m - mx)) + (mo == -INFINITY ? 0.f : so * __expf(mo - mx));
    m = mx;
  }
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    sm[w] = m;
    ss[w] = s;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float M = sm[0], Ssum = ss[0];
    for (int k = 1; k < kXentThreads / 64; ++k) {
      const float mx = fmaxf(M, sm[k]);
      Ssum = Ssum * __expf(M - mx) + ss[k] * __expf(sm[k] - mx);
      M = mx;
    }
    const float l = M + __logf(Ssum);
    int64_t t = labels[row];
    if (t < 0 || t >= V) {
      *bad = 1;
      t = t < 0 ? 0 : V - 1;
    }
    lse[row] = l;
    loss[row] = l - vin<FP16>(z[t]);
  }
}

template <bool FP16>
__global__ void __launch_bounds__(kXentThreads) xent_bwd_kernel(const uint16_t* __restrict__ logits, int64_t ld,
                                                                 const int64_t* __restrict__ labels,
                                                                 const float* __restrict__ lse,
                                                                 const float* __restrict__ dloss,
                                                                 uint16_t* __restrict__ dz, int64_t ldd, int64_t V) {
  const int64_t row = blockIdx.y;
  const uint16_t* z = logits + row * ld;
  uint16_t* d = dz + row * ldd;
  const float l = lse[row], g = dloss[row];
  int64_t t = labels[row];
  t = t < 0 ? 0 : (t >= V ? V - 1 : t);
  const int64_t nv = V / 8;
  for (int64_t i = blockIdx.x * (int64_t)kXentThreads + threadIdx.x; i < nv; i += (int64_t)gridDim.x * kXentThreads) {
    uint4 a = *reinterpret_cast<const uint4*>(z + i * 8);
    const uint16_t* e = reinterpret_cast<const uint16_t*>(&a);
    uint4 r;
    uint16_t* re = reinterpret_cast<uint16_t*>(&r);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t v = i * 8 + j;
      const float p = __expf(vin<FP16>(e[j]) - l);
      re[j] = vout<FP16>((p - (v == t ? 1.f : 0.f)) * g);
    }
    *reinterpret_cast<uint4*>(d + i * 8) = r;
  }
  if (blockIdx.x == 0)
    for (int64_t v = nv * 8 + threadIdx.x; v < V; v += kXentThreads) {
      const float p = __expf(vin<FP16>(z[v]) - l);
      d[v] = vout<FP16>((p - (v == t ? 1.f : 0.f)) * g);
    }
}

// a = b = a + b over n fp32 elements (tied-embedding gradient sum)
__global__ void tied_sum_kernel(float* __restrict__ a, float* __restrict__ b, int64_t n) {
  const int64_t nv = n / 4;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < nv; i += (int64_t)gridDim.x * blockDim.x) {
    float4 x = reinterpret_cast<float4*>(a)[i], y = reinterpret_cast<const float4*>(b)[i];
    x.x += y.x; x.y += y.y; x.z += y.z; x.w += y.w;
    reinterpret_cast<float4*>(a)[i] = x;
    reinterpret_cast<float4*>(b)[i] = x;
  }
  for (int64_t i = nv * 4 + blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const float v = a[i] + b[i];
    a[i] = v;
    b[i] = v;
  }
}

}  // namespace eth

using namespace eth;

extern "C" int eth_tied_grad_sum(float* root, float* copy, int64_t n, void* stream) {
  ETH_CHECK_ARG(n >= 0 && (n == 0 || (root && copy)), "eth_tied_grad_sum: bad arguments");
  ETH_CHECK_ARG((((uintptr_t)root) & 15) == 0 && (((uintptr_t)copy) & 15) == 0,
                "eth_tied_grad_sum: buffers must be 16-byte aligned");
  if (n == 0) return ETH_OK;
  int64_t blocks = (n / 4 + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  if (blocks < 1) blocks = 1;
  tied_sum_kernel<<<(int)blocks, 256, 0, (hipStream_t)stream>>>(root, copy, n);
  ETH_CHECK_LAUNCH("eth_tied_grad_sum");
  return ETH_OK;
}

extern "C" int eth_embedding_fwd(const int64_t* tokens, const int64_t* positions, const void* word,
                                 const void* pos, void* out, int64_t batch, int64_t seq, int64_t hidden,
                                 int64_t vocab, int64_t max_pos, int* bad_index, int dtype, void* stream) {
  ETH_CHECK_ARG(dtype == ETH_BF16 || dtype == ETH_F16, "eth_embedding_fwd: dtype must be bf16/fp16");
  ETH_CHECK_ARG(batch > 0 && seq > 0 && hidden > 0 && hidden % 8 == 0 && vocab > 0 && max_pos > 0,
                "eth_embedding_fwd: bad shape");
  ETH_CHECK_ARG(tokens && positions && word && pos && out && bad_index, "eth_embedding_fwd: null pointer");
  const int64_t rows = batch * seq;
  const int grid = (int)((rows + 3) / 4);
  hipStream_t s = (hipStream_t)stream;
  if (dtype == ETH_BF16)
    embedding_fwd_kernel<false><<<grid, 256, 0, s>>>(tokens, positions, (const uint16_t*)word, (const uint16_t*)pos,
                                                     (uint16_t*)out, (int)batch, (int)seq, (int)hidden, vocab, max_pos,
                                                     bad_index);
  else
    embedding_fwd_kernel<true><<<grid, 256, 0, s>>>(tokens, positions, (const uint16_t*)word, (const uint16_t*)pos,
                                                    (uint16_t*)out, (int)batch, (int)seq, (int)hidden, vocab, max_pos,
                                                    bad_index);
  ETH_CHECK_LAUNCH("eth_embedding_fwd");
  return ETH_OK;
}

extern "C" int eth_embedding_bwd(const int64_t* tokens, const int64_t* positions, const void* dout,
                                 float* dword, float* dpos, int64_t batch, int64_t seq, int64_t hidden,
                                 int64_t vocab, int64_t max_pos, int dtype, void* stream) {
  ETH_CHECK_ARG(dtype == ETH_BF16 || dtype == ETH_F16, "eth_embedding_bwd: dtype must be bf16/fp16");
  ETH_CHECK_ARG(batch > 0 && seq > 0 && hidden > 0 && hidden % 8 == 0, "eth_embedding_bwd: bad shape");
  ETH_CHECK_ARG(tokens && positions && dout && (dword || dpos), "eth_embedding_bwd: null pointer");
  const int64_t rows = batch * seq;
  const int grid = (int)((rows + 3) / 4);
  hipStream_t s = (hipStream_t)stream;
  if (dtype == ETH_BF16)
    embedding_bwd_kernel<false><<<grid, 256, 0, s>>>(tokens, positions, (const uint16_t*)dout, dword, dpos,
                                                     (int)batch, (int)seq, (int)hidden, vocab, max_pos);
  else
    embedding_bwd_kernel<true><<<grid, 256, 0, s>>>(tokens, positions, (const uint16_t*)dout, dword, dpos,
                                                    (int)batch, (int)seq, (int)hidden, vocab, max_pos);
  ETH_CHECK_LAUNCH("eth_embedding_bwd");
  return ETH_OK;
}

extern "C" int eth_xent_fwd(const void* logits, int64_t ld, const int64_t* labels, float* loss, float* lse,
                            int64_t rows, int64_t vocab, int* bad_index, int dtype, void* stream) {
  ETH_CHECK_ARG(dtype == ETH_BF16 || dtype == ETH_F16, "eth_xent_fwd: dtype must be bf16/fp16");
  ETH_CHECK_ARG(rows >= 0 && rows < (1LL << 31) && vocab > 0 && ld >= vocab && ld % 8 == 0,
                "eth_xent_fwd: bad shape");
  if (rows == 0) return ETH_OK;
  ETH_CHECK_ARG(logits && labels && loss && lse && bad_index, "eth_xent_fwd: null pointer");
  hipStream_t s = (hipStream_t)stream;
  if (dtype == ETH_BF16)
    xent_fwd_kernel<false><<<(int)rows, kXentThreads, 0, s>>>((const uint16_t*)logits, ld, labels, loss, lse, vocab,
                                                              bad_index);
  else
    xent_fwd_kernel<true><<<(int)rows, kXentThreads, 0, s>>>((const uint16_t*)logits, ld, labels, loss, lse, vocab,
                                                             bad_index);
  ETH_CHECK_LAUNCH("eth_xent_fwd");
  return ETH_OK;
}

extern "C" int eth_xent_bwd(const void* logits, int64_t ld, const int64_t* labels, const float* lse,
                            const float* dloss, void* dlogits, int64_t ldd, int64_t rows, int64_t vocab, int dtype,
                            void* stream) {
  ETH_CHECK_ARG(dtype == ETH_BF16 || dtype == ETH_F16, "eth_xent_bwd: dtype must be bf16/fp16");
  ETH_CHECK_ARG(rows >= 0 && rows < 65536 * 32768LL && vocab > 0 && ld >= vocab && ld % 8 == 0 && ldd >= vocab &&
                    ldd % 8 == 0,
                "eth_xent_bwd: bad shape");
  if (rows == 0) return ETH_OK;
  ETH_CHECK_ARG(rows <= 65535, "eth_xent_bwd: at most 65535 rows per launch");
  ETH_CHECK_ARG(logits && labels && lse && dloss && dlogits, "eth_xent_bwd: null pointer");
  const int64_t nv = vocab / 8;
  int gx = (int)((nv + kXentThreads - 1) / kXentThreads);
  if (gx > 16) gx = 16;
  dim3 grid(gx, (unsigned)rows);
  hipStream_t s = (hipStream_t)stream;
  if (dtype == ETH_BF16)
    xent_bwd_kernel<false><<<grid, kXentThreads, 0, s>>>((const uint16_t*)logits, ld, labels, lse, dloss,
                                                         (uint16_t*)dlogits, ldd, vocab);
  else
    xent_bwd_kernel<true><<<grid, kXentThreads, 0, s>>>((const uint16_t*)logits, ld, labels, lse, dloss,
                                                        (uint16_t*)dlogits, ldd, vocab);
  ETH_CHECK_LAUNCH("eth_xent_bwd");
  return ETH_OK;
}
