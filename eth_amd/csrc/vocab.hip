// Vocabulary-side kernels of the first / last pipeline stage.
//
//   embedding fwd   out[s, b, :] = word[tok[b, s]] + pos[pid[b, s]]   (16-bit,
//                   one rounding, written directly in the [s, b, h] layout the
//                   reference gets from .transpose(0, 1).contiguous())
//                   (Embedding_v1.forward, eth/runtime/megatron/model/flex_ops.py:450-485)
//   embedding bwd   dword[tok] += dout, dpos[pid] += dout in fp32 main grads,
//                   deterministic (sort + one owner per row; F.embedding's
//                   backward, which is a sort + segmented reduction too)
//   cross entropy   loss = log sum exp(z - max) - (z[label] - max) per row in fp32 from the
//                   16-bit logits (the `.float()` of flex_ops.py:1976-1981 is
//                   folded into the read); backward
//                   dz = (exp(z - lse) - onehot(label)) * dloss, written 16-bit
//                   (_VocabParallelCrossEntropy, mpu/cross_entropy.py:36-115, TP = 1)
//
// Token ids outside [0, V) are clamped for the memory access and reported in
// `bad_index` (set to 1), which the host checks; the reference's embedding
// would raise for them.
#include <mutex>

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

// ---------------------------------------------------------------------------
// Deterministic embedding backward: sort, then one owner per table row.
//
// For each table (word ids, position ids) a single workgroup sorts the keys
//   key = (clamped id << row_bits) | dout row        (row = s * B + b)
// in LDS with a bitonic network, so equal ids become one contiguous run
// ordered by dout row.  The accumulate kernel then gives every run to the
// workgroup of its first sorted slot, which sums the run's dout rows in fp32
// in that order and adds the sum into the fp32 main grad once: no atomics,
// and the same bits on every run.  The keys fit 32 bits when
// bits(V - 1) + bits(T - 1) <= 32; T <= kEmbSortMax keeps the LDS image at
// 128 KB (static; gfx950 gives a workgroup up to 160 KB).  Longer inputs
// run as consecutive chunks of whole sequence positions (at most
// kEmbSortMax dout rows each), one sort + accumulate per chunk in sequence
// order: each table row then receives one ordered sum per chunk.
constexpr int kEmbSortThreads = 1024;
constexpr int kEmbSortMax = 32768;

__device__ __forceinline__ int64_t clamp_id(int64_t v, int64_t n) { return v < 0 ? 0 : (v >= n ? n - 1 : v); }

// blockIdx.x = 0 sorts the token ids into keys[0, T), 1 the position ids
// into keys[T, 2T); sample b's ids start at ids + b * ld
__global__ void __launch_bounds__(kEmbSortThreads) embedding_sort_kernel(const int64_t* __restrict__ tok,
                                                                        const int64_t* __restrict__ pid,
                                                                        uint32_t* __restrict__ keys, int B, int S,
                                                                        int64_t ld, int64_t V, int64_t P,
                                                                        int row_bits, int n2) {
  __shared__ uint32_t sk[kEmbSortMax];
  const int T = B * S;
  const int64_t* ids = blockIdx.x == 0 ? tok : pid;
  const int64_t lim = blockIdx.x == 0 ? V : P;
  for (int i = threadIdx.x; i < n2; i += kEmbSortThreads) {
    uint32_t k = 0xFFFFFFFFu;
    if (i < T) {
      const int si = i / B, bi = i - si * B;  // dout row i holds (s, b)
      k = ((uint32_t)clamp_id(ids[(int64_t)bi * ld + si], lim) << row_bits) | (uint32_t)i;
    }
    sk[i] = k;
  }
  __syncthreads();
  for (int k = 2; k <= n2; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = threadIdx.x; i < (n2 >> 1); i += kEmbSortThreads) {
        const int lo = 2 * j * (i / j) + (i % j), hi = lo + j;
        const uint32_t a = sk[lo], b = sk[hi];
        if ((a > b) == ((lo & k) == 0)) {
          sk[lo] = b;
          sk[hi] = a;
        }
      }
      __syncthreads();
    }
  }
  uint32_t* out = keys + (int64_t)blockIdx.x * T;
  for (int i = threadIdx.x; i < T; i += kEmbSortThreads) out[i] = sk[i];
}

// grid (T, column chunks of 2048, tables): the workgroup at the first
// sorted slot of a run owns that table row
template <bool FP16>
__global__ void __launch_bounds__(256) embedding_accum_kernel(const uint32_t* __restrict__ keys,
                                                              const uint16_t* __restrict__ dout,
                                                              float* __restrict__ dword, float* __restrict__ dpos,
                                                              int T, int H, int row_bits) {
  const uint32_t* ks = keys + (int64_t)blockIdx.z * T;
  float* dst = blockIdx.z == 0 ? dword : dpos;
  const int j = blockIdx.x;
  const uint32_t id = ks[j] >> row_bits;
  if (dst == nullptr || (j > 0 && (ks[j - 1] >> row_bits) == id)) return;
  const int c = blockIdx.y * 2048 + threadIdx.x * 8;
  if (c >= H) return;
  const uint32_t mask = (1u << row_bits) - 1u;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  int end = j + 1;
  while (end < T && (ks[end] >> row_bits) == id) ++end;
  for (int r = j; r < end; ++r) {
    const uint4 a = *reinterpret_cast<const uint4*>(dout + (int64_t)(ks[r] & mask) * H + c);
    const uint16_t* e = reinterpret_cast<const uint16_t*>(&a);
#pragma unroll
    for (int q = 0; q < 8; ++q) acc[q] += vin<FP16>(e[q]);
  }
  float4* d = reinterpret_cast<float4*>(dst + (int64_t)id * H + c);
  float4 x0 = d[0], x1 = d[1];
  x0.x += acc[0]; x0.y += acc[1]; x0.z += acc[2]; x0.w += acc[3];
  x1.x += acc[4]; x1.y += acc[5]; x1.z += acc[6]; x1.w += acc[7];
  d[0] = x0;
  d[1] = x1;
}

static int bits_for(int64_t n) {  // bits to hold values 0 .. n-1
  int b = 0;
  while (b < 63 && (1LL << b) < n) ++b;
  return b;
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
  // one 8-element vector of the online max / sum-exp
  auto fold = [&](const uint4& a) __attribute__((always_inline)) {
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
  };
  int64_t i = threadIdx.x;
  // four vectors in flight per trip, folded in the order of the walk below
  for (; i + 3 * kXentThreads < nv; i += 4 * kXentThreads) {
    uint4 a[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) a[u] = *reinterpret_cast<const uint4*>(z + (i + u * kXentThreads) * 8);
#pragma unroll
    for (int u = 0; u < 4; ++u) fold(a[u]);
  }
  for (; i < nv; i += kXentThreads) fold(*reinterpret_cast<const uint4*>(z + i * 8));
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
    const float log_s = __logf(Ssum);
    int64_t t = labels[row];
    if (t < 0 || t >= V) {
      *bad = 1;
      t = t < 0 ? 0 : V - 1;
    }
    lse[row] = M + log_s;
    // the reference's order: log(sum exp(z - max)) - (z[t] - max), so the
    // row maximum never enters the sum with the target logit
    loss[row] = log_s - (vin<FP16>(z[t]) - M);
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

// a = b = a + b over n fp32 elements (tied-embedding gradient sum).  One
// trip per thread over kTiedVec 16-byte vectors of each operand, all loads
// in flight before the adds, nontemporal (each byte is touched once here):
// many short workgroups keep HBM busier than a grid-stride loop.
constexpr int kTiedThreads = 256, kTiedVec = 2;
typedef float tf32x4_t __attribute__((ext_vector_type(4)));
__global__ void __launch_bounds__(kTiedThreads) tied_sum_kernel(float* __restrict__ a, float* __restrict__ b,
                                                                int64_t n) {
  const int64_t nv = n / 4;
  tf32x4_t* av = reinterpret_cast<tf32x4_t*>(a);
  tf32x4_t* bv = reinterpret_cast<tf32x4_t*>(b);
  const int64_t i0 = (int64_t)blockIdx.x * (kTiedThreads * kTiedVec) + threadIdx.x;
  tf32x4_t x[kTiedVec], y[kTiedVec];
#pragma unroll
  for (int u = 0; u < kTiedVec; ++u) {
    const int64_t i = i0 + u * kTiedThreads;
    if (i < nv) {
      x[u] = __builtin_nontemporal_load(av + i);
      y[u] = __builtin_nontemporal_load(bv + i);
    }
  }
#pragma unroll
  for (int u = 0; u < kTiedVec; ++u) {
    const int64_t i = i0 + u * kTiedThreads;
    if (i < nv) {
      const tf32x4_t v = x[u] + y[u];
      __builtin_nontemporal_store(v, av + i);
      __builtin_nontemporal_store(v, bv + i);
    }
  }
  if (blockIdx.x == 0)  // the last n % 4 elements
    for (int64_t i = nv * 4 + threadIdx.x; i < n; i += kTiedThreads) {
      const float v = a[i] + b[i];
      a[i] = v;
      b[i] = v;
    }
}

// the same over 16-bit gradients: the sum is formed in fp32 and rounded
// once to the gradient dtype (a two-rank sum all-reduce in that dtype)
__global__ void tied_sum_half_kernel(uint16_t* __restrict__ a, uint16_t* __restrict__ b, int64_t n, int dtype) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const float v = load_elem(a, i, dtype) + load_elem(b, i, dtype);
    store_elem(a, i, dtype, v);
    store_elem(b, i, dtype, v);
  }
}

// The deterministic synthetic batch of a step, one thread per (sample,
// position): tokens = (id * 1103515245 + p * 12345) mod V, loss mask
// ((id + p) mod 4 != 0), position ids p; int64 products wrap in two's
// complement and the residues are taken non-negative, as torch.remainder
// gives them (grad_sync/loss.py:100-119).  The sample ids travel by value.
constexpr int kBatchIds = 64;
struct SampleIds {
  int64_t id[kBatchIds];
};
__global__ void __launch_bounds__(256) synthetic_batch_kernel(SampleIds ids, int64_t n, int64_t seq, int64_t vocab,
                                                              int64_t* __restrict__ tokens,
                                                              float* __restrict__ loss_mask,
                                                              int64_t* __restrict__ position_ids) {
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i >= n * seq) return;
  const int64_t row = i / seq, p = i - row * seq;
  const int64_t id = ids.id[row];
  const int64_t t = (int64_t)((uint64_t)id * 1103515245ull + (uint64_t)p * 12345ull);
  int64_t r = t % vocab;
  if (r < 0) r += vocab;
  int64_t m = (int64_t)((uint64_t)id + (uint64_t)p) % 4;
  if (m < 0) m += 4;
  tokens[i] = r;
  loss_mask[i] = m != 0 ? 1.0f : 0.0f;
  position_ids[i] = p;
}

}  // namespace eth

using namespace eth;

extern "C" int eth_synthetic_batch(const int64_t* sample_ids, int64_t n_samples, int64_t seq, int64_t vocab,
                                   int64_t* tokens, float* loss_mask, int64_t* position_ids, void* stream) {
  ETH_CHECK_ARG(n_samples >= 0 && seq > 0 && vocab > 0, "eth_synthetic_batch: bad sizes");
  ETH_CHECK_ARG(n_samples == 0 || (sample_ids && tokens && loss_mask && position_ids),
                "eth_synthetic_batch: null pointer");
  ETH_CHECK_ARG(seq <= (1LL << 31) / kBatchIds, "eth_synthetic_batch: sequence too long (%lld)", (long long)seq);
  for (int64_t r0 = 0; r0 < n_samples; r0 += kBatchIds) {
    const int64_t n = n_samples - r0 < kBatchIds ? n_samples - r0 : kBatchIds;
    SampleIds ids{};
    for (int64_t r = 0; r < n; ++r) ids.id[r] = sample_ids[r0 + r];
    const int64_t elems = n * seq;
    synthetic_batch_kernel<<<(int)((elems + 255) / 256), 256, 0, (hipStream_t)stream>>>(
        ids, n, seq, vocab, tokens + r0 * seq, loss_mask + r0 * seq, position_ids + r0 * seq);
    ETH_CHECK_LAUNCH("eth_synthetic_batch");
  }
  return ETH_OK;
}

extern "C" int eth_tied_grad_sum(float* root, float* copy, int64_t n, void* stream) {
  ETH_CHECK_ARG(n >= 0 && (n == 0 || (root && copy)), "eth_tied_grad_sum: bad arguments");
  ETH_CHECK_ARG((((uintptr_t)root) & 15) == 0 && (((uintptr_t)copy) & 15) == 0,
                "eth_tied_grad_sum: buffers must be 16-byte aligned");
  if (n == 0) return ETH_OK;
  int64_t blocks = (n / 4 + kTiedThreads * kTiedVec - 1) / (kTiedThreads * kTiedVec);
  if (blocks < 1) blocks = 1;  // the scalar tail alone
  ETH_CHECK_ARG(blocks < (1LL << 31), "eth_tied_grad_sum: too many elements (%lld)", (long long)n);
  tied_sum_kernel<<<(int)blocks, kTiedThreads, 0, (hipStream_t)stream>>>(root, copy, n);
  ETH_CHECK_LAUNCH("eth_tied_grad_sum");
  return ETH_OK;
}

extern "C" int eth_tied_grad_sum_half(void* root, void* copy, int64_t n, int dtype, void* stream) {
  ETH_CHECK_ARG(dtype == ETH_BF16 || dtype == ETH_F16, "eth_tied_grad_sum_half: dtype must be bf16/fp16");
  ETH_CHECK_ARG(n >= 0 && (n == 0 || (root && copy)), "eth_tied_grad_sum_half: bad arguments");
  if (n == 0) return ETH_OK;
  int64_t blocks = (n + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  tied_sum_half_kernel<<<(int)blocks, 256, 0, (hipStream_t)stream>>>((uint16_t*)root, (uint16_t*)copy, n, dtype);
  ETH_CHECK_LAUNCH("eth_tied_grad_sum_half");
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

// sequence positions per chunk: whole positions, at most kEmbSortMax dout rows
static int64_t emb_chunk_seq(int64_t batch, int64_t seq) {
  const int64_t sc = kEmbSortMax / batch;
  return sc < seq ? sc : seq;
}

extern "C" int64_t eth_embedding_bwd_workspace(int64_t batch, int64_t seq) {
  if (batch <= 0 || seq <= 0 || batch > kEmbSortMax) return 0;
  return 2 * batch * emb_chunk_seq(batch, seq) * (int64_t)sizeof(uint32_t);
}

extern "C" int eth_embedding_bwd(const int64_t* tokens, const int64_t* positions, const void* dout,
                                 float* dword, float* dpos, void* workspace, int64_t batch, int64_t seq,
                                 int64_t hidden, int64_t vocab, int64_t max_pos, int dtype, void* stream) {
  ETH_CHECK_ARG(dtype == ETH_BF16 || dtype == ETH_F16, "eth_embedding_bwd: dtype must be bf16/fp16");
  ETH_CHECK_ARG(batch > 0 && seq > 0 && hidden > 0 && hidden % 8 == 0 && vocab > 0 && max_pos > 0,
                "eth_embedding_bwd: bad shape");
  ETH_CHECK_ARG(tokens && positions && dout && workspace && (dword || dpos), "eth_embedding_bwd: null pointer");
  ETH_CHECK_ARG(batch <= kEmbSortMax, "eth_embedding_bwd: at most %d samples per call (got %lld)", kEmbSortMax,
                (long long)batch);
  // consecutive chunks of whole sequence positions, each <= kEmbSortMax rows
  const int64_t sc = emb_chunk_seq(batch, seq);
  const int row_bits = bits_for(batch * sc);
  ETH_CHECK_ARG(row_bits + bits_for(vocab) <= 32 && row_bits + bits_for(max_pos) <= 32,
                "eth_embedding_bwd: ids and rows do not fit a 32-bit sort key");
  ETH_CHECK_ARG(((uintptr_t)dword & 15) == 0 && ((uintptr_t)dpos & 15) == 0 && ((uintptr_t)workspace & 3) == 0,
                "eth_embedding_bwd: gradient tables must be 16-byte aligned");
  hipStream_t s = (hipStream_t)stream;
  uint32_t* keys = (uint32_t*)workspace;
  const uint16_t* d = (const uint16_t*)dout;
  for (int64_t s0 = 0; s0 < seq; s0 += sc) {
    const int64_t len = seq - s0 < sc ? seq - s0 : sc;
    const int64_t T = batch * len;
    int n2 = 1;
    while (n2 < T) n2 <<= 1;
    if (n2 < 2) n2 = 2;
    embedding_sort_kernel<<<2, kEmbSortThreads, 0, s>>>(tokens + s0, positions + s0, keys, (int)batch, (int)len,
                                                          seq, vocab, max_pos, row_bits, n2);
    ETH_CHECK_LAUNCH("eth_embedding_bwd (sort)");
    dim3 grid((unsigned)T, (unsigned)((hidden + 2047) / 2048), 2);
    const uint16_t* dc = d + s0 * batch * hidden;  // dout rows [s0 * B, (s0 + len) * B)
    if (dtype == ETH_BF16)
      embedding_accum_kernel<false><<<grid, 256, 0, s>>>(keys, dc, dword, dpos, (int)T, (int)hidden, row_bits);
    else
      embedding_accum_kernel<true><<<grid, 256, 0, s>>>(keys, dc, dword, dpos, (int)T, (int)hidden, row_bits);
    ETH_CHECK_LAUNCH("eth_embedding_bwd");
  }
  return ETH_OK;
}

// ---------------------------------------------------------------------------
// Allocation-free form of eth_embedding_bwd: the sort keys live in a
// file-scope device array instead of a caller workspace.  Each GPU holds its
// own copy of the array (2 * kEmbSortMax keys = 256 KiB) until the process
// ends; its device address is looked up once per device and kept.  Calls on
// one GPU share the array, so calls that overlap on one GPU race.
static __device__ __align__(256) uint32_t scratch[2 * kEmbSortMax];
constexpr int kMaxDevices = 64;
static void* g_scratch_ptr[kMaxDevices];
static std::mutex g_scratch_mutex;

static int scratch_for_current_device(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    ::eth::set_error("eth_embedding_bwd_noalloc: no usable current device (%s)", hipGetErrorString(e));
    return ETH_ERR_HIP;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr) {
      ::eth::set_error("eth_embedding_bwd_noalloc: hipGetSymbolAddress failed: %s", hipGetErrorString(e));
      return ETH_ERR_HIP;
    }
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return ETH_OK;
}

extern "C" int eth_embedding_bwd_noalloc(const int64_t* tokens, const int64_t* positions, const void* dout,
                                         float* dword, float* dpos, int64_t batch, int64_t seq, int64_t hidden,
                                         int64_t vocab, int64_t max_pos, int dtype, void* stream) {
  ETH_CHECK_ARG(batch > 0 && seq > 0 && batch * seq <= kEmbSortMax,
                "eth_embedding_bwd_noalloc: batch * seq must be in [1, %d] (the static scratch holds %d keys "
                "per table), got %lld",
                kEmbSortMax, kEmbSortMax, (long long)(batch * seq));
  void* ws = nullptr;
  const int rc = scratch_for_current_device(&ws);
  if (rc != ETH_OK) return rc;
  return eth_embedding_bwd(tokens, positions, dout, dword, dpos, ws, batch, seq, hidden, vocab, max_pos, dtype,
                           stream);
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
  ETH_CHECK_ARG(logits && labels && lse && dloss && dlogits, "eth_xent_bwd: null pointer");
  const int64_t nv = vocab / 8;
  int gx = (int)((nv + kXentThreads - 1) / kXentThreads);
  if (gx > 16) gx = 16;
  hipStream_t s = (hipStream_t)stream;
  // rows go on the grid's y dimension (at most 65535 per launch)
  constexpr int64_t kRowsPerLaunch = 65535;
  for (int64_t r0 = 0; r0 < rows; r0 += kRowsPerLaunch) {
    const int64_t n = rows - r0 < kRowsPerLaunch ? rows - r0 : kRowsPerLaunch;
    dim3 grid(gx, (unsigned)n);
    const uint16_t* z = (const uint16_t*)logits + r0 * ld;
    uint16_t* dz = (uint16_t*)dlogits + r0 * ldd;
    if (dtype == ETH_BF16)
      xent_bwd_kernel<false><<<grid, kXentThreads, 0, s>>>(z, ld, labels + r0, lse + r0, dloss + r0, dz, ldd, vocab);
    else
      xent_bwd_kernel<true><<<grid, kXentThreads, 0, s>>>(z, ld, labels + r0, lse + r0, dloss + r0, dz, ldd, vocab);
    ETH_CHECK_LAUNCH("eth_xent_bwd");
  }
  return ETH_OK;
}
