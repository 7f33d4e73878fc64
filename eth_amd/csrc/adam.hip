// Fused AdamW over a tensor table with fp32 master weights: one launch,
// kAdamSplit short workgroups per chunk, every operand streamed once with
// 16-byte accesses (R: p, g, m, v; W: p, m, v, model copy = 30 B/element
// for a 16-bit model copy).  Clip coefficient and the overflow flag are read from
// device memory, so the step never waits on the host.
//
// The per-element arithmetic restates torch.optim.AdamW's single-tensor
// step (decoupled weight decay, lerp first moment), the fallback the
// reference uses for apex FusedAdam
// (eth/runtime/megatron/optimizer/__init__.py:28-34,66-72), preceded by the
// in-place clip of grad_sync/optimizer_semantics.py:589-592 and followed by
// the master->model cast of optimizer/optimizer.py:475-479.
#include "common.h"

// Every multiply and add below is rounded on its own unless written as an
// explicit fma, so the results match the reference arithmetic bit for bit.
#pragma clang fp contract(off)

namespace eth {

// A chunk (<= 16384 elements) is cut into kAdamSplit sub-blocks of <= 1024
// elements, one workgroup of kAdamThreads each: every thread streams two
// 16-byte vectors of each operand in one trip, all eight loads in flight
// before any use.  Many short workgroups keep HBM busier than few long ones
// (5.66 vs 5.17 TB/s on MI355X for the 1.2 G-element update).
constexpr int kAdamThreads = 128;
constexpr int kAdamSplit = 16;
typedef float af32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t au32x2_t __attribute__((ext_vector_type(2)));

struct AdamScalars {
  float beta1, one_minus_beta1, beta2, one_minus_beta2, eps, bc2_sqrt;
  double bc1;
};

// Rounding follows torch's CPU kernels: lerp and addcmul are single fused
// multiply-adds, addcdiv scales the numerator before dividing.
__device__ __forceinline__ float lerp_torch(float a, float b, float w) {
  const float d = b - a;
  return (w < 0.5f) ? __builtin_fmaf(w, d, a) : __builtin_fmaf(-(1.0f - w), d, b);
}

__device__ __forceinline__ void adam_elem(float& p, float g, float& m, float& v, float decay,
                                          float neg_step, const AdamScalars& s) {
  p = p * decay;
  m = lerp_torch(m, g, s.one_minus_beta1);
  v = __builtin_fmaf(s.one_minus_beta2 * g, g, v * s.beta2);
  const float denom = __builtin_sqrtf(v) / s.bc2_sqrt + s.eps;
  p = p + (neg_step * m) / denom;
}

template <int MODEL_DT>
__global__ void __launch_bounds__(kAdamThreads) adam_kernel(const eth_adam_tensor_t* __restrict__ tensors,
                                                            const eth_adam_chunk_t* __restrict__ chunks,
                                                            AdamScalars s,
                                                            const double* __restrict__ stats,
                                                            const float* __restrict__ found_inf) {
  if (found_inf && *found_inf != 0.0f) return;
  const int sub = blockIdx.x % kAdamSplit;
  const eth_adam_chunk_t c = chunks[blockIdx.x / kAdamSplit];
  const eth_adam_tensor_t t = tensors[c.tensor];
  float clip = 1.0f;
  if (stats) {
    const double coef = stats[2];
    if (coef < 1.0) clip = (float)coef;
  }
  const float decay = (float)(1.0 - t.lr * t.weight_decay);
  const float neg_step = (float)(-(t.lr / s.bc1));
  float* __restrict__ p = reinterpret_cast<float*>(t.param) + c.start;
  const float* __restrict__ g = reinterpret_cast<const float*>(t.grad) + c.start;
  float* __restrict__ m = reinterpret_cast<float*>(t.exp_avg) + c.start;
  float* __restrict__ v = reinterpret_cast<float*>(t.exp_avg_sq) + c.start;
  uint16_t* __restrict__ out = t.model ? reinterpret_cast<uint16_t*>(t.model) + c.start : nullptr;
  const int n = c.n;
  const bool vec = (((uintptr_t)p | (uintptr_t)g | (uintptr_t)m | (uintptr_t)v) & 15u) == 0 &&
                   (((uintptr_t)out) & 7u) == 0;
  int i0 = 0;
  if (vec) {
    // this sub-block's float4 range; two float4 per thread per trip, all
    // eight loads issued before any use; nontemporal: every byte is touched
    // once per step
    const int nv = n >> 2;
    const int v0 = (int)((int64_t)nv * sub / kAdamSplit), v1 = (int)((int64_t)nv * (sub + 1) / kAdamSplit);
    auto upd = [&](int i, af32x4_t pp, af32x4_t gg, af32x4_t mm, af32x4_t vv) __attribute__((always_inline)) {
      if (clip != 1.0f) gg *= clip;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float pe = pp[e], me = mm[e], ve = vv[e];
        adam_elem(pe, gg[e], me, ve, decay, neg_step, s);
        pp[e] = pe;
        mm[e] = me;
        vv[e] = ve;
      }
      __builtin_nontemporal_store(pp, reinterpret_cast<af32x4_t*>(p) + i);
      __builtin_nontemporal_store(mm, reinterpret_cast<af32x4_t*>(m) + i);
      __builtin_nontemporal_store(vv, reinterpret_cast<af32x4_t*>(v) + i);
      if (MODEL_DT != ETH_F32 && out) {
        au32x2_t o;
        if (MODEL_DT == ETH_BF16) {
          o.x = f2bf_pair(pp.x, pp.y);
          o.y = f2bf_pair(pp.z, pp.w);
        } else {
          o.x = (uint32_t)f2h_bits(pp.x) | ((uint32_t)f2h_bits(pp.y) << 16);
          o.y = (uint32_t)f2h_bits(pp.z) | ((uint32_t)f2h_bits(pp.w) << 16);
        }
        __builtin_nontemporal_store(o, reinterpret_cast<au32x2_t*>(out) + i);
      }
    };
    const af32x4_t* p4 = reinterpret_cast<const af32x4_t*>(p);
    const af32x4_t* g4 = reinterpret_cast<const af32x4_t*>(g);
    const af32x4_t* m4 = reinterpret_cast<const af32x4_t*>(m);
    const af32x4_t* v4 = reinterpret_cast<const af32x4_t*>(v);
    int i = v0 + threadIdx.x;
    for (; i + kAdamThreads < v1; i += 2 * kAdamThreads) {
      const int j = i + kAdamThreads;
      const af32x4_t p0 = __builtin_nontemporal_load(p4 + i), g0 = __builtin_nontemporal_load(g4 + i);
      const af32x4_t m0 = __builtin_nontemporal_load(m4 + i), v0 = __builtin_nontemporal_load(v4 + i);
      const af32x4_t p1 = __builtin_nontemporal_load(p4 + j), g1 = __builtin_nontemporal_load(g4 + j);
      const af32x4_t m1 = __builtin_nontemporal_load(m4 + j), v1 = __builtin_nontemporal_load(v4 + j);
      upd(i, p0, g0, m0, v0);
      upd(j, p1, g1, m1, v1);
    }
    if (i < v1) upd(i, p4[i], g4[i], m4[i], v4[i]);
    i0 = nv << 2;
  }
  // the scalar tail of an aligned chunk once (last sub-block), an unaligned
  // chunk whole once (first sub-block)
  if (vec ? sub != kAdamSplit - 1 : sub != 0) return;
  for (int i = i0 + threadIdx.x; i < n; i += kAdamThreads) {
    float pp = p[i], mm = m[i], vv = v[i];
    float gg = g[i];
    if (clip != 1.0f) gg *= clip;
    adam_elem(pp, gg, mm, vv, decay, neg_step, s);
    p[i] = pp;
    m[i] = mm;
    v[i] = vv;
    if (MODEL_DT != ETH_F32 && out)
      out[i] = MODEL_DT == ETH_BF16 ? f2bf(pp) : f2h_bits(pp);
  }
}

}  // namespace eth

using namespace eth;

extern "C" int eth_adam_step(const eth_adam_tensor_t* tensors, const eth_adam_chunk_t* chunks,
                             int64_t n_chunks, double beta1, double beta2, double eps,
                             int64_t step, int model_dtype, const double* stats,
                             const float* found_inf, void* stream) {
  ETH_CHECK_ARG(step >= 1, "eth_adam_step: step must be positive, got %lld", (long long)step);
  ETH_CHECK_ARG(model_dtype == ETH_F32 || model_dtype == ETH_F16 || model_dtype == ETH_BF16,
                "eth_adam_step: unsupported model dtype %d", model_dtype);
  ETH_CHECK_ARG(n_chunks >= 0 && n_chunks * kAdamSplit < (1LL << 31), "eth_adam_step: bad chunk count");
  if (n_chunks == 0) return ETH_OK;
  ETH_CHECK_ARG(tensors && chunks, "eth_adam_step: null table");
  AdamScalars s;
  s.beta1 = (float)beta1;
  s.one_minus_beta1 = (float)(1.0 - beta1);
  s.beta2 = (float)beta2;
  s.one_minus_beta2 = (float)(1.0 - beta2);
  s.eps = (float)eps;
  s.bc1 = 1.0 - pow(beta1, (double)step);
  s.bc2_sqrt = (float)sqrt(1.0 - pow(beta2, (double)step));
  hipStream_t st = (hipStream_t)stream;
  if (model_dtype == ETH_BF16)
    adam_kernel<ETH_BF16><<<(int)(n_chunks * kAdamSplit), kAdamThreads, 0, st>>>(tensors, chunks, s, stats, found_inf);
  else if (model_dtype == ETH_F16)
    adam_kernel<ETH_F16><<<(int)(n_chunks * kAdamSplit), kAdamThreads, 0, st>>>(tensors, chunks, s, stats, found_inf);
  else
    adam_kernel<ETH_F32><<<(int)(n_chunks * kAdamSplit), kAdamThreads, 0, st>>>(tensors, chunks, s, stats, found_inf);
  ETH_CHECK_LAUNCH("eth_adam_step");
  return ETH_OK;
}
