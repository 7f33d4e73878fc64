// Causal flash attention for the GPT block, forward and backward, on CDNA4
// matrix cores (v_mfma_f32_32x32x16_{bf16,f16}).  Any head_dim that is a
// multiple of 8 up to 128 runs on the 64-, 96- or 128-wide kernels with the
// extra head-dim columns loaded as zeros and never stored; any sequence
// length runs on whole 128-row blocks whose rows past the end load as zeros
// (the causal mask already hides keys past every real query) and are never
// stored.
//
// Semantics: O = softmax(Q K^T / sqrt(hn) + causal -inf) V per (batch, head),
// i.e. F.scaled_dot_product_attention(q, k, v, is_causal=True) as called by
// eth/runtime/megatron/model/flex_ops.py:66-96 (ParallelFlashAtten,
// :1401-1426).  Q, K, V, O and their gradients are addressed in place through
// (row, batch, head) strides, so the [s, b, np, 3*hn] output of the QKV GEMM
// is read without the split/permute copies and dQ/dK/dV are written straight
// into the [s, b, np, 3*hn] gradient the QKV backward consumes.
//
// Layout trick.  Scores are computed transposed, S^T = K Q^T, so that each
// lane owns one query (MFMA column) and 32 of the 64 keys of a block sit in
// its registers: row max / row sum need one cross-lane exchange (lane ^ 32),
// and the per-query softmax statistics are per-lane scalars.  K rows are
// stored in LDS with bits 2 and 3 of the row index swapped, which makes the
// MFMA result layout of S^T equal to the operand layout of P^T in
// O^T = V^T P^T, so P never leaves registers.  The dK/dV kernel uses the
// mirror image (S = Q K^T, lane = key, query rows swizzled) and computes S
// and P once for both gradients, in pairs of waves that hand P over through
// LDS; dQ has its own kernel (recomputing P), so no atomics are needed and
// results are deterministic.  The dQ kernel runs first and also writes
// delta = rowsum(dO * O), which the dK/dV kernel reads.
//
// Tiles arrive through buffer loads (fixed per-thread offsets, a scalar row
// advance).  Operands that an MFMA needs transposed (V for O^T = V^T P^T, K
// for dQ^T = K^T dS^T, Q and dO for dK and dV) are kept in LDS in natural
// row order, padded to D + 32 so four k-rows fall in distinct banks, and
// read with ds_read_b64_tr_b16.  Softmax runs in fp32 base-2 (exp2) with the scale folded.
#include <type_traits>

#include "common.h"

namespace eth {

typedef __bf16 a_bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 a_f16x8 __attribute__((ext_vector_type(8)));
typedef float a_f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t a_u32x4 __attribute__((ext_vector_type(4)));

template <bool FP16>
__device__ __forceinline__ a_f32x16 mma(const uint4& a, const uint4& b, const a_f32x16& c) {
  if constexpr (FP16)
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(a_f16x8, a), __builtin_bit_cast(a_f16x8, b),
                                                  c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(a_bf16x8, a),
                                                   __builtin_bit_cast(a_bf16x8, b), c, 0, 0, 0);
}

template <bool FP16>
__device__ __forceinline__ float to_f(uint16_t v) {
  return FP16 ? h2f_bits(v) : bf2f(v);
}
template <bool FP16>
__device__ __forceinline__ uint16_t from_f(float v) {
  return FP16 ? f2h_bits(v) : f2bf(v);
}
template <bool FP16>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  if constexpr (FP16)
    return (uint32_t)f2h_bits(a) | ((uint32_t)f2h_bits(b) << 16);
  else
    return f2bf_pair(a, b);
}
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
// s_waitcnt vmcnt(0) (expcnt, lgkmcnt unconstrained) as the builtin, so the
// compiler's own wait-count tracking knows that no vector load is pending
__device__ __forceinline__ void vm_wait_all() { __builtin_amdgcn_s_waitcnt(0x0F70); }
// 8 fp32 -> one 16-byte MFMA operand
template <bool FP16>
__device__ __forceinline__ uint4 pack8(const float* v) {
  return make_uint4(pack2<FP16>(v[0], v[1]), pack2<FP16>(v[2], v[3]), pack2<FP16>(v[4], v[5]),
                    pack2<FP16>(v[6], v[7]));
}

__device__ __forceinline__ int swz(int r) {  // swap bits 2 and 3
  return (r & ~12) | ((r & 4) << 1) | ((r & 8) >> 1);
}
// index (within a 32-row MFMA tile) held by accumulator register r of a lane
// in half h, when the operand rows were swizzled
__device__ __forceinline__ int swz_row(int r, int h) { return (r < 8 ? 0 : 16) + h * 8 + (r & 7); }
// natural accumulator row of register r for half h
__device__ __forceinline__ int acc_row(int r, int h) { return (r >> 2) * 8 + h * 4 + (r & 3); }

struct AttnTensor {
  const uint16_t* p;
  int64_t ss, sb, sh;  // strides of sequence, batch, head (elements); dim contiguous
  uint32_t bytes;      // extent from p (buffer-load range)
};
struct AttnOut {
  uint16_t* p;
  int64_t ss, sb, sh;
};

struct AttnArgs {
  AttnTensor q, k, v, o, dout;
  AttnOut out, dq, dk, dv;
  float* lse;    // [B*H, S] log2-domain: m2 + log2(l)
  float* delta;  // [B*H, S] rowsum(dO * O)
  int B, H, S;
  int hd;  // head dim (<= the kernel's D; columns hd..D-1 are zero padding)
  float scale_log2;  // log2(e) / sqrt(hn)
  float scale;       // 1 / sqrt(hn)
};

constexpr int kAttnThreads = 256;
constexpr float kRescaleLog2 = 8.0f;  // forward: tolerated growth of the running max (log2 units)
constexpr int kBQ = 128;   // forward / dQ: queries per workgroup (4 waves x 32)
constexpr int kBKV = 64;   // forward / dQ: keys per step
constexpr int kBKV2 = 128; // dK/dV: keys per workgroup (4 waves x 32)
constexpr int kBQ2 = 64;   // dK/dV: queries per step
constexpr int32_t kAttnOob = (int32_t)0x80000000u;  // buffer offset past any tensor: loads read zeros
// row length (elements) of an LDS tile read with ds_read_b64_tr_b16: four
// consecutive rows then start 64 bytes apart in the bank space
constexpr int tr_row(int d) { return d % 64 == 0 ? d + 32 : d + 64; }
// 16 bytes of a row at column `col` of a strided tensor; with PAD, zeros
// past the sequence or the head dim (without, every row and column is real)
template <bool PAD>
__device__ __forceinline__ uint4 load_row16(const uint16_t* row, bool in_seq, int col, int hd) {
  if constexpr (PAD)
    return in_seq && col < hd ? *reinterpret_cast<const uint4*>(row + col) : make_uint4(0u, 0u, 0u, 0u);
  else
    return *reinterpret_cast<const uint4*>(row + col);
}

__device__ __forceinline__ const uint16_t* row_ptr(const AttnTensor& t, int s, int b, int h) {
  return t.p + (int64_t)s * t.ss + (int64_t)b * t.sb + (int64_t)h * t.sh;
}
__device__ __forceinline__ uint16_t* row_ptr(const AttnOut& t, int s, int b, int h) {
  return t.p + (int64_t)s * t.ss + (int64_t)b * t.sb + (int64_t)h * t.sh;
}

// ROWS x D tile of a strided tensor through buffer loads: each thread's
// offsets within the (batch, head) slice are fixed, the row advance is a
// scalar offset, so a load costs no address arithmetic.  Stored into LDS
// rows of LROW elements, row index optionally swizzled (SWZ).
typedef __amdgpu_buffer_rsrc_t a_rsrc_t;
template <int ROWS, int D, int LROW, bool SWZ, bool PAD>
struct BufTile {
  static constexpr int CPR = D / 8;
  static constexpr int CPT = ROWS * CPR / kAttnThreads;
  static_assert(ROWS * CPR % kAttnThreads == 0 && CPT >= 1, "tile split");
  a_u32x4 v[CPT];
  int32_t voff[CPT];
  a_rsrc_t rs;
  int32_t row_bytes;
  int rows_left;  // tensor rows (sequence length); rows past it load zeros
  int tid;        // this thread's index among the kAttnThreads that move the tile
  // columns at or past hd load zeros (an out-of-range offset)
  __device__ __forceinline__ void init(const AttnTensor& t, int b, int h, int seq, int hd) {
    init(t, b, h, seq, hd, threadIdx.x);
  }
  __device__ __forceinline__ void init(const AttnTensor& t, int b, int h, int seq, int hd, int thread) {
    tid = thread;
    rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(t.p), (short)0, (int)t.bytes, 0x00020000);
    row_bytes = (int32_t)(t.ss * 2);
    rows_left = seq;
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = tid + i * kAttnThreads;
      voff[i] = !PAD || (c % CPR) * 8 < hd
                    ? (int32_t)(((int64_t)b * t.sb + (int64_t)h * t.sh + (int64_t)(c / CPR) * t.ss + (c % CPR) * 8) * 2)
                    : kAttnOob;
    }
  }
  __device__ __forceinline__ void load(int r0) {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = tid + i * kAttnThreads;
      const int32_t off = !PAD || r0 + c / CPR < rows_left ? voff[i] : kAttnOob;
      v[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, off, r0 * row_bytes, 0);
    }
  }
  __device__ __forceinline__ void store(uint16_t* lds) const {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = tid + i * kAttnThreads;
      const int r = SWZ ? swz(c / CPR) : c / CPR;
      *reinterpret_cast<a_u32x4*>(lds + r * LROW + (c % CPR) * 8) = v[i];
    }
  }
  // the same rows in natural order into [ROWS][L2] (for transposing reads)
  template <int L2>
  __device__ __forceinline__ void store_natural(uint16_t* lds) const {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = tid + i * kAttnThreads;
      *reinterpret_cast<a_u32x4*>(lds + (c / CPR) * L2 + (c % CPR) * 8) = v[i];
    }
  }
};

typedef short a_s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) a_s16x4 a_lds_s16x4;
typedef uint32_t a_u32x2 __attribute__((ext_vector_type(2)));
// MFMA operand of 8 consecutive k from a [k][m] LDS tile (row length LROW)
// by two ds_read_b64_tr_b16: lane l passes the address of k-row
// k0 + (l%16)/4 (k0 = 8*(l/32)), element m0 + 16*((l/16)%2) + 4*(l%4)
// (tr_lane gives that offset) and receives m = m0 + l%32, k = k0..k0+7.
__device__ __forceinline__ int tr_lane(int lane, int lrow) {
  return ((lane >> 5) * 8 + ((lane & 15) >> 2)) * lrow + ((lane >> 4) & 1) * 16 + (lane & 3) * 4;
}
__device__ __forceinline__ uint4 tr_frag(const uint16_t* p, int lrow) {
  const a_u32x2 lo = __builtin_bit_cast(a_u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((a_lds_s16x4*)p));
  const a_u32x2 hi = __builtin_bit_cast(a_u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((a_lds_s16x4*)(p + 4 * lrow)));
  return make_uint4(lo.x, lo.y, hi.x, hi.y);
}

// ------------------------------------------------------------------ forward --
// 4 waves x 32 queries; K/V blocks of 64 keys double-buffered in LDS (the
// next block's global loads are in flight while this one is computed); two
// workgroups per CU, so one wave's softmax overlaps the other's MFMAs.
template <int D, bool FP16, bool PAD>
__global__ void __launch_bounds__(kAttnThreads, 2) attn_fwd_kernel(AttnArgs a) {
  constexpr int KS = D / 16;  // k-steps over the head dim
  constexpr int DT = D / 32;  // 32-row tiles over the head dim
  // K rows swizzled (see the file comment); V rows as they are, padded to
  // D + 32 so the transposing reads of O^T = V^T P^T hit distinct banks
  constexpr int VL = tr_row(D);
  __shared__ __attribute__((aligned(16))) uint16_t Ks[2][kBKV * (D + 8)];
  __shared__ __attribute__((aligned(16))) uint16_t Vs[2][kBKV * VL];

  const int BH = a.B * a.H, nqb = (a.S + kBQ - 1) / kBQ;
  const int bh = blockIdx.x % BH, qb = nqb - 1 - blockIdx.x / BH;
  const int b = bh / a.H, h = bh % a.H;
  const int lane = threadIdx.x & 63, hl = lane >> 5;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int q0 = qb * kBQ + w * 32;
  const int q = q0 + (lane & 31);
  const float sl2 = a.scale_log2;

  uint4 qf[KS];
  {
    const uint16_t* qp = row_ptr(a.q, q, b, h);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qf[ks] = load_row16<PAD>(qp, q < a.S, ks * 16 + hl * 8, a.hd);
  }
  a_f32x16 o[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[t][r] = 0.f;
  float m = -1e30f, l = 0.f;  // running max (log2 units) and sum for query q

  const int nkv = (qb * kBQ + kBQ) / kBKV;  // blocks up to the diagonal
  BufTile<kBKV, D, D + 8, true, PAD> kt;
  BufTile<kBKV, D, VL, false, PAD> vt;
  kt.init(a.k, b, h, a.S, a.hd);
  vt.init(a.v, b, h, a.S, a.hd);
  kt.load(0);
  vt.load(0);
  kt.store(Ks[0]);
  vt.store(Vs[0]);
  const int vtr = tr_lane(lane, VL);
  __syncthreads();
  // the Q fragment loads may still be in flight here; waiting for them now
  // (through the builtin, which the compiler's wait-count pass sees) keeps
  // that pass from making every iteration's first MFMAs wait for the next
  // block's prefetch loads
  vm_wait_all();

  for (int j = 0; j < nkv; ++j) {
    const int st = j & 1;
    const bool more = j + 1 < nkv;
    if (more) {
      kt.load((j + 1) * kBKV);
      vt.load((j + 1) * kBKV);
    }
    const int kv0 = j * kBKV;
    if (kv0 <= q0 + 31) {  // wave has at least one unmasked key in the block
      // S^T = K Q^T (raw scores; lane = query, registers = 32 of the keys)
      a_f32x16 s[2];
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) s[t][r] = 0.f;
      // all K fragments of the first 32-key tile are read before its MFMAs,
      // each register refilled with the second tile's fragment right after
      // its MFMA issues (order pinned: left alone, the compiler reads each
      // fragment one or two MFMAs before its use and waits on the LDS latency)
      {
        const uint16_t* kp0 = Ks[st] + (lane & 31) * (D + 8) + hl * 8;
        const uint16_t* kp1 = kp0 + 32 * (D + 8);
        uint4 kr[KS];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) kr[ks] = *reinterpret_cast<const uint4*>(kp0 + ks * 16);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          s[0] = mma<FP16>(kr[ks], qf[ks], s[0]);
          __builtin_amdgcn_sched_barrier(0);
          kr[ks] = *reinterpret_cast<const uint4*>(kp1 + ks * 16);
          __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) s[1] = mma<FP16>(kr[ks], qf[ks], s[1]);
      }
      if (kv0 + kBKV - 1 > q0) {  // diagonal block: mask keys after the query
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            if (kv0 + t * 32 + swz_row(r, hl) > q) s[t][r] = -1e30f;
      }
      float mx = s[0][0];
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[t][r]);
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float mnew = fmaxf(m, mx * sl2);
      // m is the exponent offset, kept within kRescaleLog2 below the running
      // max: O and l are rescaled only when some row's max grew past that,
      // so p = exp2(s - m) stays <= 2^kRescaleLog2 (exact in fp32, the same
      // relative precision in 16 bits) and most blocks skip the rescale;
      // O / l and lse = m + log2(l) do not depend on the offset
      if (__any(mnew > m + kRescaleLog2)) {
        const float alpha = fast_exp2(m - mnew);
        l *= alpha;
#pragma unroll
        for (int t = 0; t < DT; ++t)
#pragma unroll
          for (int r = 0; r < 16; ++r) o[t][r] *= alpha;
        m = mnew;
      }
      float rs = 0.f;
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float p = fast_exp2(__builtin_fmaf(s[t][r], sl2, -m));
          s[t][r] = p;
          rs += p;
        }
      l += rs;
      // O^T += V^T P^T over the 64 keys (4 k-steps of 16)
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const int t = kk >> 1, e0 = (kk & 1) * 8;
        const uint4 pb = make_uint4(pack2<FP16>(s[t][e0 + 0], s[t][e0 + 1]), pack2<FP16>(s[t][e0 + 2], s[t][e0 + 3]),
                                    pack2<FP16>(s[t][e0 + 4], s[t][e0 + 5]), pack2<FP16>(s[t][e0 + 6], s[t][e0 + 7]));
        const uint16_t* vp = Vs[st] + vtr + kk * 16 * VL;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) o[dt] = mma<FP16>(tr_frag(vp + dt * 32, VL), pb, o[dt]);
      }
    }
    if (more) {
      kt.store(Ks[st ^ 1]);
      vt.store(Vs[st ^ 1]);
    }
    __syncthreads();
  }
  l += __shfl_xor(l, 32, 64);
  if (PAD && q >= a.S) return;  // a padding row of the last query block
  const float inv = 1.0f / l;
  uint16_t* op = row_ptr(a.out, q, b, h);
#pragma unroll
  for (int t = 0; t < DT; ++t)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      if (PAD && t * 32 + g * 8 >= a.hd) continue;  // hd % 8 == 0: whole 8-column groups
      uint2 v;
      v.x = pack2<FP16>(o[t][g * 4 + 0] * inv, o[t][g * 4 + 1] * inv);
      v.y = pack2<FP16>(o[t][g * 4 + 2] * inv, o[t][g * 4 + 3] * inv);
      *reinterpret_cast<uint2*>(op + t * 32 + g * 8 + hl * 4) = v;
    }
  if (hl == 0) a.lse[(int64_t)bh * a.S + q] = m + log2f(l);
}

// -------------------------------------------------- forward, head_dim 128 --
// attn_fwd_kernel for D = 128 with each 64-key block of K and V in an
// XOR-swizzled LDS image (chunk c of row r at c ^ xsw(r), see
// attn_bwd_dkdv_x128_kernel), double buffered and filled by direct
// global->LDS loads a whole block ahead: no register staging, no copy
// phase, one barrier per block.  K rows are read as A operands (S^T = K Q^T)
// and V through transposing reads (O^T = V^T P^T); same arithmetic in the
// same order as attn_fwd_kernel, so the results are bit-identical.
__device__ __forceinline__ int xsw(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }
template <bool FP16, bool PAD>
__global__ void __launch_bounds__(kAttnThreads, 2) attn_fwd_x128_kernel(AttnArgs a) {
  constexpr int D = 128, KS = D / 16, DT = D / 32;
  constexpr int IMG = kBKV * D;
  __shared__ __attribute__((aligned(16))) uint16_t Kx[2 * IMG];
  __shared__ __attribute__((aligned(16))) uint16_t Vx[2 * IMG];

  const int BH = a.B * a.H, nqb = (a.S + kBQ - 1) / kBQ;
  const int bh = blockIdx.x % BH, qb = nqb - 1 - blockIdx.x / BH;
  const int b = bh / a.H, h = bh % a.H;
  const int lane = threadIdx.x & 63, hl = lane >> 5;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int q0 = qb * kBQ + w * 32;
  const int q = q0 + (lane & 31);
  const float sl2 = a.scale_log2;

  // direct loads: each wave fills 4 pieces of the K image and 4 of the V image
  const a_rsrc_t rsk = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.k.p), (short)0, (int)a.k.bytes,
                                                         0x00020000);
  const a_rsrc_t rsv = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.v.p), (short)0, (int)a.v.bytes,
                                                         0x00020000);
  int32_t koff[4], voff[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int u = (w * 4 + j) * 64 + lane;
    const int r = u >> 4, c = (u & 15) ^ xsw(r);
    koff[j] = c * 8 < a.hd ? (int32_t)(((int64_t)b * a.k.sb + (int64_t)h * a.k.sh + (int64_t)r * a.k.ss + c * 8) * 2)
                           : kAttnOob;
    voff[j] = c * 8 < a.hd ? (int32_t)(((int64_t)b * a.v.sb + (int64_t)h * a.v.sh + (int64_t)r * a.v.ss + c * 8) * 2)
                           : kAttnOob;
  }
  const int32_t krow = (int32_t)(a.k.ss * 2), vrow = (int32_t)(a.v.ss * 2);
  auto issue = [&](int slot, int r0) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bool in = !PAD || r0 + (w * 4 + j) * 4 + (lane >> 4) < a.S;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rsk, (__attribute__((address_space(3))) void*)(Kx + slot * IMG + (w * 4 + j) * 512), 16,
          in ? koff[j] : kAttnOob, r0 * krow, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rsv, (__attribute__((address_space(3))) void*)(Vx + slot * IMG + (w * 4 + j) * 512), 16,
          in ? voff[j] : kAttnOob, r0 * vrow, 0, 0);
    }
  };
  const int nkv = (qb * kBQ + kBQ) / kBKV;  // blocks up to the diagonal
  issue(0, 0);

  uint4 qf[KS];
  {
    const uint16_t* qp = row_ptr(a.q, q, b, h);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qf[ks] = load_row16<PAD>(qp, q < a.S, ks * 16 + hl * 8, a.hd);
  }
  a_f32x16 o[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[t][r] = 0.f;
  float m = -1e30f, l = 0.f;  // running max (log2 units) and sum for query q

  // K rows as A operands: row t*32 + swz(lane%32) (the swizzled key order
  // that makes S^T's result layout the B operand layout of P^T), chunk
  // 2*ks + hl
  int aoff[KS];
  {
    const int arow = swz(lane & 31), xa = xsw(arow);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) aoff[ks] = arow * D + (((2 * ks + hl) ^ xa) << 3);
  }
  // V^T through transposing reads: k-rows (keys) kk*16 + 8*(l/32) +
  // (l%16)/4 (+4 for the second read), columns dt*32 + 16*((l/16)%2) + 4*(l%4)
  int toff[DT][2];
  {
    const int R = (lane & 15) >> 2, L5 = lane >> 5, L4 = (lane >> 4) & 1, L1 = (lane >> 1) & 1;
#pragma unroll
    for (int d2 = 0; d2 < DT; ++d2)
#pragma unroll
      for (int hi = 0; hi < 2; ++hi) {
        const int row = 8 * L5 + R + 4 * hi;
        const int pc = 4 * (d2 ^ R) + ((2 * L4 + L1) ^ (2 * L5 + hi));
        toff[d2][hi] = row * D + pc * 8 + (lane & 1) * 4;
      }
  }
  vm_wait_all();
  __syncthreads();

  auto block = [&](int j, auto cur_c) __attribute__((always_inline)) {
    constexpr int cur = decltype(cur_c)::value;
    const int kv0 = j * kBKV;
    if (j + 1 < nkv) issue(cur ^ 1, kv0 + kBKV);  // the next block, a block ahead
    if (kv0 <= q0 + 31) {  // wave has at least one unmasked key in the block
      const uint16_t* ki = Kx + cur * IMG;
      const uint16_t* vi = Vx + cur * IMG;
      a_f32x16 sc[2];
      // all K fragments of the first 32-key tile are read before its MFMAs,
      // each register refilled with the second tile's fragment right after
      // its MFMA issues (order pinned)
      {
        uint4 kr[KS];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) kr[ks] = *reinterpret_cast<const uint4*>(ki + aoff[ks]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          sc[0] = mma<FP16>(kr[ks], qf[ks], ks == 0 ? a_f32x16{} : sc[0]);
          __builtin_amdgcn_sched_barrier(0);
          kr[ks] = *reinterpret_cast<const uint4*>(ki + 32 * D + aoff[ks]);
          __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) sc[1] = mma<FP16>(kr[ks], qf[ks], ks == 0 ? a_f32x16{} : sc[1]);
      }
      if (kv0 + kBKV - 1 > q0) {  // diagonal block: mask keys after the query
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            if (kv0 + t * 32 + swz_row(r, hl) > q) sc[t][r] = -1e30f;
      }
      float mx = sc[0][0];
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sc[t][r]);
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float mnew = fmaxf(m, mx * sl2);
      if (__any(mnew > m + kRescaleLog2)) {
        const float alpha = fast_exp2(m - mnew);
        l *= alpha;
#pragma unroll
        for (int t = 0; t < DT; ++t)
#pragma unroll
          for (int r = 0; r < 16; ++r) o[t][r] *= alpha;
        m = mnew;
      }
      float rs = 0.f;
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float p = fast_exp2(__builtin_fmaf(sc[t][r], sl2, -m));
          sc[t][r] = p;
          rs += p;
        }
      l += rs;
      // O^T += V^T P^T over the 64 keys (4 k-steps of 16)
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const int t = kk >> 1, e0 = (kk & 1) * 8;
        const uint4 pb = make_uint4(pack2<FP16>(sc[t][e0 + 0], sc[t][e0 + 1]), pack2<FP16>(sc[t][e0 + 2], sc[t][e0 + 3]),
                                    pack2<FP16>(sc[t][e0 + 4], sc[t][e0 + 5]), pack2<FP16>(sc[t][e0 + 6], sc[t][e0 + 7]));
        const uint16_t* vp = vi + kk * 16 * D;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          const a_u32x2 lo =
              __builtin_bit_cast(a_u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((a_lds_s16x4*)(vp + toff[dt][0])));
          const a_u32x2 hi =
              __builtin_bit_cast(a_u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((a_lds_s16x4*)(vp + toff[dt][1])));
          o[dt] = mma<FP16>(make_uint4(lo.x, lo.y, hi.x, hi.y), pb, o[dt]);
        }
      }
    }
    vm_wait_all();  // the next block's rows have landed
    __syncthreads();  // this block's images free, the next block's visible
  };
  int j = 0;
  for (; j + 1 < nkv; j += 2) {
    block(j, std::integral_constant<int, 0>{});
    block(j + 1, std::integral_constant<int, 1>{});
  }
  if (j < nkv) block(j, std::integral_constant<int, 0>{});
  l += __shfl_xor(l, 32, 64);
  if (PAD && q >= a.S) return;  // a padding row of the last query block
  const float inv = 1.0f / l;
  uint16_t* op = row_ptr(a.out, q, b, h);
#pragma unroll
  for (int t = 0; t < DT; ++t)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      if (PAD && t * 32 + g * 8 >= a.hd) continue;
      uint2 v;
      v.x = pack2<FP16>(o[t][g * 4 + 0] * inv, o[t][g * 4 + 1] * inv);
      v.y = pack2<FP16>(o[t][g * 4 + 2] * inv, o[t][g * 4 + 3] * inv);
      *reinterpret_cast<uint2*>(op + t * 32 + g * 8 + hl * 4) = v;
    }
  if (hl == 0) a.lse[(int64_t)bh * a.S + q] = m + log2f(l);
}

// ------------------------------------------------ backward: dK, dV paired --
// Eight waves: wave w < 4 (the dV wave) and wave w + 4 (the dK wave) own the
// same 32 keys and share a SIMD.  Per step of 64 queries the dV wave computes
// S = Q K^T and P and hands P (fp32) to its partner through LDS; the dK wave
// meanwhile computes dP = dO V^T and subtracts delta.  After the hand-over
// the dV wave adds P^T dO into dV while the dK wave forms dS = P (dP - delta)
// and adds dS^T Q into dK.  S and P are computed once per step (the split dV
// and dK kernels each recompute them), and on every SIMD one wave's
// exponentials or dS arithmetic overlap the other wave's MFMAs.  S = Q K^T
// is computed with lane = key (the mirror image of the forward's layout,
// query rows swizzled), so P and dS are already the A operands of
// dV += P^T dO and dK += dS^T Q.
//
// The Q and dO rows of a step are kept twice in LDS: a row-swizzled copy
// (rows of D + 8) read as A operands in the first half of the step, and a
// natural copy (rows padded for the transposing reads) read as B operands
// in the second half.  Both are filled by direct global->LDS loads, each in
// the half-step before it is read: the next step's row-swizzled copy during
// this step's second half, the next step's natural copy during its first
// half.  A step therefore has two barriers (P handed over; step done) and
// no copy phase of its own.
template <int ROWS, int D, int UPR, bool SWZ>
struct DmaCopy {
  // one LDS copy of a ROWS x D tile, rows of UPR 16-byte units (the first
  // D / 8 hold data, the rest padding), moved by the four waves of a role:
  // lane l of piece j fills unit (piece * 64 + l) of the image
  static constexpr int PIECES = ROWS * UPR / 64;
  static constexpr int PW = (PIECES + 3) / 4;  // pieces per wave (the last wave may have fewer)
  static_assert(ROWS * UPR % 64 == 0, "whole pieces");
  int32_t off[PW];
  int32_t row_in_tile[PW];  // image row of the unit (tile row via the swizzle), -1 for padding units
  int w;                    // wave within the role (wave-uniform)
  __device__ __forceinline__ void init(const AttnTensor& t, int b, int h, int hd, int wave, int lane) {
    w = wave;
#pragma unroll
    for (int j = 0; j < PW; ++j) {
      const int u = (w * PW + j) * 64 + lane;
      const int p = u / UPR, c = u % UPR;
      const int q = SWZ ? swz(p) : p;  // image row p holds tile row q
      const bool data = c < D / 8 && c * 8 < hd && p < ROWS;
      row_in_tile[j] = data ? q : -1;
      off[j] = data ? (int32_t)(((int64_t)b * t.sb + (int64_t)h * t.sh + (int64_t)q * t.ss + c * 8) * 2) : kAttnOob;
    }
  }
  // rows [r0, r0 + ROWS) of the tensor into the image at S; with PAD, rows
  // at or past `seq` read zeros
  template <bool PAD>
  __device__ __forceinline__ void issue(uint16_t* S, a_rsrc_t rs, int32_t row_bytes, int r0, int seq) const {
#pragma unroll
    for (int j = 0; j < PW; ++j) {
      if (w * PW + j >= PIECES) break;  // wave-uniform
      const int32_t o = !PAD || (row_in_tile[j] >= 0 && r0 + row_in_tile[j] < seq) ? off[j] : kAttnOob;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)(S + (w * PW + j) * 512),
                                               16, o, r0 * row_bytes, 0, 0);
    }
  }
};

template <int D, bool FP16, bool PAD>
__global__ void __launch_bounds__(2 * kAttnThreads, 1) attn_bwd_dkdv_pair_kernel(AttnArgs a) {
  constexpr int KS = D / 16, DT = D / 32;
  constexpr int QN = tr_row(D);
  constexpr int AL = D + 8;  // row length of the row-swizzled copy
  typedef DmaCopy<kBQ2, D, AL / 8, true> RowCopy;
  typedef DmaCopy<kBQ2, D, QN / 8, false> TrCopy;
  __shared__ __attribute__((aligned(16))) uint16_t Qs[RowCopy::PIECES * 512];
  __shared__ __attribute__((aligned(16))) uint16_t dOs[RowCopy::PIECES * 512];
  __shared__ __attribute__((aligned(16))) uint16_t Qn[TrCopy::PIECES * 512];
  __shared__ __attribute__((aligned(16))) uint16_t dOn[TrCopy::PIECES * 512];
  // P of a step's two 32-query tiles per key group: registers 4g..4g+3 of a
  // lane as 16 contiguous bytes, the 64 lanes side by side
  __shared__ a_u32x4 Ps[4][2][4][64];
  __shared__ float lse_s[kBQ2], del_s[kBQ2];

  const int BH = a.B * a.H;
  const int bh = blockIdx.x % BH, kb = blockIdx.x / BH;
  const int b = bh / a.H, h = bh % a.H;
  const int lane = threadIdx.x & 63, hl = lane >> 5;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int w = wv & 3;
  const bool dkw = wv >= 4;                        // the dK wave of its pair
  const int rt = threadIdx.x & (kAttnThreads - 1);  // thread index within the role
  const int k0 = kb * kBKV2 + w * 32;
  const int key = k0 + (lane & 31);

  // B operands of the first product: K rows (S = Q K^T) in the dV wave, V
  // rows (dP = dO V^T) in the dK wave
  uint4 kf[KS];
  {
    const uint16_t* kp = row_ptr(dkw ? a.v : a.k, key, b, h);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) kf[ks] = load_row16<PAD>(kp, key < a.S, ks * 16 + hl * 8, a.hd);
  }
  a_f32x16 acc[DT];  // dV in the dV wave, dK in the dK wave
#pragma unroll
  for (int t = 0; t < DT; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[t][r] = 0.f;

  // the dV waves move the Q rows, the dK waves the dO rows
  const AttnTensor& src = dkw ? a.dout : a.q;
  const a_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(src.p), (short)0, (int)src.bytes,
                                                        0x00020000);
  const int32_t row_bytes = (int32_t)(src.ss * 2);
  RowCopy rowc;
  TrCopy trc;
  rowc.init(src, b, h, a.hd, w, lane);
  trc.init(src, b, h, a.hd, w, lane);
  uint16_t* const rowimg = dkw ? dOs : Qs;
  uint16_t* const trimg = dkw ? dOn : Qn;
  const int qtr = tr_lane(lane, QN);
  const int first = (kb * kBKV2) / kBQ2, nq = (a.S + kBQ2 - 1) / kBQ2;
  // per-query statistics of a step: lse for the dV waves' P, delta for the
  // dK waves' dS (a padding query gets lse = 1e30, so P = 0)
  auto stat = [&](int qs) __attribute__((always_inline)) {
    const bool real = !PAD || qs + rt < a.S;
    const int64_t i = (int64_t)bh * a.S + qs + rt;
    return dkw ? (real ? a.delta[i] : 0.f) : (real ? a.lse[i] : 1e30f);
  };
  float stat_n = 0.f;
  rowc.template issue<PAD>(rowimg, rs, row_bytes, first * kBQ2, a.S);
  trc.template issue<PAD>(trimg, rs, row_bytes, first * kBQ2, a.S);
  if (rt < kBQ2) stat_n = stat(first * kBQ2);
  vm_wait_all();
  if (rt < kBQ2) (dkw ? del_s : lse_s)[rt] = stat_n;
  __syncthreads();
  for (int qb = first; qb < nq; ++qb) {
    const int qs0 = qb * kBQ2;
    const bool more = qb + 1 < nq;
    // the natural copy of this step (read after the hand-over barrier)
    if (qb != first) trc.template issue<PAD>(trimg, rs, row_bytes, qs0, a.S);
    // a pair whose keys all follow every query of the step skips the work
    // but not the barriers
    const bool active = qs0 + kBQ2 - 1 >= k0;
    const bool diag = qs0 < k0 + 31;
    a_f32x16 x[2];  // S, then P (dV wave); dP - delta, then dS (dK wave)
    if (active) {
#pragma unroll
      for (int t = 0; t < 2; ++t) {
#pragma unroll
        for (int r = 0; r < 16; ++r) x[t][r] = 0.f;
        const uint16_t* ap = rowimg + (t * 32 + (lane & 31)) * AL + hl * 8;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) x[t] = mma<FP16>(*reinterpret_cast<const uint4*>(ap + ks * 16), kf[ks], x[t]);
        if (!dkw) {
          // P; query index of register r = t*32 + swz_row(r, hl); the causal
          // mask only on the steps that cross the diagonal
          auto probs = [&](auto masked) __attribute__((always_inline)) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int qi = t * 32 + swz_row(r, hl);
              float p = fast_exp2(__builtin_fmaf(x[t][r], a.scale_log2, -lse_s[qi]));
              if (decltype(masked)::value && key > qs0 + qi) p = 0.f;
              x[t][r] = p;
            }
          };
          if (diag)
            probs(std::true_type{});
          else
            probs(std::false_type{});
#pragma unroll
          for (int g = 0; g < 4; ++g)
            Ps[w][t][g][lane] = a_u32x4{__float_as_uint(x[t][4 * g]), __float_as_uint(x[t][4 * g + 1]),
                                        __float_as_uint(x[t][4 * g + 2]), __float_as_uint(x[t][4 * g + 3])};
        } else {
#pragma unroll
          for (int r = 0; r < 16; ++r) x[t][r] = x[t][r] - del_s[t * 32 + swz_row(r, hl)];
        }
      }
    }
    vm_wait_all();  // this step's natural copy has landed
    __syncthreads();  // P handed over; every row-swizzled read of the step done
    // the next step's row-swizzled copy and statistics, read after the
    // step's closing barrier
    if (more) {
      rowc.template issue<PAD>(rowimg, rs, row_bytes, qs0 + kBQ2, a.S);
      if (rt < kBQ2) stat_n = stat(qs0 + kBQ2);
    }
    if (active) {
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        if (dkw) {
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const a_u32x4 pv = Ps[w][t][g][lane];
#pragma unroll
            for (int e = 0; e < 4; ++e) x[t][4 * g + e] = __uint_as_float(pv[e]) * x[t][4 * g + e];
          }
        }
        // dV += P^T dO (dV wave) or dK += dS^T Q (dK wave) over the tile's
        // 32 queries, two k-steps of 16
        const uint16_t* bp = (dkw ? Qn : dOn) + qtr;
#pragma unroll
        for (int k2 = 0; k2 < 2; ++k2) {
          const int kk = t * 2 + k2, e0 = k2 * 8;
          const uint4 pa = make_uint4(pack2<FP16>(x[t][e0 + 0], x[t][e0 + 1]), pack2<FP16>(x[t][e0 + 2], x[t][e0 + 3]),
                                      pack2<FP16>(x[t][e0 + 4], x[t][e0 + 5]), pack2<FP16>(x[t][e0 + 6], x[t][e0 + 7]));
#pragma unroll
          for (int d2 = 0; d2 < DT; ++d2) acc[d2] = mma<FP16>(pa, tr_frag(bp + kk * 16 * QN + d2 * 32, QN), acc[d2]);
        }
      }
    }
    vm_wait_all();  // the next step's row-swizzled copy and statistics have landed
    if (more && rt < kBQ2) (dkw ? del_s : lse_s)[rt] = stat_n;
    __syncthreads();  // step done: both copies and P free for the next step
  }
  // lane holds d = t*32 + lane%32 for keys k0 + acc_row(r, hl)
#pragma unroll
  for (int t = 0; t < DT; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int kr = k0 + acc_row(r, hl);
      const int d = t * 32 + (lane & 31);
      if (PAD && (kr >= a.S || d >= a.hd)) continue;
      if (dkw)
        row_ptr(a.dk, kr, b, h)[d] = from_f<FP16>(acc[t][r] * a.scale);
      else
        row_ptr(a.dv, kr, b, h)[d] = from_f<FP16>(acc[t][r]);
    }
}

// ------------------------------ backward: dK, dV paired, head_dim 128 --
// The pairing above for D = 128, skewed by half a step so that each step
// has one barrier and both waves of a SIMD mix MFMAs and VALU work: in step
// m the dV wave computes S(m) and P(m) (handing P to LDS) and then adds
// P(m)^T dO(m) into dV, while the dK wave first finishes step m-1 -- reads
// P(m-1), forms dS = P (dP - delta) and adds dS^T Q(m-1) into dK -- and then
// computes dP(m) - delta.  One wave's exponentials or dS arithmetic then
// fall between the other wave's MFMAs instead of after them.
//
// LDS holds one image per tile of 64 query rows: the 16 chunks of 8 columns
// of a row, chunk c of row r at position c ^ xsw(r); xsw swaps the two
// 2-bit fields of r mod 16, so the row reads of the A operands (16 lanes on
// 16 rows, one chunk) and the transposing reads of the B operands (4 rows x
// 64 bytes per 32 lanes) both hit distinct banks, and one image serves
// both.  Step m reads Q(m-1), Q(m) and dO(m), and the rows of step m+1 load
// directly into idle images a whole step ahead: three Q images, two dO
// images and two P buffers (145 KB in all).  The arithmetic per element is
// that of the kernel above, in the same order, with one exception: dP's
// accumulator starts at -delta instead of having delta subtracted after
// the product.  dV is therefore bit-identical to the kernel above, and dK
// may differ from it in the last bit of the 16-bit result (about 0.02 % of
// the elements at the benchmarked shape), the fp32 sum being rounded in
// another order.

template <bool FP16, bool PAD>
__global__ void __launch_bounds__(2 * kAttnThreads, 1) attn_bwd_dkdv_x128_kernel(AttnArgs a) {
  constexpr int D = 128, KS = D / 16, DT = D / 32;
  constexpr int IMG = kBQ2 * D;  // elements of one image
  __shared__ __attribute__((aligned(16))) uint16_t Qx[3 * IMG];
  __shared__ __attribute__((aligned(16))) uint16_t dOx[2 * IMG];
  __shared__ a_u32x4 Ps[2][4][2][4][64];
  __shared__ __attribute__((aligned(16))) float lse_s[2][kBQ2];
  __shared__ __attribute__((aligned(16))) float del_s[2][kBQ2];

  const int BH = a.B * a.H;
  const int bh = blockIdx.x % BH, kb = blockIdx.x / BH;
  const int b = bh / a.H, h = bh % a.H;
  const int lane = threadIdx.x & 63, hl = lane >> 5;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int w = wv & 3;
  const bool dkw = wv >= 4;  // the dK wave of its pair
  const int rt = threadIdx.x & (kAttnThreads - 1);
  const int k0 = kb * kBKV2 + w * 32;
  const int key = k0 + (lane & 31);

  // B operands of the first product: K rows (S = Q K^T) in the dV wave, V
  // rows (dP = dO V^T) in the dK wave
  uint4 kf[KS];
  {
    const uint16_t* kp = row_ptr(dkw ? a.v : a.k, key, b, h);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) kf[ks] = load_row16<PAD>(kp, key < a.S, ks * 16 + hl * 8, a.hd);
  }
  a_f32x16 acc[DT];  // dV in the dV wave, dK in the dK wave
#pragma unroll
  for (int t = 0; t < DT; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[t][r] = 0.f;

  // direct loads (the dV waves move Q, the dK waves dO): lane l of piece j
  // (4 per wave, 16 per image) fills unit (w*4 + j)*64 + l, i.e. image row
  // u / 16, position u % 16
  const AttnTensor& src = dkw ? a.dout : a.q;
  const a_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(src.p), (short)0, (int)src.bytes,
                                                        0x00020000);
  const int32_t row_bytes = (int32_t)(src.ss * 2);
  int32_t doff[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int u = (w * 4 + j) * 64 + lane;
    const int r = u >> 4, c = (u & 15) ^ xsw(r);
    doff[j] = c * 8 < a.hd ? (int32_t)(((int64_t)b * src.sb + (int64_t)h * src.sh + (int64_t)r * src.ss + c * 8) * 2)
                           : kAttnOob;
  }
  uint16_t* const ldsimg = dkw ? dOx : Qx;
  auto issue = [&](int slot, int r0) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int32_t o = !PAD || r0 + (w * 4 + j) * 4 + (lane >> 4) < a.S ? doff[j] : kAttnOob;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rs, (__attribute__((address_space(3))) void*)(ldsimg + slot * IMG + (w * 4 + j) * 512), 16, o,
          r0 * row_bytes, 0, 0);
    }
  };
  // A-operand rows: tile row t*32 + swz(lane%32), chunk 2*ks + hl at
  // position (2*ks + hl) ^ xsw(row) = 2*(ks ^ (xa >> 1)) + (hl ^ (xa & 1))
  int aoff[KS];
  {
    const int arow = swz(lane & 31), xa = xsw(arow);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) aoff[ks] = arow * D + (((2 * ks + hl) ^ xa) << 3);
  }
  // B-operand transposing reads: k-rows kk*16 + 8*(l/32) + (l%16)/4 (+4 for
  // the second read), columns d2*32 + 16*((l/16)%2) + 4*(l%4)
  int toff[DT][2];
  {
    const int R = (lane & 15) >> 2, L5 = lane >> 5, L4 = (lane >> 4) & 1, L1 = (lane >> 1) & 1;
#pragma unroll
    for (int d2 = 0; d2 < DT; ++d2)
#pragma unroll
      for (int hi = 0; hi < 2; ++hi) {
        const int row = 8 * L5 + R + 4 * hi;
        const int pc = 4 * (d2 ^ R) + ((2 * L4 + L1) ^ (2 * L5 + hi));
        toff[d2][hi] = row * D + pc * 8 + (lane & 1) * 4;
      }
  }
  auto bfrag = [&](const uint16_t* img, int kk, int d2) __attribute__((always_inline)) {
    const uint16_t* bp = img + kk * 16 * D;
    const a_u32x2 lo =
        __builtin_bit_cast(a_u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((a_lds_s16x4*)(bp + toff[d2][0])));
    const a_u32x2 hi =
        __builtin_bit_cast(a_u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((a_lds_s16x4*)(bp + toff[d2][1])));
    return make_uint4(lo.x, lo.y, hi.x, hi.y);
  };
  // acc += X^T B over a step's 64 queries: X (P or dS, one 32-query tile
  // per t) as the A operand, B from the transposing reads of `img`.  Four
  // B fragments in flight, each refilled with the next k-step's fragment of
  // its head-dim tile right after its MFMA issues (order pinned: the
  // scheduler otherwise hoists every read and runs out of registers)
  // With `pbuf` (the dK wave), tile t's X is first formed as dS = P (dP -
  // delta) from P in `pbuf`, one tile at a time.
  auto second = [&](a_f32x16 (&x)[2], const uint16_t* img, const a_u32x4 (*pbuf)[2][4][64])
                    __attribute__((always_inline)) {
    uint4 fb[DT];
#pragma unroll
    for (int d2 = 0; d2 < DT; ++d2) fb[d2] = bfrag(img, 0, d2);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      if (pbuf) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const a_u32x4 pv = pbuf[w][t][g][lane];
#pragma unroll
          for (int e = 0; e < 4; ++e) x[t][4 * g + e] = __uint_as_float(pv[e]) * x[t][4 * g + e];
        }
      }
#pragma unroll
      for (int k2 = 0; k2 < 2; ++k2) {
        const int kk = t * 2 + k2, e0 = k2 * 8;
        const uint4 pa = make_uint4(pack2<FP16>(x[t][e0 + 0], x[t][e0 + 1]), pack2<FP16>(x[t][e0 + 2], x[t][e0 + 3]),
                                    pack2<FP16>(x[t][e0 + 4], x[t][e0 + 5]), pack2<FP16>(x[t][e0 + 6], x[t][e0 + 7]));
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int d2 = 0; d2 < DT; ++d2) {
          acc[d2] = mma<FP16>(pa, fb[d2], acc[d2]);
          __builtin_amdgcn_sched_barrier(0);
          if (kk < 3) fb[d2] = bfrag(img, kk + 1, d2);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
  };
  // x = (rows of img) kf^T over the 64 queries of a step: S (dV wave) or
  // dP (dK wave), query index of register r of tile t = t*32 + swz_row(r, hl).
  // A rolling window of four A fragments, pinned like the B fragments
  // x starts at `x0(t)` (zero, or the per-query -delta of the dK wave)
  auto first_product = [&](a_f32x16 (&x)[2], const uint16_t* img, auto x0) __attribute__((always_inline)) {
    auto afrag = [&](int i) __attribute__((always_inline)) {  // fragment i = t*KS + ks
      return *reinterpret_cast<const uint4*>(img + (i / KS) * 32 * D + aoff[i % KS]);
    };
    uint4 fa[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) fa[i] = afrag(i);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int i = t * KS + ks;
        x[t] = mma<FP16>(fa[i & 3], kf[ks], ks == 0 ? x0(t) : x[t]);
        __builtin_amdgcn_sched_barrier(0);
        if (i + 4 < 2 * KS) fa[i & 3] = afrag(i + 4);
        __builtin_amdgcn_sched_barrier(0);
      }
  };

  const int first = (kb * kBKV2) / kBQ2, nq = (a.S + kBQ2 - 1) / kBQ2, n = nq - first;
  auto stat = [&](int qs) __attribute__((always_inline)) {
    const bool real = !PAD || qs + rt < a.S;
    const int64_t i = (int64_t)bh * a.S + qs + rt;
    return dkw ? (real ? -a.delta[i] : 0.f) : (real ? a.lse[i] : 1e30f);
  };
  float stat_n = 0.f;
  issue(0, first * kBQ2);
  if (rt < kBQ2) stat_n = stat(first * kBQ2);
  vm_wait_all();
  if (rt < kBQ2) (dkw ? del_s : lse_s)[0][rt] = stat_n;
  __syncthreads();

  a_f32x16 x[2];  // S then P (dV wave); dP - delta, then dS (dK wave)
  // step j = m - first (Q image j % 3; dO image, P buffer and statistics
  // j % 2 = P, a template constant)
  auto step = [&](int j, int qslot, auto par_c, auto role_c) __attribute__((always_inline)) {
    constexpr int P = decltype(par_c)::value;
    constexpr bool DKW = decltype(role_c)::value;  // the role, a constant here
    const int m = first + j, qs0 = m * kBQ2;
    const int qnext = qslot == 2 ? 0 : qslot + 1, qprev = qslot == 0 ? 2 : qslot - 1;
    if (j + 1 < n) {  // the next step's rows into idle images, a step ahead
      issue(dkw ? P ^ 1 : qnext, qs0 + kBQ2);
      if (rt < kBQ2) stat_n = stat(qs0 + kBQ2);
    }
    // a pair whose keys all follow every query of a step skips its work
    const bool active = qs0 + kBQ2 - 1 >= k0;
    const bool active_prev = j > 0 && qs0 - 1 >= k0;
    // the sub-products are fenced from each other: the scheduler otherwise
    // hoists every fragment read of the next product above the current
    // one and runs out of registers
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (!DKW) {
      if (active) {
        first_product(x, Qx + qslot * IMG, [](int) { return a_f32x16{}; });
        __builtin_amdgcn_sched_barrier(0);
        const bool diag = qs0 < k0 + 31;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          auto probs = [&](auto masked) __attribute__((always_inline)) {
            // the causal mask: query qs0 + t*32 + swz_row(r, hl) precedes the
            // key when kq > t*32 + swz_row(r, 0) (a constant per register)
            const int kq = key - qs0 - 8 * hl;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
              // lse of the 4 queries of registers 4g..4g+3 (consecutive)
              const float4 l4 = *reinterpret_cast<const float4*>(&lse_s[P][t * 32 + swz_row(4 * g, hl)]);
              const float lv[4] = {l4.x, l4.y, l4.z, l4.w};
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                const int r = 4 * g + e;
                float p = fast_exp2(__builtin_fmaf(x[t][r], a.scale_log2, -lv[e]));
                if (decltype(masked)::value && kq > t * 32 + swz_row(r, 0)) p = 0.f;
                x[t][r] = p;
              }
            }
          };
          if (diag)
            probs(std::true_type{});
          else
            probs(std::false_type{});
#pragma unroll
          for (int g = 0; g < 4; ++g)
            Ps[P][w][t][g][lane] = a_u32x4{__float_as_uint(x[t][4 * g]), __float_as_uint(x[t][4 * g + 1]),
                                           __float_as_uint(x[t][4 * g + 2]), __float_as_uint(x[t][4 * g + 3])};
        }
        __builtin_amdgcn_sched_barrier(0);
        second(x, dOx + P * IMG, nullptr);
      }
    } else {
      if (active_prev)  // finish step m-1: dS = P (dP - delta), dK += dS^T Q
        second(x, Qx + qprev * IMG, Ps[P ^ 1]);
      __builtin_amdgcn_sched_barrier(0);
      if (active) {
        // dP - delta: the accumulator starts at -delta (stored negated)
        first_product(x, dOx + P * IMG, [&](int t) __attribute__((always_inline)) {
          a_f32x16 d;
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const float4 d4 = *reinterpret_cast<const float4*>(&del_s[P][t * 32 + swz_row(4 * g, hl)]);
            d[4 * g + 0] = d4.x;
            d[4 * g + 1] = d4.y;
            d[4 * g + 2] = d4.z;
            d[4 * g + 3] = d4.w;
          }
          return d;
        });
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    vm_wait_all();  // the next step's rows and statistics have landed
    if (j + 1 < n && rt < kBQ2) (dkw ? del_s : lse_s)[P ^ 1][rt] = stat_n;
    __syncthreads();  // P(m) handed over; images of step m-1 free
  };
  // each role runs its own copy of the step loop (the same barriers in the
  // same order), so neither keeps the other's values alive
  auto run = [&](auto role_c) __attribute__((always_inline)) {
    int j = 0, qslot = 0;
    for (; j + 1 < n; j += 2) {
      step(j, qslot, std::integral_constant<int, 0>{}, role_c);
      qslot = qslot == 2 ? 0 : qslot + 1;
      step(j + 1, qslot, std::integral_constant<int, 1>{}, role_c);
      qslot = qslot == 2 ? 0 : qslot + 1;
    }
    if (j < n) {
      step(j, qslot, std::integral_constant<int, 0>{}, role_c);
      qslot = qslot == 2 ? 0 : qslot + 1;
    }
    // the dK waves finish the last step (its P is in buffer (n - 1) % 2)
    if (decltype(role_c)::value && (nq - 1) * kBQ2 + kBQ2 - 1 >= k0) {
      const int pb = (n - 1) & 1, qlast = qslot == 0 ? 2 : qslot - 1;
      second(x, Qx + qlast * IMG, Ps[pb]);
    }
  };
  if (dkw)
    run(std::true_type{});
  else
    run(std::false_type{});
  // the 32 x 128 tile of each wave (dV or dK, rounded to 16 bits) through
  // LDS, then out in 16-byte row chunks: lane holds d = t*32 + lane%32 for
  // keys acc_row(r, hl); the staging rows are padded by 8 elements
  constexpr int SL = D + 8;
  __syncthreads();  // every image and P buffer read
  // 8.5 KB per wave: the dV waves' in the Q images, the dK waves' in the P buffers
  uint16_t* stage = (dkw ? reinterpret_cast<uint16_t*>(&Ps[0][0][0][0][0]) : Qx) + w * 32 * SL;
  static_assert(4 * 32 * SL <= 3 * IMG && 4 * 32 * SL * 2 <= (int)sizeof(Ps), "staging fits");
#pragma unroll
  for (int t = 0; t < DT; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r)
      stage[acc_row(r, hl) * SL + t * 32 + (lane & 31)] = from_f<FP16>(dkw ? acc[t][r] * a.scale : acc[t][r]);
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's staging writes are done (the wave reads only its own)
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int c = i * 64 + lane, kr = c >> 4, col = (c & 15) * 8;  // key row, first column of the chunk
    const int key_g = k0 + kr;
    if (PAD && (key_g >= a.S || col >= a.hd)) continue;
    *reinterpret_cast<uint4*>(row_ptr(dkw ? a.dk : a.dv, key_g, b, h) + col) =
        *reinterpret_cast<const uint4*>(stage + kr * SL + col);
  }
}

// ------------------------------------------------------------ backward: dQ --
template <int D, bool FP16, bool PAD>
__global__ void __launch_bounds__(kAttnThreads, 2) attn_bwd_dq_kernel(AttnArgs a) {
  constexpr int KS = D / 16, DT = D / 32;
  // K and V rows swizzled for S^T and dP^T; K also in natural order, padded
  // to D + 32, for the transposing reads of dQ^T = K^T dS^T
  constexpr int KN = tr_row(D);
  __shared__ __attribute__((aligned(16))) uint16_t Ks[kBKV * (D + 8)];
  __shared__ __attribute__((aligned(16))) uint16_t Vs[kBKV * (D + 8)];
  __shared__ __attribute__((aligned(16))) uint16_t Kn[kBKV * KN];

  const int BH = a.B * a.H, nqb = (a.S + kBQ - 1) / kBQ;
  const int bh = blockIdx.x % BH, qb = nqb - 1 - blockIdx.x / BH;
  const int b = bh / a.H, h = bh % a.H;
  const int lane = threadIdx.x & 63, hl = lane >> 5;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int q0 = qb * kBQ + w * 32;
  const int q = q0 + (lane & 31);

  const bool real = !PAD || q < a.S;  // false on padding rows of the last block
  uint4 qf[KS], of[KS];
  {
    const uint16_t* qp = row_ptr(a.q, q, b, h);
    const uint16_t* op = row_ptr(a.dout, q, b, h);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      qf[ks] = load_row16<PAD>(qp, real, ks * 16 + hl * 8, a.hd);
      of[ks] = load_row16<PAD>(op, real, ks * 16 + hl * 8, a.hd);
    }
  }
  const float lse = real ? a.lse[(int64_t)bh * a.S + q] : 1e30f;
  // delta = rowsum(dO * O) for this query, from the dO fragments already in
  // registers (the two half-waves hold alternate 8-element chunks of the row);
  // written out for the dK/dV kernel, which runs next
  float del = 0.f;
  {
    const uint16_t* opp = row_ptr(a.o, q, b, h);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const uint4 ov = load_row16<PAD>(opp, real, ks * 16 + hl * 8, a.hd);
      const uint32_t ow[4] = {ov.x, ov.y, ov.z, ov.w};
      const uint32_t dw[4] = {of[ks].x, of[ks].y, of[ks].z, of[ks].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        del += to_f<FP16>((uint16_t)(ow[e] & 0xffffu)) * to_f<FP16>((uint16_t)(dw[e] & 0xffffu));
        del += to_f<FP16>((uint16_t)(ow[e] >> 16)) * to_f<FP16>((uint16_t)(dw[e] >> 16));
      }
    }
    del += __shfl_xor(del, 32, 64);
    if (hl == 0 && real) a.delta[(int64_t)bh * a.S + q] = del;
  }
  a_f32x16 dq[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) dq[t][r] = 0.f;

  BufTile<kBKV, D, D + 8, true, PAD> kt, vt;
  kt.init(a.k, b, h, a.S, a.hd);
  vt.init(a.v, b, h, a.S, a.hd);
  const int ktr = tr_lane(lane, KN);
  const int nkv = (qb * kBQ + kBQ) / kBKV;
  // the next block's K / V rows are loaded while this block computes
  kt.load(0);
  vt.load(0);
  for (int j = 0; j < nkv; ++j) {
    const int kv0 = j * kBKV;
    __syncthreads();
    kt.store(Ks);
    kt.template store_natural<KN>(Kn);
    vt.store(Vs);
    __syncthreads();
    if (j + 1 < nkv) {
      kt.load(kv0 + kBKV);
      vt.load(kv0 + kBKV);
    }
    if (kv0 > q0 + 31) continue;
    const bool diag = kv0 + kBKV - 1 > q0;
    // one 32-key tile at a time: S^T = K Q^T, dP^T = V dO^T (lane = query),
    // dS^T, then dQ^T += K^T dS^T over those 32 keys
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      a_f32x16 s, dp;
#pragma unroll
      for (int r = 0; r < 16; ++r) s[r] = dp[r] = 0.f;
      const uint16_t* kp = Ks + (t * 32 + (lane & 31)) * (D + 8) + hl * 8;
      const uint16_t* vp = Vs + (t * 32 + (lane & 31)) * (D + 8) + hl * 8;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        s = mma<FP16>(*reinterpret_cast<const uint4*>(kp + ks * 16), qf[ks], s);
        dp = mma<FP16>(*reinterpret_cast<const uint4*>(vp + ks * 16), of[ks], dp);
      }
      // causal mask only on the blocks that cross the diagonal (see dK/dV)
      auto dsoft = [&](auto masked) __attribute__((always_inline)) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float p = fast_exp2(__builtin_fmaf(s[r], a.scale_log2, -lse));
          if (decltype(masked)::value && kv0 + t * 32 + swz_row(r, hl) > q) p = 0.f;
          dp[r] = p * (dp[r] - del);
        }
      };
      if (diag)
        dsoft(std::true_type{});
      else
        dsoft(std::false_type{});
#pragma unroll
      for (int k2 = 0; k2 < 2; ++k2) {
        const int kk = t * 2 + k2, e0 = k2 * 8;
        const uint4 sb = make_uint4(pack2<FP16>(dp[e0 + 0], dp[e0 + 1]), pack2<FP16>(dp[e0 + 2], dp[e0 + 3]),
                                    pack2<FP16>(dp[e0 + 4], dp[e0 + 5]), pack2<FP16>(dp[e0 + 6], dp[e0 + 7]));
        const uint16_t* ktp = Kn + ktr + kk * 16 * KN;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) dq[dt] = mma<FP16>(tr_frag(ktp + dt * 32, KN), sb, dq[dt]);
      }
    }
  }
  if (PAD && !real) return;
  uint16_t* dqp = row_ptr(a.dq, q, b, h);
#pragma unroll
  for (int t = 0; t < DT; ++t)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      if (PAD && t * 32 + g * 8 >= a.hd) continue;
      uint2 v;
      v.x = pack2<FP16>(dq[t][g * 4 + 0] * a.scale, dq[t][g * 4 + 1] * a.scale);
      v.y = pack2<FP16>(dq[t][g * 4 + 2] * a.scale, dq[t][g * 4 + 3] * a.scale);
      *reinterpret_cast<uint2*>(dqp + t * 32 + g * 8 + hl * 4) = v;
    }
}

}  // namespace eth

using namespace eth;

static int attn_check(const eth_attn_desc_t* d) {
  ETH_CHECK_ARG(d, "attention: null descriptor");
  ETH_CHECK_ARG(d->dtype == ETH_BF16 || d->dtype == ETH_F16, "attention: dtype must be bf16/fp16");
  ETH_CHECK_ARG(d->head_dim >= 8 && d->head_dim <= 128 && d->head_dim % 8 == 0,
                "attention: head_dim must be a multiple of 8 in [8, 128] (got %d)", d->head_dim);
  ETH_CHECK_ARG(d->seq > 0, "attention: seq must be positive (got %d)", d->seq);
  ETH_CHECK_ARG(d->batch > 0 && d->heads > 0, "attention: bad batch/heads");
  return ETH_OK;
}

static AttnTensor tin(const void* p, const int64_t* st, const eth_attn_desc_t* d) {
  AttnTensor t;
  t.p = (const uint16_t*)p;
  t.ss = st[0];
  t.sb = st[1];
  t.sh = st[2];
  const int64_t extent = ((int64_t)(d->seq - 1) * st[0] + (int64_t)(d->batch - 1) * st[1] +
                          (int64_t)(d->heads - 1) * st[2] + d->head_dim) * 2;
  t.bytes = extent < (1LL << 31) ? (uint32_t)extent : 0u;
  return t;
}
static AttnOut tout(void* p, const int64_t* st) {
  AttnOut t;
  t.p = (uint16_t*)p;
  t.ss = st[0];
  t.sb = st[1];
  t.sh = st[2];
  return t;
}

static bool aligned_rows(const void* p, const int64_t* st) {
  return ((uintptr_t)p & 15) == 0 && st[0] % 8 == 0 && st[1] % 8 == 0 && st[2] % 8 == 0;
}

extern "C" int eth_attn_fwd(const eth_attn_desc_t* d, const void* q, const void* k, const void* v,
                            void* out, float* lse, void* stream) {
  if (int rc = attn_check(d)) return rc;
  ETH_CHECK_ARG(q && k && v && out && lse, "eth_attn_fwd: null pointer");
  ETH_CHECK_ARG(aligned_rows(q, d->q_strides) && aligned_rows(k, d->k_strides) && aligned_rows(v, d->v_strides) &&
                    aligned_rows(out, d->o_strides),
                "eth_attn_fwd: rows must be 16-byte aligned");
  AttnArgs a{};
  a.q = tin(q, d->q_strides, d);
  a.k = tin(k, d->k_strides, d);
  a.v = tin(v, d->v_strides, d);
  a.out = tout(out, d->o_strides);
  ETH_CHECK_ARG(a.q.bytes && a.k.bytes && a.v.bytes, "eth_attn_fwd: tensors above 2 GiB are not supported");
  a.lse = lse;
  a.B = d->batch;
  a.H = d->heads;
  a.S = d->seq;
  a.hd = d->head_dim;
  a.scale = 1.0f / sqrtf((float)d->head_dim);
  a.scale_log2 = a.scale * 1.4426950408889634f;
  const int grid = a.B * a.H * ((a.S + kBQ - 1) / kBQ);
  hipStream_t s = (hipStream_t)stream;
  const bool fp16 = d->dtype == ETH_F16;
  const int width = a.hd > 96 ? 128 : a.hd > 64 ? 96 : 64;
  // full blocks (every row and head-dim column real) take the unguarded kernels
  const bool pad = a.S % kBQ != 0 || a.hd != width;
#define ETH_ATTN_FWD(D)                                                                \
  if (pad) {                                                                           \
    if (fp16) attn_fwd_kernel<D, true, true><<<grid, kAttnThreads, 0, s>>>(a);         \
    else attn_fwd_kernel<D, false, true><<<grid, kAttnThreads, 0, s>>>(a);             \
  } else {                                                                             \
    if (fp16) attn_fwd_kernel<D, true, false><<<grid, kAttnThreads, 0, s>>>(a);        \
    else attn_fwd_kernel<D, false, false><<<grid, kAttnThreads, 0, s>>>(a);            \
  }
  if (a.hd > 96) {
    if (pad) {
      if (fp16) attn_fwd_x128_kernel<true, true><<<grid, kAttnThreads, 0, s>>>(a);
      else attn_fwd_x128_kernel<false, true><<<grid, kAttnThreads, 0, s>>>(a);
    } else {
      if (fp16) attn_fwd_x128_kernel<true, false><<<grid, kAttnThreads, 0, s>>>(a);
      else attn_fwd_x128_kernel<false, false><<<grid, kAttnThreads, 0, s>>>(a);
    }
  } else if (a.hd > 64) {
    ETH_ATTN_FWD(96)
  } else {
    ETH_ATTN_FWD(64)
  }
#undef ETH_ATTN_FWD
  ETH_CHECK_LAUNCH("eth_attn_fwd");
  return ETH_OK;
}

extern "C" int eth_attn_bwd(const eth_attn_desc_t* d, const void* q, const void* k, const void* v,
                            const void* out, const void* dout, const float* lse, float* delta, void* dq,
                            void* dk, void* dv, void* stream) {
  if (int rc = attn_check(d)) return rc;
  ETH_CHECK_ARG(q && k && v && out && dout && lse && delta && dq && dk && dv, "eth_attn_bwd: null pointer");
  ETH_CHECK_ARG(aligned_rows(q, d->q_strides) && aligned_rows(k, d->k_strides) && aligned_rows(v, d->v_strides) &&
                    aligned_rows(out, d->o_strides) && aligned_rows(dout, d->do_strides) &&
                    aligned_rows(dq, d->dq_strides) && aligned_rows(dk, d->dk_strides) &&
                    aligned_rows(dv, d->dv_strides),
                "eth_attn_bwd: rows must be 16-byte aligned");
  AttnArgs a{};
  a.q = tin(q, d->q_strides, d);
  a.k = tin(k, d->k_strides, d);
  a.v = tin(v, d->v_strides, d);
  a.o = tin(out, d->o_strides, d);
  a.dout = tin(dout, d->do_strides, d);
  a.dq = tout(dq, d->dq_strides);
  a.dk = tout(dk, d->dk_strides);
  a.dv = tout(dv, d->dv_strides);
  ETH_CHECK_ARG(a.q.bytes && a.k.bytes && a.v.bytes && a.o.bytes && a.dout.bytes,
                "eth_attn_bwd: tensors above 2 GiB are not supported");
  a.lse = (float*)lse;
  a.delta = delta;
  a.B = d->batch;
  a.H = d->heads;
  a.S = d->seq;
  a.hd = d->head_dim;
  a.scale = 1.0f / sqrtf((float)d->head_dim);
  a.scale_log2 = a.scale * 1.4426950408889634f;
  hipStream_t s = (hipStream_t)stream;
  const bool fp16 = d->dtype == ETH_F16;
  const int g_kv = a.B * a.H * ((a.S + kBKV2 - 1) / kBKV2);
  const int g_q = a.B * a.H * ((a.S + kBQ - 1) / kBQ);
  // dQ first: it also writes delta = rowsum(dO * O), which dK/dV reads
  const int width = a.hd > 96 ? 128 : a.hd > 64 ? 96 : 64;
  static_assert(kBKV2 == kBQ, "one padding rule for the three backward kernels");
  const bool pad = a.S % kBKV2 != 0 || a.hd != width;
#define ETH_ATTN_BWD_P(D, F, P)                                                    \
  attn_bwd_dq_kernel<D, F, P><<<g_q, kAttnThreads, 0, s>>>(a);                   \
  if constexpr (D == 128)                                                         \
    attn_bwd_dkdv_x128_kernel<F, P><<<g_kv, 2 * kAttnThreads, 0, s>>>(a);         \
  else                                                                            \
    attn_bwd_dkdv_pair_kernel<D, F, P><<<g_kv, 2 * kAttnThreads, 0, s>>>(a);
#define ETH_ATTN_BWD(D, F)        \
  if (pad) {                      \
    ETH_ATTN_BWD_P(D, F, true)    \
  } else {                        \
    ETH_ATTN_BWD_P(D, F, false)   \
  }
  if (a.hd > 96) {
    if (fp16) { ETH_ATTN_BWD(128, true) } else { ETH_ATTN_BWD(128, false) }
  } else if (a.hd > 64) {
    if (fp16) { ETH_ATTN_BWD(96, true) } else { ETH_ATTN_BWD(96, false) }
  } else {
    if (fp16) { ETH_ATTN_BWD(64, true) } else { ETH_ATTN_BWD(64, false) }
  }
#undef ETH_ATTN_BWD
#undef ETH_ATTN_BWD_P
  ETH_CHECK_LAUNCH("eth_attn_bwd");
  return ETH_OK;
}
