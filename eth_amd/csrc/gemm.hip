// bf16/fp16 GEMM on CDNA4 matrix cores (v_mfma_f32_32x32x16_{bf16,f16}),
// fp32 accumulation, LDS-staged double-buffered tiles.
//
//   C[m, n] (+)= alpha * sum_k A(m, k) * B(k, n)  (+ bias[n])
//
// A(m, k) is read K-contiguous (A[m*lda + k]) or M-contiguous (A[k*lda + m]);
// B(k, n) is read K-contiguous (B[n*ldb + k]) or N-contiguous (B[k*ldb + n]).
// The three GPT linear-layer products are
//   forward  Y = X W^T      : A K-contiguous, B K-contiguous
//   dgrad    dX = dY W      : A K-contiguous, B N-contiguous
//   wgrad    dW += dY^T X   : A M-contiguous, B N-contiguous, fp32 C += (the
//                             Megatron main_grad accumulation, fused)
// In the fallback kernel, M-contiguous / N-contiguous operands are
// transposed in registers on their way into LDS (4 k-rows x 8 columns per
// thread), so every LDS tile is stored K-contiguous and each MFMA operand is
// one 16-byte LDS read.
//
// Kernels:
//  * gemm256_m16_kernel / gemm256_m32_kernel, the main ones: 256x256x64
//    tiles, 4 waves (one per SIMD) of 128x128 each, 256 accumulator
//    registers per lane held in AGPRs.  Operands go global -> LDS with
//    direct loads (buffer_load ... lds) into two stages.  The k loop is
//    software-pipelined by hand: while the MFMAs of k-tile t run, k-tile
//    t+1 streams into the other stage, one 1 KB load per few MFMA gaps,
//    and the next fragments are read from LDS between the MFMAs
//    (sched_barrier fixes the order).  One barrier per k-tile.
//    Row-contiguous operands land as they are in memory and their
//    fragments come out of LDS through ds_read_b64_tr_b16.  The epilogue
//    stages each 32-row slab through LDS and writes whole rows with buffer
//    stores.  m16 (v_mfma_f32_16x16x32, single-buffered fragments) serves
//    the forward, data-gradient and weight-gradient products (for the last,
//    both operands row-contiguous, through asm MFMAs); m32
//    (v_mfma_f32_32x32x16) a row-contiguous A with a K-contiguous B.  Both
//    need K % 128 == 0, 16-byte aligned C rows and enough tiles to fill
//    the chip.
//  * gemm_kernel, the general fallback: 256x256 (8 waves) or 128x128 (4
//    waves) tiles, register-staged double buffering, any K % 8 == 0.
// Tiles are assigned XCD-aware (consecutive workgroups land on different
// XCDs, so the tile id is remapped to give each XCD a contiguous range) and
// in GROUP_M-row groups so neighbouring workgroups share A and B tiles in L2.
//
// Replaces the F.linear / cuBLAS calls of mpu/layers.py:357-370,452-470 and
// the main_grad.add_ hook of model/distributed.py:116-123.
#include <algorithm>

#include "common.h"

namespace eth {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

template <bool FP16>
__device__ __forceinline__ f32x16_t mfma32(const uint4& a, const uint4& b, const f32x16_t& c) {
  if constexpr (FP16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  }
}

constexpr int kPad = 8;  // LDS row padding (elements): 16 B breaks bank aliasing

// Workgroup barrier ordering LDS only.  __syncthreads also fences global
// memory, which makes every wave wait for its outstanding stores.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}
// The same after this wave's direct global->LDS loads have landed.
__device__ __forceinline__ void dma_barrier() {
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
}
// The same with the newest N vector-memory loads of this wave still in
// flight (loads complete in issue order): the prologues start on k-tile 0
// while k-tile 1 is still arriving.
template <int N>
__device__ __forceinline__ void dma_barrier_but() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

// Map a linear workgroup id to (tile_m, tile_n): XCD-contiguous, then
// GROUP_M-row grouped.
__device__ __forceinline__ void tile_coords(int pid, int tiles_m, int tiles_n, int& tm, int& tn) {
  constexpr int kXcds = 8, kGroupM = 4;
  const int total = tiles_m * tiles_n;
  const int per = (total + kXcds - 1) / kXcds;
  const int tall = total % kXcds == 0 ? kXcds : total % kXcds;
  const int xcd = pid % kXcds, local = pid / kXcds;
  pid = xcd < tall ? xcd * per + local : tall * per + (xcd - tall) * (per - 1) + local;
  const int in_group = kGroupM * tiles_n;
  const int first_m = (pid / in_group) * kGroupM;
  const int gm = min(tiles_m - first_m, kGroupM);
  tm = first_m + (pid % in_group) % gm;
  tn = (pid % in_group) / gm;
}

// Buffer-resource loads: 32-bit byte offsets (one VGPR per chunk, fixed for
// the whole K loop; the k advance goes in the scalar offset) and hardware
// bounds checking -- an offset of kOob reads zeros, which masks rows past
// the matrix and k past K without branches.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr int32_t kOob = (int32_t)0x80000000u;

__device__ __forceinline__ rsrc_t make_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ uint4 buf_load16(rsrc_t r, int32_t voff, int32_t soff) {
  auto v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
  return __builtin_bit_cast(uint4, v);
}

// ROWS x BK tile of a K-contiguous operand (row r at P[(r0+r)*ld + k]):
// CPT 16-byte chunks per thread.
template <int ROWS, int BK, int NT>
struct KTile {
  static constexpr int CPR = BK / 8;
  static constexpr int CPT = ROWS * CPR / NT;
  static_assert(CPT >= 1 && ROWS * CPR % NT == 0, "tile split");
  uint4 v[CPT];
  int32_t off[CPT];
  __device__ __forceinline__ void init(int64_t ld, int r0, int rows) {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = threadIdx.x + i * NT;
      const int r = c / CPR, kc = (c % CPR) * 8;
      off[i] = r0 + r < rows ? (int32_t)((((int64_t)(r0 + r)) * ld + kc) * 2) : kOob;
    }
  }
  __device__ __forceinline__ void load(rsrc_t rs, int64_t ld, int k0, int K, bool kfull) {
    const int32_t soff = k0 * 2;
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      int32_t o = off[i];
      if (!kfull && k0 + ((threadIdx.x + i * NT) % CPR) * 8 >= K) o = kOob;
      v[i] = buf_load16(rs, o, soff);
    }
  }
  __device__ __forceinline__ void store(uint16_t* S) const {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = threadIdx.x + i * NT;
      const int r = c / CPR, kc = (c % CPR) * 8;
      *reinterpret_cast<uint4*>(S + r * (BK + kPad) + kc) = v[i];
    }
  }
  // whole-tile load when K % BK == 0 (an empty resource reads zeros)
  __device__ __forceinline__ void fetch(rsrc_t rs, int64_t, int k0) {
#pragma unroll
    for (int i = 0; i < CPT; ++i) v[i] = buf_load16(rs, off[i], k0 * 2);
  }
  // part P of NP: store the staged chunks to LDS, then refill the same
  // registers with k-tile k0
  template <int P, int NP>
  __device__ __forceinline__ void cycle(uint16_t* S, rsrc_t rs, int64_t, int k0) {
#pragma unroll
    for (int i = P * CPT / NP; i < (P + 1) * CPT / NP; ++i) {
      const int c = threadIdx.x + i * NT;
      const int r = c / CPR, kc = (c % CPR) * 8;
      *reinterpret_cast<uint4*>(S + r * (BK + kPad) + kc) = v[i];
      v[i] = buf_load16(rs, off[i], k0 * 2);
    }
  }
};

// BK x ROWS tile of an operand contiguous along the row index (element
// (r, k) at P[k*ld + r0 + r]): each thread reads 4 k-rows of 8 consecutive
// r and writes them transposed (8 rows of 4 k) into LDS.  The k-group index
// varies fastest across lanes, so the 8-byte LDS writes of a wavefront
// spread over all banks (rows 8 apart would alias otherwise).
template <int ROWS, int BK, int NT>
struct RTile {
  static constexpr int RG = ROWS / 8, KG = BK / 4;
  static constexpr int BPT = RG * KG / NT;
  static_assert(BPT >= 1 && RG * KG % NT == 0, "tile split");
  uint4 v[BPT][4];
  int32_t off[BPT];
  __device__ __forceinline__ void init(int64_t ld, int r0, int rows) {
#pragma unroll
    for (int b = 0; b < BPT; ++b) {
      const int blk = threadIdx.x + b * NT;
      const int kg = blk % KG, rg = blk / KG;
      const int r = r0 + rg * 8;
      off[b] = r < rows ? (int32_t)((((int64_t)kg * 4) * ld + r) * 2) : kOob;
    }
  }
  __device__ __forceinline__ void load(rsrc_t rs, int64_t ld, int k0, int K, bool kfull) {
    const int32_t soff = (int32_t)((int64_t)k0 * ld * 2);
    const int32_t row_bytes = (int32_t)(ld * 2);
#pragma unroll
    for (int b = 0; b < BPT; ++b) {
      const int kg = (threadIdx.x + b * NT) % KG;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        int32_t o = off[b] == kOob ? kOob : off[b] + j * row_bytes;
        if (!kfull && k0 + kg * 4 + j >= K) o = kOob;
        v[b][j] = buf_load16(rs, o, soff);
      }
    }
  }
  __device__ __forceinline__ void store(uint16_t* S) const {
#pragma unroll
    for (int b = 0; b < BPT; ++b) store_block(S, b);
  }
  __device__ __forceinline__ void fetch(rsrc_t rs, int64_t ld, int k0) {
    const int32_t soff = (int32_t)((int64_t)k0 * ld * 2);
    const int32_t row_bytes = (int32_t)(ld * 2);
#pragma unroll
    for (int b = 0; b < BPT; ++b)
#pragma unroll
      for (int j = 0; j < 4; ++j) v[b][j] = buf_load16(rs, off[b] == kOob ? kOob : off[b] + j * row_bytes, soff);
  }
  template <int P, int NP>
  __device__ __forceinline__ void cycle(uint16_t* S, rsrc_t rs, int64_t ld, int k0) {
    const int32_t soff = (int32_t)((int64_t)k0 * ld * 2);
    const int32_t row_bytes = (int32_t)(ld * 2);
#pragma unroll
    for (int b = P * BPT / NP; b < (P + 1) * BPT / NP; ++b) {
      store_block(S, b);
#pragma unroll
      for (int j = 0; j < 4; ++j) v[b][j] = buf_load16(rs, off[b] == kOob ? kOob : off[b] + j * row_bytes, soff);
    }
  }
  __device__ __forceinline__ void store_block(uint16_t* S, int b) const {
    const int blk = threadIdx.x + b * NT;
    const int kg = blk % KG, rg = blk / KG;
    const uint32_t* w0 = reinterpret_cast<const uint32_t*>(&v[b][0]);
    const uint32_t* w1 = reinterpret_cast<const uint32_t*>(&v[b][1]);
    const uint32_t* w2 = reinterpret_cast<const uint32_t*>(&v[b][2]);
    const uint32_t* w3 = reinterpret_cast<const uint32_t*>(&v[b][3]);
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      // rows 2p and 2p+1 of the 8-row group
      const uint32_t a0 = w0[p], a1 = w1[p], a2 = w2[p], a3 = w3[p];
      uint2 lo, hi;
      lo.x = (a0 & 0xffffu) | (a1 << 16);
      lo.y = (a2 & 0xffffu) | (a3 << 16);
      hi.x = (a0 >> 16) | (a1 & 0xffff0000u);
      hi.y = (a2 >> 16) | (a3 & 0xffff0000u);
      uint16_t* row = S + (rg * 8 + 2 * p) * (BK + kPad) + kg * 4;
      *reinterpret_cast<uint2*>(row) = lo;
      *reinterpret_cast<uint2*>(row + (BK + kPad)) = hi;
    }
  }
};

template <int ROWS, int BK, int NT, bool KCONTIG>
struct TileLoader;
template <int ROWS, int BK, int NT>
struct TileLoader<ROWS, BK, NT, true> : KTile<ROWS, BK, NT> {};
template <int ROWS, int BK, int NT>
struct TileLoader<ROWS, BK, NT, false> : RTile<ROWS, BK, NT> {};

// BK x ROWS tile of an operand contiguous along the row index (element
// (r, k) at P[k*ld + r0 + r]), copied as it is into LDS [BK][ROWS + 32]:
// whole 512-byte k-rows per 32 lanes from global memory, 16-byte LDS
// writes, and ds_read_b64_tr_b16 transposes on the way out (tr_frag).  The
// 32-element pad puts the four k-rows one transposing read touches in
// disjoint bank ranges.
template <int ROWS, int BK, int NT>
struct MTile {
  static constexpr int CPR = ROWS / 8;  // 16-byte chunks per k-row
  static constexpr int CPT = BK * CPR / NT;
  static constexpr int LROW = ROWS + 32;
  static_assert(CPT >= 1 && BK * CPR % NT == 0, "tile split");
  u32x4_t v[CPT];
  int32_t off[CPT];
  __device__ __forceinline__ void init(int64_t ld, int r0, int rows) {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = threadIdx.x + i * NT;
      const int k = c / CPR, r = (c % CPR) * 8;
      off[i] = r0 + r < rows ? (int32_t)(((int64_t)k * ld + r0 + r) * 2) : kOob;
    }
  }
  __device__ __forceinline__ void fetch(rsrc_t rs, int64_t ld, int k0) {
    const int32_t soff = (int32_t)((int64_t)k0 * ld * 2);
#pragma unroll
    for (int i = 0; i < CPT; ++i) v[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, off[i], soff, 0);
  }
  __device__ __forceinline__ void store(uint16_t* S) const {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = threadIdx.x + i * NT;
      *reinterpret_cast<u32x4_t*>(S + (c / CPR) * LROW + (c % CPR) * 8) = v[i];
    }
  }
  template <int P, int NP>
  __device__ __forceinline__ void cycle(uint16_t* S, rsrc_t rs, int64_t ld, int k0) {
    const int32_t soff = (int32_t)((int64_t)k0 * ld * 2);
#pragma unroll
    for (int i = P * CPT / NP; i < (P + 1) * CPT / NP; ++i) {
      const int c = threadIdx.x + i * NT;
      *reinterpret_cast<u32x4_t*>(S + (c / CPR) * LROW + (c % CPR) * 8) = v[i];
      v[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, off[i], soff, 0);
    }
  }
};
template <int ROWS, int BK, int NT, bool KCONTIG>
struct Tile256;
template <int ROWS, int BK, int NT>
struct Tile256<ROWS, BK, NT, true> : KTile<ROWS, BK, NT> {};
template <int ROWS, int BK, int NT>
struct Tile256<ROWS, BK, NT, false> : MTile<ROWS, BK, NT> {};

// Tile moved by direct global->LDS loads (buffer_load_dwordx4 ... lds):
// lane i of an instruction writes its 16 bytes at the wave's LDS base +
// 16 i, so the tile's LDS image is covered by consecutive 1 KB pieces,
// PER_WAVE of them per wave.
//  * KC (K-contiguous operand): [ROWS][BK] image without padding; the
//    16-byte unit p of row r holds k-chunk p ^ kc_swizzle(r) (the lane that
//    fills unit p loads that chunk), so the fragment reads -- 16 lanes on
//    16 consecutive rows, one chunk -- hit 16 distinct bank groups.
//  * otherwise (row-contiguous operand): [BK][ROWS + 32] image as it is in
//    memory; the padding units get an out-of-range offset (they read zeros).
typedef __attribute__((address_space(3))) void lds_void_t;
__device__ __forceinline__ void dma16(rsrc_t rs, uint16_t* lds, int32_t voff, int32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void_t*)lds, 16, voff, soff, 0, 0);
}
// injective on rows 0-7 and on the even and the odd rows of 0-15 (the rows
// one 128-byte and one 256-byte bank sweep of a fragment read cover), and
// periodic in 16 rows, so every 32-row fragment block shares it
__device__ __forceinline__ int kc_swizzle(int r) { return (r & 7) ^ ((r >> 3) & 1); }
template <int ROWS, int BK, bool KC>
struct DTile {
  static constexpr int UPR = KC ? BK / 8 : ROWS / 8 + 4;  // 16-byte units per LDS row
  static constexpr int DPR = KC ? BK / 8 : ROWS / 8;      // of which data
  static constexpr int NROW = KC ? ROWS : BK;
  static constexpr int PER_WAVE = NROW * UPR / 256;
  static constexpr int IMG = NROW * UPR * 8;  // image size in elements
  static_assert(NROW * UPR % 256 == 0, "tile split");
  static_assert(!KC || BK == 64, "the swizzle covers 8 chunks per row");
  int32_t off[PER_WAVE];
  int wave;
  __device__ __forceinline__ void init(int64_t ld, int r0, int rows) {
    wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int j = 0; j < PER_WAVE; ++j) {
      const int u = (wave * PER_WAVE + j) * 64 + lane;
      const int row = u / UPR, c = u % UPR;
      if (KC)
        off[j] = r0 + row < rows ? (int32_t)((((int64_t)(r0 + row)) * ld + (c ^ kc_swizzle(row)) * 8) * 2) : kOob;
      else if (c >= DPR)
        off[j] = kOob;
      else
        off[j] = r0 + c * 8 < rows ? (int32_t)(((int64_t)row * ld + r0 + c * 8) * 2) : kOob;
    }
  }
  // pieces [J0, J1) of k-tile k0 into the LDS image at S
  template <int J0, int J1>
  __device__ __forceinline__ void issue(uint16_t* S, rsrc_t rs, int64_t ld, int k0) {
    const int32_t soff = KC ? k0 * 2 : (int32_t)((int64_t)k0 * ld * 2);
#pragma unroll
    for (int j = J0; j < J1; ++j) dma16(rs, S + (wave * PER_WAVE + j) * 512, off[j], soff);
  }
};

typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4_t lds_s16x4_t;
// MFMA operand (8 consecutive k of one row) from a [k][row] LDS tile: two
// transposing reads of 4 k each.  Lane l must pass the address of k-row
// k0 + (l%16)/4 (k0 = 8*(l/32)), element row0 + 16*((l/16)%2) + 4*(l%4);
// it then receives rows row0 + l%32, k = k0 .. k0+7.
__device__ __forceinline__ uint4 tr_frag(const uint16_t* p, int lrow) {
  const u32x2_t lo = __builtin_bit_cast(u32x2_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)p));
  const u32x2_t hi =
      __builtin_bit_cast(u32x2_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(p + 4 * lrow)));
  return make_uint4(lo.x, lo.y, hi.x, hi.y);
}

// The same for the 16x16x32 layout: lane l passes the address of k-row
// k0 + (l%16)/4 (k0 = 8*(l/16)), element row0 + 4*(l%4); it receives row
// row0 + l%16, k = k0 .. k0+7.
__device__ __forceinline__ uint4 tr_frag16(const uint16_t* p, int lrow) { return tr_frag(p, lrow); }

struct GemmArgs {
  const uint16_t* A;
  const uint16_t* B;
  uint32_t a_bytes, b_bytes;  // extent of A / B for the buffer range checks
  void* C;
  const uint16_t* bias;
  int M, N, K;
  int64_t lda, ldb, ldc;
  int c_dtype;
  int flags;
  float alpha;
  uint32_t c_bytes;  // extent of C (the gemm256 kernels' store range)
  int k_split;              // split-K: k extent per split (0: one split of K)
  int64_t c_split_stride;   // split-K: elements between the splits' C slices
};

template <int BM, int BN, int BK, int WAVES_M, int WAVES_N, bool A_K, bool B_K, bool FP16>
__global__ void __launch_bounds__(64 * WAVES_M * WAVES_N) gemm_kernel(GemmArgs g) {
  constexpr int NT = 64 * WAVES_M * WAVES_N;
  constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int LDS_ROW = BK + kPad;
  __shared__ __attribute__((aligned(16))) uint16_t As[2][BM * LDS_ROW];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[2][BN * LDS_ROW];

  const int tiles_m = (g.M + BM - 1) / BM, tiles_n = (g.N + BN - 1) / BN;
  int tm, tn;
  tile_coords(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int wm = wid / WAVES_N, wn = wid % WAVES_N;
  const int lr = lane & 31, lk = (lane >> 5) * 8;

  f32x16_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  const int nk = (g.K + BK - 1) / BK;
  // MFMA over one LDS stage; operand fragments of k-step ks+1 are read from
  // LDS while the MFMAs of k-step ks run
  auto compute = [&](int st) {
    const uint16_t* as = As[st] + (wm * WM + lr) * LDS_ROW + lk;
    const uint16_t* bs = Bs[st] + (wn * WN + lr) * LDS_ROW + lk;
    uint4 af[2][TM], bfr[2][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i) af[0][i] = *reinterpret_cast<const uint4*>(as + i * 32 * LDS_ROW);
#pragma unroll
    for (int j = 0; j < TN; ++j) bfr[0][j] = *reinterpret_cast<const uint4*>(bs + j * 32 * LDS_ROW);
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      const int cur = ks & 1, nxt = cur ^ 1;
      if (ks + 1 < BK / 16) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
          af[nxt][i] = *reinterpret_cast<const uint4*>(as + i * 32 * LDS_ROW + (ks + 1) * 16);
#pragma unroll
        for (int j = 0; j < TN; ++j)
          bfr[nxt][j] = *reinterpret_cast<const uint4*>(bs + j * 32 * LDS_ROW + (ks + 1) * 16);
      }
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = mfma32<FP16>(af[cur][i], bfr[cur][j], acc[i][j]);
    }
  };

  const rsrc_t ra = make_rsrc(g.A, g.a_bytes), rb = make_rsrc(g.B, g.b_bytes);
  const bool kfull = g.K % BK == 0;
  TileLoader<BM, BK, NT, A_K> la;
  TileLoader<BN, BK, NT, B_K> lb;
  la.init(g.lda, m0, g.M);
  lb.init(g.ldb, n0, g.N);
  la.load(ra, g.lda, 0, g.K, kfull);
  lb.load(rb, g.ldb, 0, g.K, kfull);
  la.store(As[0]);
  lb.store(Bs[0]);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int st = kt & 1;
    const bool more = kt + 1 < nk;
    if (more) {
      la.load(ra, g.lda, (kt + 1) * BK, g.K, kfull);
      lb.load(rb, g.ldb, (kt + 1) * BK, g.K, kfull);
    }
    compute(st);
    if (more) {
      la.store(As[st ^ 1]);
      lb.store(Bs[st ^ 1]);
    }
    __syncthreads();
  }

  // epilogue: lane holds column n = lane%32 and rows (r/4)*8 + (lane/32)*4 + r%4
  const bool accumulate = g.flags & ETH_GEMM_ACCUMULATE;
  const bool has_bias = (g.flags & ETH_GEMM_BIAS) && g.bias;
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int n = n0 + wn * WN + j * 32 + lr;
    if (n >= g.N) continue;
    float bn = 0.f;
    if (has_bias) bn = FP16 ? h2f_bits(g.bias[n]) : bf2f(g.bias[n]);
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + wm * WM + i * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
        if (m >= g.M) continue;
        const float v = acc[i][j][r] * g.alpha + bn;
        const int64_t off = (int64_t)m * g.ldc + n;
        if (g.c_dtype == ETH_F32) {
          float* c = reinterpret_cast<float*>(g.C) + off;
          *c = accumulate ? *c + v : v;
        } else if (g.c_dtype == ETH_BF16) {
          reinterpret_cast<uint16_t*>(g.C)[off] = f2bf(v);
        } else {
          reinterpret_cast<uint16_t*>(g.C)[off] = f2h_bits(v);
        }
      }
    }
  }
}

// 256x256x64 tiles, 4 waves of 128x128 (one per SIMD), K % 128 == 0.
//
// MFMA v_mfma_f32_16x16x32: a 128x128 wave tile is 8 x 8 blocks of 16x16,
// 4 fp32 accumulators per lane each (256 in all, AGPRs).  A k-tile of 64 is
// two k-steps of 32; a k-step is 64 MFMAs, preceded by the 16 fragment reads
// (8 A row blocks, 8 B column blocks) that feed it.  The 16x16x32 shape
// (twice the MFMA instructions of 32x32x16 for the same work) leaves more
// issue gaps between MFMAs for the fragment reads and direct loads: the same
// tile with 32x32x16 MFMAs ran 6% slower.
template <bool FP16>
__device__ __forceinline__ f32x4_t mfma16(const uint4& a, const uint4& b, const f32x4_t& c) {
  if constexpr (FP16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b),
                                                  c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  }
}

// The same MFMA as inline assembly with the accumulator tied to its AGPRs
// ("+a"), for the kernel whose operands both come through transposing
// reads: through the builtin the register allocator there keeps some 30
// accumulator tuples in VGPRs and copies them around the MFMAs every k-tile.
// The compiler still inserts the LDS waits for the operands (it sees the
// asm's register uses); the only hazard it cannot see, an accumulator read
// right after its MFMA, is covered after the k loop.
template <bool FP16>
__device__ __forceinline__ void mfma16_asm(f32x4_t& c, const uint4& a, const uint4& b) {
  if constexpr (FP16)
    asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0"
                 : "+a"(c)
                 : "v"(__builtin_bit_cast(u32x4_t, a)), "v"(__builtin_bit_cast(u32x4_t, b)));
  else
    asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0"
                 : "+a"(c)
                 : "v"(__builtin_bit_cast(u32x4_t, a)), "v"(__builtin_bit_cast(u32x4_t, b)));
}

template <bool A_K, bool B_K, bool FP16>
__global__ void __launch_bounds__(256, 1) gemm256_m16_kernel(GemmArgs g) {
  constexpr int BM = 256, BN = 256, BK = 64;
  typedef DTile<BM, BK, A_K> ATile;
  typedef DTile<BN, BK, B_K> BTile;
  constexpr int A_IMG = ATile::IMG;           // elements of the A image in a stage
  constexpr int STAGE = A_IMG + BTile::IMG;   // one LDS stage: A image then B image
  constexpr int ER = 128 + 4;                 // epilogue staging row (fp32, padded)
  constexpr int EPI = 4 * 32 * ER * 2;        // epilogue staging in elements
  // the two stages are separate arrays, so the compiler can tell the direct
  // loads into one stage from the fragment reads of the other (it would
  // otherwise wait for the loads before every read); the first also holds
  // the epilogue's staging
  __shared__ __attribute__((aligned(16))) uint16_t smem[STAGE > EPI ? STAGE : EPI];
  __shared__ __attribute__((aligned(16))) uint16_t smem1[STAGE];

  const int tiles_m = (g.M + BM - 1) / BM, tiles_n = (g.N + BN - 1) / BN;
  // split-K launches tiles * splits workgroups: split = blockIdx.x / tiles
  const int tiles = tiles_m * tiles_n;
  const int split = blockIdx.x / tiles;
  const int kb = split * g.k_split;
  int tm, tn;
  tile_coords(blockIdx.x - split * tiles, tiles_m, tiles_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int wm = wid >> 1, wn = wid & 1;
  const int l16 = lane & 15, lg = lane >> 4;
  // the 4 output columns this lane writes in the epilogue, and their bias
  // (read now so its latency is hidden behind the k loop)
  const int col = (lane & 31) * 4;
  const int n = n0 + wn * 128 + col;
  float bn[4] = {0.f, 0.f, 0.f, 0.f};
  if ((g.flags & ETH_GEMM_BIAS) && g.bias) {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (n + e < g.N) bn[e] = FP16 ? h2f_bits(g.bias[n + e]) : bf2f(g.bias[n + e]);
  }

  // acc[I][J]: C rows I*16 + lane%16, columns J*16 + 4*(lane/16) + 0..3 of
  // the wave's block (B fragment as the MFMA's first operand)
  f32x4_t acc[8][8];
  // pinned to AGPRs where they start, so the register allocator keeps each
  // block in one AGPR tuple and every MFMA accumulates in place (unpinned,
  // it parks some blocks in VGPRs and copies them around the MFMAs)
#define PIN_ACC                                          \
  _Pragma("unroll") for (int i = 0; i < 8; ++i)          \
    _Pragma("unroll") for (int j = 0; j < 8; ++j) asm volatile("" : "+a"(acc[i][j]));
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  PIN_ACC

  const int nk = (g.k_split ? g.k_split : g.K) / BK;
  const rsrc_t ra = make_rsrc(g.A, g.a_bytes), rb = make_rsrc(g.B, g.b_bytes);
  // empty ranges: the loads issued past the last k-tile read zeros
  const rsrc_t ra0 = make_rsrc(g.A, 0), rb0 = make_rsrc(g.B, 0);
  ATile la;
  BTile lb;
  // pieces per half per wave: 8 for a K-contiguous image, 9 for a padded one
  constexpr int NA = ATile::PER_WAVE, NB = BTile::PER_WAVE;
  static_assert((NA == 8 || NA == 9) && (NB == 8 || NB == 9), "the k loop's load slots");
  la.init(g.lda, m0, g.M);
  lb.init(g.ldb, n0, g.N);
  la.template issue<0, NA>(smem, ra, g.lda, kb);
  lb.template issue<0, NB>(smem + A_IMG, rb, g.ldb, kb);

  // queue item Q of a k-tile (the A pieces, then the B pieces) into stage S
#define LOAD_Q(Q, S, RSA, RSB, KK)                                      \
  if constexpr ((Q) < NA) {                                             \
    la.template issue<(Q), (Q) + 1>(S, RSA, g.lda, KK);                 \
  } else if constexpr ((Q) < NA + NB) {                                 \
    lb.template issue<(Q) - NA, (Q) - NA + 1>((S) + A_IMG, RSB, g.ldb, KK); \
  }
  // queue items 0-11 of k-tile 1 (the loop's first k-step issues the rest)
  {
    const rsrc_t rsa = nk > 1 ? ra : ra0, rsb = nk > 1 ? rb : rb0;
#define PRO_Q(Q) LOAD_Q(Q, smem1, rsa, rsb, kb + BK)
    PRO_Q(0) PRO_Q(1) PRO_Q(2) PRO_Q(3) PRO_Q(4) PRO_Q(5)
    PRO_Q(6) PRO_Q(7) PRO_Q(8) PRO_Q(9) PRO_Q(10) PRO_Q(11)
#undef PRO_Q
  }
  dma_barrier_but<12>();

  // Fragment of row block I (16 rows) for k-step KS (32 k): lane l holds row
  // l%16, k 8*(l/16) .. +7.
  // K-contiguous images ([row][64], swizzled): one 16-byte read; the unit of
  // k-chunk 4 KS + l/16 depends on KS through the swizzle, so each k-step has
  // its own lane offset, and row block I is a constant 16 rows further (the
  // swizzle has period 16).
  // Row-contiguous images ([64][256 + 32]): two transposing reads of 4 k.
  constexpr int LM = BM + 32;
  int a_frag[2], b_frag[2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    const int trl = (32 * ks + 8 * lg + (l16 >> 2)) * LM + (l16 & 3) * 4;
    const int kc = ((4 * ks + lg) ^ kc_swizzle(l16)) * 8;
    a_frag[ks] = A_K ? (wm * 128 + l16) * BK + kc : trl + wm * 128;
    b_frag[ks] = A_IMG + (B_K ? (wn * 128 + l16) * BK + kc : trl + wn * 128);
  }
  // One set of fragments, each re-read as soon as its last MFMA of the
  // k-step has issued.  A k-step's 64 MFMAs run the (row block, column
  // block) pairs column-major, first over row blocks 0-3, then over 4-7:
  //  * A0-A3 die at MFMA 31 and are re-read (next k-step) right after it;
  //  * Bj dies at MFMA 35 + 4j (row block 7) and is re-read right after it,
  //    29 MFMAs before the next k-step's first use (MFMA 4j);
  //  * A4-A7 die at MFMA 63 and are read in the next k-step's first four
  //    gaps, 28 MFMAs before their first use (MFMA 32).
  // The barrier comes 12 MFMAs into the second k-step of a k-tile, after
  // that k-step's own A4-A7 reads from the stage; then direct loads, one
  // every fourth MFMA gap, refill the stage with k-tile t+2 (12 pieces in
  // this k-step, the other 4-6 in the next).
  uint4 fa[8], fb[8];
#define SB __builtin_amdgcn_sched_barrier(0);
#define RD_A(BASE, KS, I)                                                             \
  fa[I] = A_K ? *reinterpret_cast<const uint4*>((BASE) + a_frag[KS] + (I) * 16 * BK) \
              : tr_frag((BASE) + a_frag[KS] + (I) * 16, LM);
#define RD_B(BASE, KS, J)                                                             \
  fb[J] = B_K ? *reinterpret_cast<const uint4*>((BASE) + b_frag[KS] + (J) * 16 * BK) \
              : tr_frag((BASE) + b_frag[KS] + (J) * 16, LM);
#define MM(I, J)                                  \
  if constexpr (A_K)                              \
    acc[I][J] = mfma16<FP16>(fb[J], fa[I], acc[I][J]); \
  else                                            \
    mfma16_asm<FP16>(acc[I][J], fb[J], fa[I]);
  // items 0-11 of k-tile t+2 in the barrier k-step of k-tile t, the rest
  // in the first k-step of k-tile t+1
#define LOAD_CUR(Q) LOAD_Q(Q, cur, rsa2, rsb2, k2)
#define LOAD_NXT(Q) LOAD_Q(Q, nxt, rsa1, rsb1, k1)
#define KSTEP_A(OB, OK, NB, NK)    \
  SB MM(0, 0) SB RD_A(OB, OK, 4) SB MM(1, 0) SB RD_A(OB, OK, 5) SB MM(2, 0) SB RD_A(OB, OK, 6) SB    \
  LOAD_NXT(12) SB MM(3, 0) SB RD_A(OB, OK, 7) SB MM(0, 1) SB MM(1, 1) SB MM(2, 1) SB LOAD_NXT(13) SB \
  MM(3, 1) SB MM(0, 2) SB MM(1, 2) SB MM(2, 2) SB LOAD_NXT(14) SB MM(3, 2) SB MM(0, 3) SB            \
  MM(1, 3) SB MM(2, 3) SB LOAD_NXT(15) SB MM(3, 3) SB MM(0, 4) SB MM(1, 4) SB MM(2, 4) SB            \
  LOAD_NXT(16) SB MM(3, 4) SB MM(0, 5) SB MM(1, 5) SB MM(2, 5) SB LOAD_NXT(17) SB MM(3, 5) SB        \
  MM(0, 6) SB MM(1, 6) SB MM(2, 6) SB MM(3, 6) SB MM(0, 7) SB MM(1, 7) SB MM(2, 7) SB MM(3, 7) SB    \
  MM(4, 0) SB RD_A(NB, NK, 0) SB MM(5, 0) SB RD_A(NB, NK, 1) SB MM(6, 0) SB RD_A(NB, NK, 2) SB       \
  MM(7, 0) SB RD_B(NB, NK, 0) SB MM(4, 1) SB RD_A(NB, NK, 3) SB MM(5, 1) SB MM(6, 1) SB MM(7, 1) SB  \
  RD_B(NB, NK, 1) SB MM(4, 2) SB MM(5, 2) SB MM(6, 2) SB MM(7, 2) SB RD_B(NB, NK, 2) SB MM(4, 3) SB  \
  MM(5, 3) SB MM(6, 3) SB MM(7, 3) SB RD_B(NB, NK, 3) SB MM(4, 4) SB MM(5, 4) SB MM(6, 4) SB         \
  MM(7, 4) SB RD_B(NB, NK, 4) SB MM(4, 5) SB MM(5, 5) SB MM(6, 5) SB MM(7, 5) SB RD_B(NB, NK, 5) SB  \
  MM(4, 6) SB MM(5, 6) SB MM(6, 6) SB MM(7, 6) SB RD_B(NB, NK, 6) SB MM(4, 7) SB MM(5, 7) SB         \
  MM(6, 7) SB MM(7, 7) SB RD_B(NB, NK, 7) SB
#define KSTEP_B(OB, OK, NB, NK)    \
  SB MM(0, 0) SB RD_A(OB, OK, 4) SB MM(1, 0) SB RD_A(OB, OK, 5) SB MM(2, 0) SB RD_A(OB, OK, 6) SB    \
  MM(3, 0) SB RD_A(OB, OK, 7) SB MM(0, 1) SB MM(1, 1) SB MM(2, 1) SB MM(3, 1) SB MM(0, 2) SB         \
  MM(1, 2) SB MM(2, 2) SB MM(3, 2) SB dma_barrier(); SB MM(0, 3) SB LOAD_CUR(0) SB MM(1, 3) SB       \
  MM(2, 3) SB MM(3, 3) SB MM(0, 4) SB LOAD_CUR(1) SB MM(1, 4) SB MM(2, 4) SB MM(3, 4) SB MM(0, 5) SB \
  LOAD_CUR(2) SB MM(1, 5) SB MM(2, 5) SB MM(3, 5) SB MM(0, 6) SB LOAD_CUR(3) SB MM(1, 6) SB          \
  MM(2, 6) SB MM(3, 6) SB MM(0, 7) SB LOAD_CUR(4) SB MM(1, 7) SB MM(2, 7) SB MM(3, 7) SB MM(4, 0) SB \
  LOAD_CUR(5) SB RD_A(NB, NK, 0) SB MM(5, 0) SB RD_A(NB, NK, 1) SB MM(6, 0) SB RD_A(NB, NK, 2) SB    \
  MM(7, 0) SB RD_B(NB, NK, 0) SB MM(4, 1) SB LOAD_CUR(6) SB RD_A(NB, NK, 3) SB MM(5, 1) SB           \
  MM(6, 1) SB MM(7, 1) SB RD_B(NB, NK, 1) SB MM(4, 2) SB LOAD_CUR(7) SB MM(5, 2) SB MM(6, 2) SB      \
  MM(7, 2) SB RD_B(NB, NK, 2) SB MM(4, 3) SB LOAD_CUR(8) SB MM(5, 3) SB MM(6, 3) SB MM(7, 3) SB      \
  RD_B(NB, NK, 3) SB MM(4, 4) SB LOAD_CUR(9) SB MM(5, 4) SB MM(6, 4) SB MM(7, 4) SB                  \
  RD_B(NB, NK, 4) SB MM(4, 5) SB LOAD_CUR(10) SB MM(5, 5) SB MM(6, 5) SB MM(7, 5) SB                 \
  RD_B(NB, NK, 5) SB MM(4, 6) SB LOAD_CUR(11) SB MM(5, 6) SB MM(6, 6) SB MM(7, 6) SB                 \
  RD_B(NB, NK, 6) SB MM(4, 7) SB MM(5, 7) SB MM(6, 7) SB MM(7, 7) SB RD_B(NB, NK, 7) SB

#define ITER(CUR, NXT, KT)                                \
  {                                                       \
    uint16_t* const cur = (CUR);                          \
    uint16_t* const nxt = (NXT);                          \
    const int k1 = kb + ((KT) + 1) * BK;                  \
    const int k2 = kb + ((KT) + 2) * BK;                  \
    const rsrc_t rsa1 = (KT) + 1 < nk ? ra : ra0;         \
    const rsrc_t rsb1 = (KT) + 1 < nk ? rb : rb0;         \
    const rsrc_t rsa2 = (KT) + 2 < nk ? ra : ra0;         \
    const rsrc_t rsb2 = (KT) + 2 < nk ? rb : rb0;         \
    KSTEP_A(cur, 0, cur, 1)                               \
    KSTEP_B(cur, 1, nxt, 0)                               \
  }
  SB RD_A(smem, 0, 0) SB RD_A(smem, 0, 1) SB RD_A(smem, 0, 2) SB RD_A(smem, 0, 3) SB
#pragma unroll
  for (int j = 0; j < 8; ++j) { RD_B(smem, 0, j) }
  SB
  // two k-tiles per trip, so both LDS stages have fixed addresses
  for (int kt = 0; kt < nk; kt += 2) {
    ITER(smem, smem1, kt)
    ITER(smem1, smem, kt + 1)
  }
  // asm MFMAs: wait states before any instruction reads their accumulators
  if constexpr (!A_K) asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
#undef PIN_ACC
#undef ITER
#undef KSTEP_A
#undef KSTEP_B
#undef LOAD_Q
#undef LOAD_CUR
#undef LOAD_NXT
#undef MM
#undef RD_A
#undef RD_B
#undef SB

  // Epilogue: each wave stages one 32-row slab of its 128x128 block at a
  // time in its own LDS region (fp32, padded rows) and writes it back as
  // whole rows, two rows per store instruction.  C goes through a buffer
  // resource spanning exactly its extent, so rows past M are dropped by the
  // hardware; lanes whose columns are past N get an out-of-range offset.
  float* stage = reinterpret_cast<float*>(smem) + wid * 32 * ER;
  const int esz = g.c_dtype == ETH_F32 ? 4 : 2;
  const int mode = g.c_dtype == ETH_BF16 ? 0 : g.c_dtype == ETH_F16 ? 1 : (g.flags & ETH_GEMM_ACCUMULATE) ? 3 : 2;
  const rsrc_t rc = make_rsrc(reinterpret_cast<float*>(g.C) + split * g.c_split_stride, g.c_bytes);
  const int32_t row2 = (int32_t)(2 * g.ldc * esz);
  auto write_slab = [&](const int i) __attribute__((always_inline)) {
    // the slab is private to this wave, whose LDS accesses complete in order
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    float4 v[16];
#pragma unroll
    for (int it = 0; it < 16; ++it) {
      v[it] = *reinterpret_cast<const float4*>(stage + (it * 2 + (lane >> 5)) * ER + col);
      v[it].x = v[it].x * g.alpha + bn[0];
      v[it].y = v[it].y * g.alpha + bn[1];
      v[it].z = v[it].z * g.alpha + bn[2];
      v[it].w = v[it].w * g.alpha + bn[3];
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    const int mrow = m0 + wm * 128 + i * 32 + (lane >> 5);
    const int32_t voff = n < g.N ? (int32_t)(((int64_t)mrow * g.ldc + n) * esz) : kOob;
#define OFF(IT) (voff == kOob ? kOob : voff + (IT) * row2)
    if (mode == 0) {
#pragma unroll
      for (int it = 0; it < 16; ++it) {
        u32x2_t o;
        o.x = f2bf_pair(v[it].x, v[it].y);
        o.y = f2bf_pair(v[it].z, v[it].w);
        __builtin_amdgcn_raw_buffer_store_b64(o, rc, OFF(it), 0, 0);
      }
    } else if (mode == 1) {
#pragma unroll
      for (int it = 0; it < 16; ++it) {
        u32x2_t o;
        o.x = f2h_bits(v[it].x) | ((uint32_t)f2h_bits(v[it].y) << 16);
        o.y = f2h_bits(v[it].z) | ((uint32_t)f2h_bits(v[it].w) << 16);
        __builtin_amdgcn_raw_buffer_store_b64(o, rc, OFF(it), 0, 0);
      }
    } else if (mode == 2) {
#pragma unroll
      for (int it = 0; it < 16; ++it)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, v[it]), rc, OFF(it), 0, 0);
    } else {
      // fp32 C += (the main_grad accumulation): all loads first
      u32x4_t old[16];
#pragma unroll
      for (int it = 0; it < 16; ++it) old[it] = __builtin_amdgcn_raw_buffer_load_b128(rc, OFF(it), 0, 0);
#pragma unroll
      for (int it = 0; it < 16; ++it) {
        float4 o = __builtin_bit_cast(float4, old[it]);
        o.x += v[it].x;
        o.y += v[it].y;
        o.z += v[it].z;
        o.w += v[it].w;
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, o), rc, OFF(it), 0, 0);
      }
    }
#undef OFF
  };
  dma_barrier();  // every wave is done with the k-loop stages, no load in flight
  // slab S: row blocks 2S, 2S+1 -> staging rows (I % 2) * 16 + lane % 16
#define STAGE_SLAB(S)                                                                     \
  {                                                                                       \
    _Pragma("unroll") for (int h = 0; h < 2; ++h)                                         \
      _Pragma("unroll") for (int j = 0; j < 8; ++j) {                                     \
        const f32x4_t a = acc[2 * (S) + h][j];                                            \
        *reinterpret_cast<float4*>(stage + (h * 16 + l16) * ER + j * 16 + lg * 4) =      \
            make_float4(a[0], a[1], a[2], a[3]);                                          \
      }                                                                                   \
    write_slab(S);                                                                        \
  }
  STAGE_SLAB(0) STAGE_SLAB(1) STAGE_SLAB(2) STAGE_SLAB(3)
#undef STAGE_SLAB
}

// The same tiles with v_mfma_f32_32x32x16 (4 x 4 blocks of 32x32 per wave,
// 16 accumulators per lane each), for a row-contiguous A: with transposing
// reads on both operands the 16x16x32 kernel does not keep its accumulators
// in place in AGPRs (the register allocator moves them around every MFMA).
template <bool A_K, bool B_K, bool FP16>
__global__ void __launch_bounds__(256, 1) gemm256_m32_kernel(GemmArgs g) {
  constexpr int BM = 256, BN = 256, BK = 64;
  typedef DTile<BM, BK, A_K> ATile;
  typedef DTile<BN, BK, B_K> BTile;
  constexpr int A_IMG = ATile::IMG;           // elements of the A image in a stage
  constexpr int STAGE = A_IMG + BTile::IMG;   // one LDS stage: A image then B image
  constexpr int ER = 128 + 4;                 // epilogue staging row (fp32, padded)
  constexpr int EPI = 4 * 32 * ER * 2;        // epilogue staging in elements
  // the two stages are separate arrays, so the compiler can tell the direct
  // loads into one stage from the fragment reads of the other (it would
  // otherwise wait for the loads before every read); the first also holds
  // the epilogue's staging
  __shared__ __attribute__((aligned(16))) uint16_t smem[STAGE > EPI ? STAGE : EPI];
  __shared__ __attribute__((aligned(16))) uint16_t smem1[STAGE];

  const int tiles_m = (g.M + BM - 1) / BM, tiles_n = (g.N + BN - 1) / BN;
  // split-K launches tiles * splits workgroups: split = blockIdx.x / tiles
  const int tiles = tiles_m * tiles_n;
  const int split = blockIdx.x / tiles;
  const int kb = split * g.k_split;
  int tm, tn;
  tile_coords(blockIdx.x - split * tiles, tiles_m, tiles_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int wm = wid >> 1, wn = wid & 1;
  const int lr = lane & 31, lk = (lane >> 5) * 8;
  // the 4 output columns this lane writes in the epilogue, and their bias
  // (read now so its latency is hidden behind the k loop)
  const int col = (lane & 31) * 4;
  const int n = n0 + wn * 128 + col;
  float bn[4] = {0.f, 0.f, 0.f, 0.f};
  if ((g.flags & ETH_GEMM_BIAS) && g.bias) {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (n + e < g.N) bn[e] = FP16 ? h2f_bits(g.bias[n + e]) : bf2f(g.bias[n + e]);
  }

  f32x16_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  const int nk = (g.k_split ? g.k_split : g.K) / BK;
  const rsrc_t ra = make_rsrc(g.A, g.a_bytes), rb = make_rsrc(g.B, g.b_bytes);
  // empty ranges: the loads issued past the last k-tile read zeros
  const rsrc_t ra0 = make_rsrc(g.A, 0), rb0 = make_rsrc(g.B, 0);
  ATile la;
  BTile lb;
  // pieces per half per wave: 8 for a K-contiguous image, 9 for a padded one
  constexpr int NA = ATile::PER_WAVE, NB = BTile::PER_WAVE;
  static_assert((NA == 8 || NA == 9) && (NB == 8 || NB == 9), "the k loop's load slots");
  la.init(g.lda, m0, g.M);
  lb.init(g.ldb, n0, g.N);
  la.template issue<0, NA>(smem, ra, g.lda, kb);
  lb.template issue<0, NB>(smem + A_IMG, rb, g.ldb, kb);
  // A pieces 0-7 of k-tile 1; the loop's first k-step issues a piece 8
  la.template issue<0, 8>(smem1, nk > 1 ? ra : ra0, g.lda, kb + BK);
  dma_barrier_but<8>();

  // fragment of (row block I, k-step KS): lanes 0-31 hold rows, lanes 32-63
  // the second 8 k of the 16
  // K-contiguous tiles: [row][64] swizzled, one 16-byte read per fragment
  // (the unit of k-chunk 2 KS + lane / 32 depends on KS through the
  // swizzle, so each k-step has its own lane offset; row block I is a
  // constant 32 rows further, with the same swizzle);
  // row-contiguous tiles: [BK][256 + 32], two transposing reads (tr_frag)
  constexpr int LM = BM + 32;
  const int trl = ((lane >> 5) * 8 + ((lane & 15) >> 2)) * LM + ((lane >> 4) & 1) * 16 + (lane & 3) * 4;
  int a_frag[4], b_frag[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    const int ra_ = wm * 128 + lr, rb_ = wn * 128 + lr;
    a_frag[ks] = A_K ? ra_ * BK + ((2 * ks + (lane >> 5)) ^ kc_swizzle(ra_)) * 8 : trl + wm * 128 + ks * 16 * LM;
    b_frag[ks] = A_IMG + (B_K ? rb_ * BK + ((2 * ks + (lane >> 5)) ^ kc_swizzle(rb_)) * 8 : trl + wn * 128 + ks * 16 * LM);
  }
  uint4 fa0[4], fb0[4], fa1[4], fb1[4];
#define SB __builtin_amdgcn_sched_barrier(0);
#define RD_A(FA, BASE, KS, I)                                                         \
  FA[I] = A_K ? *reinterpret_cast<const uint4*>((BASE) + a_frag[KS] + (I) * 32 * BK) \
              : tr_frag((BASE) + a_frag[KS] + (I) * 32, LM);
#define RD_B(FB, BASE, KS, J)                                                         \
  FB[J] = B_K ? *reinterpret_cast<const uint4*>((BASE) + b_frag[KS] + (J) * 32 * BK) \
              : tr_frag((BASE) + b_frag[KS] + (J) * 32, LM);
// B fragment as the MFMA's first operand: the lane then holds 4 consecutive
// output columns (r % 4) of one output row (lane % 32)
#define MMA2(FA, FB, I, J0)                                         \
  acc[I][J0] = mfma32<FP16>(FB[J0], FA[I], acc[I][J0]);             \
  acc[I][J0 + 1] = mfma32<FP16>(FB[J0 + 1], FA[I], acc[I][J0 + 1]);
// next k-step's fragments in the order its MFMA pairs consume them:
// B0 B1 A0 B2 B3 A1 A2 A3
#define RD_SEQ0(GA, GB, RB, RK) RD_B(GB, RB, RK, 0)
#define RD_SEQ1(GA, GB, RB, RK) RD_B(GB, RB, RK, 1)
#define RD_SEQ2(GA, GB, RB, RK) RD_A(GA, RB, RK, 0)
#define RD_SEQ3(GA, GB, RB, RK) RD_B(GB, RB, RK, 2)
#define RD_SEQ4(GA, GB, RB, RK) RD_B(GB, RB, RK, 3)
#define RD_SEQ5(GA, GB, RB, RK) RD_A(GA, RB, RK, 1)
#define RD_SEQ6(GA, GB, RB, RK) RD_A(GA, RB, RK, 2)
#define RD_SEQ7(GA, GB, RB, RK) RD_A(GA, RB, RK, 3)
#define MMA1(FA, FB, I, J) acc[I][J] = mfma32<FP16>(FB[J], FA[I], acc[I][J]);
// one row block of a k-step: 4 MFMAs, with two fragment reads of the next
// k-step into (GA, GB) and two direct-load slots of a tile cycle between them
#define KSTEP_ROW(FA, FB, GA, GB, RB, RK, I, S0, S1, CYC)                                        \
  SB MMA1(FA, FB, I, 0) SB S0(GA, GB, RB, RK) SB MMA1(FA, FB, I, 1) SB CYC(2 * (I)) SB MMA1(FA, FB, I, 2) \
  SB S1(GA, GB, RB, RK) SB MMA1(FA, FB, I, 3) SB CYC(2 * (I) + 1) SB
#define NOCYC(P)
// direct-load slot S (0-7) of a k-step issues one 1 KB piece: pieces 0-7
// of the A half of k-tile t+2 in the k-step after the barrier, then, one
// per slot over the next k-step and a half, the rest of k-tile t+2 (queue
// position Q: A piece 8 first when the A image has 9 pieces, then the B
// pieces) -- one load per slot, so no slot stalls the MFMA issue on a burst
// of loads (measured 3% faster than two bursts of 9)
#define CYC_A(S) la.template issue<(S), (S) + 1>(cur, rsa, g.lda, k2);
#define LOAD_Q(Q)                                                                            \
  if constexpr (NA == 9 && (Q) == 0)                                                         \
    la.template issue<8, 9>(nxt, rsa1, g.lda, k1);                                           \
  else if constexpr ((Q) - (NA - 8) < NB)                                                    \
    lb.template issue<(Q) - (NA - 8), (Q) - (NA - 8) + 1>(nxt + A_IMG, rsb, g.ldb, k1);
#define CYC_AB(S) LOAD_Q(S)
#define CYC_B2(S) LOAD_Q((S) + 8)
#define KSTEP(FA, FB, GA, GB, RB, RK, CYC)                     \
  KSTEP_ROW(FA, FB, GA, GB, RB, RK, 0, RD_SEQ0, RD_SEQ1, CYC) \
  KSTEP_ROW(FA, FB, GA, GB, RB, RK, 1, RD_SEQ2, RD_SEQ3, CYC) \
  KSTEP_ROW(FA, FB, GA, GB, RB, RK, 2, RD_SEQ4, RD_SEQ5, CYC) \
  KSTEP_ROW(FA, FB, GA, GB, RB, RK, 3, RD_SEQ6, RD_SEQ7, CYC) SB
// k-tile KT: k-steps 0-2 from stage CUR while the rest of k-tile KT+1 is
// loaded into NXT (most of its A half was started one k-step earlier); the
// barrier (after this wave's direct loads have landed) means every wave is
// done reading CUR and KT+1 is complete in NXT; k-step 3 then computes from
// registers, reads the first fragments of KT+1 from NXT and starts the A
// half of k-tile KT+2 into CUR
#define ITER(CUR, NXT, KT)                              \
  {                                                     \
    uint16_t* const cur = (CUR);                        \
    uint16_t* const nxt = (NXT);                        \
    const int k1 = kb + ((KT) + 1) * BK;                \
    const int k2 = kb + ((KT) + 2) * BK;                \
    const rsrc_t rsb = (KT) + 1 < nk ? rb : rb0;        \
    const rsrc_t rsa = (KT) + 2 < nk ? ra : ra0;        \
    const rsrc_t rsa1 = (KT) + 1 < nk ? ra : ra0;       \
    KSTEP(fa0, fb0, fa1, fb1, cur, 1, CYC_AB)           \
    KSTEP(fa1, fb1, fa0, fb0, cur, 2, CYC_B2)           \
    KSTEP(fa0, fb0, fa1, fb1, cur, 3, NOCYC)            \
    dma_barrier();                                      \
    KSTEP(fa1, fb1, fa0, fb0, nxt, 0, CYC_A)            \
  }
  SB RD_SEQ0(fa0, fb0, smem, 0) SB RD_SEQ1(fa0, fb0, smem, 0) SB RD_SEQ2(fa0, fb0, smem, 0) SB
  RD_SEQ3(fa0, fb0, smem, 0) SB RD_SEQ4(fa0, fb0, smem, 0) SB RD_SEQ5(fa0, fb0, smem, 0) SB
  RD_SEQ6(fa0, fb0, smem, 0) SB RD_SEQ7(fa0, fb0, smem, 0) SB
  // two k-tiles per trip, so both LDS stages have fixed addresses
  for (int kt = 0; kt < nk; kt += 2) {
    ITER(smem, smem1, kt)
    ITER(smem1, smem, kt + 1)
  }
#undef ITER
#undef KSTEP
#undef CYC_A
#undef CYC_AB
#undef CYC_B2
#undef LOAD_Q
#undef MMA1
#undef NOCYC
#undef KSTEP_ROW
#undef RD_SEQ0
#undef RD_SEQ1
#undef RD_SEQ2
#undef RD_SEQ3
#undef RD_SEQ4
#undef RD_SEQ5
#undef RD_SEQ6
#undef RD_SEQ7
#undef MMA2
#undef RD_A
#undef RD_B
#undef SB

  // Epilogue: each wave stages one 32-row slab of its 128x128 block at a
  // time in its own LDS region (fp32, padded rows) and writes it back as
  // whole rows, two rows per store instruction.  C goes through a buffer
  // resource spanning exactly its extent, so rows past M are dropped by the
  // hardware; lanes whose columns are past N get an out-of-range offset.
  float* stage = reinterpret_cast<float*>(smem) + wid * 32 * ER;
  const int esz = g.c_dtype == ETH_F32 ? 4 : 2;
  const int mode = g.c_dtype == ETH_BF16 ? 0 : g.c_dtype == ETH_F16 ? 1 : (g.flags & ETH_GEMM_ACCUMULATE) ? 3 : 2;
  const rsrc_t rc = make_rsrc(reinterpret_cast<float*>(g.C) + split * g.c_split_stride, g.c_bytes);
  const int32_t row2 = (int32_t)(2 * g.ldc * esz);
  auto write_slab = [&](const int i) __attribute__((always_inline)) {
    // the slab is private to this wave, whose LDS accesses complete in order
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    float4 v[16];
#pragma unroll
    for (int it = 0; it < 16; ++it) {
      v[it] = *reinterpret_cast<const float4*>(stage + (it * 2 + (lane >> 5)) * ER + col);
      v[it].x = v[it].x * g.alpha + bn[0];
      v[it].y = v[it].y * g.alpha + bn[1];
      v[it].z = v[it].z * g.alpha + bn[2];
      v[it].w = v[it].w * g.alpha + bn[3];
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    const int mrow = m0 + wm * 128 + i * 32 + (lane >> 5);
    const int32_t voff = n < g.N ? (int32_t)(((int64_t)mrow * g.ldc + n) * esz) : kOob;
#define OFF(IT) (voff == kOob ? kOob : voff + (IT) * row2)
    if (mode == 0) {
#pragma unroll
      for (int it = 0; it < 16; ++it) {
        u32x2_t o;
        o.x = f2bf_pair(v[it].x, v[it].y);
        o.y = f2bf_pair(v[it].z, v[it].w);
        __builtin_amdgcn_raw_buffer_store_b64(o, rc, OFF(it), 0, 0);
      }
    } else if (mode == 1) {
#pragma unroll
      for (int it = 0; it < 16; ++it) {
        u32x2_t o;
        o.x = f2h_bits(v[it].x) | ((uint32_t)f2h_bits(v[it].y) << 16);
        o.y = f2h_bits(v[it].z) | ((uint32_t)f2h_bits(v[it].w) << 16);
        __builtin_amdgcn_raw_buffer_store_b64(o, rc, OFF(it), 0, 0);
      }
    } else if (mode == 2) {
#pragma unroll
      for (int it = 0; it < 16; ++it)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, v[it]), rc, OFF(it), 0, 0);
    } else {
      // fp32 C += (the main_grad accumulation): all loads first
      u32x4_t old[16];
#pragma unroll
      for (int it = 0; it < 16; ++it) old[it] = __builtin_amdgcn_raw_buffer_load_b128(rc, OFF(it), 0, 0);
#pragma unroll
      for (int it = 0; it < 16; ++it) {
        float4 o = __builtin_bit_cast(float4, old[it]);
        o.x += v[it].x;
        o.y += v[it].y;
        o.z += v[it].z;
        o.w += v[it].w;
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, o), rc, OFF(it), 0, 0);
      }
    }
#undef OFF
  };
  dma_barrier();  // every wave is done with the k-loop stages, no load in flight
#define STAGE_SLAB(I)                                                                  \
  {                                                                                    \
    _Pragma("unroll") for (int j = 0; j < 4; ++j)                                      \
      _Pragma("unroll") for (int q = 0; q < 4; ++q) {                                  \
        const float4 o = make_float4(acc[I][j][q * 4 + 0], acc[I][j][q * 4 + 1],       \
                                     acc[I][j][q * 4 + 2], acc[I][j][q * 4 + 3]);      \
        *reinterpret_cast<float4*>(stage + lr * ER + j * 32 + q * 8 + (lane >> 5) * 4) = o; \
      }                                                                                \
    write_slab(I);                                                                     \
  }
  STAGE_SLAB(0) STAGE_SLAB(1) STAGE_SLAB(2) STAGE_SLAB(3)
#undef STAGE_SLAB
}

template <bool FP16>
static int launch_256(const GemmArgs& a, int a_k, int b_k, hipStream_t s, int splits = 1) {
  const int tiles = ((a.M + 255) / 256) * ((a.N + 255) / 256) * splits;
  if (a_k && b_k)
    gemm256_m16_kernel<true, true, FP16><<<tiles, 256, 0, s>>>(a);
  else if (a_k && !b_k)
    gemm256_m16_kernel<true, false, FP16><<<tiles, 256, 0, s>>>(a);
  else if (!a_k && !b_k)
    gemm256_m16_kernel<false, false, FP16><<<tiles, 256, 0, s>>>(a);
  else
    gemm256_m32_kernel<false, true, FP16><<<tiles, 256, 0, s>>>(a);
  ETH_CHECK_LAUNCH("eth_gemm");
  return ETH_OK;
}

template <int BM, int BN, int BK, int WMW, int WNW, bool FP16>
static int launch_layout(const GemmArgs& a, int a_k, int b_k, hipStream_t s) {
  const int tiles = ((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
  constexpr int NT = 64 * WMW * WNW;
  if (a_k && b_k)
    gemm_kernel<BM, BN, BK, WMW, WNW, true, true, FP16><<<tiles, NT, 0, s>>>(a);
  else if (a_k && !b_k)
    gemm_kernel<BM, BN, BK, WMW, WNW, true, false, FP16><<<tiles, NT, 0, s>>>(a);
  else if (!a_k && !b_k)
    gemm_kernel<BM, BN, BK, WMW, WNW, false, false, FP16><<<tiles, NT, 0, s>>>(a);
  else
    gemm_kernel<BM, BN, BK, WMW, WNW, false, true, FP16><<<tiles, NT, 0, s>>>(a);
  ETH_CHECK_LAUNCH("eth_gemm");
  return ETH_OK;
}

}  // namespace eth

using namespace eth;

extern "C" int eth_gemm(const void* A, int64_t lda, int a_kcontig, const void* B, int64_t ldb,
                        int b_kcontig, void* C, int64_t ldc, int c_dtype, const void* bias,
                        int64_t M, int64_t N, int64_t K, int in_dtype, int flags, float alpha,
                        void* stream) {
  ETH_CHECK_ARG(in_dtype == ETH_BF16 || in_dtype == ETH_F16, "eth_gemm: inputs must be bf16 or fp16");
  ETH_CHECK_ARG(valid_dtype(c_dtype), "eth_gemm: bad output dtype %d", c_dtype);
  ETH_CHECK_ARG(M > 0 && N > 0 && K > 0 && M < (1LL << 31) && N < (1LL << 31) && K < (1LL << 31),
                "eth_gemm: bad shape %lld x %lld x %lld", (long long)M, (long long)N, (long long)K);
  ETH_CHECK_ARG(A && B && C, "eth_gemm: null operand");
  ETH_CHECK_ARG(K % 8 == 0, "eth_gemm: K (%lld) must be a multiple of 8", (long long)K);
  ETH_CHECK_ARG(lda % 8 == 0 && ldb % 8 == 0, "eth_gemm: lda/ldb must be multiples of 8");
  ETH_CHECK_ARG(((uintptr_t)A & 15) == 0 && ((uintptr_t)B & 15) == 0, "eth_gemm: A/B must be 16-byte aligned");
  ETH_CHECK_ARG(a_kcontig ? lda >= K : (M % 8 == 0 && lda >= M), "eth_gemm: bad A layout");
  ETH_CHECK_ARG(b_kcontig ? ldb >= K : (N % 8 == 0 && ldb >= N), "eth_gemm: bad B layout");
  ETH_CHECK_ARG(ldc >= N, "eth_gemm: ldc < N");
  ETH_CHECK_ARG(!(flags & ETH_GEMM_ACCUMULATE) || c_dtype == ETH_F32, "eth_gemm: accumulate needs fp32 C");
  ETH_CHECK_ARG(!(flags & ETH_GEMM_BIAS) || bias, "eth_gemm: bias flag without bias");
  // extents: A spans M rows of lda (K-contiguous) or K rows of lda; same for B
  const int64_t a_elems = a_kcontig ? (M - 1) * lda + K : (K - 1) * lda + M;
  const int64_t b_elems = b_kcontig ? (N - 1) * ldb + K : (K - 1) * ldb + N;
  ETH_CHECK_ARG(a_elems * 2 < (1LL << 31) && b_elems * 2 < (1LL << 31),
                "eth_gemm: operands above 2 GiB are not supported");
  GemmArgs a;
  a.A = (const uint16_t*)A;
  a.B = (const uint16_t*)B;
  a.a_bytes = (uint32_t)(a_elems * 2);
  a.b_bytes = (uint32_t)(b_elems * 2);
  a.C = C;
  a.bias = (const uint16_t*)bias;
  a.M = (int)M;
  a.N = (int)N;
  a.K = (int)K;
  a.lda = lda;
  a.ldb = ldb;
  a.ldc = ldc;
  a.c_dtype = c_dtype;
  a.flags = flags;
  a.alpha = alpha;
  hipStream_t s = (hipStream_t)stream;
  const int64_t big_tiles = ((M + 255) / 256) * ((N + 255) / 256);
  // the pipelined 256x256 kernel: K in whole k-tile pairs, C rows 16-byte
  // aligned (vector stores), C extent plus one tile of rows below 2 GiB (its
  // buffer offsets), and at least half a wave of tiles per chip
  const int esz = c_dtype == ETH_F32 ? 4 : 2;
  const int64_t c_extent = ((M - 1) * ldc + N) * esz;
  const bool c_vec = ldc % 4 == 0 && N % 4 == 0 && ((uintptr_t)C % (4 * esz)) == 0;
  a.k_split = 0;
  a.c_split_stride = 0;
  if (K % 128 == 0 && c_vec && big_tiles >= 128 && c_extent + 256 * ldc * esz < (1LL << 31)) {
    a.c_bytes = (uint32_t)c_extent;
    return in_dtype == ETH_BF16 ? launch_256<false>(a, a_kcontig, b_kcontig, s)
                                : launch_256<true>(a, a_kcontig, b_kcontig, s);
  }
  a.c_bytes = 0;
  // otherwise 256x256 tiles (8 waves of 128x64) when the grid still fills
  // the chip, 128x128 (4 waves of 64x64) below that
  const bool big = big_tiles >= 192;
  if (in_dtype == ETH_BF16)
    return big ? launch_layout<256, 256, 64, 2, 4, false>(a, a_kcontig, b_kcontig, s)
               : launch_layout<128, 128, 64, 2, 2, false>(a, a_kcontig, b_kcontig, s);
  return big ? launch_layout<256, 256, 64, 2, 4, true>(a, a_kcontig, b_kcontig, s)
             : launch_layout<128, 128, 64, 2, 2, true>(a, a_kcontig, b_kcontig, s);
}

namespace eth {
// C[m, n] += sum_s W[s][m*N + n], splits added in order (deterministic)
__global__ void splitk_reduce_kernel(const float* __restrict__ W, int splits, int64_t stride, float* __restrict__ C,
                                     int64_t ldc, int M, int N, int accumulate) {
  const int nq = N / 4;
  const int64_t total = (int64_t)M * nq;
  for (int64_t q = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; q < total; q += (int64_t)gridDim.x * blockDim.x) {
    const int m = (int)(q / nq), n = (int)(q % nq) * 4;
    float4 acc = *reinterpret_cast<const float4*>(W + (int64_t)m * N + n);
    for (int sp = 1; sp < splits; ++sp) {
      const float4 w = *reinterpret_cast<const float4*>(W + sp * stride + (int64_t)m * N + n);
      acc.x += w.x;
      acc.y += w.y;
      acc.z += w.z;
      acc.w += w.w;
    }
    float4* c = reinterpret_cast<float4*>(C + (int64_t)m * ldc + n);
    if (accumulate) {
      const float4 o = *c;
      acc.x = o.x + acc.x;
      acc.y = o.y + acc.y;
      acc.z = o.z + acc.z;
      acc.w = o.w + acc.w;
    }
    *c = acc;
  }
}
}  // namespace eth

extern "C" int64_t eth_gemm_splitk_workspace(int64_t M, int64_t N, int splits) {
  return splits > 0 && M > 0 && N > 0 ? (int64_t)splits * M * N * 4 : 0;
}

extern "C" int eth_gemm_splitk(const void* A, int64_t lda, int a_kcontig, const void* B, int64_t ldb, int b_kcontig,
                               float* C, int64_t ldc, int64_t M, int64_t N, int64_t K, int in_dtype, int splits,
                               int accumulate, float* workspace, void* stream) {
  ETH_CHECK_ARG(in_dtype == ETH_BF16 || in_dtype == ETH_F16, "eth_gemm_splitk: inputs must be bf16 or fp16");
  ETH_CHECK_ARG(A && B && C && workspace, "eth_gemm_splitk: null operand");
  ETH_CHECK_ARG(splits >= 1 && splits <= 16, "eth_gemm_splitk: splits must be in [1, 16] (got %d)", splits);
  ETH_CHECK_ARG(M > 0 && N > 0 && K > 0 && M < (1LL << 31) && N < (1LL << 31) && K < (1LL << 31),
                "eth_gemm_splitk: bad shape %lld x %lld x %lld", (long long)M, (long long)N, (long long)K);
  ETH_CHECK_ARG(K % (128LL * splits) == 0, "eth_gemm_splitk: K (%lld) must be a multiple of 128 * splits",
                (long long)K);
  ETH_CHECK_ARG(N % 4 == 0 && ldc % 4 == 0 && ldc >= N && ((uintptr_t)C & 15) == 0 && ((uintptr_t)workspace & 15) == 0,
                "eth_gemm_splitk: C and the workspace need 16-byte aligned rows (N %% 4 == 0)");
  ETH_CHECK_ARG(lda % 8 == 0 && ldb % 8 == 0, "eth_gemm_splitk: lda/ldb must be multiples of 8");
  ETH_CHECK_ARG(((uintptr_t)A & 15) == 0 && ((uintptr_t)B & 15) == 0, "eth_gemm_splitk: A/B must be 16-byte aligned");
  ETH_CHECK_ARG(a_kcontig ? lda >= K : (M % 8 == 0 && lda >= M), "eth_gemm_splitk: bad A layout");
  ETH_CHECK_ARG(b_kcontig ? ldb >= K : (N % 8 == 0 && ldb >= N), "eth_gemm_splitk: bad B layout");
  const int64_t a_elems = a_kcontig ? (M - 1) * lda + K : (K - 1) * lda + M;
  const int64_t b_elems = b_kcontig ? (N - 1) * ldb + K : (K - 1) * ldb + N;
  const int64_t slice = M * N;
  ETH_CHECK_ARG(a_elems * 2 < (1LL << 31) && b_elems * 2 < (1LL << 31) && (slice + 256 * N) * 4 < (1LL << 31),
                "eth_gemm_splitk: operands above 2 GiB are not supported");
  GemmArgs a{};
  a.A = (const uint16_t*)A;
  a.B = (const uint16_t*)B;
  a.a_bytes = (uint32_t)(a_elems * 2);
  a.b_bytes = (uint32_t)(b_elems * 2);
  a.C = workspace;
  a.bias = nullptr;
  a.M = (int)M;
  a.N = (int)N;
  a.K = (int)K;
  a.lda = lda;
  a.ldb = ldb;
  a.ldc = N;
  a.c_dtype = ETH_F32;
  a.flags = 0;
  a.alpha = 1.0f;
  a.c_bytes = (uint32_t)(slice * 4);
  a.k_split = (int)(K / splits);
  a.c_split_stride = slice;
  hipStream_t s = (hipStream_t)stream;
  const int rc = in_dtype == ETH_BF16 ? launch_256<false>(a, a_kcontig, b_kcontig, s, splits)
                                      : launch_256<true>(a, a_kcontig, b_kcontig, s, splits);
  if (rc != ETH_OK) return rc;
  const int64_t quads = M * (N / 4);
  const int grid = (int)std::min<int64_t>((quads + 255) / 256, 2048);
  splitk_reduce_kernel<<<grid, 256, 0, s>>>(workspace, splits, slice, C, ldc, (int)M, (int)N, accumulate);
  ETH_CHECK_LAUNCH("eth_gemm_splitk");
  return ETH_OK;
}
