// MFMA GEMM mainloop for gfx950: acc[M_tile x N_tile] = A[M x K] . B[N x K]^T
// with both operands K-contiguous ("NT"), fp32 accumulation.
//
//  * bf16 inputs use v_mfma_f32_32x32x16_bf16: lane l supplies 8 consecutive
//    k of row (l % 32), k-half (l / 32).
//  * f32 inputs use v_mfma_f32_32x32x2_f32: lane l supplies one k of row
//    (l % 32); four MFMAs consume a 16-byte k-slab per lane half, the half
//    h = l / 32 covering k = 4h .. 4h+3 of each 8-wide group (the sum over k
//    is order-free, so this permutation of k between the MFMAs is exact).
//  * Accumulator (32x32, 16 fp32 per lane): register r of lane l holds
//    row 8 * (r / 4) + 4 * (l / 32) + (r % 4), column l % 32.
//
// A K-stage is 128 bytes of every tile row (64 bf16 / 32 f32).  Rows are
// staged in LDS with a 144-byte pitch, which makes both the 16-byte row
// writes and the 16-byte MFMA operand reads (eight lanes, eight distinct
// rows) bank-conflict free.  Two LDS stages plus a register prefetch of the
// next stage give one barrier per K-stage.
#pragma once

#include "nf_device.h"

namespace nf {
namespace gemm {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

template <typename TI_, int BM_, int BN_, int WM_, int WN_>
struct Cfg {
  using TI = TI_;
  static constexpr int BM = BM_, BN = BN_, WM = WM_, WN = WN_;
  static constexpr int NT = WM * WN * 64;        // threads per block
  static constexpr int WTM = BM / WM;            // wave tile rows
  static constexpr int WTN = BN / WN;            // wave tile cols
  static constexpr int TM = WTM / 32;            // 32x32 MFMA tiles per wave (M)
  static constexpr int TN = WTN / 32;            // 32x32 MFMA tiles per wave (N)
  static constexpr int VE = 16 / sizeof(TI);     // elements per 16-byte vector
  static constexpr int BK = 128 / sizeof(TI);    // k per stage
  static constexpr int KV = 8;                   // 16-byte vectors per row per stage
  static constexpr int PITCH = 144;              // LDS row pitch, bytes
  static constexpr int STAGE = (BM + BN) * PITCH;
  static constexpr int LDS_BYTES = 2 * STAGE;
  static constexpr int AV = BM * KV / NT;        // A vectors per thread per stage
  static constexpr int BV = BN * KV / NT;        // B vectors per thread per stage
  static_assert(BM % (WM * 32) == 0 && BN % (WN * 32) == 0, "tile/wave mismatch");
  static_assert((BM * KV) % NT == 0 && (BN * KV) % NT == 0, "loader mismatch");
};

// One 16-byte vector of a tile row: rows >= nrows or k >= K read as zero.
// VK: every row start is 16-byte aligned and K is a multiple of VE, so a
// vector is either wholly inside or wholly outside [0, K).
template <typename TI, bool VK>
__device__ __forceinline__ u32x4 load_vec(const TI *base, int64_t ld,
                                          int64_t row, int64_t nrows,
                                          int64_t k, int64_t K) {
  constexpr int VE = 16 / sizeof(TI);
  u32x4 r = {0u, 0u, 0u, 0u};
  if (row < nrows && k < K) {
    const TI *p = base + row * ld + k;
    if (VK) {
      r = *reinterpret_cast<const u32x4 *>(p);
    } else {
      TI e[VE];
#pragma unroll
      for (int i = 0; i < VE; ++i) e[i] = (k + i < K) ? p[i] : static_cast<TI>(0.f);
      __builtin_memcpy(&r, e, 16);
    }
  }
  return r;
}

template <class C, bool VK>
__device__ __forceinline__ void load_stage(const typename C::TI *A, int64_t lda,
                                           int64_t M, const typename C::TI *B,
                                           int64_t ldb, int64_t N, int64_t K,
                                           int64_t m0, int64_t n0, int64_t k0,
                                           u32x4 (&ra)[C::AV],
                                           u32x4 (&rb)[C::BV]) {
  const int t = threadIdx.x;
#pragma unroll
  for (int i = 0; i < C::AV; ++i) {
    const int v = t + i * C::NT;
    ra[i] = load_vec<typename C::TI, VK>(A, lda, m0 + v / C::KV, M,
                                         k0 + (v % C::KV) * C::VE, K);
  }
#pragma unroll
  for (int i = 0; i < C::BV; ++i) {
    const int v = t + i * C::NT;
    rb[i] = load_vec<typename C::TI, VK>(B, ldb, n0 + v / C::KV, N,
                                         k0 + (v % C::KV) * C::VE, K);
  }
}

template <class C>
__device__ __forceinline__ void store_stage(char *stage, const u32x4 (&ra)[C::AV],
                                            const u32x4 (&rb)[C::BV]) {
  const int t = threadIdx.x;
#pragma unroll
  for (int i = 0; i < C::AV; ++i) {
    const int v = t + i * C::NT;
    *reinterpret_cast<u32x4 *>(stage + (v / C::KV) * C::PITCH + (v % C::KV) * 16) = ra[i];
  }
  char *bs = stage + C::BM * C::PITCH;
#pragma unroll
  for (int i = 0; i < C::BV; ++i) {
    const int v = t + i * C::NT;
    *reinterpret_cast<u32x4 *>(bs + (v / C::KV) * C::PITCH + (v % C::KV) * 16) = rb[i];
  }
}

template <typename TI>
__device__ __forceinline__ void mfma_slab(const u32x4 &a, const u32x4 &b,
                                          floatx16 &acc);

template <>
__device__ __forceinline__ void mfma_slab<bf16>(const u32x4 &a, const u32x4 &b,
                                                floatx16 &acc) {
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
      __builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), acc, 0, 0, 0);
}

template <>
__device__ __forceinline__ void mfma_slab<float>(const u32x4 &a, const u32x4 &b,
                                                 floatx16 &acc) {
#pragma unroll
  for (int j = 0; j < 4; ++j)
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a[j]),
                                               __uint_as_float(b[j]), acc, 0, 0, 0);
}

template <class C>
__device__ __forceinline__ void compute_stage(const char *stage, int wm, int wn,
                                              floatx16 (&acc)[C::TM][C::TN]) {
  const int l = threadIdx.x & 63;
  const char *as = stage + (wm * C::WTM + (l & 31)) * C::PITCH + (l >> 5) * 16;
  const char *bs = stage + (C::BM + wn * C::WTN + (l & 31)) * C::PITCH + (l >> 5) * 16;
#pragma unroll
  for (int kg = 0; kg < 4; ++kg) {
    u32x4 a[C::TM], b[C::TN];
#pragma unroll
    for (int i = 0; i < C::TM; ++i)
      a[i] = *reinterpret_cast<const u32x4 *>(as + i * 32 * C::PITCH + kg * 32);
#pragma unroll
    for (int j = 0; j < C::TN; ++j)
      b[j] = *reinterpret_cast<const u32x4 *>(bs + j * 32 * C::PITCH + kg * 32);
#pragma unroll
    for (int i = 0; i < C::TM; ++i)
#pragma unroll
      for (int j = 0; j < C::TN; ++j) mfma_slab<typename C::TI>(a[i], b[j], acc[i][j]);
  }
}

// Full K loop for the block tile at (m0, n0).  `smem` holds C::LDS_BYTES.
// Ends with a barrier, so the caller may reuse smem for its epilogue.
template <class C, bool VK>
__device__ __forceinline__ void mainloop(const typename C::TI *A, int64_t lda,
                                         const typename C::TI *B, int64_t ldb,
                                         int64_t M, int64_t N, int64_t K,
                                         int64_t m0, int64_t n0, char *smem,
                                         floatx16 (&acc)[C::TM][C::TN]) {
  const int w = threadIdx.x >> 6;
  const int wm = w / C::WN, wn = w % C::WN;
#pragma unroll
  for (int i = 0; i < C::TM; ++i)
#pragma unroll
    for (int j = 0; j < C::TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  const int64_t nk = (K + C::BK - 1) / C::BK;
  u32x4 ra[C::AV], rb[C::BV];
  load_stage<C, VK>(A, lda, M, B, ldb, N, K, m0, n0, 0, ra, rb);
  store_stage<C>(smem, ra, rb);
  __syncthreads();
  for (int64_t kt = 0; kt < nk; ++kt) {
    char *cur = smem + (kt & 1) * C::STAGE;
    char *nxt = smem + ((kt + 1) & 1) * C::STAGE;
    const bool more = kt + 1 < nk;
    if (more) load_stage<C, VK>(A, lda, M, B, ldb, N, K, m0, n0, (kt + 1) * C::BK, ra, rb);
    compute_stage<C>(cur, wm, wn, acc);
    if (more) store_stage<C>(nxt, ra, rb);
    __syncthreads();
  }
}

// Position of accumulator element (i, j, r) of this lane inside the block
// tile: local row and local column.
template <class C>
__device__ __forceinline__ int acc_row(int wm, int i, int r) {
  const int l = threadIdx.x & 63;
  return wm * C::WTM + i * 32 + 8 * (r >> 2) + 4 * (l >> 5) + (r & 3);
}
template <class C>
__device__ __forceinline__ int acc_col(int wn, int j) {
  const int l = threadIdx.x & 63;
  return wn * C::WTN + j * 32 + (l & 31);
}

}  // namespace gemm
}  // namespace nf
