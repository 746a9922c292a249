// MFMA GEMM mainloop for gfx950: acc[M_tile x N_tile] = A[M x K] . B[N x K]^T
// with both operands K-contiguous ("NT"), or B N-major, fp32 accumulation.
//
//  * bf16 inputs use v_mfma_f32_32x32x16_bf16 (lane l supplies 8 consecutive
//    k of row (l % 32), k-half (l / 32)) or, on the direct-to-LDS path with B
//    K-contiguous, four v_mfma_f32_16x16x32_bf16 per 32x32 tile brought to
//    the same accumulator layout (mainloop_dtl16).
//  * f32 inputs use v_mfma_f32_32x32x2_f32: lane l supplies one k of row
//    (l % 32); four MFMAs consume a 16-byte k-slab per lane half, the half
//    h = l / 32 covering k = 4h .. 4h+3 of each 8-wide group (the sum over k
//    is order-free, so this permutation of k between the MFMAs is exact).
//  * Accumulator (32x32, 16 fp32 per lane): register r of lane l holds
//    row 8 * (r / 4) + 4 * (l / 32) + (r % 4), column l % 32.
//
// Two stagings of the operand tiles in LDS:
//  * Cfg (bf16 and f32): a K-stage is 128 bytes of every tile row (64 bf16 /
//    32 f32), loaded into registers and written to LDS with a 144-byte row
//    pitch, which makes both the 16-byte row writes and the 16-byte MFMA
//    operand reads (eight lanes, eight distinct rows) bank-conflict free.
//  * DCfg (bf16): a K-stage is BK = 32 or 64 k of every tile row (64 or 128
//    bytes), copied global -> LDS by the buffer unit (buffer_load_dwordx4 ...
//    lds) with no register staging.  One such load writes 1 KB contiguously
//    (lane i at +16 i), i.e. 16 or 8 unpadded rows; the 16-byte vectors of a
//    row are stored XOR-swizzled by row (dtl_slot), which keeps the MFMA
//    operand reads conflict free.
#pragma once

#include "nf_device.h"

// Kernel attributes for a GEMM block of configuration C: its thread count,
// and exactly the wavefronts per SIMD that one block brings (one block per
// CU at these LDS sizes), so the compiler does not trade registers for an
// occupancy the LDS cannot give anyway.
#define NF_GEMM_BOUNDS(C) \
  __launch_bounds__(C::NT) __attribute__((amdgpu_waves_per_eu(C::NT / 256, C::NT / 256)))

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
  // K-stages of global loads in flight ahead of the MFMAs (register sets):
  // 2 for small wave tiles, whose short compute stage hides little latency,
  // 1 where a second set would not fit beside the accumulators.
  static constexpr int PF = (NT <= 256 && TM * TN <= 4) ? 2 : 1;
  static constexpr bool DTL = false;
  static_assert(BM % (WM * 32) == 0 && BN % (WN * 32) == 0, "tile/wave mismatch");
  static_assert((BM * KV) % NT == 0 && (BN * KV) % NT == 0, "loader mismatch");
};

// Direct-to-LDS bf16 configuration (see the file comment): BK k per stage
// (32 or 64: LDS rows of 64 or 128 bytes), STAGES stage buffers.
template <int BM_, int BN_, int WM_, int WN_, int STAGES_ = 2, int BK_ = 64>
struct DCfg {
  using TI = bf16;
  static constexpr bool DTL = true;
  static constexpr int BM = BM_, BN = BN_, WM = WM_, WN = WN_, STAGES = STAGES_;
  static constexpr int NW = WM * WN;              // wavefronts per block
  static constexpr int NT = NW * 64;
  static constexpr int WTM = BM / WM, WTN = BN / WN;
  static constexpr int TM = WTM / 32, TN = WTN / 32;
  static constexpr int VE = 8;                    // bf16 per 16-byte vector
  static constexpr int BK = BK_;                  // k per stage
  static constexpr int KVEC = BK / 8;             // 16-byte vectors per LDS row
  static constexpr int ROW = BK * 2;              // LDS row, bytes
  static constexpr int RPC = 64 / KVEC;           // rows per 1 KB direct copy
  static constexpr int KG = BK / 16;              // MFMA k-groups per stage
  static constexpr int STAGE = (BM + BN) * ROW;
  static constexpr int LDS_BYTES = STAGES * STAGE;
  static constexpr int ACW = BM / RPC / NW;       // 1 KB A copies per wave per stage
  static constexpr int BCW = BN / RPC / NW;       // 1 KB B copies per wave per stage
  static constexpr int PF = 0;
  static_assert(BK == 32 || BK == 64, "BK is 32 or 64");
  static_assert(BM % (WM * 32) == 0 && BN % (WN * 32) == 0, "tile/wave mismatch");
  static_assert((BM / RPC) % NW == 0 && (BN / RPC) % NW == 0, "chunk/wave mismatch");
  static_assert(WTM % 16 == 0 && WTN % 16 == 0, "swizzle assumes 16-row alignment");
  static_assert(STAGES >= 2 && STAGES <= 5 && (STAGES - 1) * (ACW + BCW) <= 63,
                "vmcnt range");
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

// Operand source for the K loop.  BUF (the fast path): a buffer resource
// over the whole operand, each thread's 16-byte vectors addressed by one
// 32-bit base offset plus uniform strides; a vector whose row is past the
// matrix or whose k is past K gets an out-of-range offset, which the buffer
// unit turns into zeros (no branches, no 64-bit address math).  Requires
// K % VE == 0, 16-byte aligned rows and an operand under 2 GiB.
// !BUF: plain pointer loads with per-element masking (any K, any alignment).
template <class C, bool BUF>
struct Operand {
  using TI = typename C::TI;
  const TI *base;
  int64_t ld, rows, K, r0;
  __amdgpu_buffer_rsrc_t rsrc;
  uint32_t off0;       // byte offset of this thread's first vector at k = 0
  uint32_t row_step;   // bytes between this thread's successive vectors
  __device__ __forceinline__ void init(const TI *p, int64_t ld_, int64_t rows_, int64_t K_,
                                       int64_t r0_) {
    base = p; ld = ld_; rows = rows_; K = K_; r0 = r0_;
    if constexpr (BUF) {
      rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<TI *>(p), (short)0,
                                               (int)(rows_ * ld_ * (int64_t)sizeof(TI)),
                                               0x00020000);
      const int t = threadIdx.x;
      off0 = (uint32_t)(((r0_ + t / C::KV) * ld_ + (t % C::KV) * C::VE) * (int64_t)sizeof(TI));
      row_step = (uint32_t)((C::NT / C::KV) * ld_ * (int64_t)sizeof(TI));
    }
  }
  // vector i (0 <= i < count) of the stage starting at k0
  template <int COUNT>
  __device__ __forceinline__ void load(int64_t k0, u32x4 (&r)[COUNT]) const {
    const int t = threadIdx.x;
    if constexpr (BUF) {
      const int64_t kk = k0 + (t % C::KV) * C::VE;
      const bool kin = kk < K;
      const uint32_t kb = (uint32_t)(k0 * (int64_t)sizeof(TI));
#pragma unroll
      for (int i = 0; i < COUNT; ++i) {
        const bool in = kin && (r0 + t / C::KV + (int64_t)i * (C::NT / C::KV)) < rows;
        const uint32_t off = in ? off0 + (uint32_t)i * row_step + kb : 0x80000000u;
        r[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, off, 0, 0));
      }
    } else {
#pragma unroll
      for (int i = 0; i < COUNT; ++i) {
        const int v = t + i * C::NT;
        r[i] = load_vec<TI, false>(base, ld, r0 + v / C::KV, rows, k0 + (v % C::KV) * C::VE, K);
      }
    }
  }
};

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
__device__ __forceinline__ void read_operands(const char *as, const char *bs, int kg,
                                              u32x4 (&a)[C::TM], u32x4 (&b)[C::TN]) {
#pragma unroll
  for (int i = 0; i < C::TM; ++i)
    a[i] = *reinterpret_cast<const u32x4 *>(as + i * 32 * C::PITCH + kg * 32);
#pragma unroll
  for (int j = 0; j < C::TN; ++j)
    b[j] = *reinterpret_cast<const u32x4 *>(bs + j * 32 * C::PITCH + kg * 32);
}

template <class C>
__device__ __forceinline__ void mfma_block(const u32x4 (&a)[C::TM], const u32x4 (&b)[C::TN],
                                           floatx16 (&acc)[C::TM][C::TN]) {
#pragma unroll
  for (int i = 0; i < C::TM; ++i)
#pragma unroll
    for (int j = 0; j < C::TN; ++j) mfma_slab<typename C::TI>(a[i], b[j], acc[i][j]);
}

// Scheduling hint for one k-group: the (TM + TN) LDS operand reads of the
// next k-group are spread between this k-group's TM * TN MFMAs, so their
// latency hides behind matrix work instead of stalling the wavefront (one
// wavefront per SIMD leaves no other wave to switch to).  The MFMAs left over
// after one per read go first (2 for 8 MFMAs and 6 reads): measured against
// putting them last, CE cfg4 2.04-2.05 ms against 2.05-2.07 ms and the
// gate/up fwd+bwd 187-190 us against 191-193 us.
template <class C, int kReads = C::TM + C::TN>
__device__ __forceinline__ void interleave_hint() {
  constexpr int kMfma = C::TM * C::TN * (sizeof(typename C::TI) == 2 ? 1 : 4);
  constexpr int kPer = kMfma / kReads > 0 ? kMfma / kReads : 1;
  constexpr int kLead = kMfma - kReads * kPer;  // MFMAs issued before the first read
  if constexpr (kLead > 0) __builtin_amdgcn_sched_group_barrier(0x008, kLead, 0);
#pragma unroll
  for (int r = 0; r < kReads; ++r) {
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);     // 1 DS read
    __builtin_amdgcn_sched_group_barrier(0x008, kPer, 0);  // kPer MFMAs
  }
}

template <class C>
__device__ __forceinline__ void compute_stage(const char *stage, int wm, int wn,
                                              floatx16 (&acc)[C::TM][C::TN]) {
  const int l = threadIdx.x & 63;
  const char *as = stage + (wm * C::WTM + (l & 31)) * C::PITCH + (l >> 5) * 16;
  const char *bs = stage + (C::BM + wn * C::WTN + (l & 31)) * C::PITCH + (l >> 5) * 16;
  // operands double-buffered across the four 32-byte k-groups of a stage
  u32x4 a0[C::TM], b0[C::TN], a1[C::TM], b1[C::TN];
  read_operands<C>(as, bs, 0, a0, b0);
#pragma unroll
  for (int kg = 0; kg < 4; kg += 2) {
    read_operands<C>(as, bs, kg + 1, a1, b1);
    mfma_block<C>(a0, b0, acc);
    interleave_hint<C>();
    if (kg + 2 < 4) {
      read_operands<C>(as, bs, kg + 2, a0, b0);
      mfma_block<C>(a1, b1, acc);
      interleave_hint<C>();
    } else {
      mfma_block<C>(a1, b1, acc);
    }
  }
}

// ---- direct-to-LDS path (DCfg) ----------------------------------------------

// A K-stage row of the tile holds KVEC = BK / 8 16-byte k-vectors; one 1 KB
// direct copy covers RPC = 64 / KVEC consecutive rows, lane l writing LDS
// slot (l % KVEC) of row (l / KVEC).  Slots are XOR-swizzled by row so the
// 32 rows an MFMA operand read touches at one k-vector spread over all banks:
//   KVEC 4 (64-byte rows):  slot = kvec ^ ((row >> 2) & 3)
//   KVEC 8 (128-byte rows): slot = kvec ^ ((row >> 1) & 7)
// (both maps are involutions, so the same formula gives kvec from slot).
template <class C>
__device__ __forceinline__ int dtl_slot(int row, int kv) {
  if constexpr (C::KVEC == 4)
    return kv ^ ((row >> 2) & 3);
  else
    return kv ^ ((row >> 1) & 7);
}

typedef __attribute__((address_space(3))) void *lds_ptr_t;

// One operand (A or B) of the block tile: CW chunks per wavefront.  Chunk
// g = wave * CW + c covers tile rows [g * RPC, g * RPC + RPC); the lane's
// swizzled k-vector depends only on the parity of g (dtl_slot of row
// g * RPC + l / KVEC), so two base offsets describe all chunks and a chunk's
// offset is base[g & 1] + c * RPC rows.
template <class C, int CW>
struct DtlOperand {
  using TI = typename C::TI;
  static constexpr bool kKRows = false;
  const TI *base;
  int64_t ld, rows, K, r0;  // r0: matrix row of tile row 0
  __amdgpu_buffer_rsrc_t rsrc;
  uint32_t off_p[2];  // byte offset at k = 0 of chunk parity p (rows assumed in range)
  int kvec_p[2];      // k-vector this lane copies for chunk parity p
  int lrow;           // l / KVEC: the lane's row inside a chunk
  int rows_left;      // rows from this wave's first chunk on that exist (clamped)
  uint32_t cstride;   // bytes between the first rows of consecutive chunks
  static constexpr uint32_t kOob = 0x80000000u;

  __device__ __forceinline__ void init(const TI *p, int64_t ld_, int64_t rows_, int64_t K_,
                                       int64_t r0_, int wave) {
    base = p; ld = ld_; rows = rows_; K = K_; r0 = r0_;
    rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<TI *>(p), (short)0,
                                             (int)(rows_ * ld_ * (int64_t)sizeof(TI)),
                                             0x00020000);
    const int l = threadIdx.x & 63;
    lrow = l / C::KVEC;
    const int g0 = wave * CW;
    const int64_t first = r0_ + (int64_t)g0 * C::RPC;  // first row of chunk g0
    const int64_t left = rows_ - first;
    rows_left = (int)(left < 0 ? 0 : (left > CW * C::RPC ? CW * C::RPC : left));
    cstride = (uint32_t)((int64_t)C::RPC * ld_ * (int64_t)sizeof(TI));
#pragma unroll
    for (int q = 0; q < 2; ++q) {  // q: chunk g0 + q's parity
      kvec_p[q] = dtl_slot<C>((g0 + q) * C::RPC + lrow, l % C::KVEC);
      // chunk c's offset is off_p[c & 1] + c * cstride
      off_p[q] = (uint32_t)(((first + lrow) * ld_ + kvec_p[q] * C::VE) * (int64_t)sizeof(TI));
    }
  }
  // copy the stage starting at k0 into `region` (this operand's part of a stage)
  __device__ __forceinline__ void issue(int64_t k0, char *region, int wave) const {
    const uint32_t kb = (uint32_t)(k0 * (int64_t)sizeof(TI));
    const bool kin0 = k0 + kvec_p[0] * C::VE < K, kin1 = k0 + kvec_p[1] * C::VE < K;
#pragma unroll
    for (int c = 0; c < CW; ++c) {
      const bool in = lrow + c * C::RPC < rows_left && ((c & 1) ? kin1 : kin0);
      const uint32_t o = off_p[c & 1] + (uint32_t)c * cstride + kb;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rsrc, (lds_ptr_t)(region + (wave * CW + c) * 1024), 16, in ? o : kOob, 0, 0, 0);
    }
  }
  // the same copy through registers and ds_write (any alignment, any K)
  __device__ __forceinline__ void copy_sync(int64_t k0, int wave, char *region) const {
    const int l = threadIdx.x & 63;
#pragma unroll
    for (int c = 0; c < CW; ++c) {
      const int g = wave * CW + c;
      const u32x4 v = load_vec<TI, false>(base, ld, r0 + g * C::RPC + lrow, rows,
                                          k0 + kvec_p[c & 1] * C::VE, K);
      *reinterpret_cast<u32x4 *>(region + g * 1024 + l * 16) = v;
    }
  }
};

// s_waitcnt vmcnt(N) lgkmcnt(0), then s_barrier: after it the direct LDS
// copies of the stage about to be read are complete in every wavefront, and
// so are every wavefront's reads of the buffer about to be refilled.  The
// wait is the builtin (so the compiler's own counter bookkeeping sees it);
// the empty asm statements with memory clobbers keep LDS accesses from
// moving across.  gfx9 encoding: vmcnt[3:0] bits 3:0, expcnt bits 6:4,
// lgkmcnt bits 11:8, vmcnt[5:4] bits 15:14.
template <int N>
__device__ __forceinline__ void wait_vm_barrier() {
  static_assert(N >= 0 && N <= 63, "vmcnt range");
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (0 << 8) | ((N >> 4) << 14));
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

template <class C>
__device__ __forceinline__ void wait_stage(int n_after) {
  constexpr int L = C::ACW + C::BCW;  // copies per wavefront per stage
  static_assert((C::STAGES - 1) * L <= 63, "vmcnt range");
  switch (n_after) {  // stages whose copies may still be in flight
    case 0: wait_vm_barrier<0>(); break;
    case 1: wait_vm_barrier<(1 * L < 63 ? 1 * L : 63)>(); break;
    case 2: wait_vm_barrier<(2 * L < 63 ? 2 * L : 63)>(); break;
    case 3: wait_vm_barrier<(3 * L < 63 ? 3 * L : 63)>(); break;
    default: wait_vm_barrier<(4 * L < 63 ? 4 * L : 63)>(); break;
  }
}

// Operands of one 16-wide k-group of a stage, for this lane: k-vector
// 2 * kg + (lane / 32) of rows (lane % 32) + 32 i.  Tile row offsets are
// multiples of 16, so the swizzle only depends on lane % 32.
template <class C>
__device__ __forceinline__ void read_kgroup_dtl(const char *stage, int wm, int wn, int kg,
                                                u32x4 (&a)[C::TM], u32x4 (&b)[C::TN]) {
  const int l = threadIdx.x & 63;
  const int sw = dtl_slot<C>(l & 31, 2 * kg + (l >> 5)) * 16;
  const char *as = stage + (wm * C::WTM + (l & 31)) * C::ROW + sw;
  const char *bs = stage + (C::BM + wn * C::WTN + (l & 31)) * C::ROW + sw;
#pragma unroll
  for (int i = 0; i < C::TM; ++i) a[i] = *reinterpret_cast<const u32x4 *>(as + i * 32 * C::ROW);
#pragma unroll
  for (int j = 0; j < C::TN; ++j) b[j] = *reinterpret_cast<const u32x4 *>(bs + j * 32 * C::ROW);
}

// ---- B given N-major ([K, N], unit-stride N) ---------------------------------
// For products whose B operand is stored with N contiguous (the cross
// entropy's dW product reads E, rows of tokens by vocabulary, this way).  A
// stage holds the BK k-rows of the tile's BN columns, 2 * BN bytes per k-row,
// the k-row's 16-byte vectors XOR-swizzled by kn_swz(k-row); one 1 KB direct
// copy covers 1024 / (2 * BN) k-rows.  The MFMA operand (8 consecutive k of
// one column per lane) comes from two transposing reads
// (ds_read_b64_tr_b16, 4 k each): in each 16-lane group, lane i receives
// element i % 4 of the 8-byte pieces addressed by lanes i / 4 + 4 q
// (q = 0..3), so lane a + 4 q addresses k-row k0 + q at columns 4 a .. 4 a + 3
// and lane i receives column i at k0 .. k0 + 3.  One read instruction of a
// wavefront covers k-rows {0..3, 8..11} + 16 kg (+ 4 for the second) x 64
// bytes of columns; kn_swz gives those eight k-rows eight different groups of
// four vector slots, so the 512 bytes spread evenly over the banks.
template <class C>
__device__ __forceinline__ int kn_swz(int krow) {
  return 4 * ((krow & 3) | (((krow >> 3) & 1) << 2));
}

template <class C>
struct DtlOperandKN {
  using TI = typename C::TI;
  static constexpr bool kKRows = true;
  static constexpr int VPR = C::BN / 8;           // 16-byte vectors per k-row
  static constexpr int KPC = 64 / VPR;            // k-rows per 1 KB copy
  static constexpr int CW = C::BK / KPC / C::NW;  // copies per wavefront per stage
  static_assert(VPR == 32 && KPC == 2 && CW == 4, "N-major B: BN = 256, BK = 64, 8 wavefronts");
  // The lane's k-row in copy c is r0 + 2 c (r0 = 8 wave + lane / 32), whose
  // swizzle depends on c's parity only, so copies c and c + 2 read the same
  // columns 4 k-rows apart: two offsets describe all four.
  const TI *base;
  int64_t ld, ncols, K, c0;  // ncols: columns that may be read; c0: column of tile column 0
  __amdgpu_buffer_rsrc_t rsrc;
  uint32_t off_p[2];  // byte offset at k = 0 of copy parity p's vector
  bool cin_p[2];      // that vector lies inside [0, ncols)
  int r0;             // k-row of copy 0
  uint32_t kbytes;    // bytes per k-row
  static constexpr uint32_t kOob = 0x80000000u;

  __device__ __forceinline__ void init(const TI *p, int64_t ld_, int64_t ncols_, int64_t K_,
                                       int64_t c0_, int wave) {
    base = p; ld = ld_; ncols = ncols_; K = K_; c0 = c0_;
    rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<TI *>(p), (short)0,
                                             (int)(K_ * ld_ * (int64_t)sizeof(TI)), 0x00020000);
    kbytes = (uint32_t)(ld_ * (int64_t)sizeof(TI));
    const int l = threadIdx.x & 63;
    r0 = wave * (CW * KPC) + l / VPR;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int row = r0 + 2 * q;
      const int64_t col = c0_ + ((l % VPR) ^ kn_swz<C>(row)) * C::VE;
      cin_p[q] = col < ncols_;
      off_p[q] = (uint32_t)((row * ld_ + col) * (int64_t)sizeof(TI));
    }
  }
  __device__ __forceinline__ void issue(int64_t k0, char *region, int wave) const {
    const uint32_t kb = (uint32_t)k0 * kbytes;
#pragma unroll
    for (int c = 0; c < CW; ++c) {
      const bool in = cin_p[c & 1] && k0 + r0 + 2 * c < K;
      const uint32_t o = off_p[c & 1] + (uint32_t)(c >> 1) * (4 * kbytes) + kb;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rsrc, (lds_ptr_t)(region + (wave * CW + c) * 1024), 16, in ? o : kOob, 0, 0, 0);
    }
  }
  __device__ __forceinline__ void copy_sync(int64_t k0, int wave, char *region) const {
    const int l = threadIdx.x & 63;
#pragma unroll
    for (int c = 0; c < CW; ++c) {
      const int row = r0 + 2 * c;
      const int v = (l % VPR) ^ kn_swz<C>(row);
      const u32x4 x = load_vec<TI, false>(base, ld, k0 + row, K, c0 + v * C::VE, ncols);
      *reinterpret_cast<u32x4 *>(region + (wave * CW + c) * 1024 + l * 16) = x;
    }
  }
};

// Operands of one 16-wide k-group, B from the N-major stage layout above
// (A as read_kgroup_dtl).  The lane's first read is k-row r = 16 kg +
// 8 (lane / 32) + (lane % 16) / 4, whose swizzle does not depend on kg and is
// the same at r + 4; and MFMA tile j + 1's 16-byte slot differs from tile j's
// in bit 2 only.  So one address per tile j (at kg = 0) and immediate offsets
// (8 KB per k-group, 2 KB for the second read) cover every read.
template <class C>
__device__ __forceinline__ void read_kgroup_kn(const char *stage, int wm, int wn, int kg,
                                               u32x4 (&a)[C::TM], u32x4 (&b)[C::TN]) {
  typedef short v4s __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) v4s *lds_v4s;
  static_assert(C::BN == 256 && C::WTN == 64 && C::TN == 2, "N-major B tiling");
  const int l = threadIdx.x & 63;
  const int sw = dtl_slot<C>(l & 31, 2 * kg + (l >> 5)) * 16;
  const char *as = stage + (wm * C::WTM + (l & 31)) * C::ROW + sw;
#pragma unroll
  for (int i = 0; i < C::TM; ++i) a[i] = *reinterpret_cast<const u32x4 *>(as + i * 32 * C::ROW);
  const int j16 = l & 15;
  const int r = 8 * (l >> 5) + (j16 >> 2);  // k-row at kg = 0
  const int col = wn * C::WTN + 16 * ((l >> 4) & 1) + 4 * (j16 & 3);  // tile j = 0
  const int off0 = r * (2 * C::BN) + (((col >> 3) ^ kn_swz<C>(r)) << 4) + (col & 7) * 2;
  const char *bs = stage + C::BM * C::ROW + kg * 16 * (2 * C::BN);
#pragma unroll
  for (int j = 0; j < C::TN; ++j) {
    const char *p = bs + (j ? (off0 ^ 64) : off0);
    const v4s x = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s)p);
    const v4s y = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s)(p + 4 * (2 * C::BN)));
    b[j] = __builtin_bit_cast(u32x4, __builtin_shufflevector(x, y, 0, 1, 2, 3, 4, 5, 6, 7));
  }
}

// ---- 16x16x32 products on K-contiguous operands -------------------------------
#ifndef NF_MFMA16
#define NF_MFMA16 1
#endif
constexpr bool kMfma16 = NF_MFMA16 != 0;

// v_mfma_f32_16x16x32_bf16 sustains ~14% more than v_mfma_f32_32x32x16_bf16
// on this chip under its power limit (register-held random bf16 operands, one
// wavefront per SIMD: 2.06-2.09 against 1.80-1.83 PFLOP/s).  With K-contiguous
// B the mainloop computes each 32 x 32 accumulator tile of the wavefront as
// four 16 x 16 products over 32-wide k-groups, product s = 2 ti + tj in the
// tile's registers 4 s .. 4 s + 3, and hands the tile over in the 32x32x16
// layout, so every epilogue sees the layout it was written for.  Product
// (ti, tj) leaves in lane l column 16 tj + l % 16 and rows
// rA(ti, 4 (l / 16) + q), q = 0..3, where rA(ti, i) is the tile row lane i
// of its A operand supplies; taking rA(ti, i) = 16 ti + (i with bits 2 and 3
// swapped), one v_permlane16_swap per register pair (tj = 0, tj = 1) leaves
// lane l holding column l % 32 and rows 8 (r / 4) + 4 (l / 32) + r % 4, the
// 32x32x16 layout (the swap is its own inverse, so it also takes a loaded
// accumulator into the 16 x 16 form).
template <class C>
struct Mfma16 {
  static constexpr int NA = 2 * C::TM, NB = 2 * C::TN;  // operand vectors per k-group
  static constexpr int KG = C::BK / 32;                 // k-groups per stage
};

// Operands of 32-wide k-group kg: A vector i = 2 I + ti for tile rows
// 32 I + rA(ti, lane % 16), B vector j = 2 J + tj for tile columns
// 32 J + 16 tj + lane % 16, k-vector 4 kg + lane / 16.  Tile row offsets are
// multiples of 16, so the swizzle only depends on the row's low four bits.
template <class C>
__device__ __forceinline__ void read_kgroup16(const char *stage, int wm, int wn, int kg,
                                              u32x4 (&a)[Mfma16<C>::NA],
                                              u32x4 (&b)[Mfma16<C>::NB]) {
  const int l = threadIdx.x & 63;
  const int r16 = l & 15;
  const int ra = (r16 & 3) | ((r16 & 4) << 1) | ((r16 & 8) >> 1);
  const int kv = 4 * kg + (l >> 4);
  const char *as = stage + (wm * C::WTM + ra) * C::ROW + dtl_slot<C>(ra, kv) * 16;
  const char *bs = stage + (C::BM + wn * C::WTN + r16) * C::ROW + dtl_slot<C>(r16, kv) * 16;
#pragma unroll
  for (int i = 0; i < Mfma16<C>::NA; ++i)
    a[i] = *reinterpret_cast<const u32x4 *>(as + i * 16 * C::ROW);
#pragma unroll
  for (int j = 0; j < Mfma16<C>::NB; ++j)
    b[j] = *reinterpret_cast<const u32x4 *>(bs + j * 16 * C::ROW);
}

template <class C>
__device__ __forceinline__ void mfma_block16(const u32x4 (&a)[Mfma16<C>::NA],
                                             const u32x4 (&b)[Mfma16<C>::NB],
                                             floatx16 (&acc)[C::TM][C::TN]) {
#pragma unroll
  for (int i = 0; i < C::TM; ++i)
#pragma unroll
    for (int j = 0; j < C::TN; ++j)
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        floatx4 c = {acc[i][j][4 * s], acc[i][j][4 * s + 1], acc[i][j][4 * s + 2],
                     acc[i][j][4 * s + 3]};
        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            __builtin_bit_cast(bf16x8, a[2 * i + (s >> 1)]),
            __builtin_bit_cast(bf16x8, b[2 * j + (s & 1)]), c, 0, 0, 0);
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[i][j][4 * s + e] = c[e];
      }
}

// Between the two layouts of a tile, in place: registers (8 ti + r,
// 8 ti + 4 + r) hold products (2 ti, 2 ti + 1) at element r in the 16 x 16
// form and rows (16 ti + r, 16 ti + 8 + r) (plus 4 for lanes 32-63) in the
// 32x32x16 layout; v_permlane16_swap of each pair goes either way.
__device__ __forceinline__ void acc_swap16(floatx16 &acc) {
#pragma unroll
  for (int ti = 0; ti < 2; ++ti)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const auto v = __builtin_amdgcn_permlane16_swap(__float_as_uint(acc[8 * ti + r]),
                                                      __float_as_uint(acc[8 * ti + 4 + r]),
                                                      false, false);
      acc[8 * ti + r] = __uint_as_float(v[0]);
      acc[8 * ti + 4 + r] = __uint_as_float(v[1]);
    }
}

// As interleave_hint for a 16x16x32 k-group: 4 TM TN MFMAs, 2 (TM + TN) reads.
template <class C>
__device__ __forceinline__ void interleave_hint16() {
  constexpr int kMfma = 4 * C::TM * C::TN;
  constexpr int kReads = Mfma16<C>::NA + Mfma16<C>::NB;
  constexpr int kPer = kMfma / kReads > 0 ? kMfma / kReads : 1;
  constexpr int kLead = kMfma - kReads * kPer;
  if constexpr (kLead > 0) __builtin_amdgcn_sched_group_barrier(0x008, kLead, 0);
#pragma unroll
  for (int r = 0; r < kReads; ++r) {
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, kPer, 0);
  }
}

// The K loop of mainloop_dtl_ops in 16x16x32 products (K-contiguous B, BK 64);
// ZERO: acc holds zeros, which both layouts share.
template <class C, bool BUF, bool ZERO>
__device__ __forceinline__ void mainloop_dtl16(const DtlOperand<C, C::ACW> &opa,
                                               const DtlOperand<C, C::BCW> &opb, int64_t K,
                                               char *smem, floatx16 (&acc)[C::TM][C::TN]) {
  using Q = Mfma16<C>;
  static_assert(Q::KG == 2, "two 32-wide k-groups per stage");
  const int w = threadIdx.x >> 6;
  const int wave = __builtin_amdgcn_readfirstlane(w);
  const int wm = w / C::WN, wn = w % C::WN;
  const int64_t nk = (K + C::BK - 1) / C::BK;
  if constexpr (!ZERO) {
#pragma unroll
    for (int i = 0; i < C::TM; ++i)
#pragma unroll
      for (int j = 0; j < C::TN; ++j) acc_swap16(acc[i][j]);
  }
  u32x4 a0[Q::NA], b0[Q::NB], a1[Q::NA], b1[Q::NB];
  if constexpr (BUF) {
    // the stage hand-over of mainloop_dtl_ops, with two k-groups per stage
#pragma unroll
    for (int s = 0; s < C::STAGES; ++s)
      if (s < nk) {
        char *st = smem + s * C::STAGE;
        opa.issue((int64_t)s * C::BK, st, wave);
        opb.issue((int64_t)s * C::BK, st + C::BM * C::ROW, wave);
      }
    if (nk > 0) {
      wait_stage<C>(nk - 1 < C::STAGES - 1 ? (int)(nk - 1) : C::STAGES - 1);
      read_kgroup16<C>(smem, wm, wn, 0, a0, b0);
    }
    int cur = 0;
    for (int64_t kt = 0; kt < nk; ++kt) {
      const char *st = smem + cur * C::STAGE;
      read_kgroup16<C>(st, wm, wn, 1, a1, b1);
      mfma_block16<C>(a0, b0, acc);
      interleave_hint16<C>();
      mfma_block16<C>(a1, b1, acc);
      interleave_hint16<C>();
      if (kt + 1 < nk) {
        if constexpr (C::STAGES == 2) {
          wait_vm_barrier<0>();
        } else {
          const int64_t later = nk - 2 - kt;
          wait_stage<C>(later < C::STAGES - 2 ? (int)later : C::STAGES - 2);
        }
        if (kt + C::STAGES < nk) {
          char *re = smem + cur * C::STAGE;
          opa.issue((kt + C::STAGES) * C::BK, re, wave);
          opb.issue((kt + C::STAGES) * C::BK, re + C::BM * C::ROW, wave);
        }
        cur = cur + 1 == C::STAGES ? 0 : cur + 1;
        read_kgroup16<C>(smem + cur * C::STAGE, wm, wn, 0, a0, b0);
      }
    }
  } else {
    for (int64_t kt = 0; kt < nk; ++kt) {
      opa.copy_sync(kt * C::BK, wave, smem);
      opb.copy_sync(kt * C::BK, wave, smem + C::BM * C::ROW);
      __syncthreads();
      read_kgroup16<C>(smem, wm, wn, 0, a0, b0);
      read_kgroup16<C>(smem, wm, wn, 1, a1, b1);
      mfma_block16<C>(a0, b0, acc);
      mfma_block16<C>(a1, b1, acc);
      __syncthreads();
    }
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < C::TM; ++i)
#pragma unroll
    for (int j = 0; j < C::TN; ++j) acc_swap16(acc[i][j]);
}

// k-group operands for B operand type OpB
template <class C, class OpB>
__device__ __forceinline__ void read_kgroup_op(const char *stage, int wm, int wn, int kg,
                                               u32x4 (&a)[C::TM], u32x4 (&b)[C::TN]) {
  if constexpr (OpB::kKRows)
    read_kgroup_kn<C>(stage, wm, wn, kg, a, b);
  else
    read_kgroup_dtl<C>(stage, wm, wn, kg, a, b);
}

template <class C, bool BUF, bool ZERO = false, class OpB>
__device__ __forceinline__ void mainloop_dtl_ops(const DtlOperand<C, C::ACW> &opa,
                                                 const OpB &opb, int64_t K,
                                                 char *smem, floatx16 (&acc)[C::TM][C::TN]);

template <class C, bool BUF, bool ZERO>
__device__ __forceinline__ void mainloop_dtl(const bf16 *A, int64_t lda, const bf16 *B,
                                             int64_t ldb, int64_t M, int64_t N, int64_t K,
                                             int64_t m0, int64_t n0, char *smem,
                                             floatx16 (&acc)[C::TM][C::TN]) {
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  if constexpr (ZERO) {
#pragma unroll
    for (int i = 0; i < C::TM; ++i)
#pragma unroll
      for (int j = 0; j < C::TN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
  }
  DtlOperand<C, C::ACW> opa;
  DtlOperand<C, C::BCW> opb;
  opa.init(A, lda, M, K, m0, wave);
  opb.init(B, ldb, N, K, n0, wave);
  mainloop_dtl_ops<C, BUF, ZERO>(opa, opb, K, smem, acc);
}

// As mainloop_dtl with B given N-major: B[k, n] at B[k * ldb + n], k-rows
// past K read as zero, columns at or past nb_cols read as zero (16-byte
// vectors, so nb_cols is a multiple of 8 on the buffer path).
template <class C, bool BUF, bool ZERO>
__device__ __forceinline__ void mainloop_kn(const bf16 *A, int64_t lda, const bf16 *B,
                                            int64_t ldb, int64_t M, int64_t nb_cols, int64_t K,
                                            int64_t m0, int64_t n0, char *smem,
                                            floatx16 (&acc)[C::TM][C::TN]) {
  static_assert(DtlOperandKN<C>::CW == C::BCW, "stage copies per wavefront (wait counts)");
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  if constexpr (ZERO) {
#pragma unroll
    for (int i = 0; i < C::TM; ++i)
#pragma unroll
      for (int j = 0; j < C::TN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
  }
  DtlOperand<C, C::ACW> opa;
  DtlOperandKN<C> opb;
  opa.init(A, lda, M, K, m0, wave);
  opb.init(B, ldb, nb_cols, K, n0, wave);
  mainloop_dtl_ops<C, BUF, ZERO>(opa, opb, K, smem, acc);
}

// The K loop over operands the caller has set up (a kernel may point each
// wavefront's share of a tile at a different matrix).  acc is not cleared.
// OpB: DtlOperand (B K-contiguous) or DtlOperandKN (B N-major).  ZERO: acc
// holds zeros on entry.
template <class C, bool BUF, bool ZERO, class OpB>
__device__ __forceinline__ void mainloop_dtl_ops(const DtlOperand<C, C::ACW> &opa,
                                                 const OpB &opb, int64_t K,
                                                 char *smem, floatx16 (&acc)[C::TM][C::TN]) {
  if constexpr (!OpB::kKRows && C::BK == 64 && kMfma16) {
    mainloop_dtl16<C, BUF, ZERO>(opa, opb, K, smem, acc);
    return;
  }
  // LDS read instructions per k-group: an N-major B takes two per MFMA tile
  constexpr int kReadsB = C::TM + (OpB::kKRows ? 2 : 1) * C::TN;
  const int w = threadIdx.x >> 6;
  const int wave = __builtin_amdgcn_readfirstlane(w);
  const int wm = w / C::WN, wn = w % C::WN;
  const int64_t nk = (K + C::BK - 1) / C::BK;
  u32x4 a0[C::TM], b0[C::TN], a1[C::TM], b1[C::TN];
  if constexpr (BUF) {
    // Stage kt lives in buffer kt % STAGES.  Every buffer is filled up front;
    // buffer kt % STAGES is refilled with stage kt + STAGES right after the
    // barrier that follows the last read of stage kt.  The operands of the
    // KG k-groups of a stage alternate between two register sets, each read
    // from LDS while the MFMAs of the other run.  The last k-group's MFMAs go
    // out before the wait for the next stage, so the matrix pipe has work
    // queued while the wavefront waits at the barrier (measured against
    // issuing them after the hand-over: +1% on 8192^3 and the cross-entropy
    // products, cfg4 fwd+bwd 1.456-1.463 against 1.465-1.478 ms).
#pragma unroll
    for (int s = 0; s < C::STAGES; ++s)
      if (s < nk) {
        char *st = smem + s * C::STAGE;
        opa.issue((int64_t)s * C::BK, st, wave);
        opb.issue((int64_t)s * C::BK, st + C::BM * C::ROW, wave);
      }
    if (nk > 0) {
      wait_stage<C>(nk - 1 < C::STAGES - 1 ? (int)(nk - 1) : C::STAGES - 1);
      read_kgroup_op<C, OpB>(smem, wm, wn, 0, a0, b0);
    }
    int cur = 0;  // buffer of stage kt
    static_assert(C::KG % 2 == 0, "k-groups alternate register sets in pairs");
    for (int64_t kt = 0; kt < nk; ++kt) {
      const char *st = smem + cur * C::STAGE;
#pragma unroll
      for (int kg = 0; kg + 1 < C::KG; kg += 2) {
        read_kgroup_op<C, OpB>(st, wm, wn, kg + 1, a1, b1);
        mfma_block<C>(a0, b0, acc);
        interleave_hint<C, kReadsB>();
        if (kg + 2 < C::KG) {
          read_kgroup_op<C, OpB>(st, wm, wn, kg + 2, a0, b0);
          mfma_block<C>(a1, b1, acc);
          interleave_hint<C, kReadsB>();
        }
      }
      mfma_block<C>(a1, b1, acc);  // the last k-group, then the hand-over
      interleave_hint<C, kReadsB>();
      if (kt + 1 < nk) {
        if constexpr (C::STAGES == 2) {
          // stage kt + 1 is the only one in flight: wait for all of it
          wait_vm_barrier<0>();
        } else {
          const int64_t later = nk - 2 - kt;  // stages issued beyond kt + 1 (>= 0)
          wait_stage<C>(later < C::STAGES - 2 ? (int)later : C::STAGES - 2);
        }
        if (kt + C::STAGES < nk) {
          char *re = smem + cur * C::STAGE;
          opa.issue((kt + C::STAGES) * C::BK, re, wave);
          opb.issue((kt + C::STAGES) * C::BK, re + C::BM * C::ROW, wave);
        }
        cur = cur + 1 == C::STAGES ? 0 : cur + 1;
        read_kgroup_op<C, OpB>(smem + cur * C::STAGE, wm, wn, 0, a0, b0);
      }
    }
  } else {
    for (int64_t kt = 0; kt < nk; ++kt) {
      opa.copy_sync(kt * C::BK, wave, smem);
      opb.copy_sync(kt * C::BK, wave, smem + C::BM * C::ROW);
      __syncthreads();
#pragma unroll
      for (int kg = 0; kg < C::KG; kg += 2) {
        read_kgroup_op<C, OpB>(smem, wm, wn, kg, a0, b0);
        read_kgroup_op<C, OpB>(smem, wm, wn, kg + 1, a1, b1);
        mfma_block<C>(a0, b0, acc);
        mfma_block<C>(a1, b1, acc);
      }
      __syncthreads();
    }
  }
  __syncthreads();
}

// Full K loop for the block tile at (m0, n0).  `smem` holds C::LDS_BYTES.
// With C::PF == 2, global loads run two K-stages ahead of the MFMAs in two
// alternating register sets (while stage k is multiplied out of LDS, stage
// k+1 sits in registers waiting for the other LDS buffer and stage k+2 is in
// flight): a small wave tile's compute stage is too short to hide HBM/MALL
// latency alone.  With C::PF == 1 one register set holds stage k+1 while
// stage k is computed: large wave tiles (and a second wavefront per SIMD)
// cover the latency, and a second set would not fit beside the accumulators.
// Ends with a barrier, so the caller may reuse smem for its epilogue.
// ZERO: start from acc = 0; otherwise the caller has loaded acc (C += A B^T).
template <class C, bool BUF, bool ZERO = true>
__device__ __forceinline__ void mainloop(const typename C::TI *A, int64_t lda,
                                         const typename C::TI *B, int64_t ldb,
                                         int64_t M, int64_t N, int64_t K,
                                         int64_t m0, int64_t n0, char *smem,
                                         floatx16 (&acc)[C::TM][C::TN]) {
  if constexpr (C::DTL) {
    mainloop_dtl<C, BUF, ZERO>(A, lda, B, ldb, M, N, K, m0, n0, smem, acc);
    return;
  } else {
  const int w = threadIdx.x >> 6;
  const int wm = w / C::WN, wn = w % C::WN;
  if constexpr (ZERO) {
#pragma unroll
    for (int i = 0; i < C::TM; ++i)
#pragma unroll
      for (int j = 0; j < C::TN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
  }

  Operand<C, BUF> opa, opb;
  opa.init(A, lda, M, K, m0);
  opb.init(B, ldb, N, K, n0);
  const int64_t nk = (K + C::BK - 1) / C::BK;
  char *const lds0 = smem;
  char *const lds1 = smem + C::STAGE;
  if constexpr (C::PF == 2) {
    u32x4 ra0[C::AV], rb0[C::BV], ra1[C::AV], rb1[C::BV];
    opa.load(0, ra0);
    opb.load(0, rb0);
    store_stage<C>(lds0, ra0, rb0);
    if (nk > 1) { opa.load(C::BK, ra1); opb.load(C::BK, rb1); }
    if (nk > 2) { opa.load(2 * C::BK, ra0); opb.load(2 * C::BK, rb0); }
    __syncthreads();
    for (int64_t kt = 0; kt < nk; kt += 2) {
      // even stage kt in lds0; stage kt+1 in (ra1, rb1); stage kt+2 in (ra0, rb0)
      compute_stage<C>(lds0, wm, wn, acc);
      if (kt + 1 < nk) {
        store_stage<C>(lds1, ra1, rb1);
        if (kt + 3 < nk) { opa.load((kt + 3) * C::BK, ra1); opb.load((kt + 3) * C::BK, rb1); }
      }
      __syncthreads();
      if (kt + 1 >= nk) break;
      // odd stage kt+1 in lds1; stage kt+2 in (ra0, rb0); stage kt+3 in (ra1, rb1)
      compute_stage<C>(lds1, wm, wn, acc);
      if (kt + 2 < nk) {
        store_stage<C>(lds0, ra0, rb0);
        if (kt + 4 < nk) { opa.load((kt + 4) * C::BK, ra0); opb.load((kt + 4) * C::BK, rb0); }
      }
      __syncthreads();
    }
  } else {
    u32x4 ra[C::AV], rb[C::BV];
    opa.load(0, ra);
    opb.load(0, rb);
    store_stage<C>(lds0, ra, rb);
    if (nk > 1) { opa.load(C::BK, ra); opb.load(C::BK, rb); }
    __syncthreads();
    for (int64_t kt = 0; kt < nk; ++kt) {
      // stage kt in LDS buffer kt&1; stage kt+1 in (ra, rb)
      char *const cur = (kt & 1) ? lds1 : lds0;
      char *const nxt = (kt & 1) ? lds0 : lds1;
      compute_stage<C>(cur, wm, wn, acc);
      if (kt + 1 < nk) {
        store_stage<C>(nxt, ra, rb);
        if (kt + 2 < nk) { opa.load((kt + 2) * C::BK, ra); opb.load((kt + 2) * C::BK, rb); }
      }
      __syncthreads();
    }
  }
  }
}

// Output tile of a one-dimensional grid's block b, for `total` = tiles_m *
// tiles_n tiles.  Workgroups are dealt to the 8 XCDs round-robin (block b to
// XCD b % 8) and each XCD has its own L2, so XCD x is given a contiguous
// range of a grouped tile order (a bijection of [0, total)): the order walks
// groups of G tile rows, row-fastest inside a group (group_tile), so the
// ~32 blocks an XCD runs at once cover a G x (32 / G) rectangle and share
// its A and B K-slices in that L2.  xcd_order gives block b's position in
// that order.
constexpr int kXcds = 8;
__device__ __forceinline__ int xcd_order(int b, int total) {
  const int q = total / kXcds, r = total % kXcds;
  const int x = b % kXcds, loc = b / kXcds;
  return x * q + (x < r ? x : r) + loc;
}
// Tile (tm, tn) at position k of the grouped order over tiles_m x tiles_n.
__device__ __forceinline__ void group_tile(int k, int tiles_m, int tiles_n, int G, int &tm,
                                           int &tn) {
  const int per_group = G * tiles_n;
  const int grp = k / per_group, in = k % per_group;
  const int first = grp * G;
  const int rows = tiles_m - first < G ? tiles_m - first : G;
  tm = first + in % rows;
  tn = in / rows;
}
constexpr int kTileGroup = 4;

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
