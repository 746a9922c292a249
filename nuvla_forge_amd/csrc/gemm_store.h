// GEMM with a store epilogue on the MFMA core of gemm_core.h, shared by the
// kernels that need a plain product C = scale * (Cin + A B^T): one or two
// independent jobs per launch, optional split-K with a fixed-order reduce,
// output in fp32 / bf16 / fp16.  Plus the 2-D transposes that make operands
// K-contiguous, and the launch helpers.
#pragma once

#include "gemm_core.h"

namespace nf {
namespace gemm {

// Can an operand of `rows` x K (row stride ld) use the buffer-load path?
template <typename TI>
inline bool buf_ok(const void *p, int64_t ld, int64_t rows, int64_t K) {
  constexpr int VE = 16 / sizeof(TI);
  return K % VE == 0 && ld % VE == 0 && aligned16(p) &&
         rows * ld * (int64_t)sizeof(TI) < ((int64_t)1 << 31) - 64;
}


// ---------------------------------------------------------------------------
// Branch-free epilogue stores.  With SB, a store goes through a buffer
// resource over the destination (which must be under 2 GiB); a masked
// element gets an out-of-range offset and the buffer unit drops it, so no
// lane diverges.  Without SB, plain stores under a per-element condition.
// ---------------------------------------------------------------------------
constexpr uint32_t kOobOffset = 0x80000000u;

template <bool SB>
struct OutBuf {
  char *base;
  __amdgpu_buffer_rsrc_t rsrc;
  __device__ __forceinline__ void init(void *p, int64_t bytes) {
    base = static_cast<char *>(p);
    if constexpr (SB)
      rsrc = __builtin_amdgcn_make_buffer_rsrc(p, (short)0, (int)bytes, 0x00020000);
  }
  __device__ __forceinline__ void st32(int64_t off, bool ok, float v) const {
    if constexpr (SB)
      __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), rsrc,
                                            ok ? (uint32_t)off : kOobOffset, 0, 0);
    else if (ok)
      *reinterpret_cast<float *>(base + off) = v;
  }
  __device__ __forceinline__ float ld32(int64_t off, bool ok) const {
    if constexpr (SB)
      return __uint_as_float(
          __builtin_amdgcn_raw_buffer_load_b32(rsrc, ok ? (uint32_t)off : kOobOffset, 0, 0));
    else
      return ok ? *reinterpret_cast<const float *>(base + off) : 0.f;
  }
  __device__ __forceinline__ void st16(int64_t off, bool ok, uint16_t v) const {
    if constexpr (SB)
      __builtin_amdgcn_raw_buffer_store_b16(v, rsrc, ok ? (uint32_t)off : kOobOffset, 0, 0);
    else if (ok)
      *reinterpret_cast<uint16_t *>(base + off) = v;
  }
  __device__ __forceinline__ void st64(int64_t off, bool ok, u32x2 v) const {
    if constexpr (SB)
      __builtin_amdgcn_raw_buffer_store_b64(v, rsrc, ok ? (uint32_t)off : kOobOffset, 0, 0);
    else if (ok)
      *reinterpret_cast<u32x2 *>(base + off) = v;
  }
  __device__ __forceinline__ void st128(int64_t off, bool ok, u32x4 v) const {
    if constexpr (SB)
      __builtin_amdgcn_raw_buffer_store_b128(v, rsrc, ok ? (uint32_t)off : kOobOffset, 0, 0);
    else if (ok)
      *reinterpret_cast<u32x4 *>(base + off) = v;
  }
};

inline bool sb_ok(int64_t bytes) { return bytes < ((int64_t)1 << 31) - 64; }

// ---------------------------------------------------------------------------
// plain store epilogue, C[m, n] = scale * (Cin[m, n] + A B^T), for one or two
// independent GEMMs in one launch (the dW and dH products of a vocabulary
// chunk: each alone is too few 256x256 tiles to fill the chip, together they
// do).  A job with Cin loads that fp32 tile into the accumulators before the
// K loop, so the load latency overlaps the first operand copies and the
// epilogue only stores.  C has element type cdt (fp32, bf16 or fp16: the
// last product of a gradient goes straight to the caller's type) and
// scale, when given, is a device fp32 scalar (the loss's grad_output), and
// row_scale a device fp32 vector over the rows of C (a per-row factor that
// could not enter the product: the cross entropy's softmax normaliser).
// ---------------------------------------------------------------------------
// A job with ksplit > 1 divides K into slices of kslice (a multiple of the
// stage width): block (tile, s) writes the partial product over slice s to
// part[s] ([M, N], dense, fp32) and splitk_reduce_kernel adds the slices in
// order, then Cin, scales and converts.
//
// A job with `dyn` set takes one extent from device memory, so a caller can
// size work by a count it never reads back: e = clamp(*dyn - dyn_base, 0, X)
// replaces M (dyn_rows: blocks past the e rows exit, rows past e are not
// written) or K (rounded up to 8; the operands must hold zeros between e and
// that).  The static M, N, K still give the grid and the buffer extents.
template <typename TI>
struct GemmJob {
  const TI *A;
  const TI *B;
  const float *Cin;    // fp32 [M, ldc] added to the product, or null
  void *C;             // [M, ldc] of cdt
  const float *scale;  // device scalar multiplying the result, or null
  const float *row_scale;  // device fp32 per output row multiplying it, or null
  int64_t lda, ldb, ldc, M, N, K;
  int cdt;       // NF_DTYPE_F32 / BF16 / F16
  int tiles_m;   // tiles along M
  int tiles;     // blocks of this job: tiles_m * tiles_n * ksplit
  int ksplit;    // K slices (1: no split)
  int64_t kslice;
  float *part;   // [ksplit, M, N] partial products when ksplit > 1
  const int *dyn;    // device count giving the dynamic extent, or null
  int64_t dyn_base;  // the extent is *dyn - dyn_base, clamped to [0, M or K]
  int dyn_rows;      // 1: the dynamic extent is M; 0: it is K
  // bt: B is given N-major, B[k, n] at B[k * ldb + n] (columns up to ldb may
  // be read; 16-bit inputs, DCfg only).  ct: C is stored
  // transposed, element (m, n) at C[n * ldc + m] (no K split); Cin keeps
  // [M, ldcin].
  int bt, ct;
  int ct_vec;     // ct with M and ldc multiples of 8: the LDS-transposed store
  int64_t ldcin;  // row stride of Cin (make_job: ldc)
};

// The job's (M, K) after its dynamic extent, if any.
template <typename TI>
__device__ __forceinline__ void job_extents(const GemmJob<TI> &j, int64_t &M, int64_t &K) {
  M = j.M;
  K = j.K;
  if (j.dyn) {
    int64_t e = (int64_t)__builtin_amdgcn_readfirstlane(*j.dyn) - j.dyn_base;
    const int64_t cap = j.dyn_rows ? j.M : j.K;
    e = e < 0 ? 0 : (e > cap ? cap : e);
    if (j.dyn_rows) {
      M = e;
    } else {
      e = (e + 7) / 8 * 8;
      K = e < j.K ? e : j.K;
    }
  }
}

__host__ __device__ inline int dtype_bytes(int dt) { return dt == NF_DTYPE_F32 ? 4 : 2; }

__device__ __forceinline__ uint16_t to_half_bits(float v, int dt) {
  uint16_t bits;
  if (dt == NF_DTYPE_BF16) {
    const bf16 h = static_cast<bf16>(v);
    __builtin_memcpy(&bits, &h, 2);
  } else {
    const f16 h = static_cast<f16>(v);
    __builtin_memcpy(&bits, &h, 2);
  }
  return bits;
}

// Tilings the N-major B path (DtlOperandKN, read_kgroup_kn) and the
// LDS-transposed C store are written for.
template <class C>
constexpr bool kn_tiling() {
  if constexpr (!C::DTL)
    return false;
  else
    return C::BN == 256 && C::BK == 64 && C::NW == 8 && C::WTN == 64 && C::TN == 2;
}
template <class C>
constexpr bool ct_vec_tiling() {
  if constexpr (!C::DTL)
    return false;
  else
    return C::WTN == 64 && C::WN * C::WTN == C::BN && C::BM == 256;
}

// One block's tile of job j: the K loop (B K-contiguous, or N-major when BT)
// and the store epilogue.  The kernel instantiates it once per B layout in
// separate branches, so the two K loops never share a merge point (which
// would force one register assignment on both and spill).
template <class C, bool BUF, bool SB, bool BT>
__device__ __forceinline__ void store_tile(const GemmJob<typename C::TI> &j, int64_t M,
                                           int64_t K, int ks, int64_t m0, int64_t n0,
                                           char *smem) {
  const int64_t N = j.N;
  const bool split = j.ksplit > 1;
  const int64_t k0 = ks * j.kslice;
  int64_t klen = K - k0 < j.kslice ? K - k0 : j.kslice;
  if (klen < 0) klen = 0;
  // a split block writes its fp32 partial densely; the reduce does the rest
  const int64_t ldc = split ? N : j.ldc;
  const int cdt = split ? NF_DTYPE_F32 : j.cdt;
  const bool preload = !split && j.Cin != nullptr;
  // element (m, n) of C sits at idx(m, n); of Cin at m * ldcin + n
  const bool ct = !split && j.ct;
  auto idx = [&](int64_t m, int64_t n) { return ct ? n * ldc + m : m * ldc + n; };
  const int64_t c_rows = ct ? N : j.M;
  OutBuf<SB> out, cin;
  out.init(split ? static_cast<void *>(j.part + ks * j.M * N) : j.C,
           c_rows * ldc * (int64_t)dtype_bytes(cdt));
  cin.init(const_cast<float *>(j.Cin), j.M * j.ldcin * (int64_t)sizeof(float));
  const int w = threadIdx.x >> 6, wm = w / C::WN, wn = w % C::WN;
  // element (i, jj, r) of this lane sits at byte offset base + i * 32 rows
  // + 8 * (r / 4) + (r % 4) rows + jj * 32 columns
  const int64_t row0 = m0 + gemm::acc_row<C>(wm, 0, 0);
  const int64_t col0 = n0 + gemm::acc_col<C>(wn, 0);
  floatx16 acc[C::TM][C::TN];
#pragma unroll
  for (int i = 0; i < C::TM; ++i)
#pragma unroll
    for (int jj = 0; jj < C::TN; ++jj)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int dr = i * 32 + 8 * (r >> 2) + (r & 3);
        const bool ok = row0 + dr < M && col0 + jj * 32 < N;
        acc[i][jj][r] =
            preload ? cin.ld32(((row0 + dr) * j.ldcin + col0 + jj * 32) * 4, ok) : 0.f;
      }
  if constexpr (BT)
    gemm::mainloop_kn<C, BUF, false>(j.A + k0, j.lda, j.B + k0 * j.ldb, j.ldb, M, j.ldb, klen,
                                     m0, n0, smem, acc);
  else
    gemm::mainloop<C, BUF, false>(j.A + k0, j.lda, j.B + k0, j.ldb, M, N, klen, m0, n0, smem, acc);
  const float g = (!split && j.scale) ? *j.scale : 1.f;
  if constexpr (ct_vec_tiling<C>()) {
  if (ct && j.ct_vec) {
    // Transposed store through LDS (free after the K loop), so that global
    // stores are whole 16-byte vectors along m: in pass p the wavefronts of
    // column p (tile columns 64 p .. 64 p + 63) put their scaled accumulators
    // into LDS as 64 rows n of 256 m (row pitch 256 elements + 16 bytes, so
    // the 32 rows a write instruction touches start on different banks), then
    // every thread stores row vectors.  Needs M and ldc multiples of 8.
    const int es = dtype_bytes(cdt);
    const int pitch = 256 * es + 16;
    const int l = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int wm = w / C::WN, wn = w % C::WN;
    const int vpr = 256 * es / 16;  // 16-byte vectors per LDS row
#pragma unroll 1
    for (int p = 0; p < C::WN; ++p) {
      if (wn == p) {
#pragma unroll
        for (int i = 0; i < C::TM; ++i)
#pragma unroll
          for (int jj = 0; jj < C::TN; ++jj)
#pragma unroll
            for (int rq = 0; rq < 4; ++rq) {
              const int ml = wm * C::WTM + i * 32 + 8 * rq + 4 * (l >> 5);
              char *dst = smem + (jj * 32 + (l & 31)) * pitch + ml * es;
              float v[4];
#pragma unroll
              for (int q = 0; q < 4; ++q) v[q] = acc[i][jj][4 * rq + q] * g;
              if (es == 4) {
                u32x4 x;
                x.x = __float_as_uint(v[0]); x.y = __float_as_uint(v[1]);
                x.z = __float_as_uint(v[2]); x.w = __float_as_uint(v[3]);
                *reinterpret_cast<u32x4 *>(dst) = x;
              } else {
                u32x2 x;
                x.x = (uint32_t)to_half_bits(v[0], cdt) | ((uint32_t)to_half_bits(v[1], cdt) << 16);
                x.y = (uint32_t)to_half_bits(v[2], cdt) | ((uint32_t)to_half_bits(v[3], cdt) << 16);
                *reinterpret_cast<u32x2 *>(dst) = x;
              }
            }
      }
      __syncthreads();
      for (int e = threadIdx.x; e < 64 * vpr; e += C::NT) {
        const int nl = e / vpr, vi = e % vpr;
        const int64_t n = n0 + p * 64 + nl, m = m0 + (int64_t)vi * (16 / es);
        const u32x4 x = *reinterpret_cast<const u32x4 *>(smem + nl * pitch + vi * 16);
        out.st128((n * ldc + m) * es, n < N && m < M, x);
      }
      __syncthreads();
    }
    return;
  }
  }
  // the per-row factor of the lane's 16 rows of MFMA tile i (rows past M: 0)
  const float *rsc = split ? nullptr : j.row_scale;
  auto row_factors = [&](int i, float (&f)[16]) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int64_t row = row0 + i * 32 + 8 * (r >> 2) + (r & 3);
      f[r] = rsc ? (row < M ? rsc[row] * g : 0.f) : g;
    }
  };
  if (cdt == NF_DTYPE_F32) {
#pragma unroll
    for (int i = 0; i < C::TM; ++i) {
      float f[16];
      row_factors(i, f);
#pragma unroll
      for (int jj = 0; jj < C::TN; ++jj)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int dr = i * 32 + 8 * (r >> 2) + (r & 3);
          const bool ok = row0 + dr < M && col0 + jj * 32 < N;
          out.st32(idx(row0 + dr, col0 + jj * 32) * 4, ok, acc[i][jj][r] * f[r]);
        }
    }
  } else {
#pragma unroll
    for (int i = 0; i < C::TM; ++i) {
      float f[16];
      row_factors(i, f);
#pragma unroll
      for (int jj = 0; jj < C::TN; ++jj)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int dr = i * 32 + 8 * (r >> 2) + (r & 3);
          const bool ok = row0 + dr < M && col0 + jj * 32 < N;
          out.st16(idx(row0 + dr, col0 + jj * 32) * 2, ok,
                   to_half_bits(acc[i][jj][r] * f[r], cdt));
        }
    }
  }
}

template <class C, bool BUF, bool SB>
__global__ NF_GEMM_BOUNDS(C) void gemm_store_kernel(GemmJob<typename C::TI> j0,
                                                    GemmJob<typename C::TI> j1) {
  __shared__ __attribute__((aligned(16))) char smem[C::LDS_BYTES];
  // The job comes from the raw block index, so j0's blocks are dispatched
  // first and spread over all 8 XCDs (block b runs on XCD b % 8); the
  // XCD-grouped tile order applies within each job.  (Grouping the two jobs
  // together put a long first job on the first XCDs only: the cross-entropy
  // gradient launch with 256 long split-K blocks ahead of 1000 short ones
  // ran 2.4x its work on 64 of the 256 CUs.)  A job starting at a block
  // index that is not a multiple of 8 has its XCD groups rotated, which
  // keeps each group on one XCD.
  const bool second = (int)blockIdx.x >= j0.tiles;
  const GemmJob<typename C::TI> &j = second ? j1 : j0;
  const int b = second ? (int)blockIdx.x - j0.tiles : (int)blockIdx.x;
  int64_t M, K;
  job_extents(j, M, K);
  // With a device row count the job's tiles are renumbered over the rows
  // that exist, so its real blocks are the first ones and the rest exit at
  // once.  The dispatcher hands out blocks in order, round-robin over the
  // XCDs; exiting blocks left among the real ones (the last tile row of every
  // K slice) gathered on two XCDs, which then filled all their CUs with long
  // blocks and held up the dispatch of every later block.
  const int tiles_n = j.tiles / j.ksplit / j.tiles_m;
  int tiles_m = j.tiles_m, tiles = j.tiles;
  if (j.dyn && j.dyn_rows) {
    tiles_m = (int)((M + C::BM - 1) / C::BM);
    tiles = tiles_m * tiles_n * j.ksplit;
  }
  if (b >= tiles) return;
  int t = gemm::xcd_order(b, tiles);
  const int per_split = tiles_m * tiles_n;
  const int ks = t / per_split;  // K slice of this block
  int tm, tn;
  gemm::group_tile(t % per_split, tiles_m, tiles_n, gemm::kTileGroup, tm, tn);
  const int64_t m0 = (int64_t)tm * C::BM;
  const int64_t n0 = (int64_t)tn * C::BN;
  if constexpr (kn_tiling<C>()) {
    if (j.bt) {
      store_tile<C, BUF, SB, true>(j, M, K, ks, m0, n0, smem);
      return;
    }
  }
  store_tile<C, BUF, SB, false>(j, M, K, ks, m0, n0, smem);
}

// C[m, n] = scale * row_scale[m] * (Cin[m, n] + sum over s = 0 .. S-1 of
// part[s, m, n]), the slices added in order; C of element type cdt.  With `dyn`, only the
// first clamp(*dyn - dyn_base, 0, M) rows (the slices keep their M x N size).
static __global__ __launch_bounds__(256) void splitk_reduce_kernel(const float *__restrict__ part,
                                                            int S, int64_t M, int64_t N,
                                                            const float *Cin, void *C,
                                                            int64_t ldc, int cdt,
                                                            const float *scale,
                                                            const float *row_scale,
                                                            const int *dyn, int64_t dyn_base) {
  const int64_t total = M * N;  // slice stride
  int64_t rows = M;
  if (dyn) {
    rows = (int64_t)*dyn - dyn_base;
    rows = rows < 0 ? 0 : (rows > M ? M : rows);
  }
  const int64_t live = rows * N;
  const float g = scale ? *scale : 1.f;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < live;
       i += (int64_t)gridDim.x * 256) {
    // slices added in order 0 .. S-1; 8 loads in flight per batch
    constexpr int kBatch = 8;
    float a = 0.f;
    for (int k0 = 0; k0 < S; k0 += kBatch) {
      float v[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) v[u] = k0 + u < S ? part[(k0 + u) * total + i] : 0.f;
#pragma unroll
      for (int u = 0; u < kBatch; ++u)
        if (k0 + u < S) a += v[u];
    }
    const int64_t o = ldc == N ? i : (i / N) * ldc + i % N;  // dense C skips the division
    if (Cin) a = Cin[o] + a;
    store_dyn(C, cdt, o, a * (row_scale ? row_scale[i / N] * g : g));
  }
}


// ---------------------------------------------------------------------------
// transpose with zero padding: out[c, r] = in[r, c] (r < R), 0 for R <= r < ldo
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void transpose_pad_kernel(
    const T *__restrict__ in, int64_t R, int64_t Cn, int64_t ldi,
    T *__restrict__ out, int64_t ldo) {
  __shared__ T tile[64][65];
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  const int64_t r0 = (int64_t)blockIdx.x * 64, c0 = (int64_t)blockIdx.y * 64;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int64_t r = r0 + ty + 4 * i, c = c0 + tx;
    tile[ty + 4 * i][tx] = (r < R && c < Cn) ? in[r * ldi + c] : static_cast<T>(0.f);
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int64_t c = c0 + ty + 4 * i, r = r0 + tx;
    if (c < Cn && r < ldo) out[c * ldo + r] = tile[tx][ty + 4 * i];
  }
}

// 16-bit elements, 16-byte accesses: a 64 x 64 tile is read as 8-element row
// vectors and written as 8-element column vectors through LDS.  Requires
// Cn, ldi, ldo multiples of 8 and 16-byte aligned bases (a vector is then
// wholly inside or outside the matrix).
constexpr int kTpPitch = 66;  // LDS row pitch in elements (spreads column reads over banks)

static __global__ __launch_bounds__(256) void transpose16_kernel(
    const uint16_t *__restrict__ in, int64_t R, int64_t Cn, int64_t ldi,
    uint16_t *__restrict__ out, int64_t ldo) {
  __shared__ uint16_t tile[64 * kTpPitch];
  const int t = threadIdx.x;
  const int64_t r0 = (int64_t)blockIdx.x * 64, c0 = (int64_t)blockIdx.y * 64;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int row = t / 8 + 32 * i, vec = t % 8;
    const int64_t r = r0 + row, c = c0 + 8 * vec;
    u32x4 v = {0u, 0u, 0u, 0u};
    if (r < R && c < Cn) v = *reinterpret_cast<const u32x4 *>(in + r * ldi + c);
    uint16_t e[8];
    __builtin_memcpy(e, &v, 16);
#pragma unroll
    for (int q = 0; q < 8; ++q) tile[row * kTpPitch + 8 * vec + q] = e[q];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int oc = t / 8 + 32 * i, seg = t % 8;
    const int64_t c = c0 + oc, r = r0 + 8 * seg;
    uint16_t e[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) e[q] = tile[(8 * seg + q) * kTpPitch + oc];
    u32x4 v;
    __builtin_memcpy(&v, e, 16);
    if (c < Cn && r < ldo) *reinterpret_cast<u32x4 *>(out + c * ldo + r) = v;
  }
}


// The same transpose as one region of work inside another kernel (a GEMM
// launch whose last blocks transpose while its final partial wave of tiles
// leaves CUs idle): rows [r0, r0 + 256) x columns [c0, c0 + 128) of `in`
// become the corresponding columns / rows of `out`, rows R .. ldo - 1 of the
// region written as zeros.  NTH threads (a multiple of 256), all of which
// call it; `lds` holds kTpRegionRows * kTpRegionPitch elements.  Same
// requirements as transpose16_kernel.  Every thread first issues its eight
// 16-byte row loads, then writes them to LDS as 32-bit pairs; a half-wave's
// column reads cover 8 row segments x 4 column pairs, 32 distinct banks
// (pitch 130 elements: 8 rows = 520 dwords, 8 mod 64).
constexpr int kTpRegionRows = 256, kTpRegionCols = 128, kTpRegionPitch = 130;
template <int NTH>
__device__ __forceinline__ void transpose16_region(const uint16_t *__restrict__ in, int64_t R,
                                                   int64_t Cn, int64_t ldi,
                                                   uint16_t *__restrict__ out, int64_t ldo,
                                                   int64_t r0, int64_t c0, uint16_t *lds) {
  constexpr int VPR = kTpRegionCols / 8;           // 16-byte vectors per input row
  constexpr int NV = kTpRegionRows * VPR / NTH;    // input vectors per thread
  constexpr int SEGS = kTpRegionRows / 8;          // 16-byte vectors per output row
  constexpr int NO = kTpRegionCols * SEGS / NTH;   // output vectors per thread
  static_assert(NTH % 256 == 0 && NV >= 1 && NO >= 1 && NV * NTH == kTpRegionRows * VPR &&
                    NO * NTH == kTpRegionCols * SEGS, "region / thread mismatch");
  const int t = threadIdx.x;
  u32x4 v[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int idx = t + i * NTH, row = idx / VPR, vec = idx % VPR;
    const int64_t r = r0 + row, c = c0 + 8 * vec;
    v[i] = u32x4{0u, 0u, 0u, 0u};
    if (r < R && c < Cn) v[i] = *reinterpret_cast<const u32x4 *>(in + r * ldi + c);
  }
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int idx = t + i * NTH, row = idx / VPR, vec = idx % VPR;
    uint32_t *d = reinterpret_cast<uint32_t *>(lds + row * kTpRegionPitch + 8 * vec);
    d[0] = v[i][0]; d[1] = v[i][1]; d[2] = v[i][2]; d[3] = v[i][3];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < NO; ++i) {
    // lanes: 8 consecutive row segments x 8 columns; seg = low 3 bits of t
    // plus 8 per pair of iterations, column = t / 8 + 64 * (i % 2) (NTH 512)
    const int idx = t + i * NTH;
    const int seg = (idx % 8) + 8 * (idx / (8 * kTpRegionCols));
    const int oc = (idx / 8) % kTpRegionCols;
    const int64_t c = c0 + oc, r = r0 + 8 * seg;
    uint16_t e[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) e[q] = lds[(8 * seg + q) * kTpRegionPitch + oc];
    u32x4 o;
    __builtin_memcpy(&o, e, 16);
    if (c < Cn && r < ldo) *reinterpret_cast<u32x4 *>(out + c * ldo + r) = o;
  }
}

// Transposes folded into a launch: up to two 16-bit matrices, each cut into
// regions of kTpRegionRows x kTpRegionCols (rb x cb of them); `n` regions in
// all (0: none).
struct TpJobs {
  const uint16_t *in[2];
  uint16_t *out[2];
  int64_t R[2], Cn[2], ldi[2], ldo[2];
  int rb[2], cb[2];
  int n;
};

// Region `q` of the jobs (q < n): which matrix, and its region row / column.
template <int NTH>
__device__ __forceinline__ void tp_jobs_run(const TpJobs &tp, int q, uint16_t *lds) {
  const int n0 = tp.rb[0] * tp.cb[0];
  const int j = q < n0 ? 0 : 1;
  const int k = j ? q - n0 : q;
  const int rr = k % tp.rb[j], cc = k / tp.rb[j];
  transpose16_region<NTH>(tp.in[j], tp.R[j], tp.Cn[j], tp.ldi[j], tp.out[j], tp.ldo[j],
                          (int64_t)rr * kTpRegionRows, (int64_t)cc * kTpRegionCols, lds);
}

// rows x cols 16-bit elements of a matrix with row stride ld set to zero (a
// kernel rather than hipMemset2DAsync, so that a captured graph holds no
// memset node)
static __global__ __launch_bounds__(256) void zero16_kernel(uint16_t *__restrict__ p, int64_t ld,
                                                            int64_t rows, int64_t cols) {
  const int64_t total = rows * cols;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * 256)
    p[(i / cols) * ld + i % cols] = 0;
}

inline int launch_zero16(void *p, int64_t ld, int64_t rows, int64_t cols, hipStream_t s) {
  const int64_t total = rows * cols;
  if (total <= 0) return NF_OK;
  int64_t blocks = (total + 255) / 256;
  if (blocks > 1024) blocks = 1024;
  zero16_kernel<<<(unsigned)blocks, 256, 0, s>>>(static_cast<uint16_t *>(p), ld, rows, cols);
  return check_launch("zero16");
}

// bf16: 256x256 block tiles, 8 wavefronts of 128x64 (two per SIMD, so one
// wavefront's LDS waits and epilogue overlap the other's MFMAs), operands
// copied global -> LDS directly in 64-wide K-stages, two stage buffers; f32
// (correctness path): 128x128 tiles staged through registers.
template <typename TI>
struct MainCfgT;
template <>
struct MainCfgT<bf16> { using type = gemm::DCfg<256, 256, 2, 4, 2, 64>; };
template <>
struct MainCfgT<float> { using type = Cfg<float, 128, 128, 2, 2>; };
template <typename TI>
using MainCfg = typename MainCfgT<TI>::type;

inline int64_t round_up(int64_t x, int64_t m) { return (x + m - 1) / m * m; }
inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

template <class C>
GemmJob<typename C::TI> make_job(const typename C::TI *A, int64_t lda, const typename C::TI *B,
                                 int64_t ldb, const float *Cin, void *Cout, int cdt,
                                 const float *scale, int64_t ldc, int64_t M, int64_t N,
                                 int64_t K) {
  GemmJob<typename C::TI> j;
  j.A = A; j.B = B; j.Cin = Cin; j.C = Cout; j.scale = scale; j.row_scale = nullptr;
  j.lda = lda; j.ldb = ldb; j.ldc = ldc; j.M = M; j.N = N; j.K = K;
  j.cdt = cdt;
  j.tiles_m = (int)((M + C::BM - 1) / C::BM);
  j.tiles = j.tiles_m * (int)((N + C::BN - 1) / C::BN);
  j.ksplit = 1;
  j.kslice = K;
  j.part = nullptr;
  j.dyn = nullptr;
  j.dyn_base = 0;
  j.dyn_rows = 0;
  j.bt = 0;
  j.ct = 0;
  j.ct_vec = 0;
  j.ldcin = ldc;
  return j;
}

template <typename TI>
bool job_buf_ok(const GemmJob<TI> &j) {
  if (j.tiles == 0) return true;
  if (j.bt)  // B's K rows of ldb elements, read as whole 16-byte vectors
    return buf_ok<TI>(j.A, j.lda, j.M, j.K) && buf_ok<TI>(j.B, j.ldb, j.K, j.ldb);
  return buf_ok<TI>(j.A, j.lda, j.M, j.K) && buf_ok<TI>(j.B, j.ldb, j.N, j.K);
}
// every buffer the epilogue addresses through a 32-bit offset is under 2 GiB
template <typename TI>
bool job_sb_ok(const GemmJob<TI> &j) {
  if (j.tiles == 0) return true;
  if (j.ksplit > 1) return sb_ok(j.M * j.N * (int64_t)sizeof(float));
  const int64_t rows = j.ct ? j.N : j.M;
  return sb_ok(rows * j.ldc * (int64_t)dtype_bytes(j.cdt)) &&
         (!j.Cin || sb_ok(j.M * j.ldcin * (int64_t)sizeof(float)));
}

// Both jobs in one grid (j1 may be empty: tiles == 0), then the split-K
// reductions of a split job (unless `reduce` is false: the caller then adds
// the slices itself, as splitk_reduce_kernel would).
template <class C>
int launch_gemm_store(const GemmJob<typename C::TI> &j0_in, const GemmJob<typename C::TI> &j1_in,
                      hipStream_t s, bool reduce = true) {
  GemmJob<typename C::TI> j0 = j0_in, j1 = j1_in;
  for (auto *jp : {&j0, &j1})  // the LDS-transposed store where it applies
    jp->ct_vec = ct_vec_tiling<C>() && jp->ct && !jp->row_scale && jp->M % 8 == 0 &&
                 jp->ldc % 8 == 0;
  const int64_t total = (int64_t)j0.tiles + j1.tiles;
  if (total == 0) return NF_OK;
  if (total > 0x7fffffffLL) return set_error(NF_ERR_ARG, "gemm: too many tiles");
  for (const auto *jp : {&j0, &j1}) {
    if (jp->tiles == 0) continue;
    if (jp->bt && !kn_tiling<C>())
      return set_error(NF_ERR_ARG, "gemm: an N-major B needs the 16-bit 256-column tiling");
    if (jp->ct && jp->ksplit > 1)
      return set_error(NF_ERR_ARG, "gemm: a transposed C cannot be split along K");
  }
  const dim3 grid((unsigned)total);
  const bool sb = job_sb_ok(j0) && job_sb_ok(j1);
  const bool buf = job_buf_ok(j0) && job_buf_ok(j1);
  if (buf && sb)
    gemm_store_kernel<C, true, true><<<grid, C::NT, 0, s>>>(j0, j1);
  else if (buf)
    gemm_store_kernel<C, true, false><<<grid, C::NT, 0, s>>>(j0, j1);
  else
    gemm_store_kernel<C, false, false><<<grid, C::NT, 0, s>>>(j0, j1);
  if (int e = check_launch("gemm_store")) return e;
  if (!reduce) return NF_OK;
  for (const auto *jp : {&j0, &j1}) {
    if (jp->tiles == 0 || jp->ksplit <= 1) continue;
    int64_t blocks = (jp->M * jp->N + 255) / 256;
    if (blocks > 2048) blocks = 2048;
    splitk_reduce_kernel<<<(unsigned)blocks, 256, 0, s>>>(
        jp->part, jp->ksplit, jp->M, jp->N, jp->Cin, jp->C, jp->ldc, jp->cdt, jp->scale,
        jp->row_scale,
        jp->dyn_rows ? jp->dyn : nullptr, jp->dyn_base);
    if (int e = check_launch("splitk_reduce")) return e;
  }
  return NF_OK;
}

template <typename T>
int launch_transpose(const void *in, int64_t R, int64_t Cn, int64_t ldi, void *out,
                     int64_t ldo, hipStream_t s) {
  dim3 grid((unsigned)((ldo + 63) / 64), (unsigned)((Cn + 63) / 64));
  if (sizeof(T) == 2 && Cn % 8 == 0 && ldi % 8 == 0 && ldo % 8 == 0 && aligned16(in) &&
      aligned16(out))
    transpose16_kernel<<<grid, 256, 0, s>>>((const uint16_t *)in, R, Cn, ldi, (uint16_t *)out,
                                            ldo);
  else
    transpose_pad_kernel<T><<<grid, 256, 0, s>>>((const T *)in, R, Cn, ldi, (T *)out, ldo);
  return check_launch("transpose");
}


}  // namespace gemm
}  // namespace nf
