// SwiGLU as the epilogue of the gate/up projection GEMM:
//   a = x W_gate^T,  b = x W_up^T,  act = silu(a) * b
// in one MFMA kernel (the reference's SwiGLUMLP runs two GEMMs that write a
// and b to HBM and a SwiGLU kernel that reads them back, model/dit.py:96-110).
//
// Tiling.  A 256 x 256 block tile of the combined product x [W_gate; W_up]^T
// covers 256 tokens and 128 hidden units: tile columns 64 q .. 64 q + 31 are
// gate units u0 + 32 q .. + 31 and columns 64 q + 32 .. 64 q + 63 the up
// projections of the same units (u0 = 128 * tile column).  The direct-to-LDS
// loader hands each wavefront 32 consecutive tile rows of the B operand, so
// wavefront w simply copies its rows from W_up (w odd) or W_gate (w even):
// the interleave costs nothing and the weights are used in place.  With 8
// wavefronts of 128 x 64, a lane's two 32-column accumulator tiles are then
// a and b of the same (token, unit) pairs, and the epilogue is element-wise
// in registers: fp32 silu(a) * b rounded once, plus a and b rounded to the
// input type (what the backward needs; the caller may skip them).
#include "gemm_store.h"

namespace nf {
namespace swiglu_gemm {

using C = gemm::DCfg<256, 256, 2, 4, 2, 64>;
using gemm::floatx16;
static_assert(C::BN == 256 && C::NW == 8 && C::WM == 2 && C::WN == 4, "tiling assumed below");
static_assert(C::BCW * C::RPC == 32, "each wavefront must copy one 32-row group of B");
static_assert(C::TN == 2, "a lane's two column tiles are the gate and up halves");

constexpr uint32_t kOob = 0x80000000u;

struct Args {
  const bf16 *x;
  const bf16 *wg;
  const bf16 *wu;
  bf16 *a;    // [M, ldo] or null
  bf16 *b;    // [M, ldo] or null
  bf16 *act;  // [M, ldo]
  int64_t ldx, ldg, ldu, ldo, M, D, H;  // ldg / ldu: row strides of W_gate / W_up
  int tiles_m, tiles_n;
};

// 2-byte store through a buffer resource over a [M, ldo] output; masked
// elements get an out-of-range offset (dropped by the buffer unit).
__device__ __forceinline__ void st_bf16(__amdgpu_buffer_rsrc_t r, uint32_t off, bool ok, float v) {
  const bf16 h = static_cast<bf16>(v);
  uint16_t bits;
  __builtin_memcpy(&bits, &h, 2);
  __builtin_amdgcn_raw_buffer_store_b16(bits, r, ok ? off : kOob, 0, 0);
}

template <bool BUF>
__global__ NF_GEMM_BOUNDS(C) void gate_up_swiglu_kernel(Args p) {
  __shared__ __attribute__((aligned(16))) char smem[C::LDS_BYTES];
  int tm, tn;
  gemm::group_tile(gemm::xcd_order(blockIdx.x, p.tiles_m * p.tiles_n), p.tiles_m, p.tiles_n,
                   gemm::kTileGroup, tm, tn);
  const int64_t m0 = (int64_t)tm * C::BM;
  const int64_t u0 = (int64_t)tn * (C::BN / 2);  // first hidden unit of the tile
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));

  floatx16 acc[C::TM][C::TN];
#pragma unroll
  for (int i = 0; i < C::TM; ++i)
#pragma unroll
    for (int j = 0; j < C::TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
  gemm::DtlOperand<C, C::ACW> opa;
  gemm::DtlOperand<C, C::BCW> opb;
  opa.init(p.x, p.ldx, p.M, p.D, m0, wave);
  // wavefront w copies tile rows 32 w .. 32 w + 31: units u0 + 32 (w / 2) + 0..31
  // of W_up (w odd) or W_gate (w even); r0 makes tile row 32 w that matrix row
  const int64_t unit0 = u0 + 32 * (wave >> 1);
  opb.init((wave & 1) ? p.wu : p.wg, (wave & 1) ? p.ldu : p.ldg, p.H, p.D, unit0 - 32 * wave,
           wave);
  gemm::mainloop_dtl_ops<C, BUF, true>(opa, opb, p.D, smem, acc);

  const int l = threadIdx.x & 63;
  const int w = threadIdx.x >> 6, wm = w / C::WN, wn = w % C::WN;
  const int64_t unit = u0 + 32 * wn + (l & 31);
  const int64_t row0 = m0 + wm * C::WTM + 4 * (l >> 5);
  const int64_t bytes = p.M * p.ldo * 2;
  const __amdgpu_buffer_rsrc_t ract =
      __builtin_amdgcn_make_buffer_rsrc(p.act, (short)0, (int)bytes, 0x00020000);
  __amdgpu_buffer_rsrc_t ra = ract, rb = ract;
  if (p.a) ra = __builtin_amdgcn_make_buffer_rsrc(p.a, (short)0, (int)bytes, 0x00020000);
  if (p.b) rb = __builtin_amdgcn_make_buffer_rsrc(p.b, (short)0, (int)bytes, 0x00020000);
  const bool save = p.a != nullptr;
#pragma unroll
  for (int i = 0; i < C::TM; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int64_t row = row0 + i * 32 + 8 * (r >> 2) + (r & 3);
      const bool ok = row < p.M && unit < p.H;
      const uint32_t off = (uint32_t)((row * p.ldo + unit) * 2);
      const float av = acc[i][0][r], bv = acc[i][1][r];
      st_bf16(ract, off, ok, av * sigmoid(av) * bv);
      if (save) {
        st_bf16(ra, off, ok, av);
        st_bf16(rb, off, ok, bv);
      }
    }
}

// ---------------------------------------------------------------------------
// Weight gradients of the gate/up projection: dW_gate = da^T x and
// dW_up = db^T x (the Linears' weight gradients in the reference's
// SwiGLUMLP backward, model/dit.py:104-110).  Long in K (the tokens) and small
// in output (H x D), these are the shape a library GEMM handles worst; here
// da, db and x are transposed to K-contiguous [H, M] and [D, M] copies, both
// products run in one launch split along K so that it fills the chip, and the
// fixed-order split-K reduce writes the bf16 gradients.
// ---------------------------------------------------------------------------
// rows x ld elements of `es` bytes stay under 2 GiB (32-bit buffer offsets);
// divides instead of multiplying, so absurd sizes cannot overflow the test
inline bool under_2gib(int64_t rows, int64_t ld, int64_t es) {
  const int64_t lim = ((int64_t)1 << 31) - 64;
  if (rows < 0 || ld <= 0) return false;
  if (ld > lim / es) return rows == 0;
  return rows <= (lim - 1) / (ld * es);
}

namespace wgrad {
struct Layout {
  int64_t ldt;     // row stride of the transposed copies (tokens, padded to 8)
  int S;           // K slices per product
  int64_t kslice;  // tokens per slice (a multiple of the stage width)
  size_t off_dat, off_dbt, off_xt, off_part, total;
};
inline Layout layout(int64_t M, int64_t D, int64_t H) {
  using C = gemm::DCfg<256, 256, 2, 4, 2, 64>;
  Layout L{};
  L.ldt = gemm::round_up(M, 8);
  const int64_t tiles = ((H + C::BM - 1) / C::BM) * ((D + C::BN - 1) / C::BN);
  // fill one wave of 256 blocks with both products, slices of >= 256 tokens
  int64_t S = 256 / (2 * tiles);
  const int64_t smax = (L.ldt + 255) / 256;
  if (S > smax) S = smax;
  if (S > 64) S = 64;
  if (S < 1) S = 1;
  L.kslice = gemm::round_up((L.ldt + S - 1) / S, C::BK);
  L.S = (int)((L.ldt + L.kslice - 1) / L.kslice);
  size_t o = 0;
  auto take = [&](size_t bytes) { const size_t at = o; o = gemm::align256(o + bytes); return at; };
  L.off_dat = take((size_t)H * L.ldt * 2);
  L.off_dbt = take((size_t)H * L.ldt * 2);
  L.off_xt = take((size_t)D * L.ldt * 2);
  L.off_part = take(L.S > 1 ? (size_t)2 * L.S * H * D * sizeof(float) : 0);
  L.total = o;
  return L;
}
}  // namespace wgrad

}  // namespace swiglu_gemm
}  // namespace nf

using namespace nf;

extern "C" int nf_gemm_swiglu(const void *x, int64_t ldx, const void *w_gate, int64_t ld_gate,
                              const void *w_up, int64_t ld_up, void *a, void *b, void *act,
                              int64_t ldo, int64_t M, int64_t D, int64_t H, int dtype,
                              void *stream) {
  using namespace nf::swiglu_gemm;
  if (M < 0 || D <= 0 || H <= 0)
    return set_error(NF_ERR_ARG, "nf_gemm_swiglu: bad shape M=%lld D=%lld H=%lld",
                     (long long)M, (long long)D, (long long)H);
  if (M == 0) return NF_OK;
  if (dtype != NF_DTYPE_BF16)
    return set_error(NF_ERR_DTYPE, "nf_gemm_swiglu: dtype %d unsupported (bf16 only)", dtype);
  if (!x || !w_gate || !w_up || !act || (!a) != (!b))
    return set_error(NF_ERR_ARG, "nf_gemm_swiglu: null pointer (a and b: both or neither)");
  if (ldx < D || ld_gate < D || ld_up < D || ldo < H)
    return set_error(NF_ERR_ARG, "nf_gemm_swiglu: bad leading dimension");
  // 32-bit buffer offsets: every operand and output under 2 GiB
  if (!under_2gib(M, ldx, 2) || !under_2gib(H, ld_gate, 2) || !under_2gib(H, ld_up, 2) ||
      !under_2gib(M, ldo, 2))
    return set_error(NF_ERR_ARG, "nf_gemm_swiglu: an operand exceeds 2 GiB");
  const int64_t tiles_m = (M + C::BM - 1) / C::BM, tiles_n = (H + C::BN / 2 - 1) / (C::BN / 2);
  if (tiles_m * tiles_n > 0x7fffffffLL)
    return set_error(NF_ERR_ARG, "nf_gemm_swiglu: grid too large");
  Args args{static_cast<const bf16 *>(x), static_cast<const bf16 *>(w_gate),
            static_cast<const bf16 *>(w_up), static_cast<bf16 *>(a), static_cast<bf16 *>(b),
            static_cast<bf16 *>(act), ldx, ld_gate, ld_up, ldo, M, D, H, (int)tiles_m,
            (int)tiles_n};
  const bool buf = D % 8 == 0 && ldx % 8 == 0 && ld_gate % 8 == 0 && ld_up % 8 == 0 &&
                   aligned16(x) && aligned16(w_gate) && aligned16(w_up);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const unsigned grid = (unsigned)(tiles_m * tiles_n);
  if (buf)
    gate_up_swiglu_kernel<true><<<grid, C::NT, 0, s>>>(args);
  else
    gate_up_swiglu_kernel<false><<<grid, C::NT, 0, s>>>(args);
  return check_launch("nf_gemm_swiglu");
}

extern "C" size_t nf_gemm_swiglu_wgrad_workspace(int64_t M, int64_t D, int64_t H) {
  const int64_t big = (int64_t)1 << 31;  // beyond what the entry point accepts
  if (M <= 0 || D <= 0 || H <= 0 || M > big || D > big || H > big) return 0;
  return nf::swiglu_gemm::wgrad::layout(M, D, H).total;
}

extern "C" int nf_gemm_swiglu_wgrad(const void *da, const void *db, int64_t ld_ab, const void *x,
                                    int64_t ldx, void *dw_gate, void *dw_up, int64_t ldw,
                                    int64_t M, int64_t D, int64_t H, int dtype, void *workspace,
                                    size_t workspace_bytes, void *stream) {
  using namespace nf::gemm;
  using C = DCfg<256, 256, 2, 4, 2, 64>;
  if (M < 0 || D <= 0 || H <= 0)
    return set_error(NF_ERR_ARG, "nf_gemm_swiglu_wgrad: bad shape M=%lld D=%lld H=%lld",
                     (long long)M, (long long)D, (long long)H);
  if (dtype != NF_DTYPE_BF16)
    return set_error(NF_ERR_DTYPE, "nf_gemm_swiglu_wgrad: dtype %d unsupported (bf16 only)",
                     dtype);
  if (!dw_gate || !dw_up || (M > 0 && (!da || !db || !x)))
    return set_error(NF_ERR_ARG, "nf_gemm_swiglu_wgrad: null pointer");
  if (ld_ab < H || ldx < D || ldw < D)
    return set_error(NF_ERR_ARG, "nf_gemm_swiglu_wgrad: bad leading dimension");
  using nf::swiglu_gemm::under_2gib;
  if (!under_2gib(M, ld_ab, 2) || !under_2gib(M, ldx, 2) || !under_2gib(H, ldw, 2))
    return set_error(NF_ERR_ARG, "nf_gemm_swiglu_wgrad: an operand exceeds 2 GiB");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (M == 0) {  // no tokens: zero gradients
    int e = launch_zero16(dw_gate, ldw, H, D, s);
    return e ? e : launch_zero16(dw_up, ldw, H, D, s);
  }
  const nf::swiglu_gemm::wgrad::Layout L = nf::swiglu_gemm::wgrad::layout(M, D, H);
  if (!workspace || workspace_bytes < L.total || !aligned16(workspace))
    return set_error(NF_ERR_WORKSPACE, "nf_gemm_swiglu_wgrad: workspace %zu bytes < required %zu",
                     workspace_bytes, L.total);
  if (!under_2gib(H, L.ldt, 2) || !under_2gib(D, L.ldt, 2) ||
      (L.S > 1 && !under_2gib(H, D, sizeof(float))))
    return set_error(NF_ERR_ARG, "nf_gemm_swiglu_wgrad: a transposed operand exceeds 2 GiB");
  char *ws = static_cast<char *>(workspace);
  bf16 *dat = reinterpret_cast<bf16 *>(ws + L.off_dat);
  bf16 *dbt = reinterpret_cast<bf16 *>(ws + L.off_dbt);
  bf16 *xt = reinterpret_cast<bf16 *>(ws + L.off_xt);
  float *part = reinterpret_cast<float *>(ws + L.off_part);
  int e;
  if ((e = launch_transpose<uint16_t>(da, M, H, ld_ab, dat, L.ldt, s))) return e;
  if ((e = launch_transpose<uint16_t>(db, M, H, ld_ab, dbt, L.ldt, s))) return e;
  if ((e = launch_transpose<uint16_t>(x, M, D, ldx, xt, L.ldt, s))) return e;
  auto jg = make_job<C>(dat, L.ldt, xt, L.ldt, nullptr, dw_gate, NF_DTYPE_BF16, nullptr, ldw, H,
                        D, L.ldt);
  auto ju = make_job<C>(dbt, L.ldt, xt, L.ldt, nullptr, dw_up, NF_DTYPE_BF16, nullptr, ldw, H,
                        D, L.ldt);
  if (L.S > 1) {
    jg.ksplit = ju.ksplit = L.S;
    jg.kslice = ju.kslice = L.kslice;
    jg.tiles *= L.S;
    ju.tiles *= L.S;
    jg.part = part;
    ju.part = part + (size_t)L.S * H * D;
  }
  return launch_gemm_store<C>(jg, ju, s);
}
