// Chunked cross entropy on the MFMA GEMM core of gemm_core.h, in two calls,
// all on the caller's stream with fixed reduction orders (no atomics).
//
// Only valid rows (target != ignore_index, inside [0, V)) do any work: the
// forward compacts them on the device (no count reaches the host), and every
// later kernel sizes itself by that device count.  The logits are formed once
// per row (6 * n_valid * V * D flops in all: logits, dH, dW), never twice.
//
// Forward (nf_ce_fwd):
//   1. ce_compact: the valid rows in order -> rows[], their target columns,
//      pos[m] (compacted index or -1), n_valid, inv = 1 / max(n_valid, 1).
//   2. ce_gather: Hc = H[rows] ([M, D], zero past n_valid) and each valid
//      row's target logit mref = Hc[r] . W[target], the row's reference.
//      Wt = W^T [D, V] (zero-padded; the dH product's K-contiguous B
//      operand) is formed by the first logits launch's last blocks (16-bit
//      inputs) or by a transpose launch here (fp32).
//   3. per chunk of `crows` compacted rows:
//      ce_logits: S = Hc_c W^T tile by tile (formed transposed, W Hc_c^T, so a
//                 lane holds each token's logits along the vocabulary); per
//                 (vocabulary tile of WTM rows, token) the max and the sum of
//                 exp(S - max), the target logit, and E = exp(S - mref) in
//                 the input type, row-major [crows, ldp] and (unless E is
//                 held once: "single", see Plan) transposed [V, crows];
//      ce_lse:    lse per row from the tile statistics (fixed order), the
//                 row's loss lse - S[target], the row factor cfac =
//                 exp(mref - lse) / n, and the one-hot term folded into E's
//                 target entry, so cfac * E = (softmax - onehot) / n; rows
//                 whose maximum lies far above mref are rescaled to it;
//      ce_scale_hct: Hct = (cfac * Hc_c)^T, the dW product's B operand; in
//                 the last chunk's launch, also the mean loss;
//      gradient products of every chunk but the last (one launch):
//                 dW_acc (+)= E^T_c Hct_c^T  (fp32 [V, D], K = the chunk's rows;
//                             single: dW_acc^T (+)= Hct_c E_c, fp32 [D, V],
//                             E read N-major)
//                 dHc_c   = cfac * (E_c Wt^T) (fp32, K = V, split along K)
// Backward (nf_ce_bwd, with the loss's grad_output g): the last chunk's
// products, dW = g * (dW_acc + E^T Hct^T) written in dweight's type (single:
// formed transposed and stored through LDS as [V, D]), and the scatter of
// dHc back to the hidden rows as g * dH (0 for ignored rows).
//
// Memory: the state kept between the calls holds one chunk's E (once, for
// twice the rows, when single), W^T, the scaled Hc^T and the fp32 dH rows,
// plus the fp32 dW accumulator when there is more than one chunk; E and the
// accumulator stay within the bytes the reference's chunk loop holds for
// them (see make_plan), so E covers every row at once only where that fits.
#include <type_traits>

#include "gemm_store.h"

namespace nf {
namespace ce {

using namespace gemm;

__device__ __forceinline__ float log_f32(float x) {
  constexpr float kLn2 = 0.6931471805599453f;  // ln(2)
  return __builtin_amdgcn_logf(x) * kLn2;       // log2 on the hardware
}

__device__ __forceinline__ float2 combine_stats(float2 a, float2 b) {
  const float m = fmaxf(a.x, b.x);
  if (m == -INFINITY) return make_float2(m, 0.f);
  return make_float2(m, a.y * exp_f32(a.x - m) + b.y * exp_f32(b.x - m));
}

__device__ __forceinline__ int64_t chunk_count(const int *n_ptr, int64_t j0, int64_t crows) {
  const int64_t c = (int64_t)__builtin_amdgcn_readfirstlane(*n_ptr) - j0;
  return c < 0 ? 0 : (c > crows ? crows : c);
}

// ---------------------------------------------------------------------------
// 1. compaction of the valid rows, in order.  One block; each round takes
// 4 x 1024 targets, each wavefront ranks its lanes by a ballot, and the
// per-wavefront counts are prefixed through LDS in wavefront order.
// ---------------------------------------------------------------------------
constexpr int kCompactThreads = 1024, kCompactSub = 4;

__global__ __launch_bounds__(kCompactThreads) void ce_compact_kernel(
    const int64_t *__restrict__ targets, int64_t M, int64_t V, int64_t ignore_index,
    int *__restrict__ rows, int *__restrict__ tcol, int *__restrict__ pos, int *n_out,
    float *inv_out, int *bad_out) {
  constexpr int kWaves = kCompactThreads / 64;
  __shared__ int wsum[kCompactSub][kWaves];
  __shared__ int wbad[kCompactSub][kWaves];
  const int l = threadIdx.x & 63, w = threadIdx.x >> 6;
  const uint64_t below = (1ull << l) - 1ull;
  int carry = 0, bad_total = 0;  // the same in every thread
  for (int64_t base = 0; base < M; base += kCompactThreads * kCompactSub) {
    int64_t tg[kCompactSub];
    bool valid[kCompactSub];
    int before[kCompactSub];
#pragma unroll
    for (int u = 0; u < kCompactSub; ++u) {
      const int64_t m = base + (int64_t)u * kCompactThreads + threadIdx.x;
      tg[u] = m < M ? targets[m] : ignore_index;
      const bool in_range = tg[u] >= 0 && tg[u] < V;
      valid[u] = m < M && tg[u] != ignore_index && in_range;
      const bool bad = m < M && tg[u] != ignore_index && !in_range;
      const uint64_t vm = __ballot(valid[u]);
      const uint64_t bm = __ballot(bad);
      before[u] = __popcll(vm & below);
      if (l == 0) {
        wsum[u][w] = __popcll(vm);
        wbad[u][w] = __popcll(bm);
      }
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < kCompactSub; ++u) {
      int off = carry, tot = 0, btot = 0;
      for (int k = 0; k < kWaves; ++k) {
        off += k < w ? wsum[u][k] : 0;
        tot += wsum[u][k];
        btot += wbad[u][k];
      }
      const int64_t m = base + (int64_t)u * kCompactThreads + threadIdx.x;
      if (m < M) {
        if (valid[u]) {
          const int idx = off + before[u];
          rows[idx] = (int)m;
          tcol[idx] = (int)tg[u];
          pos[m] = idx;
        } else {
          pos[m] = -1;
        }
      }
      carry += tot;
      bad_total += btot;
    }
    __syncthreads();  // wsum / wbad are rewritten by the next round
  }
  if (threadIdx.x == 0) {
    *n_out = carry;
    *inv_out = 1.f / (float)(carry > 1 ? carry : 1);
    if (bad_out) *bad_out = bad_total;
  }
}

// ---------------------------------------------------------------------------
// 2. Hc[r, :] = H[rows[r], :] for r < n_valid, 0 for n_valid <= r < R, and
// the row's reference logit mref[r] = H[rows[r], :] . W[tcol[r], :] (fp32, a
// fixed-order sum; 0 past n_valid).  One wavefront per row.  E is stored
// relative to mref (exp(S - mref)), so mref needs only to lie within the
// exponent range of the row's largest logit; the target logit does for every
// row whose loss is below ~50 nats, and for any other row the logits pass
// keeps E in range and the statistics pass rescales it (ce_lse_kernel).
// VEC: 16-byte vectors
// (D a multiple of the vector width, aligned rows).
// ---------------------------------------------------------------------------
constexpr int kGatherThreads = 256;

template <typename T, bool VEC>
__global__ __launch_bounds__(kGatherThreads) void ce_gather_kernel(
    const T *__restrict__ H, const T *__restrict__ W, int64_t D, const int *__restrict__ rows,
    const int *__restrict__ tcol, const int *n_ptr, int64_t R, T *__restrict__ Hc,
    float *__restrict__ mref) {
  constexpr int kWaves = kGatherThreads / 64;
  const int64_t n = *n_ptr;
  constexpr int VE = VEC ? 16 / (int)sizeof(T) : 1;
  const int l = threadIdx.x & 63;
  for (int64_t r = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6); r < R;
       r += (int64_t)gridDim.x * kWaves) {
    const bool live = r < n;
    const T *h = live ? H + (int64_t)rows[r] * D : nullptr;
    const T *w = live ? W + (int64_t)tcol[r] * D : nullptr;
    float dot = 0.f;
    for (int64_t c = (int64_t)l * VE; c < D; c += 64 * VE) {
      if constexpr (VEC) {
        u32x4 hv = {0u, 0u, 0u, 0u}, wv = {0u, 0u, 0u, 0u};
        if (live) {
          hv = *reinterpret_cast<const u32x4 *>(h + c);
          wv = *reinterpret_cast<const u32x4 *>(w + c);
        }
        *reinterpret_cast<u32x4 *>(Hc + r * D + c) = hv;
        T he[VE], we[VE];
        __builtin_memcpy(he, &hv, 16);
        __builtin_memcpy(we, &wv, 16);
#pragma unroll
        for (int q = 0; q < VE; ++q) dot += static_cast<float>(he[q]) * static_cast<float>(we[q]);
      } else {
        const T hv = live ? h[c] : static_cast<T>(0.f);
        Hc[r * D + c] = hv;
        if (live) dot += static_cast<float>(hv) * static_cast<float>(w[c]);
      }
    }
    dot = wave_sum(dot);
    if (l == 0) mref[r] = live ? dot : 0.f;
  }
}

// ---------------------------------------------------------------------------
// 3. logits of one chunk, their tile statistics and E = exp(S - mref) in the
// input type, row-major and transposed.  The product is formed transposed,
// acc = W_tile Hc_tile^T (rows: vocabulary entries, columns: tokens), so each
// lane holds 16 * TM logits of each of its TN tokens: a wavefront's max and
// sum of exp over its WTM vocabulary rows are reductions in registers plus
// one exchange between the lane halves.  Statistics tile t covers vocabulary
// rows [t * WTM, (t + 1) * WTM): stats[t * crows + token] = (max, sum
// exp(S - max)), taken from the sum of E (see the epilogue).  The target
// logit comes from the one lane holding it.  E = exp(S - mref) goes out
// row-major [token, ldp] (columns V..ldp zero, tokens past the chunk's rows
// zero up to a multiple of 8) and, when ET is given, transposed [V, ldet]
// (tokens past the chunk's rows zero up to a multiple of 8): with 16-bit
// 256 x 256 tiles through LDS (free once the K loop ends) -- element (t, c)
// at byte t * 512 + 2 * (c ^ e_swz(t)), the XOR moving whole 8-element
// vectors so rows still read as 16-byte vectors while the writes of a
// half-wave spread over the banks, and a column gathers its 8 tokens per
// vector from 8 rows; otherwise straight from the accumulators.  With a row
// factor P = inv * exp(mref - lse) (ce_lse_kernel), P * E is the softmax.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int e_swz(int t) { return 8 * (((t >> 3) ^ (t & 7)) & 31); }
constexpr float kStatsGap = 64.f;  // exp(-64) of a row maximum is below fp32 resolution
// E entries relative to mref stay below exp(kBaseGap): a wavefront whose
// maximum for a token lies further above mref stores that token's E relative
// to its own maximum instead (see the epilogue)
constexpr float kBaseGap = 60.f;

// Blocks past the vtiles x ttiles logits tiles run the transpose regions of
// `tp` (16-bit inputs only): dispatched last, they fill the CUs that the
// final partial wave of tiles leaves idle.
template <class C, bool BUF, bool SB>
__global__ NF_GEMM_BOUNDS(C) void ce_logits_kernel(
    const typename C::TI *W, const typename C::TI *Hc, int64_t V, int64_t D, int64_t j0,
    int64_t crows, const int *n_ptr, const int *tcol, const float *mref, float2 *stats,
    float *tgt, typename C::TI *E, int64_t ldp, typename C::TI *ET, int64_t ldet, int vtiles,
    int ttiles, gemm::TpJobs tp) {
  using TI = typename C::TI;
  constexpr int ES = (int)sizeof(TI);
  // one LDS buffer only: a second __shared__ object makes the compiler wait
  // for every direct-to-LDS copy in flight before each operand read of the
  // K loop; the E staging and the transposes reuse the operand stages
  __shared__ __attribute__((aligned(16))) char smem[C::LDS_BYTES];
  if constexpr (ES == 2) {
    static_assert(C::LDS_BYTES >= gemm::kTpRegionRows * gemm::kTpRegionPitch * 2,
                  "transpose region does not fit the LDS");
    const int q = (int)blockIdx.x - vtiles * ttiles;
    if (q >= 0) {
      if (q < tp.n) gemm::tp_jobs_run<C::NT>(tp, q, reinterpret_cast<uint16_t *>(smem));
      return;
    }
  }
  int vt, tt;
  gemm::group_tile(gemm::xcd_order(blockIdx.x, vtiles * ttiles), vtiles, ttiles,
                   gemm::kTileGroup, vt, tt);
  const int64_t cnt = chunk_count(n_ptr, j0, crows);
  const int64_t v0 = (int64_t)vt * C::BM;
  const int64_t t0 = (int64_t)tt * C::BN;  // first token of the tile, chunk-local
  if (t0 >= cnt) return;
  floatx16 acc[C::TM][C::TN];
  gemm::mainloop<C, BUF>(W, D, Hc + j0 * D, D, V, cnt, D, v0, t0, smem, acc);

  const int l = threadIdx.x & 63, half = l >> 5;
  const int w = threadIdx.x >> 6, wm = w / C::WN, wn = w % C::WN;
  const int64_t vtile0 = v0 + wm * C::WTM;      // first vocabulary row of this wavefront
  const int64_t crow0 = vtile0 + 4 * half;      // vocabulary row of (i = 0, r = 0)
  const int stile = vt * C::WM + wm;            // statistics tile
  // Rows past the vocabulary (only in a wavefront whose rows reach V) are set
  // to -inf once, so the max, the sum and E need no per-element masks.
  if (vtile0 + C::WTM > V) {
    const int vlim = (int)(V - crow0 < C::WTM ? V - crow0 : C::WTM);
#pragma unroll
    for (int i = 0; i < C::TM; ++i)
#pragma unroll
      for (int j = 0; j < C::TN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (i * 32 + 8 * (r >> 2) + (r & 3) >= vlim) acc[i][j][r] = -INFINITY;
  }
  constexpr bool kStaged = ES == 2 && C::BM == 256 && C::BN == 256 && C::NT == 512 &&
                           C::LDS_BYTES >= 256 * 512;
  OutBuf<SB> eout, etout;
  eout.init(E, crows * ldp * ES);
  etout.init(ET, V * ldet * ES);
  const int64_t cnt8 = (cnt + 7) / 8 * 8;
#pragma unroll
  for (int j = 0; j < C::TN; ++j) {
    const int tl = wn * C::WTN + j * 32 + (l & 31);  // token within the tile
    const int64_t tok = t0 + tl;                     // token within the chunk
    const float mr = tok < cnt ? mref[j0 + tok] : 0.f;  // the row's reference
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < C::TM; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, acc[i][j][r]);
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    // the target logit, from the one lane that holds it (before the exp)
    if (tok < cnt) {
      const int64_t loc64 = (int64_t)tcol[j0 + tok] - vtile0;
      const int loc = (int)(loc64 >= 0 && loc64 < C::WTM ? loc64 : -1);
      if (loc >= 0 && ((loc >> 2) & 1) == half) {
        const int want = ((loc >> 5) << 4) | (((loc & 31) >> 3) << 2) | (loc & 3);
        float z = 0.f;
#pragma unroll
        for (int i = 0; i < C::TM; ++i)
#pragma unroll
          for (int r = 0; r < 16; ++r) z = (i * 16 + r == want) ? acc[i][j][r] : z;
        tgt[tok] = z;
      }
    }
    // E = exp(S - mref) relative to the row's reference (rows past V are -inf
    // and give 0; S - mref is exact where S is near mref, so the target's own
    // entry is exactly 1).  The tile's statistics
    // follow from its sum: s = sum exp(S - mx) = exp(mref - mx) * sum E.  A
    // tile more than kStatsGap below mref keeps s = 1: its share of the row
    // total, below exp(-kStatsGap) of the row maximum's, is under fp32
    // resolution.  Where the maximum lies more than kBaseGap above mref (a
    // row far from its reference), E = exp(S - mx) instead, so no entry
    // leaves the exponent range, and s = sum E is stored negated: the
    // statistics pass then rescales the row to its maximum.  A wavefront
    // with no row inside the vocabulary keeps (-inf, 0).
    const bool own = mx - mr > kBaseGap;
    const float base = own ? mx : mr;
#pragma unroll
    for (int i = 0; i < C::TM; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = exp_f32(acc[i][j][r] - base);
    float se = 0.f;
#pragma unroll
    for (int i = 0; i < C::TM; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) se += acc[i][j][r];
    se += __shfl_xor(se, 32);
    const float s = mx == -INFINITY ? 0.f
                    : own           ? -se
                    : (mr - mx > kStatsGap ? 1.f : se * exp_f32(mr - mx));
    if (half == 0 && tok < cnt) stats[(int64_t)stile * crows + tok] = make_float2(mx, s);

#pragma unroll
    for (int i = 0; i < C::TM; ++i)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int o = i * 32 + 8 * g;  // offset of r = 4g from crow0
        TI ev[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) ev[q] = static_cast<TI>(acc[i][j][4 * g + q]);
        if constexpr (kStaged) {
          const int cl = wm * C::WTM + 4 * half + o;  // tile column (vocabulary)
          u32x2 packed;
          __builtin_memcpy(&packed, ev, 8);
          *reinterpret_cast<u32x2 *>(smem + tl * 512 + 2 * (cl ^ e_swz(tl))) = packed;
        } else {
          // straight from the accumulators: E row-major and E^T (zero past
          // the chunk's rows, up to the K padding of the dW product)
          const int64_t c = crow0 + o;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const TI e = tok < cnt ? ev[q] : static_cast<TI>(0.f);
            if constexpr (ES == 2) {
              uint16_t bits;
              __builtin_memcpy(&bits, &e, 2);
              eout.st16((tok * ldp + c + q) * ES, tok < cnt && c + q < ldp, bits);
              etout.st16(((c + q) * ldet + tok) * ES, c + q < V && tok < cnt8, bits);
            } else {
              eout.st32((tok * ldp + c + q) * ES, tok < cnt && c + q < ldp,
                        static_cast<float>(e));
              etout.st32(((c + q) * ldet + tok) * ES, c + q < V && tok < cnt8,
                         static_cast<float>(e));
            }
          }
        }
      }
  }
  if constexpr (kStaged) {
    __syncthreads();
    // wavefront w stores tile rows (tokens) 32 w .. 32 w + 31, two per
    // instruction (one per half-wave), as 16-byte vectors; ldp is a multiple
    // of 8, so a vector is wholly inside or outside the row.  Rows from the
    // chunk's count up to a multiple of 8 are zero (K padding of the dW
    // product when it reads E N-major).
    const int hv = l >> 5, c8 = 8 * (l & 31);
#pragma unroll 4
    for (int it = 0; it < 16; ++it) {
      const int t = 32 * w + 2 * it + hv;
      const int64_t tok = t0 + t, c = v0 + c8;
      const u32x4 v = tok < cnt ? *reinterpret_cast<const u32x4 *>(smem + t * 512 +
                                                                    2 * (c8 ^ e_swz(t)))
                                : u32x4{0u, 0u, 0u, 0u};
      eout.st128((tok * ldp + c) * ES, tok < cnt8 && c < ldp, v);
    }
    if (ET == nullptr) return;  // E held once (the dW product reads it N-major)
    // E^T through transposing LDS reads (ds_read_b64_tr_b16: in each 16-lane
    // group, lane i receives element i % 4 of the 8-byte chunks addressed by
    // lanes i / 4 + 4 q, q = 0..3).  Lane j of a group addresses token row
    // T + 8 (j % 4) + j / 4 (+ 4 for the second read) at tile columns c0 ..
    // c0 + 3, so lane i gets tokens T + 8 (i / 4) .. + 7 of column c0 + i % 4:
    // one 16-byte E^T vector.  A wavefront covers 16 columns x 32 tokens per
    // step, wavefront w columns 32 w .. 32 w + 31; tokens past the chunk's
    // rows are zero up to cnt8 (the dW product's K padding), none beyond.
    typedef short v4s __attribute__((ext_vector_type(4)));
    const int grp = l >> 4, j = l & 15;
#pragma unroll 2
    for (int k = 0; k < 16; ++k) {
      const int C0 = 32 * w + 16 * (k >> 3), T = 32 * (k & 7);
      const int c0 = C0 + 4 * grp;
      const int ra = T + 8 * (j & 3) + (j >> 2), rb = ra + 4;
      const v4s a = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) v4s *)(smem + ra * 512 + 2 * (c0 ^ e_swz(ra))));
      const v4s b = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) v4s *)(smem + rb * 512 + 2 * (c0 ^ e_swz(rb))));
      const int64_t v = v0 + c0 + (j & 3), tok = t0 + T + 8 * (j >> 2);
      uint16_t e[8];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        e[q] = tok + q < cnt ? (uint16_t)a[q] : (uint16_t)0;
        e[4 + q] = tok + 4 + q < cnt ? (uint16_t)b[q] : (uint16_t)0;
      }
      u32x4 pk;
      __builtin_memcpy(&pk, e, 16);
      etout.st128((v * ldet + tok) * ES, v < V && tok < cnt8, pk);
    }
  }
}

// ---------------------------------------------------------------------------
// 4. lse per row of a chunk: a block takes 16 rows and 16 parts; part q
// combines statistics tiles q, q + 16, q + 32, ... of its row in that order
// (sixteen tiles' loads issued before their combines: one round of loads for
// vocabularies up to 32768), then the first part
// combines the 16 partial results in order.  A row of 16 tokens is 128
// contiguous bytes of the [ntiles][crows] statistics.
// ---------------------------------------------------------------------------
// The row factor cfac = inv * exp(mref - lse), so that cfac * E is the
// softmax over the row scaled by 1 / n.  The one-hot term goes into E itself:
// the target entry becomes exp(z - mref) - exp(lse - mref), so cfac * E is
// (softmax - onehot) / n, the gradient of the mean loss by the logits.
// The fast path holds while (lse - mref) + ln n <= kFactorGap: cfac (which
// multiplies Hc into the dW product's operand, rounded to the input type)
// then stays above exp(-kFactorGap), far inside the normal range of bf16 and
// fp32, and every E entry below exp(kFactorGap), far from overflow in the
// products' sums (lse is at least the row's largest logit).  Any other row
// (a loss above kFactorGap - ln n nats, ~52 at n = 4096, which includes every
// row with a tile stored relative to its own maximum; also a NaN / inf row)
// is rescaled by its block to the row's maximum M: each entry of statistics
// tile t is multiplied by exp(base_t - M), base_t being the reference that
// tile's E was formed with (mref, or the tile's maximum where its sum is
// negated), and the target entry becomes exp(z - M) - exp(lse - M); both
// layouts are rewritten, and mref becomes M (cfac is then at least
// 1 / (n V)).  No E entry left the exponent range in the logits pass, so
// nothing is lost but one rounding of the rescaled entries.
constexpr float kFactorGap = 60.f;
static_assert(kBaseGap <= kFactorGap, "a row with a tile of its own base must take the rescale");
constexpr int kLseRows = 16, kLseParts = 16, kLseThreads = kLseRows * kLseParts;

template <typename TI>
__global__ __launch_bounds__(kLseThreads) void ce_lse_kernel(
    const float2 *__restrict__ stats, int ntiles, int wtm, int64_t crows, const float *tgt,
    const int *n_ptr, int64_t j0, const float *inv_ptr, const int *__restrict__ tcol,
    float *__restrict__ mref, float *__restrict__ cfac, float *loss_row, TI *P, int64_t ldp,
    TI *PT, int64_t ldet, int64_t V) {
  __shared__ float2 part[kLseParts][kLseRows];
  __shared__ int own[kLseParts][kLseRows];
  __shared__ int redo[kLseRows];
  __shared__ float2 rowst[kLseRows];
  __shared__ float mold[kLseRows];  // mref as the logits pass used it
  const int64_t cnt = chunk_count(n_ptr, j0, crows);
  const int rl = threadIdx.x % kLseRows, q = threadIdx.x / kLseRows;
  const int64_t row = (int64_t)blockIdx.x * kLseRows + rl;
  if ((int64_t)blockIdx.x * kLseRows >= cnt) return;  // the whole block is past the chunk
  float2 a = make_float2(-INFINITY, 0.f);
  int flag = 0;
  if (row < cnt) {
    constexpr int kBatch = 16;
    for (int t0 = q; t0 < ntiles; t0 += kLseParts * kBatch) {
      float2 v[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int t = t0 + u * kLseParts;
        v[u] = t < ntiles ? stats[(int64_t)t * crows + row] : make_float2(-INFINITY, 0.f);
      }
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        flag |= v[u].y < 0.f;
        a = combine_stats(a, make_float2(v[u].x, fabsf(v[u].y)));
      }
    }
  }
  part[q][rl] = a;
  own[q][rl] = flag;
  __syncthreads();
  const float inv = *inv_ptr;
  if (q == 0) {
    int again = 0;
    if (row < cnt) {
#pragma unroll
      for (int k = 1; k < kLseParts; ++k) {
        a = combine_stats(a, part[k][rl]);
        flag |= own[k][rl];
      }
      const float ls = a.x + log_f32(a.y);
      const float z = tgt[row];
      loss_row[j0 + row] = ls - z;
      const float m = mref[j0 + row];
      again = flag || !(ls - m - log_f32(inv) <= kFactorGap);  // also for a NaN / inf row
      if (!again) {
        cfac[j0 + row] = inv * exp_f32(m - ls);
        const int64_t tc = tcol[j0 + row];
        const TI e = static_cast<TI>(exp_f32(z - m) - exp_f32(ls - m));
        P[row * ldp + tc] = e;
        if (PT) PT[tc * ldet + row] = e;
      }
    }
    redo[rl] = again;
    rowst[rl] = a;
    mold[rl] = row < cnt ? mref[j0 + row] : 0.f;
  }
  __syncthreads();
  // The rows outside the reference's range (rare), all of the block's rows
  // together: a thread takes 8 entries (ldp and wtm are multiples of 8, so
  // the eight lie in one statistics tile; rows of P are 16-byte aligned) of
  // each row and rescales those of the rows off the fast path.  With E also
  // held transposed it then writes the block's 16 columns of E^T for those 8
  // vocabulary entries from all 16 rows (the other rows' entries are final
  // and go back unchanged; rows past the chunk's count give zeros, the K
  // padding of the dW product).
  int any = 0;
#pragma unroll
  for (int k = 0; k < kLseRows; ++k) any |= redo[k];
  if (!any) return;  // uniform across the block
  constexpr int kVec = 8, kWords = kVec * (int)sizeof(TI) / 16;
  constexpr int kColWords = kLseRows * (int)sizeof(TI) / 16;
  const int64_t r0 = (int64_t)blockIdx.x * kLseRows;
  for (int64_t v0 = (int64_t)threadIdx.x * kVec; v0 < ldp; v0 += (int64_t)kLseThreads * kVec) {
    TI ev[kLseRows][kVec];
#pragma unroll
    for (int k = 0; k < kLseRows; ++k) {
      if ((redo[k] || PT) && r0 + k < cnt) {
        u32x4 raw[kWords];
#pragma unroll
        for (int w = 0; w < kWords; ++w)
          raw[w] = reinterpret_cast<const u32x4 *>(P + (r0 + k) * ldp + v0)[w];
        __builtin_memcpy(ev[k], raw, sizeof(ev[k]));
      } else {
#pragma unroll
        for (int i = 0; i < kVec; ++i) ev[k][i] = static_cast<TI>(0.f);
      }
    }
#pragma unroll
    for (int k = 0; k < kLseRows; ++k) {
      if (!redo[k]) continue;
      const int64_t r = r0 + k;
      const float mx = rowst[k].x, ls = rowst[k].x + log_f32(rowst[k].y);
      float f = 0.f;
      if (v0 < V) {
        const float2 ts = stats[(v0 / wtm) * crows + r];
        f = exp_f32((ts.y < 0.f ? ts.x : mold[k]) - mx);
      }
      const int64_t tc = tcol[j0 + r];
#pragma unroll
      for (int i = 0; i < kVec; ++i) {
        const int64_t v = v0 + i;
        const float e = v >= V   ? 0.f
                        : v == tc ? exp_f32(tgt[r] - mx) - exp_f32(ls - mx)
                                  : static_cast<float>(ev[k][i]) * f;
        ev[k][i] = static_cast<TI>(e);
      }
      u32x4 raw[kWords];
      __builtin_memcpy(raw, ev[k], sizeof(ev[k]));
#pragma unroll
      for (int w = 0; w < kWords; ++w) reinterpret_cast<u32x4 *>(P + r * ldp + v0)[w] = raw[w];
    }
    if (PT) {
#pragma unroll
      for (int i = 0; i < kVec; ++i) {
        if (v0 + i >= V) break;
        TI col[kLseRows];
#pragma unroll
        for (int k = 0; k < kLseRows; ++k) col[k] = ev[k][i];
        u32x4 raw[kColWords];
        __builtin_memcpy(raw, col, sizeof(col));
#pragma unroll
        for (int w = 0; w < kColWords; ++w)
          reinterpret_cast<u32x4 *>(PT + (v0 + i) * ldet + r0)[w] = raw[w];
      }
    }
  }
  if (threadIdx.x < kLseRows && redo[threadIdx.x]) {
    const int k = threadIdx.x;
    const float mx = rowst[k].x, ls = rowst[k].x + log_f32(rowst[k].y);
    mref[j0 + r0 + k] = mx;
    cfac[j0 + r0 + k] = inv * exp_f32(mx - ls);
  }
}

// ---------------------------------------------------------------------------
// 5. The dW product's B operand for a chunk: Hct[d, j0 + r] = cfac[j0 + r] *
// Hc[j0 + r, d] in the input type for r < count, 0 for count <= r <
// round_up(count, 8) (the product's K padding): the row factor enters the
// product over the rows through this operand.  64 x 64 tiles through LDS;
// VEC: 16-byte row vectors in and column vectors out (D a multiple of the
// vector width), else one element per access.
// With `loss` set (the last chunk's launch, when every row's loss is known),
// block (0, 0) first writes the mean loss: each thread sums a strided share
// of the n valid rows' losses, each wavefront reduces its lanes (fixed
// butterfly), and thread 0 adds the 4 wavefront sums in order.  This saves
// the launch a one-block loss kernel would cost.
// ---------------------------------------------------------------------------
constexpr int kPrepThreads = 256;

template <typename TI, bool VEC>
__global__ __launch_bounds__(kPrepThreads) void ce_scale_hct_kernel(
    const TI *__restrict__ Hc, int64_t D, const float *__restrict__ cfac,
    const int *n_ptr, int64_t j0, int64_t crows, TI *__restrict__ Hct, int64_t ldht,
    const float *__restrict__ loss_row, const float *inv_ptr, float *loss) {
  using U = typename std::conditional<sizeof(TI) == 2, uint16_t, uint32_t>::type;
  constexpr int VE = VEC ? 16 / (int)sizeof(TI) : 1;  // elements per access
  constexpr int PITCH = 64 + (sizeof(TI) == 2 ? 2 : 1);
  __shared__ U tile[64 * PITCH];
  if (loss != nullptr && blockIdx.x == 0 && blockIdx.y == 0) {
    __shared__ float sl[kPrepThreads / 64];
    const int64_t n = *n_ptr;
    float a = 0.f;
    for (int64_t i = threadIdx.x; i < n; i += kPrepThreads) a += loss_row[i];
    a = wave_sum(a);
    if ((threadIdx.x & 63) == 0) sl[threadIdx.x >> 6] = a;
    __syncthreads();
    if (threadIdx.x == 0) {
      float tl = 0.f;
      for (int k = 0; k < kPrepThreads / 64; ++k) tl += sl[k];
      *loss = tl * *inv_ptr;
    }
  }
  const int64_t cnt = chunk_count(n_ptr, j0, crows);
  const int64_t cnt8 = (cnt + 7) / 8 * 8;
  const int64_t r0 = (int64_t)blockIdx.x * 64, d0 = (int64_t)blockIdx.y * 64;
  if (r0 >= cnt8) return;
  const int t = threadIdx.x;
  constexpr int VPR = 64 / VE;  // accesses per 64-element tile row
  for (int idx = t; idx < 64 * VPR; idx += kPrepThreads) {
    const int rr = idx / VPR, cv = idx % VPR;
    const int64_t r = r0 + rr, d = d0 + (int64_t)cv * VE;
    TI e[VE];
    const float f = r < cnt ? cfac[j0 + r] : 0.f;
    if constexpr (VEC) {
      u32x4 v = {0u, 0u, 0u, 0u};
      if (r < cnt && d < D) v = *reinterpret_cast<const u32x4 *>(Hc + (j0 + r) * D + d);
      __builtin_memcpy(e, &v, 16);
    } else {
      e[0] = (r < cnt && d < D) ? Hc[(j0 + r) * D + d] : static_cast<TI>(0.f);
    }
#pragma unroll
    for (int q = 0; q < VE; ++q) {
      const TI sc = static_cast<TI>(static_cast<float>(e[q]) * f);
      U bits;
      __builtin_memcpy(&bits, &sc, sizeof(U));
      tile[rr * PITCH + cv * VE + q] = bits;
    }
  }
  __syncthreads();
  for (int idx = t; idx < 64 * VPR; idx += kPrepThreads) {
    const int dc = idx / VPR, rv = idx % VPR;  // output row (d), row vector
    const int64_t d = d0 + dc, r = r0 + (int64_t)rv * VE;
    if (d >= D || r >= cnt8) continue;  // cnt8 is a multiple of VE
    U e[VE];
#pragma unroll
    for (int q = 0; q < VE; ++q) e[q] = tile[(rv * VE + q) * PITCH + dc];
    if constexpr (VEC) {
      *reinterpret_cast<u32x4 *>(Hct + d * ldht + j0 + r) = *reinterpret_cast<const u32x4 *>(e);
    } else {
      __builtin_memcpy(Hct + d * ldht + j0 + r, e, sizeof(U));
    }
  }
}

// ---------------------------------------------------------------------------
// 6. dH[m, :] = g * dHc[pos[m], :] in dH's type, 0 where pos[m] < 0.
// ---------------------------------------------------------------------------
// VE elements per thread step (4 when D is a multiple of 4: one 16-byte load).
// With sp.S > 1 the last chunk's dH product was left in S fp32 slices
// (`part`, [S, crows, D]): for its rows (compacted index >= sp.j0) the kernel
// forms (sum of the slices in order 0 .. S-1) * (cfac * 1) as
// splitk_reduce_kernel would have written to dHc, then scales by g: the same
// operations in the same order, so the same bits, with one launch and one
// fp32 pass over the rows fewer.
struct SplitRows {
  const float *part;
  int S;
  int64_t j0, crows;
  const float *cfac;
};
template <int VE>
__global__ __launch_bounds__(256) void ce_scatter_dh_kernel(const float *__restrict__ dHc,
                                                            int64_t D,
                                                            const int *__restrict__ pos,
                                                            int64_t M, const float *g_ptr,
                                                            void *dH, int dt, SplitRows sp) {
  const float g = g_ptr ? *g_ptr : 1.f;
  const int64_t dv = D / VE;
  const int64_t total = M * dv;
  const int64_t slice = sp.crows * D;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * 256) {
    const int64_t m = i / dv, c = (i - m * dv) * VE;
    const int p = pos[m];
    float v[VE];
    if (sp.S > 1 && p >= sp.j0) {
      const float *src = sp.part + (p - sp.j0) * D + c;
      float a[VE];
#pragma unroll
      for (int k = 0; k < VE; ++k) a[k] = 0.f;
      // slices added in order, 8 loads in flight per batch
      constexpr int kBatch = 8;
      for (int q0 = 0; q0 < sp.S; q0 += kBatch) {
        float t[kBatch][VE];
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
          if (q0 + u < sp.S) {
            if constexpr (VE == 4) {
              const float4 w = *reinterpret_cast<const float4 *>(src + (q0 + u) * slice);
              t[u][0] = w.x; t[u][1] = w.y; t[u][2] = w.z; t[u][3] = w.w;
            } else {
              t[u][0] = src[(q0 + u) * slice];
            }
          }
        }
#pragma unroll
        for (int u = 0; u < kBatch; ++u)
          if (q0 + u < sp.S)
#pragma unroll
            for (int k = 0; k < VE; ++k) a[k] += t[u][k];
      }
      const float f = sp.cfac[p] * 1.f;
#pragma unroll
      for (int k = 0; k < VE; ++k) v[k] = a[k] * f;
    } else if constexpr (VE == 4) {
      const float4 q = p >= 0 ? *reinterpret_cast<const float4 *>(dHc + (int64_t)p * D + c)
                              : make_float4(0.f, 0.f, 0.f, 0.f);
      v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
    } else {
      v[0] = p >= 0 ? dHc[(int64_t)p * D + c] : 0.f;
    }
#pragma unroll
    for (int k = 0; k < VE; ++k) store_dyn(dH, dt, m * D + c + k, v[k] * g);
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

// K split of a chunk's dH product.  The launch holding a chunk's gradient
// products has the dW blocks (K = the chunk's rows, crows) and the dH blocks
// (K = V, long); dH is split into S slices to balance them: S minimises the
// launch's makespan, max(longest block, total work / 256 CUs), plus the
// write and read of the S fp32 slices, all in units of one 64-deep K stage of
// a 256 x 256 tile (~2 us per CU at ~1.1 PFLOP/s, against ~5 TB/s of HBM).
// At cfg4 in one chunk (3687 rows) it does not split (128 dH blocks of K
// 32000 beside 1000 dW blocks of K 3687 balance by themselves): measured
// against forcing slices of at most 2048 / 4096 / 8192 / 16384 (16 / 8 / 4 /
// 2 slices), 1.64-1.66 ms against 1.85 / 1.77-1.80 / 1.72-1.74 / 1.67-1.69 ms
// per fwd+bwd: the extra fp32 slice traffic costs more than shorter blocks
// gain.  (This holds with the long job's blocks spread over all XCDs, see
// gemm_store_kernel.)
struct Split {
  int S;
  int64_t kslice;
};
template <class C>
inline Split dh_split(int64_t crows, int64_t D, int64_t V, int64_t ldp, bool single) {
  const int64_t tn = (D + C::BN - 1) / C::BN;
  const double tw = (double)((V + C::BM - 1) / C::BM * tn);
  const double th = (double)((crows + C::BM - 1) / C::BM * tn);
  // the N-major dW product (single) issues 8 LDS reads per 8 MFMAs against
  // 6: ~12% longer stages measured at K = 2048 / 4096
  const double kw = (double)crows / C::BK * (single ? 1.12 : 1.0);
  const double stage_s = 2e-6, hbm_bps = 5e12;
  Split best{1, ldp};
  double best_t = -1.0;
  for (int S = 1; S <= 64; ++S) {
    const int64_t ks = round_up((ldp + S - 1) / S, C::BK);
    const int64_t se = (ldp + ks - 1) / ks;
    const double kh = (double)ks / C::BK;
    const double work = tw * kw + th * (double)se * kh;
    double t = work / 256.0;
    if (kh > t) t = kh;
    if (kw > t) t = kw;
    if (se > 1) t += 2.0 * se * crows * D * 4.0 / hbm_bps / stage_s;
    if (best_t < 0 || t < best_t - 1e-9) {
      best_t = t;
      best = {(int)se, ks};
    }
  }
  return best;
}

struct Plan {
  int64_t crows, nch;     // compacted rows per chunk (a multiple of 256), chunks
  int64_t ldp, ldwt, ldht;
  int wtm, ntiles;        // statistics tile height and count
  int vtiles, ttiles;     // logits grid
  Split split;            // dH product's K split
  // single: E is held once, as P (16-bit inputs): the dW product reads it
  // N-major, so a chunk holds twice the rows of the two-layout form in the
  // same bytes, and the fp32 dW accumulator is kept transposed, [D, ldp]
  bool single;
  // state (kept from nf_ce_fwd to nf_ce_bwd)
  size_t s_scal, s_pos, s_cfac, s_wt, s_hct, s_p, s_pt, s_dhc, s_dwacc, s_total;
  // forward scratch
  size_t f_hc, f_rows, f_tcol, f_mref, f_stats, f_tgt, f_loss, f_part, f_total;
  // backward scratch
  size_t b_part, b_total;
};

template <typename TI>
inline Plan make_plan(int64_t M, int64_t D, int64_t V, int64_t chunk_rows) {
  using C = MainCfg<TI>;
  const size_t es = sizeof(TI);
  Plan P{};
  const int64_t mcap = round_up(M, 256);
  const int64_t want = chunk_rows < 1 ? 1 : (chunk_rows > mcap ? mcap : chunk_rows);
  if (sizeof(TI) == 2) {
    // chunk_rows bounds E and the dW accumulator together by what the
    // reference's chunk loop holds for the same roles: an fp32
    // [chunk_rows, V] logits tile and an fp32 [V, D] dW accumulator, i.e.
    // 2 (chunk_rows + D) rows of 16-bit E.  The first form inside it of:
    //  * one chunk, E in both layouts (2 mcap rows), for D >= 2048 only:
    //    the dW product on K-contiguous operands (one chunk, V 32000, fwd+bwd:
    //    M4096 D4096 2.96 ms against 3.06 held once; M8192 D2048 3.02
    //    against 3.05; M4096 D2048 level);
    //  * one chunk, E held once (mcap rows), no accumulator pass (at D 384 -
    //    1024 also faster than both layouts: M4096 D384 0.52 ms against
    //    0.55, M2048 D384 0.28 against 0.30-0.32, M1024 D1024 0.31 against
    //    0.33; at cfg4, M4096 D2048 with 3687 valid rows, the accumulator
    //    alone is the bytes of E for every row, and chunk_size 1024 runs in
    //    1.41-1.46 ms against 1.64 in two chunks);
    //  * chunks of 2 chunk_rows rows held once, beside the fp32 accumulator.
    const int64_t budget = 2 * ((chunk_rows < M ? chunk_rows : M) + D);
    P.single = D < 2048 || 2 * mcap > budget;
    const int64_t cr = P.single && mcap > budget ? round_up(2 * want, 256) : mcap;
    P.crows = cr > mcap ? mcap : cr;
  } else {
    // fp32: chunks of chunk_rows rows in both layouts (E alone is the
    // reference's tile) with the fp32 accumulator between them
    P.single = false;
    const int64_t cr = round_up(want, 256);
    P.crows = cr > mcap ? mcap : cr;
  }
  P.nch = (M + P.crows - 1) / P.crows;
  P.ldp = round_up(V, 8);
  P.ldwt = P.ldp;
  P.ldht = round_up(M, 8);
  P.wtm = C::WTM;
  P.vtiles = (int)((V + C::BM - 1) / C::BM);
  P.ntiles = P.vtiles * C::WM;
  P.ttiles = (int)(P.crows / C::BN);
  P.split = dh_split<C>(P.crows, D, V, P.ldp, P.single);
  const size_t part = P.split.S > 1 ? (size_t)P.split.S * P.crows * D * sizeof(float) : 0;
  size_t o = 0;
  auto take = [&](size_t bytes) { const size_t at = o; o = align256(o + bytes); return at; };
  P.s_scal = take(64);  // n_valid (int), inv (float)
  P.s_pos = take((size_t)M * sizeof(int));
  P.s_cfac = take((size_t)M * sizeof(float));
  P.s_wt = take((size_t)D * P.ldwt * es);
  P.s_hct = take((size_t)D * P.ldht * es);
  P.s_p = take((size_t)P.crows * P.ldp * es);
  P.s_pt = take(P.single ? 0 : (size_t)V * P.crows * es);
  P.s_dhc = take((size_t)M * D * sizeof(float));
  P.s_dwacc = take(P.nch > 1 ? (size_t)(P.single ? D * P.ldp : V * D) * sizeof(float) : 0);
  P.s_total = o;
  o = 0;
  P.f_hc = take((size_t)M * D * es);
  P.f_rows = take((size_t)M * sizeof(int));
  P.f_tcol = take((size_t)M * sizeof(int));
  P.f_mref = take((size_t)M * sizeof(float));
  P.f_stats = take((size_t)P.ntiles * P.crows * sizeof(float2));
  P.f_tgt = take((size_t)P.crows * sizeof(float));
  P.f_loss = take((size_t)M * sizeof(float));
  P.f_part = take(P.nch > 1 ? part : 0);
  P.f_total = o;
  o = 0;
  P.b_part = take(part);
  P.b_total = o;
  return P;
}

// Pointers into the state.
template <typename TI>
struct StateView {
  int *n;
  float *inv;
  int *pos;
  float *cfac;  // per compacted row: inv * exp(mref - lse)
  TI *Wt, *Hct, *P, *PT;
  float *dHc, *dWacc;
  StateView(const Plan &L, char *s)
      : n(reinterpret_cast<int *>(s + L.s_scal)),
        inv(reinterpret_cast<float *>(s + L.s_scal + 16)),
        pos(reinterpret_cast<int *>(s + L.s_pos)),
        cfac(reinterpret_cast<float *>(s + L.s_cfac)),
        Wt(reinterpret_cast<TI *>(s + L.s_wt)),
        Hct(reinterpret_cast<TI *>(s + L.s_hct)),
        P(reinterpret_cast<TI *>(s + L.s_p)),
        PT(reinterpret_cast<TI *>(s + L.s_pt)),
        dHc(reinterpret_cast<float *>(s + L.s_dhc)),
        dWacc(reinterpret_cast<float *>(s + L.s_dwacc)) {}
};

// The gradient products of chunk c in one launch: dW (+)= E^T_c Hct_c^T (E^T
// in the PT buffer; Hct holding the chunk's rows already times their factor
// cfac) and dHc_c = cfac_c * (E_c Wt^T) (E in the P buffer; the factor per
// output row, split along K).  dW goes
// to `dw_out` (type dt_w, scaled by g when given) on top of `dw_in` when
// given.
// reduce_dh = false leaves a split dH's fp32 slices in `part` for the
// caller (the backward's scatter adds them).
template <typename TI>
int launch_grads(const Plan &L, const StateView<TI> &S, int64_t c, int64_t D, int64_t V,
                 const float *dw_in, void *dw_out, int dt_w, const float *g, float *part,
                 hipStream_t s, bool final_dw, bool reduce_dh = true) {
  using C = MainCfg<TI>;
  const int64_t j0 = c * L.crows;
  // single: dW^T (+)= Hct_c P_c, [D, V], with P read N-major; the fp32
  // accumulator holds dW^T [D, ldp] and the final product stores dW [V, D]
  // transposed (final_dw: dw_out is the caller's gradient).
  auto jw = L.single ? make_job<C>(S.Hct + j0, L.ldht, S.P, L.ldp, dw_in, dw_out, dt_w, g,
                                   final_dw ? D : L.ldp, D, V, L.crows)
                     : make_job<C>(S.PT, L.crows, S.Hct + j0, L.ldht, dw_in, dw_out, dt_w, g,
                                   D, V, D, L.crows);
  if (L.single) {
    jw.bt = 1;
    jw.ct = final_dw ? 1 : 0;
    jw.ldcin = L.ldp;
  }
  jw.dyn = S.n;
  jw.dyn_base = j0;
  jw.dyn_rows = 0;  // K: the chunk's rows
  auto jh = make_job<C>(S.P, L.ldp, S.Wt, L.ldwt, nullptr, S.dHc + j0 * D, NF_DTYPE_F32,
                        nullptr, D, L.crows, D, L.ldp);
  jh.dyn = S.n;
  jh.dyn_base = j0;
  jh.dyn_rows = 1;  // M: the chunk's rows
  jh.row_scale = S.cfac + j0;
  if (L.split.S > 1) {
    jh.ksplit = L.split.S;
    jh.kslice = L.split.kslice;
    jh.part = part;
    jh.tiles *= L.split.S;
  }
  // the longest blocks go first (the dW job is never split)
  return L.split.kslice > L.crows ? launch_gemm_store<C>(jh, jw, s, reduce_dh)
                                  : launch_gemm_store<C>(jw, jh, s, reduce_dh);
}

template <typename TI>
int ce_fwd_run(const TI *H, const TI *W, const int64_t *targets, int64_t M, int64_t D,
               int64_t V, int64_t ignore_index, int64_t chunk_rows, float *loss, int32_t *bad,
               char *state, char *ws, hipStream_t s) {
  using C = MainCfg<TI>;
  using U = typename std::conditional<sizeof(TI) == 2, uint16_t, uint32_t>::type;
  const Plan L = make_plan<TI>(M, D, V, chunk_rows);
  const StateView<TI> S(L, state);
  TI *Hc = reinterpret_cast<TI *>(ws + L.f_hc);
  int *rows = reinterpret_cast<int *>(ws + L.f_rows);
  int *tcol = reinterpret_cast<int *>(ws + L.f_tcol);
  float2 *stats = reinterpret_cast<float2 *>(ws + L.f_stats);
  float *tgt = reinterpret_cast<float *>(ws + L.f_tgt);
  float *mref = reinterpret_cast<float *>(ws + L.f_mref);
  float *loss_row = reinterpret_cast<float *>(ws + L.f_loss);
  float *part = reinterpret_cast<float *>(ws + L.f_part);
  int e;

  ce_compact_kernel<<<1, kCompactThreads, 0, s>>>(targets, M, V, ignore_index, rows, tcol,
                                                  S.pos, S.n, S.inv, bad);
  if ((e = check_launch("ce_compact"))) return e;
  const bool vec = D % (16 / (int64_t)sizeof(TI)) == 0 && aligned16(H) && aligned16(W) &&
                   aligned16(Hc);
  {
    constexpr int kRowsPerBlock = kGatherThreads / 64;
    int64_t blocks = (M + kRowsPerBlock - 1) / kRowsPerBlock;
    if (blocks > 4096) blocks = 4096;
    if (vec)
      ce_gather_kernel<TI, true><<<(unsigned)blocks, kGatherThreads, 0, s>>>(
          H, W, D, rows, tcol, S.n, M, Hc, mref);
    else
      ce_gather_kernel<TI, false><<<(unsigned)blocks, kGatherThreads, 0, s>>>(
          H, W, D, rows, tcol, S.n, M, Hc, mref);
    if ((e = check_launch("ce_gather"))) return e;
  }
  // W^T is only read by the dH product: with 16-bit elements and 16-byte
  // rows it is formed by extra blocks at the end of the first logits launch,
  // otherwise by its own launch here
  gemm::TpJobs tp{};
  const bool fold = sizeof(TI) == 2 && D % 8 == 0 && L.ldwt % 8 == 0 && aligned16(W) &&
                    aligned16(S.Wt);
  if (fold) {
    tp.in[0] = reinterpret_cast<const uint16_t *>(W);
    tp.out[0] = reinterpret_cast<uint16_t *>(S.Wt);
    tp.R[0] = V;
    tp.Cn[0] = D;
    tp.ldi[0] = D;
    tp.ldo[0] = L.ldwt;
    tp.rb[0] = (int)((L.ldwt + gemm::kTpRegionRows - 1) / gemm::kTpRegionRows);
    tp.cb[0] = (int)((D + gemm::kTpRegionCols - 1) / gemm::kTpRegionCols);
    tp.n = tp.rb[0] * tp.cb[0];
  } else if ((e = launch_transpose<U>(W, V, D, D, S.Wt, L.ldwt, s))) {
    return e;
  }
  const gemm::TpJobs none{};

  const bool vk = buf_ok<TI>(Hc, D, M, D) && buf_ok<TI>(W, D, V, D);
  const bool sb = sb_ok(L.crows * L.ldp * (int64_t)sizeof(TI));
  const unsigned glog = (unsigned)(L.vtiles * L.ttiles);
  TI *const PT = L.single ? nullptr : S.PT;
  const dim3 gprep((unsigned)(L.crows / 64), (unsigned)((D + 63) / 64));
  for (int64_t c = 0; c < L.nch; ++c) {
    const int64_t j0 = c * L.crows;
    const gemm::TpJobs &tj = c == 0 ? tp : none;
    const unsigned grid = glog + (unsigned)tj.n;
    if (vk && sb)
      ce_logits_kernel<C, true, true><<<grid, C::NT, 0, s>>>(
          W, Hc, V, D, j0, L.crows, S.n, tcol, mref, stats, tgt, S.P, L.ldp, PT, L.crows,
          L.vtiles, L.ttiles, tj);
    else if (vk)
      ce_logits_kernel<C, true, false><<<grid, C::NT, 0, s>>>(
          W, Hc, V, D, j0, L.crows, S.n, tcol, mref, stats, tgt, S.P, L.ldp, PT, L.crows,
          L.vtiles, L.ttiles, tj);
    else
      ce_logits_kernel<C, false, false><<<grid, C::NT, 0, s>>>(
          W, Hc, V, D, j0, L.crows, S.n, tcol, mref, stats, tgt, S.P, L.ldp, PT, L.crows,
          L.vtiles, L.ttiles, tj);
    if ((e = check_launch("ce_logits"))) return e;
    ce_lse_kernel<TI><<<(unsigned)(L.crows / kLseRows), kLseThreads, 0, s>>>(
        stats, L.ntiles, L.wtm, L.crows, tgt, S.n, j0, S.inv, tcol, mref, S.cfac, loss_row, S.P,
        L.ldp, PT, L.crows, V);
    if ((e = check_launch("ce_lse"))) return e;
    const bool last = c + 1 == L.nch;  // the mean loss comes with the last chunk's launch
    if (vec)
      ce_scale_hct_kernel<TI, true><<<gprep, kPrepThreads, 0, s>>>(
          Hc, D, S.cfac, S.n, j0, L.crows, S.Hct, L.ldht, loss_row, S.inv, last ? loss : nullptr);
    else
      ce_scale_hct_kernel<TI, false><<<gprep, kPrepThreads, 0, s>>>(
          Hc, D, S.cfac, S.n, j0, L.crows, S.Hct, L.ldht, loss_row, S.inv, last ? loss : nullptr);
    if ((e = check_launch("ce_scale_hct"))) return e;
    if (!last &&
        (e = launch_grads<TI>(L, S, c, D, V, c > 0 ? S.dWacc : nullptr, S.dWacc, NF_DTYPE_F32,
                              nullptr, part, s, /*final_dw=*/false)))
      return e;
  }
  return NF_OK;
}

template <typename TI>
int ce_bwd_run(int64_t M, int64_t D, int64_t V, int64_t chunk_rows, char *state,
               const float *g, void *dH, int dt_h, void *dW, int dt_w, char *ws, hipStream_t s) {
  const Plan L = make_plan<TI>(M, D, V, chunk_rows);
  const StateView<TI> S(L, state);
  float *part = reinterpret_cast<float *>(ws + L.b_part);
  int e;
  // the last chunk's split dH slices are added by the scatter below
  if ((e = launch_grads<TI>(L, S, L.nch - 1, D, V, L.nch > 1 ? S.dWacc : nullptr, dW, dt_w, g,
                            part, s, /*final_dw=*/true, /*reduce_dh=*/false)))
    return e;
  const SplitRows sp{part, L.split.S, (L.nch - 1) * L.crows, L.crows, S.cfac};
  const bool vec = D % 4 == 0;  // dHc rows and slices are then 16-byte aligned
  int64_t blocks = (M * (vec ? D / 4 : D) + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  if (vec)
    ce_scatter_dh_kernel<4><<<(unsigned)blocks, 256, 0, s>>>(S.dHc, D, S.pos, M, g, dH, dt_h,
                                                             sp);
  else
    ce_scatter_dh_kernel<1><<<(unsigned)blocks, 256, 0, s>>>(S.dHc, D, S.pos, M, g, dH, dt_h,
                                                             sp);
  return check_launch("ce_scatter_dh");
}

}  // namespace ce
}  // namespace nf

using namespace nf;
using namespace nf::ce;

namespace {
// Sizes whose buffers could exist: M, V, D within int32 and each operand
// under 2^40 elements, so every byte count below fits int64 / size_t.
bool ce_sizes_ok(int64_t M, int64_t D, int64_t V) {
  const int64_t i32 = 0x7fffffffLL, cap = (int64_t)1 << 40;
  return M > 0 && D > 0 && V > 0 && M <= i32 && V <= i32 && D <= i32 && M * D <= cap &&
         V * D <= cap && M * V <= cap;
}
int ce_check_shape(const char *fn, int64_t M, int64_t D, int64_t V) {
  if (M <= 0 || D <= 0 || V <= 0)
    return set_error(NF_ERR_ARG, "%s: bad shape M=%lld D=%lld V=%lld", fn, (long long)M,
                     (long long)D, (long long)V);
  if (!ce_sizes_ok(M, D, V))
    return set_error(NF_ERR_ARG, "%s: M, V or D exceeds int32, or an operand 2^40 elements",
                     fn);
  return NF_OK;
}
int ce_check_dtype(const char *fn, int dtype) {
  if (dtype != NF_DTYPE_BF16 && dtype != NF_DTYPE_F32)
    return set_error(NF_ERR_DTYPE, "%s: dtype %d unsupported (bf16 or f32)", fn, dtype);
  return NF_OK;
}
bool dtype_ok(int dtype) { return dtype == NF_DTYPE_BF16 || dtype == NF_DTYPE_F32; }
Plan plan_of(int64_t M, int64_t D, int64_t V, int64_t chunk_rows, int dtype) {
  return dtype == NF_DTYPE_BF16 ? make_plan<bf16>(M, D, V, chunk_rows)
                                : make_plan<float>(M, D, V, chunk_rows);
}
}  // namespace

extern "C" size_t nf_ce_state_bytes(int64_t M, int64_t D, int64_t V, int64_t chunk_rows,
                                    int dtype) {
  if (!ce_sizes_ok(M, D, V) || chunk_rows <= 0 || !dtype_ok(dtype)) return 0;
  return plan_of(M, D, V, chunk_rows, dtype).s_total;
}

extern "C" size_t nf_ce_fwd_workspace(int64_t M, int64_t D, int64_t V, int64_t chunk_rows,
                                      int dtype) {
  if (!ce_sizes_ok(M, D, V) || chunk_rows <= 0 || !dtype_ok(dtype)) return 0;
  return plan_of(M, D, V, chunk_rows, dtype).f_total;
}

extern "C" size_t nf_ce_bwd_workspace(int64_t M, int64_t D, int64_t V, int64_t chunk_rows,
                                      int dtype) {
  if (!ce_sizes_ok(M, D, V) || chunk_rows <= 0 || !dtype_ok(dtype)) return 0;
  const size_t b = plan_of(M, D, V, chunk_rows, dtype).b_total;
  return b > 0 ? b : 256;  // never 0 for a valid shape (0 marks a refusal)
}

extern "C" int nf_ce_fwd(const void *hidden, const void *weight, const int64_t *targets,
                         int64_t M, int64_t D, int64_t V, int64_t ignore_index,
                         int64_t chunk_rows, int dtype, float *loss, int32_t *bad_targets,
                         void *state, size_t state_bytes, void *workspace,
                         size_t workspace_bytes, void *stream) {
  if (int e = ce_check_shape("nf_ce_fwd", M, D, V)) return e;
  if (chunk_rows <= 0) return set_error(NF_ERR_ARG, "nf_ce_fwd: chunk_rows must be > 0");
  if (!hidden || !weight || !targets || !loss || !state)
    return set_error(NF_ERR_ARG, "nf_ce_fwd: null pointer");
  if (int e = ce_check_dtype("nf_ce_fwd", dtype)) return e;
  const Plan L = plan_of(M, D, V, chunk_rows, dtype);
  if (state_bytes < L.s_total || !aligned16(state))
    return set_error(NF_ERR_WORKSPACE, "nf_ce_fwd: state %zu bytes < required %zu",
                     state_bytes, L.s_total);
  if (!workspace || workspace_bytes < L.f_total || !aligned16(workspace))
    return set_error(NF_ERR_WORKSPACE, "nf_ce_fwd: workspace %zu bytes < required %zu",
                     workspace_bytes, L.f_total);
  hipStream_t s = static_cast<hipStream_t>(stream);
  char *st = static_cast<char *>(state), *ws = static_cast<char *>(workspace);
  if (dtype == NF_DTYPE_BF16)
    return ce_fwd_run<bf16>((const bf16 *)hidden, (const bf16 *)weight, targets, M, D, V,
                            ignore_index, chunk_rows, loss, bad_targets, st, ws, s);
  return ce_fwd_run<float>((const float *)hidden, (const float *)weight, targets, M, D, V,
                           ignore_index, chunk_rows, loss, bad_targets, st, ws, s);
}

extern "C" int nf_ce_bwd(int64_t M, int64_t D, int64_t V, int64_t chunk_rows, int dtype,
                         void *state, size_t state_bytes, const float *grad_output,
                         void *dhidden, int dt_hidden, void *dweight, int dt_weight,
                         void *workspace, size_t workspace_bytes, void *stream) {
  if (int e = ce_check_shape("nf_ce_bwd", M, D, V)) return e;
  if (chunk_rows <= 0) return set_error(NF_ERR_ARG, "nf_ce_bwd: chunk_rows must be > 0");
  if (!state || !dhidden || !dweight) return set_error(NF_ERR_ARG, "nf_ce_bwd: null pointer");
  if (int e = ce_check_dtype("nf_ce_bwd", dtype)) return e;
  if (!is_dtype(dt_hidden) || !is_dtype(dt_weight))
    return set_error(NF_ERR_DTYPE, "nf_ce_bwd: gradient dtypes %d, %d", dt_hidden, dt_weight);
  const Plan L = plan_of(M, D, V, chunk_rows, dtype);
  if (state_bytes < L.s_total || !aligned16(state))
    return set_error(NF_ERR_WORKSPACE, "nf_ce_bwd: state %zu bytes < required %zu",
                     state_bytes, L.s_total);
  const size_t need = nf_ce_bwd_workspace(M, D, V, chunk_rows, dtype);
  if (!workspace || workspace_bytes < need || !aligned16(workspace))
    return set_error(NF_ERR_WORKSPACE, "nf_ce_bwd: workspace %zu bytes < required %zu",
                     workspace_bytes, need);
  hipStream_t s = static_cast<hipStream_t>(stream);
  char *st = static_cast<char *>(state), *ws = static_cast<char *>(workspace);
  if (dtype == NF_DTYPE_BF16)
    return ce_bwd_run<bf16>(M, D, V, chunk_rows, st, grad_output, dhidden, dt_hidden, dweight,
                            dt_weight, ws, s);
  return ce_bwd_run<float>(M, D, V, chunk_rows, st, grad_output, dhidden, dt_hidden, dweight,
                           dt_weight, ws, s);
}

// one call: [state | forward and backward scratch, overlapped]
extern "C" size_t nf_ce_workspace(int64_t M, int64_t D, int64_t V, int64_t chunk_rows,
                                  int dtype) {
  const size_t st = nf_ce_state_bytes(M, D, V, chunk_rows, dtype);
  const size_t f = nf_ce_fwd_workspace(M, D, V, chunk_rows, dtype);
  const size_t b = nf_ce_bwd_workspace(M, D, V, chunk_rows, dtype);
  if (!st || !f || !b) return 0;
  return st + (f > b ? f : b);
}

extern "C" int nf_ce_fwd_bwd(const void *hidden, const void *weight, const int64_t *targets,
                             int64_t M, int64_t D, int64_t V, int64_t ignore_index,
                             int64_t chunk_rows, int dtype, float *loss, float *dhidden,
                             float *dweight, int32_t *bad_targets, void *workspace,
                             size_t workspace_bytes, void *stream) {
  if (int e = ce_check_shape("nf_ce_fwd_bwd", M, D, V)) return e;
  if (chunk_rows <= 0) return set_error(NF_ERR_ARG, "nf_ce_fwd_bwd: chunk_rows must be > 0");
  if (!hidden || !weight || !targets || !loss || !dhidden || !dweight)
    return set_error(NF_ERR_ARG, "nf_ce_fwd_bwd: null pointer");
  if (int e = ce_check_dtype("nf_ce_fwd_bwd", dtype)) return e;
  const size_t need = nf_ce_workspace(M, D, V, chunk_rows, dtype);
  if (!workspace || workspace_bytes < need || !aligned16(workspace))
    return set_error(NF_ERR_WORKSPACE, "nf_ce_fwd_bwd: workspace %zu bytes < required %zu",
                     workspace_bytes, need);
  const size_t sb = nf_ce_state_bytes(M, D, V, chunk_rows, dtype);
  char *ws = static_cast<char *>(workspace);
  if (int e = nf_ce_fwd(hidden, weight, targets, M, D, V, ignore_index, chunk_rows, dtype, loss,
                        bad_targets, ws, sb, ws + sb, workspace_bytes - sb, stream))
    return e;
  return nf_ce_bwd(M, D, V, chunk_rows, dtype, ws, sb, nullptr, dhidden, NF_DTYPE_F32, dweight,
                   NF_DTYPE_F32, ws + sb, workspace_bytes - sb, stream);
}
