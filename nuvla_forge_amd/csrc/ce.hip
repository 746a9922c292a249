// Chunked cross entropy on the MFMA GEMM core of gemm_core.h, in two calls
// (all on the caller's stream, fixed reduction orders throughout).
//
// Forward (nf_ce_fwd):
//   1. ce_stats:  S^T = W H^T tile by tile; per (vocabulary tile, token) the
//      max and sum of exp(S - max), plus S[m, t_m] for the target column.
//      S itself is never stored.
//   2. ce_lse:    lse[m] = combine of the tile partials (fixed order);
//                 loss_row[m] = lse - S[m, t_m] for valid rows.
//   3. ce_loss:   one block: n_valid, loss = sum(loss_row) / max(n, 1),
//                 inv = 1 / max(n, 1).
//   lse, the target columns and inv are the state the backward reads.
// Backward (nf_ce_bwd, with the loss's grad_output g):
//   4. transpose  W [V, D] -> Wt [D, ldwt],  H [M, D] -> Ht [D, ldht]
//      (zero-padded columns), so every GEMM below is K-contiguous (NT).
//   5. per vocabulary chunk c of `vocab_chunk` columns:
//      ce_prob:  recompute S_c^T = W_c H^T; P_c = inv * (softmax - onehot)
//                (0 for ignored rows) in the input type, written row-major
//                [M, Vc] and transposed [Vc, M];
//      dW_c  = g * P_c^T H    (gemm_store, K = M)   -> dweight rows of c, in
//                                                     dweight's type
//      dH   += P_c   W_c      (gemm_store, K = Vc)  -> an fp32 accumulator;
//                                                     the last chunk writes
//                                                     g * dH in dhidden's type
// Memory is O(M * vocab_chunk) for P; the [M, V] logits never exist.
#include <type_traits>

#include "gemm_store.h"

namespace nf {
namespace ce {

using namespace gemm;


// bf16: 256x256 block tiles, 8 wavefronts of 128x64 (two per SIMD, so one
// wavefront's LDS waits and epilogue overlap the other's MFMAs), operands
// copied global -> LDS directly in 64-wide K-stages, two stage buffers (one
// barrier per 64 k: measured ~12% faster than 32-wide stages with four
// buffers); f32 (correctness path): 128x128 tiles staged through registers.
template <typename TI>
struct MainCfgT;
template <>
struct MainCfgT<bf16> { using type = gemm::DCfg<256, 256, 2, 4, 2, 64>; };
template <>
struct MainCfgT<float> { using type = Cfg<float, 128, 128, 2, 2>; };
template <typename TI>
using MainCfg = typename MainCfgT<TI>::type;

__device__ __forceinline__ float log_f32(float x) {
  constexpr float kLn2 = 0.6931471805599453f;  // ln(2)
  return __builtin_amdgcn_logf(x) * kLn2;       // log2 on the hardware
}

// ---------------------------------------------------------------------------
// Logit statistics of one (vocabulary tile, token tile) block.  The product
// is formed transposed, acc = W_tile H_tile^T (rows: vocabulary entries,
// columns: tokens), so each lane holds 16 * TM logits of each of its TN
// tokens and the per-token max / sum of exp are reductions in registers,
// then one exchange between the two lane halves and a fixed-order combine
// of the WM wavefronts that share the token (through LDS).  Writes
// stats[vtile * M + token] = (max, sum exp(logit - max)) over the tile, and
// tgt_logit[token] from the block holding the token's target column.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float2 combine_stats(float2 a, float2 b) {
  const float m = fmaxf(a.x, b.x);
  if (m == -INFINITY) return make_float2(m, 0.f);
  return make_float2(m, a.y * exp_f32(a.x - m) + b.y * exp_f32(b.x - m));
}

template <class C, bool BUF>
__global__ NF_GEMM_BOUNDS(C) void ce_stats_kernel(
    const typename C::TI *W, const typename C::TI *H, int64_t V, int64_t M, int64_t D,
    const int64_t *targets, float2 *stats, float *tgt_logit, int vtiles, int mtiles) {
  // one LDS buffer only: a second __shared__ object makes the compiler wait
  // for every direct-to-LDS copy in flight before each operand read of the
  // K loop (it cannot tell the copies do not write that object); the
  // per-wavefront partials reuse the operand stages after the K loop
  __shared__ __attribute__((aligned(16))) char smem[C::LDS_BYTES];
  static_assert(sizeof(float2) * C::WM * C::BN <= C::LDS_BYTES, "partials do not fit");
  float2(*red)[C::BN] = reinterpret_cast<float2(*)[C::BN]>(smem);
  int vt, mt;
  gemm::group_tile(gemm::xcd_order(blockIdx.x, vtiles * mtiles), vtiles, mtiles,
                   gemm::kTileGroup, vt, mt);
  const int64_t v0 = (int64_t)vt * C::BM;
  const int64_t m0 = (int64_t)mt * C::BN;
  floatx16 acc[C::TM][C::TN];
  gemm::mainloop<C, BUF>(W, D, H, D, V, M, D, v0, m0, smem, acc);

  const int l = threadIdx.x & 63, half = l >> 5;
  const int w = threadIdx.x >> 6, wm = w / C::WN, wn = w % C::WN;
  // vocabulary row of acc[i][*][r]: v0 + wm * WTM + 4 * half + i * 32 + 8 * (r / 4) + r % 4
  const int64_t vrow0 = v0 + wm * C::WTM + 4 * half;
  // Rows past the vocabulary (only in a wavefront whose rows reach V) are set
  // to -inf once, so the max and the sum below need no per-element masks
  // (masks kept live across both loops would cost 64 scalar register pairs).
  if (v0 + wm * C::WTM + C::WTM > V) {
    const int vlim = (int)(V - vrow0 < C::WTM ? V - vrow0 : C::WTM);
#pragma unroll
    for (int i = 0; i < C::TM; ++i)
#pragma unroll
      for (int j = 0; j < C::TN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (i * 32 + 8 * (r >> 2) + (r & 3) >= vlim) acc[i][j][r] = -INFINITY;
  }
#pragma unroll
  for (int j = 0; j < C::TN; ++j) {
    const int tl = wn * C::WTN + j * 32 + (l & 31);
    const int64_t tok = m0 + tl;
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < C::TM; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, acc[i][j][r]);
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    // a column with no row inside the vocabulary keeps (-inf, 0)
    const float mref = mx == -INFINITY ? 0.f : mx;
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < C::TM; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) s += exp_f32(acc[i][j][r] - mref);
    s += __shfl_xor(s, 32);
    if (half == 0) red[wm][tl] = make_float2(mx, s);

    // the target logit, from the one lane that holds it
    if (tok < M) {
      const int64_t loc64 = targets[tok] - (v0 + wm * C::WTM);
      const int loc = (int)(loc64 >= 0 && loc64 < C::WTM ? loc64 : -1);
      if (loc >= 0 && ((loc >> 2) & 1) == half) {
        const int want = ((loc >> 5) << 4) | (((loc & 31) >> 3) << 2) | (loc & 3);
        float z = 0.f;
#pragma unroll
        for (int i = 0; i < C::TM; ++i)
#pragma unroll
          for (int r = 0; r < 16; ++r) z = (i * 16 + r == want) ? acc[i][j][r] : z;
        tgt_logit[tok] = z;
      }
    }
  }
  __syncthreads();
  for (int t = threadIdx.x; t < C::BN; t += C::NT) {
    const int64_t tok = m0 + t;
    if (tok >= M) continue;
    float2 a = red[0][t];
#pragma unroll
    for (int q = 1; q < C::WM; ++q) a = combine_stats(a, red[q][t]);
    stats[(int64_t)vt * M + tok] = a;
  }
}

// ---------------------------------------------------------------------------
// lse per token: a block takes 16 tokens and 16 parts; part q combines
// vocabulary tiles q, q + 16, q + 32, ... of its token in that order (the
// loads of four tiles issued before their combines, so a part waits for one
// load latency per four tiles, not per tile), then the first part combines
// the 16 partial results in order.  A row of 16 tokens is 128 contiguous
// bytes of the [ntiles][M] stats.
// ---------------------------------------------------------------------------
constexpr int kLseRows = 16, kLseParts = 16;

__global__ __launch_bounds__(kLseRows * kLseParts) void ce_lse_kernel(
    const float2 *__restrict__ stats, int ntiles, const float *tgt_logit,
    const int64_t *targets, int64_t M, int64_t V, int64_t ignore_index,
    float *lse, int *tcol, float *loss_row, int *flags) {
  __shared__ float2 part[kLseParts][kLseRows];
  const int rl = threadIdx.x % kLseRows, q = threadIdx.x / kLseRows;
  const int64_t row = (int64_t)blockIdx.x * kLseRows + rl;
  float2 a = make_float2(-INFINITY, 0.f);
  if (row < M) {
    constexpr int kBatch = 4;
    for (int t0 = q; t0 < ntiles; t0 += kLseParts * kBatch) {
      float2 v[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int t = t0 + u * kLseParts;
        v[u] = t < ntiles ? stats[(int64_t)t * M + row] : make_float2(-INFINITY, 0.f);
      }
#pragma unroll
      for (int u = 0; u < kBatch; ++u) a = combine_stats(a, v[u]);
    }
  }
  part[q][rl] = a;
  __syncthreads();
  if (q != 0 || row >= M) return;
#pragma unroll
  for (int k = 1; k < kLseParts; ++k) a = combine_stats(a, part[k][rl]);
  const float ls = a.x + log_f32(a.y);
  const int64_t tg = targets[row];
  const bool in_range = tg >= 0 && tg < V;
  const bool valid = tg != ignore_index && in_range;
  lse[row] = ls;
  tcol[row] = valid ? (int)tg : -1;
  loss_row[row] = valid ? ls - tgt_logit[row] : 0.f;
  flags[row] = (valid ? 1 : 0) | ((tg != ignore_index && !in_range) ? 2 : 0);
}

// ---------------------------------------------------------------------------
// loss, n_valid, inv_count: one block; each thread sums a strided share of
// the rows, each wavefront reduces its lanes (fixed butterfly), and thread 0
// adds the 16 wavefront sums in order.
// ---------------------------------------------------------------------------
constexpr int kLossThreads = 1024;

__device__ __forceinline__ int wave_sum_int(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

__global__ __launch_bounds__(kLossThreads) void ce_loss_kernel(
    const float *loss_row, const int *flags, int64_t M, float *loss,
    float *inv_out, int *bad_out) {
  constexpr int kWaves = kLossThreads / 64;
  __shared__ float sl[kWaves];
  __shared__ int sn[kWaves], sb[kWaves];
  float a = 0.f;
  int n = 0, bad = 0;
  for (int64_t i = threadIdx.x; i < M; i += kLossThreads) {
    a += loss_row[i];
    n += flags[i] & 1;
    bad += (flags[i] >> 1) & 1;
  }
  a = wave_sum(a);
  n = wave_sum_int(n);
  bad = wave_sum_int(bad);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    sl[w] = a;
    sn[w] = n;
    sb[w] = bad;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float tl = 0.f;
    int tn = 0, tb = 0;
    for (int k = 0; k < kWaves; ++k) {
      tl += sl[k];
      tn += sn[k];
      tb += sb[k];
    }
    const float inv = 1.f / (float)(tn > 1 ? tn : 1);
    *loss = tl * inv;
    *inv_out = inv;
    if (bad_out) *bad_out = tb;
  }
}

// ---------------------------------------------------------------------------
// probability epilogue: P = inv * (softmax - onehot) for one vocabulary
// chunk, from the transposed product acc = Wc_tile H_tile^T (rows: chunk
// columns, columns: tokens).  Each lane's TN tokens bring their lse, target
// and scale in registers.  Writes P [M, ldp] (token rows; columns [Vc, kpad)
// zero) and PT [Vc, ldpt] (chunk-column rows; tokens [M, ldpt) zero).
//
// 16-bit tiles of 256 x 256 go through LDS (free once the K loop ends): the
// lanes write their values as a [token][chunk column] tile, 4 columns (8
// bytes) at a time, and both outputs then leave as 16-byte row vectors, P
// from the tile's rows and PT from its columns (8 two-byte LDS reads per
// vector).  A lane's own values would give 8-byte P stores spread over 64
// rows and 2-byte PT stores.  Element (t, c) sits at byte
// t * 512 + 2 * (c ^ prob_swz(t)): the XOR term moves whole 8-element
// vectors, so rows still read as vectors, and spreads the column reads of a
// half-wave (tokens 8 l + k, l < 32) over the banks.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int prob_swz(int t) { return 8 * (((t >> 3) ^ (t & 7)) & 31); }

template <class C, bool BUF, bool SB>
__global__ NF_GEMM_BOUNDS(C) void ce_prob_kernel(
    const typename C::TI *Wc, const typename C::TI *H, int64_t Vc, int64_t M, int64_t D,
    int64_t vbase, const int *tcol, const float *lse, const float *inv_ptr,
    typename C::TI *P, int64_t ldp, int64_t kpad, typename C::TI *PT, int64_t ldpt, int vtiles,
    int mtiles) {
  using TI = typename C::TI;
  constexpr int ES = (int)sizeof(TI);
  __shared__ __attribute__((aligned(16))) char smem[C::LDS_BYTES];
  int vt, mt;
  gemm::group_tile(gemm::xcd_order(blockIdx.x, vtiles * mtiles), vtiles, mtiles,
                   gemm::kTileGroup, vt, mt);
  const int64_t v0 = (int64_t)vt * C::BM;
  const int64_t m0 = (int64_t)mt * C::BN;
  floatx16 acc[C::TM][C::TN];
  gemm::mainloop<C, BUF>(Wc, D, H, D, Vc, M, D, v0, m0, smem, acc);
  const float inv = *inv_ptr;

  const int l = threadIdx.x & 63, half = l >> 5;
  const int w = threadIdx.x >> 6, wm = w / C::WN, wn = w % C::WN;
  const int64_t crow0 = v0 + wm * C::WTM + 4 * half;  // chunk column of (i = 0, r = 0)
  OutBuf<SB> pout, ptout;
  pout.init(P, M * ldp * ES);
  ptout.init(PT, Vc * ldpt * ES);
  constexpr bool kStaged = ES == 2 && C::BM == 256 && C::BN == 256 && C::NT == 512 &&
                           C::LDS_BYTES >= 256 * 512;
  // Rows past the chunk (only in a wavefront whose rows reach Vc) are set to
  // -inf once, so their probabilities come out 0 without per-element masks
  // (masks kept live through the loop would cost 64 scalar register pairs).
  if (v0 + wm * C::WTM + C::WTM > Vc) {
    const int vlim = (int)(Vc - crow0 < C::WTM ? Vc - crow0 : C::WTM);
#pragma unroll
    for (int i = 0; i < C::TM; ++i)
#pragma unroll
      for (int j = 0; j < C::TN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (i * 32 + 8 * (r >> 2) + (r & 3) >= vlim) acc[i][j][r] = -INFINITY;
  }
#pragma unroll
  for (int j = 0; j < C::TN; ++j) {
    const int64_t tok = m0 + wn * C::WTN + j * 32 + (l & 31);
    const int tc = tok < M ? tcol[tok] : -1;
    const float ls = tok < M ? lse[tok] : 0.f;
    const bool keep = tc >= 0;  // counted token: P row = inv * (softmax - onehot)
    // the target's offset from crow0 when it lies in this chunk's Vc columns,
    // else -1 (a row past Vc may be a later chunk's column: no onehot there)
    const int64_t tin = (int64_t)tc - vbase;
    const int tloc = (keep && tin >= 0 && tin < Vc) ? (int)(tin - crow0) : -1;
#pragma unroll
    for (int i = 0; i < C::TM; ++i)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int o = i * 32 + 8 * g;  // offset of r = 4g from crow0
        float p[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float e = exp_f32(acc[i][j][4 * g + q] - ls) - (tloc == o + q ? 1.f : 0.f);
          p[q] = keep ? e * inv : 0.f;
        }
        TI pv[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) pv[q] = static_cast<TI>(p[q]);
        const int64_t c = crow0 + o;
        if constexpr (kStaged) {
          const int t = wn * C::WTN + j * 32 + (l & 31);  // tile token
          const int cl = wm * C::WTM + 4 * half + o;       // tile chunk column
          u32x2 packed;
          __builtin_memcpy(&packed, pv, 8);
          *reinterpret_cast<u32x2 *>(smem + t * 512 + 2 * (cl ^ prob_swz(t))) = packed;
        } else if constexpr (ES == 2) {
          u32x2 packed;
          __builtin_memcpy(&packed, pv, 8);
          pout.st64((tok * ldp + c) * ES, tok < M && c < kpad, packed);
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            uint16_t bits;
            __builtin_memcpy(&bits, &pv[q], 2);
            ptout.st16(((c + q) * ldpt + tok) * ES, c + q < Vc && tok < ldpt, bits);
          }
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            pout.st32((tok * ldp + c + q) * ES, tok < M && c + q < kpad, p[q]);
            ptout.st32(((c + q) * ldpt + tok) * ES, c + q < Vc && tok < ldpt, p[q]);
          }
        }
      }
  }
  if constexpr (kStaged) {
    __syncthreads();
    // Out-of-range tokens and chunk columns hold zeros in the tile; a vector
    // is stored when its first element is in range (kpad and ldpt are
    // multiples of 8, so a vector is wholly inside or outside).  Wavefront w
    // stores tile rows (P) and tile columns (PT) 32 w .. 32 w + 31, two per
    // instruction, one per half-wave.
    const int hv = l >> 5, c8 = 8 * (l & 31);
#pragma unroll 4
    for (int it = 0; it < 16; ++it) {
      const int t = 32 * w + 2 * it + hv;
      const u32x4 v = *reinterpret_cast<const u32x4 *>(smem + t * 512 + 2 * (c8 ^ prob_swz(t)));
      const int64_t tok = m0 + t, c = v0 + c8;
      pout.st128((tok * ldp + c) * ES, tok < M && c < kpad, v);
    }
#pragma unroll 4
    for (int it = 0; it < 16; ++it) {
      const int c = 32 * w + 2 * it + hv;
      uint16_t e[8];
#pragma unroll
      for (int k = 0; k < 8; ++k)
        e[k] = *reinterpret_cast<const uint16_t *>(smem + (c8 + k) * 512 +
                                                   2 * (c ^ prob_swz(c8 + k)));
      u32x4 v;
      __builtin_memcpy(&v, e, 16);
      const int64_t crow = v0 + c, tok = m0 + c8;
      ptout.st128((crow * ldpt + tok) * ES, crow < Vc && tok < ldpt, v);
    }
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

// K splits of a vocabulary chunk's two gradient products.  The chunk's dW
// blocks (K = tokens) and dH blocks (K = chunk columns) run in one launch.
// When that launch fits in one wave of the 256 CUs, its time is the longest
// block's K; splitting the job with the longer K into S slices shortens it
// at the cost of more blocks.  S is chosen (1 .. 64) to minimise
// waves(blocks) x longest slice, ties to fewer slices: e.g. the reasoning
// head (M 512, D 384, the whole vocabulary in one chunk: 4 dH tiles of K
// 32000 beside 250 dW tiles of K 512) splits dH 63 ways, M 16384 with D 384
// and 2048-column chunks (16 dW tiles of K 16384) splits dW 8 ways, and the
// BASELINE shape (128 + 128 tiles of K 4096) is not split.  Slices are summed
// by splitk_reduce_kernel in a fixed order.
struct Split {
  int S;
  int64_t kslice;
};
struct SplitPlan {
  Split w, h;  // dW, dH
};
template <class C>
inline Split best_split(int64_t t_short, int64_t k_short, int64_t t_long, int64_t k_long) {
  Split best{1, k_long};
  int64_t best_t = -1;
  for (int64_t S = 1; S <= 64; ++S) {
    const int64_t ks = round_up((k_long + S - 1) / S, C::BK);
    const int64_t se = (k_long + ks - 1) / ks;
    const int64_t waves = (t_short + t_long * se + 255) / 256;
    const int64_t t = waves * (k_short > ks ? k_short : ks);
    if (best_t < 0 || t < best_t) {
      best_t = t;
      best = {(int)se, ks};
    }
  }
  return best;
}
template <class C>
inline SplitPlan chunk_split(int64_t vc, int64_t M, int64_t D) {
  const int64_t tn = (D + C::BN - 1) / C::BN;
  const int64_t tw = (vc + C::BM - 1) / C::BM * tn, th = (M + C::BM - 1) / C::BM * tn;
  const int64_t kh = round_up(vc, 8), kw = round_up(M, 8);
  SplitPlan p{{1, kw}, {1, kh}};
  if (tw + th >= 256) return p;  // a full wave or more: the blocks already balance
  if (kh >= kw)
    p.h = best_split<C>(tw, kw, th, kh);
  else
    p.w = best_split<C>(th, kh, tw, kw);
  return p;
}

// Per-row state the backward reads: lse [M], the target column [M] (-1: the
// row has no gradient) and the scalars (inv = 1 / max(n_valid, 1)).
struct StateLayout {
  size_t off_lse, off_tcol, off_scal, total;
};
inline StateLayout state_layout(int64_t M) {
  StateLayout L{};
  size_t o = 0;
  auto take = [&](size_t bytes) { const size_t at = o; o = align256(o + bytes); return at; };
  L.off_lse = take((size_t)M * sizeof(float));
  L.off_tcol = take((size_t)M * sizeof(int));
  L.off_scal = take(64);
  L.total = o;
  return L;
}

// Forward scratch: per (vocabulary tile, token) stats, the target logits,
// the row losses and the row flags.
struct FwdLayout {
  int64_t ntiles;
  size_t off_stats, off_tgt, off_loss, off_flags, total;
};
inline FwdLayout fwd_layout(int64_t M, int64_t V, int es) {
  FwdLayout L{};
  const int64_t bm = es == 2 ? MainCfg<bf16>::BM : MainCfg<float>::BM;
  L.ntiles = (V + bm - 1) / bm;  // vocabulary tiles
  size_t o = 0;
  auto take = [&](size_t bytes) { const size_t at = o; o = align256(o + bytes); return at; };
  L.off_stats = take((size_t)L.ntiles * M * sizeof(float2));  // [ntiles][M]
  L.off_tgt = take((size_t)M * sizeof(float));
  L.off_loss = take((size_t)M * sizeof(float));
  L.off_flags = take((size_t)M * sizeof(int));
  L.total = o;
  return L;
}

template <class C>
inline size_t partial_bytes(int64_t M, int64_t D, int64_t V, int64_t vc) {
  size_t most = 0;
  for (int64_t vb = 0; vb < V; vb += vc) {
    const int64_t c = V - vb < vc ? V - vb : vc;
    const SplitPlan sp = chunk_split<C>(c, M, D);
    const size_t bw = sp.w.S > 1 ? (size_t)sp.w.S * c * D * sizeof(float) : 0;
    const size_t bh = sp.h.S > 1 ? (size_t)sp.h.S * M * D * sizeof(float) : 0;
    const size_t b = bw > bh ? bw : bh;  // at most one of the two is split
    if (b > most) most = b;
  }
  return most;
}

// Backward scratch: W^T, H^T, one chunk's P and P^T, split-K partials, and
// the fp32 dH accumulator when the vocabulary takes more than one chunk.
struct BwdLayout {
  int64_t ldwt, ldht, vc, ldp;
  size_t off_wt, off_ht, off_p, off_pt, off_part, off_dh, total;
};
inline BwdLayout bwd_layout(int64_t M, int64_t D, int64_t V, int64_t vocab_chunk, int es) {
  BwdLayout L{};
  L.ldwt = round_up(V, 8);
  L.ldht = round_up(M, 8);
  L.vc = round_up(vocab_chunk < V ? vocab_chunk : V, 8);
  L.ldp = L.vc;
  const size_t part = es == 2 ? partial_bytes<MainCfg<bf16>>(M, D, V, L.vc)
                              : partial_bytes<MainCfg<float>>(M, D, V, L.vc);
  size_t o = 0;
  auto take = [&](size_t bytes) { const size_t at = o; o = align256(o + bytes); return at; };
  L.off_wt = take((size_t)D * L.ldwt * es);
  L.off_ht = take((size_t)D * L.ldht * es);
  L.off_p = take((size_t)M * L.ldp * es);
  L.off_pt = take((size_t)L.vc * L.ldht * es);
  L.off_part = take(part);
  L.off_dh = take(V > L.vc ? (size_t)M * D * sizeof(float) : 0);
  L.total = o;
  return L;
}

// Forward: stats over the whole vocabulary, per-row lse and loss, the mean.
// Writes loss, the state (lse, target columns, inv) and the bad-target count.
template <typename TI>
int ce_fwd_run(const TI *H, const TI *W, const int64_t *targets, int64_t M, int64_t D,
               int64_t V, int64_t ignore_index, float *loss, int32_t *bad, char *state,
               char *ws, hipStream_t s) {
  using C = MainCfg<TI>;
  const StateLayout S = state_layout(M);
  const FwdLayout L = fwd_layout(M, V, sizeof(TI));
  float *lse = reinterpret_cast<float *>(state + S.off_lse);
  int *tcol = reinterpret_cast<int *>(state + S.off_tcol);
  float *inv = reinterpret_cast<float *>(state + S.off_scal);
  float2 *stats = reinterpret_cast<float2 *>(ws + L.off_stats);
  float *tgt = reinterpret_cast<float *>(ws + L.off_tgt);
  float *loss_row = reinterpret_cast<float *>(ws + L.off_loss);
  int *flags = reinterpret_cast<int *>(ws + L.off_flags);
  int e;
  // blocks (vocabulary tile, token tile); the product is W H^T
  const bool vk = buf_ok<TI>(H, D, M, D) && buf_ok<TI>(W, D, V, D);
  const int mtiles = (int)((M + C::BN - 1) / C::BN);
  const unsigned gs = (unsigned)(L.ntiles * mtiles);
  if (vk)
    ce_stats_kernel<C, true><<<gs, C::NT, 0, s>>>(W, H, V, M, D, targets, stats, tgt,
                                                  (int)L.ntiles, mtiles);
  else
    ce_stats_kernel<C, false><<<gs, C::NT, 0, s>>>(W, H, V, M, D, targets, stats, tgt,
                                                   (int)L.ntiles, mtiles);
  if ((e = check_launch("ce_stats"))) return e;
  ce_lse_kernel<<<(unsigned)((M + kLseRows - 1) / kLseRows), kLseRows * kLseParts, 0, s>>>(
      stats, (int)L.ntiles, tgt, targets, M, V, ignore_index, lse, tcol, loss_row, flags);
  if ((e = check_launch("ce_lse"))) return e;
  ce_loss_kernel<<<1, kLossThreads, 0, s>>>(loss_row, flags, M, loss, inv, bad);
  return check_launch("ce_loss");
}

// Backward: per vocabulary chunk, P = inv * (softmax - onehot) from the
// saved lse, then dW_c = g * P_c^T H and dH (+)= P_c W_c; the last chunk's dH
// and every dW chunk are written scaled, in the caller's element types.
template <typename TI>
int ce_bwd_run(const TI *H, const TI *W, int64_t M, int64_t D, int64_t V, int64_t vocab_chunk,
               const char *state, const float *g, void *dH, int dt_h, void *dW, int dt_w,
               char *ws, hipStream_t s) {
  using C = MainCfg<TI>;
  const StateLayout S = state_layout(M);
  const BwdLayout L = bwd_layout(M, D, V, vocab_chunk, sizeof(TI));
  const float *lse = reinterpret_cast<const float *>(state + S.off_lse);
  const int *tcol = reinterpret_cast<const int *>(state + S.off_tcol);
  const float *inv = reinterpret_cast<const float *>(state + S.off_scal);
  TI *Wt = reinterpret_cast<TI *>(ws + L.off_wt);
  TI *Ht = reinterpret_cast<TI *>(ws + L.off_ht);
  TI *P = reinterpret_cast<TI *>(ws + L.off_p);
  TI *PT = reinterpret_cast<TI *>(ws + L.off_pt);
  float *part = reinterpret_cast<float *>(ws + L.off_part);
  float *dh_acc = reinterpret_cast<float *>(ws + L.off_dh);  // used when V > vc
  int e;

  using U = typename std::conditional<sizeof(TI) == 2, uint16_t, uint32_t>::type;
  if ((e = launch_transpose<U>(W, V, D, D, Wt, L.ldwt, s))) return e;
  if ((e = launch_transpose<U>(H, M, D, D, Ht, L.ldht, s))) return e;

  const bool vk = buf_ok<TI>(H, D, M, D) && buf_ok<TI>(W, D, V, D);
  const int mtiles = (int)((M + C::BN - 1) / C::BN);
  for (int64_t vb = 0; vb < V; vb += L.vc) {
    const int64_t vc = (V - vb < L.vc) ? V - vb : L.vc;  // columns in this chunk
    const int64_t kpad = round_up(vc, 8);
    const TI *Wc = W + vb * D;
    // blocks (chunk-column tile, token tile); the product is W_c H^T
    const int vtiles = (int)((vc + C::BM - 1) / C::BM);
    const unsigned gp = (unsigned)(vtiles * mtiles);
    const bool sb = sb_ok(M * L.ldp * (int64_t)sizeof(TI)) &&
                    sb_ok(vc * L.ldht * (int64_t)sizeof(TI));
    const bool vb_ok = vk && buf_ok<TI>(Wc, D, vc, D);
    if (vb_ok && sb)
      ce_prob_kernel<C, true, true><<<gp, C::NT, 0, s>>>(Wc, H, vc, M, D, vb, tcol, lse, inv, P,
                                                         L.ldp, kpad, PT, L.ldht, vtiles, mtiles);
    else if (vb_ok)
      ce_prob_kernel<C, true, false><<<gp, C::NT, 0, s>>>(Wc, H, vc, M, D, vb, tcol, lse, inv, P,
                                                          L.ldp, kpad, PT, L.ldht, vtiles,
                                                          mtiles);
    else
      ce_prob_kernel<C, false, false><<<gp, C::NT, 0, s>>>(Wc, H, vc, M, D, vb, tcol, lse, inv,
                                                           P, L.ldp, kpad, PT, L.ldht, vtiles,
                                                           mtiles);
    if ((e = check_launch("ce_prob"))) return e;
    // dW[vb:vb+vc, :] = g * P_c^T H   (K = tokens, zero-padded to ldht), final;
    // dH (+)= P_c W_c                 (K = chunk columns, zero-padded to kpad)
    // into the fp32 accumulator, the last chunk scaled into dH itself
    const bool first = vb == 0, last = vb + L.vc >= V;
    char *dw_c = static_cast<char *>(dW) + vb * D * dtype_bytes(dt_w);
    auto jw = make_job<C>(PT, L.ldht, Ht, L.ldht, nullptr, dw_c, dt_w, g, D, vc, D, L.ldht);
    auto jh = make_job<C>(P, L.ldp, Wt + vb, L.ldwt, first ? nullptr : dh_acc,
                          last ? dH : static_cast<void *>(dh_acc),
                          last ? dt_h : NF_DTYPE_F32, last ? g : nullptr, D, M, D, kpad);
    const SplitPlan sp = chunk_split<C>(vc, M, D);
    for (auto *jp : {&jw, &jh}) {
      const Split &q = jp == &jw ? sp.w : sp.h;
      if (q.S > 1) {
        jp->ksplit = q.S;
        jp->kslice = q.kslice;
        jp->part = part;
        jp->tiles *= q.S;
      }
    }
    // a split job's slices are the longest blocks: dispatch them first
    if ((e = sp.h.S > 1 ? launch_gemm_store<C>(jh, jw, s) : launch_gemm_store<C>(jw, jh, s)))
      return e;
  }
  return NF_OK;
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
         V * D <= cap;
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
size_t es_of(int dtype) { return dtype == NF_DTYPE_BF16 ? 2 : 4; }
}  // namespace

extern "C" size_t nf_ce_state_bytes(int64_t M) {
  return M > 0 && M <= 0x7fffffffLL ? state_layout(M).total : 0;
}

extern "C" size_t nf_ce_fwd_workspace(int64_t M, int64_t D, int64_t V, int dtype) {
  if (!ce_sizes_ok(M, D, V)) return 0;
  if (dtype != NF_DTYPE_BF16 && dtype != NF_DTYPE_F32) return 0;
  return fwd_layout(M, V, (int)es_of(dtype)).total;
}

extern "C" size_t nf_ce_bwd_workspace(int64_t M, int64_t D, int64_t V, int64_t vocab_chunk,
                                      int dtype) {
  if (!ce_sizes_ok(M, D, V) || vocab_chunk <= 0) return 0;
  if (dtype != NF_DTYPE_BF16 && dtype != NF_DTYPE_F32) return 0;
  return bwd_layout(M, D, V, vocab_chunk, (int)es_of(dtype)).total;
}

extern "C" int nf_ce_fwd(const void *hidden, const void *weight, const int64_t *targets,
                         int64_t M, int64_t D, int64_t V, int64_t ignore_index, int dtype,
                         float *loss, int32_t *bad_targets, void *state, size_t state_bytes,
                         void *workspace, size_t workspace_bytes, void *stream) {
  if (int e = ce_check_shape("nf_ce_fwd", M, D, V)) return e;
  if (!hidden || !weight || !targets || !loss || !state)
    return set_error(NF_ERR_ARG, "nf_ce_fwd: null pointer");
  if (int e = ce_check_dtype("nf_ce_fwd", dtype)) return e;
  const size_t need_s = nf_ce_state_bytes(M), need = nf_ce_fwd_workspace(M, D, V, dtype);
  if (state_bytes < need_s || !aligned16(state))
    return set_error(NF_ERR_WORKSPACE, "nf_ce_fwd: state %zu bytes < required %zu",
                     state_bytes, need_s);
  if (!workspace || workspace_bytes < need || !aligned16(workspace))
    return set_error(NF_ERR_WORKSPACE, "nf_ce_fwd: workspace %zu bytes < required %zu",
                     workspace_bytes, need);
  hipStream_t s = static_cast<hipStream_t>(stream);
  char *st = static_cast<char *>(state), *ws = static_cast<char *>(workspace);
  if (dtype == NF_DTYPE_BF16)
    return ce_fwd_run<bf16>((const bf16 *)hidden, (const bf16 *)weight, targets, M, D, V,
                            ignore_index, loss, bad_targets, st, ws, s);
  return ce_fwd_run<float>((const float *)hidden, (const float *)weight, targets, M, D, V,
                           ignore_index, loss, bad_targets, st, ws, s);
}

extern "C" int nf_ce_bwd(const void *hidden, const void *weight, int64_t M, int64_t D,
                         int64_t V, int64_t vocab_chunk, int dtype, const void *state,
                         size_t state_bytes, const float *grad_output, void *dhidden,
                         int dt_hidden, void *dweight, int dt_weight, void *workspace,
                         size_t workspace_bytes, void *stream) {
  if (int e = ce_check_shape("nf_ce_bwd", M, D, V)) return e;
  if (vocab_chunk <= 0) return set_error(NF_ERR_ARG, "nf_ce_bwd: vocab_chunk must be > 0");
  if (!hidden || !weight || !state || !dhidden || !dweight)
    return set_error(NF_ERR_ARG, "nf_ce_bwd: null pointer");
  if (int e = ce_check_dtype("nf_ce_bwd", dtype)) return e;
  if (!is_dtype(dt_hidden) || !is_dtype(dt_weight))
    return set_error(NF_ERR_DTYPE, "nf_ce_bwd: gradient dtypes %d, %d", dt_hidden, dt_weight);
  const size_t need_s = nf_ce_state_bytes(M), need = nf_ce_bwd_workspace(M, D, V, vocab_chunk,
                                                                         dtype);
  if (state_bytes < need_s || !aligned16(state))
    return set_error(NF_ERR_WORKSPACE, "nf_ce_bwd: state %zu bytes < required %zu",
                     state_bytes, need_s);
  if (!workspace || workspace_bytes < need || !aligned16(workspace))
    return set_error(NF_ERR_WORKSPACE, "nf_ce_bwd: workspace %zu bytes < required %zu",
                     workspace_bytes, need);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const char *st = static_cast<const char *>(state);
  char *ws = static_cast<char *>(workspace);
  if (dtype == NF_DTYPE_BF16)
    return ce_bwd_run<bf16>((const bf16 *)hidden, (const bf16 *)weight, M, D, V, vocab_chunk, st,
                            grad_output, dhidden, dt_hidden, dweight, dt_weight, ws, s);
  return ce_bwd_run<float>((const float *)hidden, (const float *)weight, M, D, V, vocab_chunk,
                           st, grad_output, dhidden, dt_hidden, dweight, dt_weight, ws, s);
}

// one call: [state | forward and backward scratch, overlapped]
extern "C" size_t nf_ce_workspace(int64_t M, int64_t D, int64_t V, int64_t vocab_chunk,
                                  int dtype) {
  const size_t f = nf_ce_fwd_workspace(M, D, V, dtype);
  const size_t b = nf_ce_bwd_workspace(M, D, V, vocab_chunk, dtype);
  if (!f || !b) return 0;
  return nf_ce_state_bytes(M) + (f > b ? f : b);
}

extern "C" int nf_ce_fwd_bwd(const void *hidden, const void *weight, const int64_t *targets,
                             int64_t M, int64_t D, int64_t V, int64_t ignore_index,
                             int64_t vocab_chunk, int dtype, float *loss, float *dhidden,
                             float *dweight, int32_t *bad_targets, void *workspace,
                             size_t workspace_bytes, void *stream) {
  if (int e = ce_check_shape("nf_ce_fwd_bwd", M, D, V)) return e;
  if (vocab_chunk <= 0) return set_error(NF_ERR_ARG, "nf_ce_fwd_bwd: vocab_chunk must be > 0");
  if (!hidden || !weight || !targets || !loss || !dhidden || !dweight)
    return set_error(NF_ERR_ARG, "nf_ce_fwd_bwd: null pointer");
  if (int e = ce_check_dtype("nf_ce_fwd_bwd", dtype)) return e;
  const size_t need = nf_ce_workspace(M, D, V, vocab_chunk, dtype);
  if (!workspace || workspace_bytes < need || !aligned16(workspace))
    return set_error(NF_ERR_WORKSPACE, "nf_ce_fwd_bwd: workspace %zu bytes < required %zu",
                     workspace_bytes, need);
  const size_t sb = nf_ce_state_bytes(M);
  char *ws = static_cast<char *>(workspace);
  if (int e = nf_ce_fwd(hidden, weight, targets, M, D, V, ignore_index, dtype, loss,
                        bad_targets, ws, sb, ws + sb, workspace_bytes - sb, stream))
    return e;
  return nf_ce_bwd(hidden, weight, M, D, V, vocab_chunk, dtype, ws, sb, nullptr, dhidden,
                   NF_DTYPE_F32, dweight, NF_DTYPE_F32, ws + sb, workspace_bytes - sb, stream);
}

extern "C" int nf_gemm_nt(const void *A, int64_t lda, const void *B, int64_t ldb, float *C,
                          int64_t ldc, int64_t M, int64_t N, int64_t K, int dtype,
                          void *stream) {
  if (M < 0 || N < 0 || K < 0) return set_error(NF_ERR_ARG, "nf_gemm_nt: negative size");
  if (M > 0x7fffffffLL || N > 0x7fffffffLL || K > 0x7fffffffLL)
    return set_error(NF_ERR_ARG, "nf_gemm_nt: a size exceeds int32");
  if (M == 0 || N == 0) return NF_OK;
  if (!A || !B || !C) return set_error(NF_ERR_ARG, "nf_gemm_nt: null pointer");
  if (lda < K || ldb < K || ldc < N) return set_error(NF_ERR_ARG, "nf_gemm_nt: bad leading dim");
  // tiles are at least 128 x 128; the grid is one-dimensional
  if (((M + 127) / 128) * ((N + 127) / 128) > 0x7fffffffLL)
    return set_error(NF_ERR_ARG, "nf_gemm_nt: grid too large");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == NF_DTYPE_BF16) {
    using C16 = MainCfg<bf16>;
    const GemmJob<bf16> none{};
    return launch_gemm_store<C16>(
        make_job<C16>((const bf16 *)A, lda, (const bf16 *)B, ldb, nullptr, C, NF_DTYPE_F32,
                      nullptr, ldc, M, N, K),
        none, s);
  }
  if (dtype == NF_DTYPE_F32) {
    using C32 = MainCfg<float>;
    const GemmJob<float> none{};
    return launch_gemm_store<C32>(
        make_job<C32>((const float *)A, lda, (const float *)B, ldb, nullptr, C, NF_DTYPE_F32,
                      nullptr, ldc, M, N, K),
        none, s);
  }
  return set_error(NF_ERR_DTYPE, "nf_gemm_nt: dtype %d unsupported", dtype);
}
