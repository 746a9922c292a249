// adaLN-Zero seam: gated residual add + RMSNorm + modulation, fwd and bwd.
//
// Layout.  x, y, h, out, dh_up, dout, dx, dy are [M, N] row-major (unit
// stride along N); row m belongs to sample b = m / T.  gate, scale, shift are
// [B, N] with an arbitrary row stride (0 for a broadcast view), weight is [N].
//
// Row mapping.  A row is owned by R = 64 * WPR threads (WPR wavefronts); each
// thread holds K 8-element chunks of the row in registers, chunk k of thread
// r covering columns [(k * R + r) * 8, +8), so every load instruction of a
// wavefront touches one contiguous 1 KiB (bf16) or 2 KiB (f32) span.  With
// WPR == 1 the row's sum of squares is a pure DPP wavefront reduction; with
// WPR > 1 the per-wave sums meet in LDS.
//
// Forward.  Each row group walks a contiguous run of rows.  When the run lies
// in one sample (16-bit inputs), it is taken in batches of RB rows whose
// loads are all issued before any math and whose RB sums of squares share one
// LDS round; otherwise row by row, issuing the loads of row r+1 before working
// on row r and keeping the per-sample conditioning in registers while the
// sample does not change.
//
// Backward.  Block (b, j) owns a contiguous run of rows of sample b; its G row
// groups take every G-th row, with the next row's (or batch's) four inputs
// loaded before the current one is processed.  Each thread accumulates three
// per-column partials over its rows:
//   A = sum dout * xhat,  S = sum dout,  G = sum dh * y
// (dscale = weight * A, dshift = S, dgate = G, dweight = sum_b (1+scale_b) A_b);
// the row groups combine them in LDS in a fixed order and the block writes
// one [3, N] fp32 partial row.  adaln_reduce_kernel (adaln.hip) then sums the
// partial rows in a fixed order: no atomics, bit-identical run to run.
#pragma once
#include "nf_device.h"

namespace nf {
namespace adaln {

constexpr int kMaxN = 16384;  // 64 lanes * 16 waves * 8 elems * 2 chunks

struct FwdArgs {
  const void *x;
  const void *y;
  const void *gate;
  const void *weight;
  const void *scale;
  const void *shift;
  void *h;
  void *out;
  float *rstd;
  int64_t ld_x, ld_y, ld_gate, ld_scale, ld_shift;
  int64_t M, T;
  int N;
  int rows_per_group;  // contiguous rows walked by one row group
  float eps;
  int dt_gate, dt_weight, dt_scale, dt_shift;
};

struct BwdArgs {
  const void *dh_up;
  const void *dout;
  const void *x;
  const void *y;
  const void *gate;
  const void *weight;
  const void *scale;
  const float *rstd;
  void *dx;
  void *dy;
  float *partial;  // [B * J, 3, N]
  int64_t ld_x, ld_y, ld_gate, ld_scale;
  int64_t M, T;
  int N;
  int J;               // blocks per sample
  int rows_per_block;  // ceil(T / J)
  int dt_gate, dt_weight, dt_scale;
};

// Block shapes: a row is owned by R = 64 * WPR threads, a block holds
// G = BLK / R row groups, BLK = max(R, MINB).  The forward's MINB depends on
// the chunks per thread: with one (rows up to 1024 elements on two
// wavefronts) 128-thread blocks, one row group each, run the bf16
// [8192, 1024] fwd+bwd step 1.3-3.6% faster than 256- or 512-thread blocks
// (the forward alone: 10.3 against 10.5 us); with two (bf16 [65536, 2048])
// 256-thread blocks are 1.3% faster than 128.
template <int K>
constexpr int fwd_min_block() {
  return K == 1 ? 128 : 256;
}
template <int WPR, int MINB>
struct FwdShape {
  static constexpr int R = 64 * WPR;
  static constexpr int BLK = R < MINB ? MINB : R;
  static constexpr int G = BLK / R;
};
template <int WPR, int MINB = 512>
struct BwdShape {
  static constexpr int R = 64 * WPR;
  static constexpr int BLK = R < MINB ? MINB : R;
  static constexpr int G = BLK / R;
};

__device__ __forceinline__ int chunk_valid(int N, int col) {
  const int v = N - col;
  return v < 0 ? 0 : (v > 8 ? 8 : v);
}

// Sum over the WPR wavefronts that share one row.  `red` holds G * WPR
// floats; every thread of the block must call this (it may synchronise).
template <int WPR>
__device__ __forceinline__ float row_sum(float v, float *red, int g, int rt) {
  v = wave_sum(v);
  if constexpr (WPR == 1) {
    return v;
  } else {
    if ((rt & 63) == 0) red[g * WPR + (rt >> 6)] = v;
    __syncthreads();
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < WPR; ++i) t += red[g * WPR + i];
    __syncthreads();
    return t;
  }
}

// row_sum for RB rows at once: one LDS round (two barriers) for all RB sums.
// `red` holds G * WPR * RB floats.
template <int WPR, int RB>
__device__ __forceinline__ void row_sum_batch(float (&v)[RB], float *red, int g, int rt) {
#pragma unroll
  for (int q = 0; q < RB; ++q) v[q] = wave_sum(v[q]);
  if constexpr (WPR > 1) {
    if ((rt & 63) == 0) {
#pragma unroll
      for (int q = 0; q < RB; ++q) red[(g * WPR + (rt >> 6)) * RB + q] = v[q];
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < RB; ++q) {
      float t = 0.f;
#pragma unroll
      for (int i = 0; i < WPR; ++i) t += red[(g * WPR + i) * RB + q];
      v[q] = t;
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// forward
// ---------------------------------------------------------------------------
template <typename TX, typename TY, int K, int WPR, bool VEC, bool NT,
          int MINB = fwd_min_block<K>()>
__global__ __launch_bounds__((FwdShape<WPR, MINB>::BLK)) void adaln_fwd_kernel(
    FwdArgs p) {
  using S = FwdShape<WPR, MINB>;
  // 1024-thread blocks (16 wavefronts per row, 128 VGPRs per thread) hold
  // neither the weight nor the next row nor h: the weight is read again when
  // the sample changes, each row is loaded at the top of its iteration, and h
  // is formed again for the output (same operations, same values)
  constexpr bool LEAN = S::BLK > 512;
  __shared__ float red[S::G * WPR];
  const int g = threadIdx.x / S::R;
  const int rt = threadIdx.x % S::R;
  const int64_t first = ((int64_t)blockIdx.x * S::G + g) * p.rows_per_group;
  const int64_t last = first + p.rows_per_group < p.M ? first + p.rows_per_group : p.M;
  const TX *const xp = static_cast<const TX *>(p.x);
  const TY *const yp = static_cast<const TY *>(p.y);

  float wv[K][8];
  if constexpr (!LEAN) {
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int col = (k * S::R + rt) * 8;
      const int valid = chunk_valid(p.N, col);
      if (valid > 0) load8_dyn<VEC>(p.weight, p.dt_weight, col, valid, wv[k]);
    }
  }

  Raw8<TX> xc[K], xn[K];
  Raw8<TY> yc[K], yn[K];
  auto load_row = [&](int64_t row, Raw8<TX>(&xa)[K], Raw8<TY>(&ya)[K]) {
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int col = (k * S::R + rt) * 8;
      const int valid = chunk_valid(p.N, col);
      if (valid > 0) {
        xa[k].template load<VEC>(xp + row * p.ld_x + col, valid);
        ya[k].template load<VEC>(yp + row * p.ld_y + col, valid);
      } else {
        xa[k].zero();
        ya[k].zero();
      }
    }
  };
  if (!LEAN && first < last) load_row(first, xc, yc);

  float gv[K][8], wo[K][8], shv[K][8];
  int64_t cur_b = -1;
  for (int r = 0; r < p.rows_per_group; ++r) {
    const int64_t row = first + r;
    const bool active = row < last;
    if constexpr (LEAN) {
      if (active) load_row(row, xc, yc);
    } else {
      if (row + 1 < last) load_row(row + 1, xn, yn);
    }
    if (active) {
      const int64_t b = row / p.T;
      if (b != cur_b) {  // uniform across the row group
        cur_b = b;
#pragma unroll
        for (int k = 0; k < K; ++k) {
          const int col = (k * S::R + rt) * 8;
          const int valid = chunk_valid(p.N, col);
          float sv[8];
          if (valid > 0) {
            if constexpr (LEAN) load8_dyn<VEC>(p.weight, p.dt_weight, col, valid, wv[k]);
            load8_dyn<VEC>(p.gate, p.dt_gate, b * p.ld_gate + col, valid, gv[k]);
            load8_dyn<VEC>(p.scale, p.dt_scale, b * p.ld_scale + col, valid, sv);
            load8_dyn<VEC>(p.shift, p.dt_shift, b * p.ld_shift + col, valid, shv[k]);
#pragma unroll
            for (int i = 0; i < 8; ++i) wo[k][i] = wv[k][i] * (1.f + sv[i]);
          }
        }
      }
    }

    float hv[K][8];
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int col = (k * S::R + rt) * 8;
      const int valid = active ? chunk_valid(p.N, col) : 0;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        hv[k][i] = valid > 0 ? xc[k][i] + gv[k][i] * yc[k][i] : 0.f;
        ss += hv[k][i] * hv[k][i];
      }
      if (valid > 0)
        store8_hint<TX, VEC, NT>(static_cast<TX *>(p.h) + row * (int64_t)p.N + col, valid,
                                 hv[k]);
    }
    ss = row_sum<WPR>(ss, red, g, rt);
    const float rstd = 1.f / __builtin_sqrtf(ss / (float)p.N + p.eps);
    if (active && rt == 0) p.rstd[row] = rstd;
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int col = (k * S::R + rt) * 8;
      const int valid = active ? chunk_valid(p.N, col) : 0;
      if (valid > 0) {
        float o[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float hh = LEAN ? xc[k][i] + gv[k][i] * yc[k][i] : hv[k][i];
          o[i] = (hh * rstd) * wo[k][i] + shv[k][i];
        }
        store8_hint<TX, VEC, NT>(static_cast<TX *>(p.out) + row * (int64_t)p.N + col, valid,
                                 o);
      }
    }
    if constexpr (!LEAN) {
#pragma unroll
      for (int k = 0; k < K; ++k) {
        xc[k] = xn[k];
        yc[k] = yn[k];
      }
    }
  }
}

// Forward in batches of RB rows: every row group's rows lie in one sample
// (the host uses it only when T is a multiple of rows_per_group), so the
// conditioning is loaded once; each batch issues all its x / y loads before
// any math (2 * RB * K loads in flight per thread) and reduces its RB sums of
// squares with one LDS round.
template <typename TX, typename TY, int K, int WPR, bool VEC, bool NT, int RB, bool NTL>
__global__ __launch_bounds__((FwdShape<WPR, fwd_min_block<K>()>::BLK)) void adaln_fwd_batch_kernel(
    FwdArgs p) {
  using S = FwdShape<WPR, fwd_min_block<K>()>;
  __shared__ float red[S::G * WPR * RB];
  const int g = threadIdx.x / S::R;
  const int rt = threadIdx.x % S::R;
  const int64_t first = ((int64_t)blockIdx.x * S::G + g) * p.rows_per_group;
  const int64_t last = first + p.rows_per_group < p.M ? first + p.rows_per_group : p.M;
  const TX *const xp = static_cast<const TX *>(p.x);
  const TY *const yp = static_cast<const TY *>(p.y);

  float gv[K][8], wo[K][8], shv[K][8];
  if (first < last) {
    const int64_t b = first / p.T;
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int col = (k * S::R + rt) * 8;
      const int valid = chunk_valid(p.N, col);
      float wv[8], sv[8];
      if (valid > 0) {
        load8_dyn<VEC>(p.weight, p.dt_weight, col, valid, wv);
        load8_dyn<VEC>(p.gate, p.dt_gate, b * p.ld_gate + col, valid, gv[k]);
        load8_dyn<VEC>(p.scale, p.dt_scale, b * p.ld_scale + col, valid, sv);
        load8_dyn<VEC>(p.shift, p.dt_shift, b * p.ld_shift + col, valid, shv[k]);
#pragma unroll
        for (int i = 0; i < 8; ++i) wo[k][i] = wv[i] * (1.f + sv[i]);
      }
    }
  }
  for (int r = 0; r < p.rows_per_group; r += RB) {
    Raw8<TX> xs[RB][K];
    Raw8<TY> ys[RB][K];
#pragma unroll
    for (int q = 0; q < RB; ++q) {
      const int64_t row = first + r + q;
#pragma unroll
      for (int k = 0; k < K; ++k) {
        const int col = (k * S::R + rt) * 8;
        const int valid = row < last ? chunk_valid(p.N, col) : 0;
        if (valid > 0) {
          xs[q][k].template load<VEC, NTL>(xp + row * p.ld_x + col, valid);
          ys[q][k].template load<VEC, NTL>(yp + row * p.ld_y + col, valid);
        } else {
          xs[q][k].zero();
          ys[q][k].zero();
        }
      }
    }
    float hv[RB][K][8], ss[RB];
#pragma unroll
    for (int q = 0; q < RB; ++q) {
      const int64_t row = first + r + q;
      ss[q] = 0.f;
#pragma unroll
      for (int k = 0; k < K; ++k) {
        const int col = (k * S::R + rt) * 8;
        const int valid = row < last ? chunk_valid(p.N, col) : 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          hv[q][k][i] = valid > 0 ? xs[q][k][i] + gv[k][i] * ys[q][k][i] : 0.f;
          ss[q] += hv[q][k][i] * hv[q][k][i];
        }
        if (valid > 0)
          store8_hint<TX, VEC, NT>(static_cast<TX *>(p.h) + row * (int64_t)p.N + col, valid,
                                   hv[q][k]);
      }
    }
    row_sum_batch<WPR, RB>(ss, red, g, rt);
#pragma unroll
    for (int q = 0; q < RB; ++q) {
      const int64_t row = first + r + q;
      const float rstd = 1.f / __builtin_sqrtf(ss[q] / (float)p.N + p.eps);
      if (row < last && rt == 0) p.rstd[row] = rstd;
#pragma unroll
      for (int k = 0; k < K; ++k) {
        const int col = (k * S::R + rt) * 8;
        const int valid = row < last ? chunk_valid(p.N, col) : 0;
        if (valid > 0) {
          float o[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) o[i] = (hv[q][k][i] * rstd) * wo[k][i] + shv[k][i];
          store8_hint<TX, VEC, NT>(static_cast<TX *>(p.out) + row * (int64_t)p.N + col, valid,
                                   o);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// backward: per-row gradients + per-block partial rows
// ---------------------------------------------------------------------------

// Sum one accumulator over the G row groups of the block (group order
// 0, 1, ..., G-1) and store the result row.  All threads must call it.
template <int K, int G, int R, bool VEC>
__device__ __forceinline__ void combine_store(float (&acc)[K][8], float *comb,
                                              int g, int rt, float *dst,
                                              int N) {
  constexpr int kRowElems = R * K * 8;
  if constexpr (G > 1) {
    if (g > 0) {
#pragma unroll
      for (int k = 0; k < K; ++k)
#pragma unroll
        for (int i = 0; i < 8; ++i)
          comb[(g - 1) * kRowElems + (k * R + rt) * 8 + i] = acc[k][i];
    }
    __syncthreads();
    if (g == 0) {
#pragma unroll
      for (int gg = 1; gg < G; ++gg)
#pragma unroll
        for (int k = 0; k < K; ++k)
#pragma unroll
          for (int i = 0; i < 8; ++i)
            acc[k][i] += comb[(gg - 1) * kRowElems + (k * R + rt) * 8 + i];
    }
    __syncthreads();
  }
  if (g == 0) {
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int col = (k * R + rt) * 8;
      const int valid = chunk_valid(N, col);
      if (valid > 0) store8<float, VEC>(dst + col, valid, acc[k]);
    }
  }
}

template <typename TX, typename TY, int K>
struct BwdRow {
  Raw8<TX> x[K], dout[K], dh[K];
  Raw8<TY> y[K];
};

// CL: the per-column conditioning factors (weight * (1 + scale), gate) sit in
// LDS instead of registers, each thread reading back its own columns at the
// start of every row (no barrier: nothing is shared).  For 1024-thread blocks
// (16 wavefronts per row, 128 VGPRs per thread), whose registers cannot hold
// them beside the row and the column partials.
template <typename TX, typename TY, int K, int WPR, bool VEC, bool NT, bool PF, int MINB = 512,
          bool CL = false>
__global__ __launch_bounds__((BwdShape<WPR, MINB>::BLK)) void adaln_bwd_kernel(
    BwdArgs p) {
  using S = BwdShape<WPR, MINB>;
  static_assert(!CL || !PF, "LDS conditioning is for the loop without prefetch");
  __shared__ __attribute__((aligned(16))) float cond[CL ? 2 * kMaxN : 1];
  __shared__ float red[S::G * WPR];
  // combine buffer for the G row groups: (G - 1) x (R * K * 8) floats
  __shared__ float comb[S::G > 1 ? (S::G - 1) * S::R * K * 8 : 1];

  const int g = threadIdx.x / S::R;
  const int rt = threadIdx.x % S::R;
  const int64_t b = blockIdx.x / p.J;
  const int j = blockIdx.x % p.J;
  const int64_t t0 = (int64_t)j * p.rows_per_block;
  int64_t t1 = t0 + p.rows_per_block;
  if (t1 > p.T) t1 = p.T;

  // per-sample conditioning, held in registers across the rows:
  // wo = weight * (1 + scale[b]) (the dout -> dxhat factor) and gate[b]
  float wo[K][8], gv[K][8];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int col = (k * S::R + rt) * 8;
    const int valid = chunk_valid(p.N, col);
    float wv[8], sv[8];
    if (valid > 0) {
      load8_dyn<VEC>(p.weight, p.dt_weight, col, valid, wv);
      load8_dyn<VEC>(p.scale, p.dt_scale, b * p.ld_scale + col, valid, sv);
      load8_dyn<VEC>(p.gate, p.dt_gate, b * p.ld_gate + col, valid, gv[k]);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) wv[i] = sv[i] = gv[k][i] = 0.f;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) wo[k][i] = wv[i] * (1.f + sv[i]);
    if constexpr (CL) {
      float *cw = cond + (k * S::R + rt) * 8, *cg = cw + kMaxN;
#pragma unroll
      for (int i = 0; i < 8; i += 4) {
        *reinterpret_cast<float4 *>(cw + i) = make_float4(wo[k][i], wo[k][i + 1], wo[k][i + 2],
                                                          wo[k][i + 3]);
        *reinterpret_cast<float4 *>(cg + i) = make_float4(gv[k][i], gv[k][i + 1], gv[k][i + 2],
                                                          gv[k][i + 3]);
      }
    }
  }

  float accA[K][8], accS[K][8], accG[K][8];
#pragma unroll
  for (int k = 0; k < K; ++k)
#pragma unroll
    for (int i = 0; i < 8; ++i) accA[k][i] = accS[k][i] = accG[k][i] = 0.f;

  const TX *const xp = static_cast<const TX *>(p.x);
  const TY *const yp = static_cast<const TY *>(p.y);
  const TX *const dop = static_cast<const TX *>(p.dout);
  const TX *const dhp = static_cast<const TX *>(p.dh_up);

  auto load_row = [&](int64_t t, BwdRow<TX, TY, K> &rw) {
    const int64_t row = b * p.T + t;
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int col = (k * S::R + rt) * 8;
      const int valid = t < t1 ? chunk_valid(p.N, col) : 0;
      if (valid > 0) {
        rw.x[k].template load<VEC>(xp + row * p.ld_x + col, valid);
        rw.y[k].template load<VEC>(yp + row * p.ld_y + col, valid);
        if (dop) rw.dout[k].template load<VEC>(dop + row * (int64_t)p.N + col, valid);
        else rw.dout[k].zero();
        if (dhp) rw.dh[k].template load<VEC>(dhp + row * (int64_t)p.N + col, valid);
        else rw.dh[k].zero();
      } else {
        rw.x[k].zero(); rw.y[k].zero(); rw.dout[k].zero(); rw.dh[k].zero();
      }
    }
  };

  const int64_t nrows = t1 > t0 ? t1 - t0 : 0;
  const int64_t iters = (nrows + S::G - 1) / S::G;
  BwdRow<TX, TY, K> cur, nxt;
  if (PF && iters > 0) load_row(t0 + g, cur);
  for (int64_t it = 0; it < iters; ++it) {
    const int64_t t = t0 + it * S::G + g;
    const bool active = t < t1;
    const int64_t row = b * p.T + t;
    if constexpr (PF) {
      if (it + 1 < iters) load_row(t + S::G, nxt);
    } else {
      load_row(t, cur);
    }
    const float rstd = active ? p.rstd[row] : 0.f;

    // chunk k's conditioning factors: from registers, or (CL) read back from
    // LDS where they are used, so they are never all live at once
    auto cond_of = [&](int k, float (&w8)[8], float (&g8)[8]) {
      if constexpr (CL) {
        const float *cw = cond + (k * S::R + rt) * 8, *cg = cw + kMaxN;
#pragma unroll
        for (int i = 0; i < 8; i += 4) {
          const float4 a = *reinterpret_cast<const float4 *>(cw + i);
          const float4 e = *reinterpret_cast<const float4 *>(cg + i);
          w8[i] = a.x; w8[i + 1] = a.y; w8[i + 2] = a.z; w8[i + 3] = a.w;
          g8[i] = e.x; g8[i + 1] = e.y; g8[i + 2] = e.z; g8[i + 3] = e.w;
        }
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          w8[i] = wo[k][i];
          g8[i] = gv[k][i];
        }
      }
    };
    // xhat = (x + gate * y) * rstd (h recomputed in fp32, never re-read);
    // with CL formed again after the exchange (same operations, same
    // values) instead of held across it
    float xh[K][8];
    float dot = 0.f;
#pragma unroll
    for (int k = 0; k < K; ++k) {
      float w8[8], g8[8];
      cond_of(k, w8, g8);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float xv = (cur.x[k][i] + g8[i] * cur.y[k][i]) * rstd;
        if constexpr (!CL) xh[k][i] = xv;
        dot += (cur.dout[k][i] * w8[i]) * xv;
      }
    }
    dot = row_sum<WPR>(dot, red, g, rt);
    const float c = dot / (float)p.N;

#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int col = (k * S::R + rt) * 8;
      const int valid = active ? chunk_valid(p.N, col) : 0;
      if (valid > 0) {
        float w8[8], g8[8];
        cond_of(k, w8, g8);
        float dh[8], dyv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float d = cur.dout[k][i];
          const float xv = CL ? (cur.x[k][i] + g8[i] * cur.y[k][i]) * rstd : xh[k][i];
          dh[i] = cur.dh[k][i] + rstd * (d * w8[i] - xv * c);
          dyv[i] = dh[i] * g8[i];
          accA[k][i] += d * xv;
          accS[k][i] += d;
          accG[k][i] += dh[i] * cur.y[k][i];
        }
        store8_hint<TX, VEC, NT>(static_cast<TX *>(p.dx) + row * (int64_t)p.N + col, valid, dh);
        store8_hint<TY, VEC, NT>(static_cast<TY *>(p.dy) + row * (int64_t)p.N + col, valid, dyv);
      }
    }
    if constexpr (PF) cur = nxt;
  }

  // combine the G row groups in a fixed order (group 0 + 1 + ... + G-1) and
  // write the block's [3, N] partial row
  float *dst = p.partial + (int64_t)blockIdx.x * 3 * p.N;
  combine_store<K, S::G, S::R, VEC>(accA, comb, g, rt, dst, p.N);
  combine_store<K, S::G, S::R, VEC>(accS, comb, g, rt, dst + p.N, p.N);
  combine_store<K, S::G, S::R, VEC>(accG, comb, g, rt, dst + 2 * (int64_t)p.N, p.N);
}

// ---------------------------------------------------------------------------
// backward, software-pipelined: the rows of block (b, j) as in
// adaln_bwd_kernel (row group g takes rows t0 + g, t0 + g + G, ...), in
// batches of RB per row group, with batch i + 1's loads issued before batch
// i's math and stores (two register buffers in turn, the loop unrolled by
// two).  Per-row arithmetic, accumulation order and the final combine are
// adaln_bwd_kernel's, so the results are bit-identical to it.
// Host conditions: 16-bit x and y, vector I/O, one 8-element chunk per lane.
// ---------------------------------------------------------------------------
template <typename TX, typename TY, int K, int RB>
struct BwdBatch {
  BwdRow<TX, TY, K> rw[RB];
  float rs[RB];
};

template <typename TX, typename TY, int K, int WPR, bool NT, int RB, bool NTL>
__global__ __launch_bounds__((BwdShape<WPR>::BLK)) void adaln_bwd_pipe_kernel(BwdArgs p) {
  using S = BwdShape<WPR>;
  __shared__ float red[S::G * WPR * RB];
  __shared__ float comb[S::G > 1 ? (S::G - 1) * S::R * K * 8 : 1];

  const int g = threadIdx.x / S::R;
  const int rt = threadIdx.x % S::R;
  const int64_t b = blockIdx.x / p.J;
  const int j = blockIdx.x % p.J;
  const int64_t t0 = (int64_t)j * p.rows_per_block;
  int64_t t1 = t0 + p.rows_per_block;
  if (t1 > p.T) t1 = p.T;

  float wo[K][8], gv[K][8];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int col = (k * S::R + rt) * 8;
    float wv[8], sv[8];
    if (col < p.N) {
      load8_dyn<true>(p.weight, p.dt_weight, col, 8, wv);
      load8_dyn<true>(p.scale, p.dt_scale, b * p.ld_scale + col, 8, sv);
      load8_dyn<true>(p.gate, p.dt_gate, b * p.ld_gate + col, 8, gv[k]);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) wv[i] = sv[i] = gv[k][i] = 0.f;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) wo[k][i] = wv[i] * (1.f + sv[i]);
  }

  float accA[K][8], accS[K][8], accG[K][8];
#pragma unroll
  for (int k = 0; k < K; ++k)
#pragma unroll
    for (int i = 0; i < 8; ++i) accA[k][i] = accS[k][i] = accG[k][i] = 0.f;

  const TX *const xp = static_cast<const TX *>(p.x);
  const TY *const yp = static_cast<const TY *>(p.y);
  const TX *const dop = static_cast<const TX *>(p.dout);
  const TX *const dhp = static_cast<const TX *>(p.dh_up);
  using VX = typename Raw8<TX>::vtype;
  using VY = typename Raw8<TY>::vtype;

  using Batch = BwdBatch<TX, TY, K, RB>;
  auto load_batch = [&](int64_t it, Batch &bt) {
#pragma unroll
    for (int q = 0; q < RB; ++q) {
      const int64_t t = t0 + (it + q) * S::G + g;
      const int64_t row = b * p.T + t;
      BwdRow<TX, TY, K> &rw = bt.rw[q];
#pragma unroll
      for (int k = 0; k < K; ++k) {
        const int col = (k * S::R + rt) * 8;
        if (t < t1 && col < p.N) {
          rw.x[k].v = stream_load_vec<VX, NTL>(xp + row * p.ld_x + col);
          rw.y[k].v = stream_load_vec<VY, NTL>(yp + row * p.ld_y + col);
          if (dop) rw.dout[k].v = stream_load_vec<VX, NTL>(dop + row * (int64_t)p.N + col);
          else rw.dout[k].zero();
          if (dhp) rw.dh[k].v = stream_load_vec<VX, NTL>(dhp + row * (int64_t)p.N + col);
          else rw.dh[k].zero();
        } else {
          rw.x[k].zero(); rw.y[k].zero(); rw.dout[k].zero(); rw.dh[k].zero();
        }
      }
      bt.rs[q] = t < t1 ? p.rstd[row] : 0.f;
    }
  };
  auto work_batch = [&](int64_t it, const Batch &bt) {
    float xh[RB][K][8], dot[RB];
#pragma unroll
    for (int q = 0; q < RB; ++q) {
      dot[q] = 0.f;
#pragma unroll
      for (int k = 0; k < K; ++k)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          xh[q][k][i] = (bt.rw[q].x[k][i] + gv[k][i] * bt.rw[q].y[k][i]) * bt.rs[q];
          dot[q] += (bt.rw[q].dout[k][i] * wo[k][i]) * xh[q][k][i];
        }
    }
    row_sum_batch<WPR, RB>(dot, red, g, rt);
#pragma unroll
    for (int q = 0; q < RB; ++q) {
      const int64_t t = t0 + (it + q) * S::G + g;
      const int64_t row = b * p.T + t;
      const float c = dot[q] / (float)p.N;
#pragma unroll
      for (int k = 0; k < K; ++k) {
        const int col = (k * S::R + rt) * 8;
        if (t < t1 && col < p.N) {
          float dh[8], dyv[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const float d = bt.rw[q].dout[k][i];
            dh[i] = bt.rw[q].dh[k][i] + bt.rs[q] * (d * wo[k][i] - xh[q][k][i] * c);
            dyv[i] = dh[i] * gv[k][i];
            accA[k][i] += d * xh[q][k][i];
            accS[k][i] += d;
            accG[k][i] += dh[i] * bt.rw[q].y[k][i];
          }
          store8_hint<TX, true, NT>(static_cast<TX *>(p.dx) + row * (int64_t)p.N + col, 8, dh);
          store8_hint<TY, true, NT>(static_cast<TY *>(p.dy) + row * (int64_t)p.N + col, 8, dyv);
        }
      }
    }
  };

  const int64_t nrows = t1 > t0 ? t1 - t0 : 0;
  const int64_t iters = (nrows + S::G - 1) / S::G;  // the same in every row group
  Batch A, B;
  if (iters > 0) load_batch(0, A);
  for (int64_t it = 0; it < iters; it += 2 * RB) {
    if (it + RB < iters) load_batch(it + RB, B);
    work_batch(it, A);
    if (it + RB < iters) {
      if (it + 2 * RB < iters) load_batch(it + 2 * RB, A);
      work_batch(it + RB, B);
    }
  }

  float *dst = p.partial + (int64_t)blockIdx.x * 3 * p.N;
  combine_store<K, S::G, S::R, true>(accA, comb, g, rt, dst, p.N);
  combine_store<K, S::G, S::R, true>(accS, comb, g, rt, dst + p.N, p.N);
  combine_store<K, S::G, S::R, true>(accG, comb, g, rt, dst + 2 * (int64_t)p.N, p.N);
}

// ---------------------------------------------------------------------------
// planning
// ---------------------------------------------------------------------------
struct Plan {
  int fwd_wpr;  // forward: wavefronts per row (1, 2, 4, 8, 16)
  int fwd_k;    // forward: 8-element chunks per thread (1, 2)
  int fwd_rpg;  // forward: contiguous rows per row group
  int bwd_wpr;  // backward: wavefronts per row (1, 2, 4, 8, 16)
  int bwd_k;    // backward: 8-element chunks per thread (1, 2)
  int bwd_rb;   // pipelined backward (16-bit rows, one chunk per lane): rows per batch
  int J;        // backward blocks per sample
  int rows_per_block;
  int64_t B;
};

// Launch shapes for the 256-CU MI355X, from sweeps at the BASELINE shapes
// (bf16 [8,1024,1024] and [32,2048,2048]).  More wavefronts in flight beat
// deeper per-thread buffering for these streaming kernels, so rows of
// N >= 1024 are split over >= 2 wavefronts in the forward and the backward
// keeps one 8-element chunk per thread up to N = 4096 (8 wavefronts), two
// beyond (8 wavefronts up to N = 8192, 16 up to 16384).
// Forward: each row group walks clamp(M / 2048, 1, 8) consecutive rows
// (clamp(M / 256, 1, 8) for rows of 8 or more wavefronts).
// Backward: at most 256 blocks of 512 threads (1 per CU), each a run of one
// sample's rows, so the partial rows (B * J * 3 * N floats written, then
// reduced) are half those of 512 blocks.  16-bit rows of one chunk per lane
// take the pipelined kernel (adaln_bwd_pipe_kernel): batches of 2 rows per
// row group when a row group has at most 16 rows, of 1 row beyond (A/B on
// one box, fwd -> bwd -> reduce step, bit-identical): bf16 [8192, 1024]
// (8 rows per row group) 35.4 us with 2-row batches, 36.1 with 1-row, 36.3
// for the one-round kernel with 4-row batches it replaces; bf16 [65536,
// 2048] (128 rows per row group) 489 us with 1-row batches, 516 with
// 2-row, 503 one-round.  512 blocks lost at both shapes (38.4-39.7 us).
constexpr int kBwdBlocksTarget = 256;
constexpr int kBwdRb2MaxRows = 16;
// A cap on the blocks (and so the partial rows) per sample: past it more
// blocks only add partial rows for the reduction to read.
constexpr int kMaxBlocksPerSample = 1024;
constexpr int kFwdGroupsTarget = 2048;
// Rows of 8 or more wavefronts (N > 4096 with two chunks per lane) fill a
// block each; for them ~256 row groups (one per CU, 2-4 rows each, taken in
// batches) beat one row per block: bf16 [1024, 8192] forward 14.5 us with 4
// rows per group against 23.3 us with 1, [512, 16384] 14.4 us with 2 against
// 22.0 us with 1 (and 16.8 us with 4).
constexpr int kFwdWideGroupsTarget = 256;
constexpr int kFwdMaxRowsPerGroup = 8;

inline int pick_wpr(int64_t N, int max_k) {
  int wpr = 1;
  while ((int64_t)64 * wpr * 8 * max_k < N) wpr *= 2;
  return wpr;
}
inline int pick_k(int64_t N, int wpr) {
  const int64_t per_chunk = (int64_t)64 * wpr * 8;
  const int64_t k = (N + per_chunk - 1) / per_chunk;
  return k <= 1 ? 1 : (k <= 2 ? 2 : 4);
}

// Launch choices make_plan takes from its caller; the defaults are the
// shipped plan (a measurement build sweeps them).
struct Knobs {
  int fwd_groups = kFwdGroupsTarget;  // forward row groups aimed at
  int bwd_blocks = kBwdBlocksTarget;  // backward blocks aimed at
  int fwd_rpg = 0;  // rows per forward row group (0: M / fwd_groups, capped)
  int bwd_rb = 0;   // pipelined backward rows per batch, 1 or 2 (0: planned)
};

inline Plan make_plan(int64_t M, int64_t N, int64_t T, const Knobs &kn = Knobs()) {
  Plan pl{};
  int fwd_groups = kn.fwd_groups;
  const int bwd_blocks = kn.bwd_blocks;
  pl.fwd_wpr = pick_wpr(N, 2);
  if (N >= 1024 && pl.fwd_wpr < 2) pl.fwd_wpr = 2;
  pl.fwd_k = pick_k(N, pl.fwd_wpr);
  if (pl.fwd_wpr >= 8 && fwd_groups == kFwdGroupsTarget) fwd_groups = kFwdWideGroupsTarget;
  {
    int64_t rpg = M / fwd_groups;
    if (rpg > kFwdMaxRowsPerGroup) rpg = kFwdMaxRowsPerGroup;
    pl.fwd_rpg = (int)(rpg < 1 ? 1 : rpg);
  }
  if (kn.fwd_rpg > 0) pl.fwd_rpg = kn.fwd_rpg;
  // One chunk per lane up to N = 4096 (8 wavefronts); wider rows take two
  // chunks per lane, so rows up to 8192 stay on 512-thread blocks (256
  // VGPRs, no spills: bf16 [1024, 8192] backward 24.5 us) instead of
  // 1024-thread blocks whose 128-VGPR budget spills the row (134 us).
  pl.bwd_wpr = pick_wpr(N, N > 4096 ? 2 : 1);
  if (pl.bwd_wpr > 16) pl.bwd_wpr = 16;
  pl.bwd_k = pick_k(N, pl.bwd_wpr);
  pl.B = M / T;
  const int R = 64 * pl.bwd_wpr;
  const int G = (R < 512 ? 512 : R) / R;
  // At most bwd_blocks blocks in all: the backward kernels hold one
  // 512-thread block per CU (151-251 VGPRs a lane), so blocks past 256 run as
  // a second, nearly empty round (bf16 [24, 2048, 2048] with 11 blocks per
  // sample, 264 blocks: 361 us against 235 us with 10).
  int64_t J = pl.B > 0 ? bwd_blocks / pl.B : 1;
  const int64_t jmax = (T + 2 * G - 1) / (2 * G);  // >= 2 rows per row group
  if (J > jmax) J = jmax;
  if (J > kMaxBlocksPerSample) J = kMaxBlocksPerSample;
  if (J < 1) J = 1;
  pl.rows_per_block = (int)((T + J - 1) / J);
  pl.J = (int)((T + pl.rows_per_block - 1) / pl.rows_per_block);
  const int64_t group_rows = (pl.rows_per_block + G - 1) / G;
  pl.bwd_rb = kn.bwd_rb > 0 ? (kn.bwd_rb >= 2 ? 2 : 1) : (group_rows <= kBwdRb2MaxRows ? 2 : 1);
  return pl;
}

inline size_t workspace_bytes(const Plan &pl, int64_t N) {
  return (size_t)(pl.B * pl.J * 3 * N) * sizeof(float);
}

// blocks of shape S covering M rows, pl.fwd_rpg consecutive rows per row group
template <class S>
inline unsigned fwd_grid(const Plan &pl, int64_t M) {
  const int64_t per_block = (int64_t)S::G * pl.fwd_rpg;
  return (unsigned)((M + per_block - 1) / per_block);
}

// ---------------------------------------------------------------------------
// dispatch over (TX, TY) x K x WPR x VEC (stores: non-temporal; backward:
// next-row prefetch)
// ---------------------------------------------------------------------------
constexpr bool kFwdNT = true;
constexpr bool kBwdNT = true;

// The batched forward (adaln_fwd_batch_kernel) takes RB rows per step: 4 with
// one 8-element chunk per thread, 2 with two; 16-bit x and y only (fp32 rows
// would not fit the registers), and only when every row group's rows lie in
// one sample and split into whole batches.  Measured at bf16 [8192, 1024]:
// 10.5 us against 12.3 us for the one-row-at-a-time kernel, bit-identical.
template <typename TX, typename TY, int K>
constexpr int fwd_batch_rows() {
  return (sizeof(TX) == 2 && sizeof(TY) == 2) ? (K == 1 ? 4 : 2) : 1;
}
template <typename TX, typename TY, bool VEC, int WPR, int K>
int launch_fwd_t(const FwdArgs &a, const Plan &pl, hipStream_t s) {
  using S = FwdShape<WPR, fwd_min_block<K>()>;  // the shape of both kernels below
  constexpr int RB = fwd_batch_rows<TX, TY, K>();
  if constexpr (VEC && RB > 1) {
    if (a.rows_per_group % RB == 0 && a.T % a.rows_per_group == 0) {
      if (nt_loads_for(a.M * a.N * (int64_t)(sizeof(TX) + sizeof(TY))))
        adaln_fwd_batch_kernel<TX, TY, K, WPR, VEC, kFwdNT, RB, true>
            <<<fwd_grid<S>(pl, a.M), S::BLK, 0, s>>>(a);
      else
        adaln_fwd_batch_kernel<TX, TY, K, WPR, VEC, kFwdNT, RB, false>
            <<<fwd_grid<S>(pl, a.M), S::BLK, 0, s>>>(a);
      return check_launch("nf_adaln_fwd");
    }
  }
  adaln_fwd_kernel<TX, TY, K, WPR, VEC, kFwdNT><<<fwd_grid<S>(pl, a.M), S::BLK, 0, s>>>(a);
  return check_launch("nf_adaln_fwd");
}
// The pipelined backward takes 16-bit rows of one 8-element chunk per lane
// on the vector path; the others run adaln_bwd_kernel one row at a time
// (with the next-row prefetch when a thread holds two chunks per row).
template <typename TX, typename TY, int K>
constexpr bool bwd_pipelined() {
  return sizeof(TX) == 2 && sizeof(TY) == 2 && K == 1;
}
template <typename TX, typename TY, bool VEC, int WPR, int K>
int launch_bwd_t(const BwdArgs &a, const Plan &pl, hipStream_t s) {
  using S = BwdShape<WPR>;
  const unsigned grid = (unsigned)(pl.B * a.J);
  if constexpr (VEC && bwd_pipelined<TX, TY, K>()) {
    const int64_t in_row = (int64_t)(sizeof(TX) * (1 + (a.dout ? 1 : 0) + (a.dh_up ? 1 : 0)) +
                                     sizeof(TY));
    const bool ntl = nt_loads_for(a.M * a.N * in_row);
    if (pl.bwd_rb == 2 && ntl)
      adaln_bwd_pipe_kernel<TX, TY, K, WPR, kBwdNT, 2, true><<<grid, S::BLK, 0, s>>>(a);
    else if (pl.bwd_rb == 2)
      adaln_bwd_pipe_kernel<TX, TY, K, WPR, kBwdNT, 2, false><<<grid, S::BLK, 0, s>>>(a);
    else if (ntl)
      adaln_bwd_pipe_kernel<TX, TY, K, WPR, kBwdNT, 1, true><<<grid, S::BLK, 0, s>>>(a);
    else
      adaln_bwd_pipe_kernel<TX, TY, K, WPR, kBwdNT, 1, false><<<grid, S::BLK, 0, s>>>(a);
  } else {
    // The next-row prefetch needs a second row of registers; 1024-thread
    // blocks (16 wavefronts per row, N > 8192) have 128 VGPRs and spill less
    // without it (bf16 [512, 16384]: 66 us against 116 us).
    constexpr bool PF = K > 1 && S::BLK <= 512;
    constexpr bool CL = S::BLK > 512;
    adaln_bwd_kernel<TX, TY, K, WPR, VEC, kBwdNT, PF, 512, CL><<<grid, S::BLK, 0, s>>>(a);
  }
  return check_launch("nf_adaln_bwd");
}

// (wavefronts per row, chunks per lane) pairs make_plan gives on the vector
// path, so only those are compiled: forward one chunk up to 2 wavefronts (N <=
// 1024), two chunks otherwise; backward one chunk up to 8 wavefronts (N <=
// 4096), two chunks from 8 (N > 4096).  The element-wise path always takes two.
// make_plan never asks for more than two chunks per lane (pick_wpr widens the
// row first); a plan that did is refused rather than run on a kernel that
// would cover only part of the row.
template <int WPR, int K>
constexpr bool fwd_planned() {
  return K == 2 || WPR <= 2;
}
template <int WPR, int K>
constexpr bool bwd_planned() {
  return K == 1 ? WPR <= 8 : WPR >= 8;
}
inline int unplanned(const char *who, int wpr, int k) {
  return set_error(NF_ERR_ARG, "%s: no kernel for %d wavefronts x %d chunks per row", who, wpr,
                   k);
}

template <typename TX, typename TY, bool VEC, int WPR>
int fwd_k(const FwdArgs &a, const Plan &pl, hipStream_t s) {
  if constexpr (!VEC) {
    return launch_fwd_t<TX, TY, false, WPR, 2>(a, pl, s);
  } else {
    if (pl.fwd_k == 1) {
      if constexpr (fwd_planned<WPR, 1>()) return launch_fwd_t<TX, TY, true, WPR, 1>(a, pl, s);
      return unplanned("nf_adaln_fwd", WPR, 1);
    }
    if (pl.fwd_k != 2) return unplanned("nf_adaln_fwd", WPR, pl.fwd_k);
    if constexpr (fwd_planned<WPR, 2>()) return launch_fwd_t<TX, TY, true, WPR, 2>(a, pl, s);
    return unplanned("nf_adaln_fwd", WPR, 2);
  }
}
template <typename TX, typename TY, bool VEC, int WPR>
int bwd_k(const BwdArgs &a, const Plan &pl, hipStream_t s) {
  if constexpr (!VEC) {
    return launch_bwd_t<TX, TY, false, WPR, 2>(a, pl, s);
  } else {
    if (pl.bwd_k == 1) {
      if constexpr (bwd_planned<WPR, 1>()) return launch_bwd_t<TX, TY, true, WPR, 1>(a, pl, s);
      return unplanned("nf_adaln_bwd", WPR, 1);
    }
    if (pl.bwd_k != 2) return unplanned("nf_adaln_bwd", WPR, pl.bwd_k);
    if constexpr (bwd_planned<WPR, 2>()) return launch_bwd_t<TX, TY, true, WPR, 2>(a, pl, s);
    return unplanned("nf_adaln_bwd", WPR, 2);
  }
}

template <typename TX, typename TY, bool VEC>
int fwd_w(const FwdArgs &a, const Plan &pl, hipStream_t s) {
  switch (pl.fwd_wpr) {
    case 1: return fwd_k<TX, TY, VEC, 1>(a, pl, s);
    case 2: return fwd_k<TX, TY, VEC, 2>(a, pl, s);
    case 4: return fwd_k<TX, TY, VEC, 4>(a, pl, s);
    case 8: return fwd_k<TX, TY, VEC, 8>(a, pl, s);
    default: return fwd_k<TX, TY, VEC, 16>(a, pl, s);
  }
}
template <typename TX, typename TY, bool VEC>
int bwd_w(const BwdArgs &a, const Plan &pl, hipStream_t s) {
  switch (pl.bwd_wpr) {
    case 1: return bwd_k<TX, TY, VEC, 1>(a, pl, s);
    case 2: return bwd_k<TX, TY, VEC, 2>(a, pl, s);
    case 4: return bwd_k<TX, TY, VEC, 4>(a, pl, s);
    case 8: return bwd_k<TX, TY, VEC, 8>(a, pl, s);
    default: return bwd_k<TX, TY, VEC, 16>(a, pl, s);
  }
}

// Explicitly instantiated once per (TX, TY) pair in adaln_inst_*.hip so the
// kernel variants compile in parallel translation units.
template <typename TX, typename TY>
int fwd_v(const FwdArgs &a, const Plan &pl, bool vec, hipStream_t s) {
  return vec ? fwd_w<TX, TY, true>(a, pl, s) : fwd_w<TX, TY, false>(a, pl, s);
}
template <typename TX, typename TY>
int bwd_v(const BwdArgs &a, const Plan &pl, bool vec, hipStream_t s) {
  return vec ? bwd_w<TX, TY, true>(a, pl, s) : bwd_w<TX, TY, false>(a, pl, s);
}

// supported (x, y) type pairs: equal types, or fp32 residual with a 16-bit
// branch output (the autocast mix of the DiT seams)
template <class F>
inline int dispatch_xy(int dt_x, int dt_y, const char *who, F &&f) {
  if (dt_x == NF_DTYPE_F32 && dt_y == NF_DTYPE_F32) return f(float(), float());
  if (dt_x == NF_DTYPE_BF16 && dt_y == NF_DTYPE_BF16) return f(bf16(), bf16());
  if (dt_x == NF_DTYPE_F16 && dt_y == NF_DTYPE_F16) return f(f16(), f16());
  if (dt_x == NF_DTYPE_F32 && dt_y == NF_DTYPE_BF16) return f(float(), bf16());
  if (dt_x == NF_DTYPE_F32 && dt_y == NF_DTYPE_F16) return f(float(), f16());
  return set_error(NF_ERR_DTYPE, "%s: unsupported (x, y) dtypes (%d, %d)", who,
                   dt_x, dt_y);
}

inline int check_shape(const char *who, int64_t M, int64_t N, int64_t T) {
  if (M < 0 || N <= 0 || T <= 0)
    return set_error(NF_ERR_ARG, "%s: bad shape M=%lld N=%lld T=%lld", who,
                     (long long)M, (long long)N, (long long)T);
  if (M % T != 0)
    return set_error(NF_ERR_ARG, "%s: M=%lld is not a multiple of T=%lld", who,
                     (long long)M, (long long)T);
  if (N > kMaxN)
    return set_error(NF_ERR_ARG, "%s: N=%lld exceeds %d", who, (long long)N, kMaxN);
  if (M > ((int64_t)1 << 40) / N)  // keeps grids and byte counts far from overflow
    return set_error(NF_ERR_ARG, "%s: M x N exceeds 2^40 elements", who);
  return NF_OK;
}

}  // namespace adaln
}  // namespace nf
