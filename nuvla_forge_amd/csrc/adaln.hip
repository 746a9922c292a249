// adaLN seam C entry points and the fixed-order partial reductions.  The
// forward/backward row kernels live in adaln_impl.h and are instantiated per
// (x, y) element-type pair in adaln_inst_*.hip.
#include "adaln_impl.h"

namespace nf {
namespace adaln {

#define NF_ADALN_EXTERN(TX, TY)                                              \
  extern template int fwd_v<TX, TY>(const FwdArgs &, const Plan &, bool,     \
                                    hipStream_t);                            \
  extern template int bwd_v<TX, TY>(const BwdArgs &, const Plan &, bool,     \
                                    hipStream_t);
NF_ADALN_EXTERN(float, float)
NF_ADALN_EXTERN(bf16, bf16)
NF_ADALN_EXTERN(f16, f16)
NF_ADALN_EXTERN(float, bf16)
NF_ADALN_EXTERN(float, f16)
#undef NF_ADALN_EXTERN

// ---------------------------------------------------------------------------
// fixed-order reductions of the partial rows
// ---------------------------------------------------------------------------
struct ReduceArgs {
  const float *partial;  // [B * J, 3, N]
  const void *weight;
  const void *scale;
  void *dgate;
  void *dscale;
  void *dshift;
  float *q;  // [B, N]: (1 + scale_b) * A_b, for dweight
  int64_t ld_scale;
  int N, J, B;
  int dt_weight, dt_scale, dt_gate, dt_shift;
};

constexpr int kRedCols = 64;
constexpr int kRedSplit = 4;

// grid (ceil(N / 64), B); thread (c, s) sums partial rows j = s, s+4, ...
__global__ __launch_bounds__(kRedCols *kRedSplit) void adaln_reduce_samples(
    ReduceArgs p) {
  __shared__ float part[3][kRedSplit][kRedCols];
  const int c = threadIdx.x % kRedCols;
  const int s = threadIdx.x / kRedCols;
  const int col = blockIdx.x * kRedCols + c;
  const int64_t b = blockIdx.y;
  float a0 = 0.f, a1 = 0.f, a2 = 0.f;
  if (col < p.N) {
    for (int j = s; j < p.J; j += kRedSplit) {
      const float *src = p.partial + ((b * p.J + j) * 3) * (int64_t)p.N + col;
      a0 += src[0];
      a1 += src[p.N];
      a2 += src[2 * (int64_t)p.N];
    }
  }
  part[0][s][c] = a0;
  part[1][s][c] = a1;
  part[2][s][c] = a2;
  __syncthreads();
  if (s == 0 && col < p.N) {
    float A = 0.f, Sh = 0.f, G = 0.f;
#pragma unroll
    for (int i = 0; i < kRedSplit; ++i) {
      A += part[0][i][c];
      Sh += part[1][i][c];
      G += part[2][i][c];
    }
    const int64_t o = b * p.N + col;
    if (p.dgate) store_dyn(p.dgate, p.dt_gate, o, G);
    if (p.dshift) store_dyn(p.dshift, p.dt_shift, o, Sh);
    if (p.dscale || p.q) {
      float w[8], sc[8];
      load8_dyn<false>(p.weight, p.dt_weight, col, 1, w);
      if (p.dscale) store_dyn(p.dscale, p.dt_scale, o, w[0] * A);
      if (p.q) {
        load8_dyn<false>(p.scale, p.dt_scale, b * p.ld_scale + col, 1, sc);
        p.q[o] = (1.f + sc[0]) * A;
      }
    }
  }
}

// dweight[n] = sum_b q[b, n], b ascending
__global__ __launch_bounds__(256) void adaln_reduce_weight(
    const float *__restrict__ q, void *dweight, int dt_weight, int N, int B) {
  const int col = blockIdx.x * 256 + threadIdx.x;
  if (col >= N) return;
  float acc = 0.f;
  for (int b = 0; b < B; ++b) acc += q[(int64_t)b * N + col];
  store_dyn(dweight, dt_weight, col, acc);
}

}  // namespace adaln
}  // namespace nf

using namespace nf;
using namespace nf::adaln;
extern "C" int nf_adaln_fwd(const void *x, int64_t ld_x, const void *y,
                            int64_t ld_y, const void *gate, int64_t ld_gate,
                            const void *weight, const void *scale,
                            int64_t ld_scale, const void *shift,
                            int64_t ld_shift, void *h, void *out, float *rstd,
                            int64_t M, int64_t N, int64_t T, float eps,
                            int dt_x, int dt_y, int dt_gate, int dt_weight,
                            int dt_scale, int dt_shift, void *stream) {
  if (int e = check_shape("nf_adaln_fwd", M, N, T)) return e;
  if (M == 0) return NF_OK;
  if (!x || !y || !gate || !weight || !scale || !shift || !h || !out || !rstd)
    return set_error(NF_ERR_ARG, "nf_adaln_fwd: null pointer");
  if (ld_x < N || ld_y < N || ld_gate < 0 || ld_scale < 0 || ld_shift < 0)
    return set_error(NF_ERR_ARG, "nf_adaln_fwd: bad row stride");
  if (!is_dtype(dt_gate) || !is_dtype(dt_weight) || !is_dtype(dt_scale) ||
      !is_dtype(dt_shift))
    return set_error(NF_ERR_DTYPE, "nf_adaln_fwd: bad conditioning dtype");
  const bool vec = N % 8 == 0 && ld_x % 8 == 0 && ld_y % 8 == 0 &&
                   ld_gate % 8 == 0 && ld_scale % 8 == 0 && ld_shift % 8 == 0 &&
                   aligned16(x) && aligned16(y) && aligned16(gate) &&
                   aligned16(weight) && aligned16(scale) && aligned16(shift) &&
                   aligned16(h) && aligned16(out);
  FwdArgs a{x, y, gate, weight, scale, shift, h, out, rstd,
            ld_x, ld_y, ld_gate, ld_scale, ld_shift, M, T, (int)N, eps,
            dt_gate, dt_weight, dt_scale, dt_shift};
  const Plan pl = make_plan(M, N, T);
  hipStream_t s = static_cast<hipStream_t>(stream);
  return dispatch_xy(dt_x, dt_y, "nf_adaln_fwd", [&](auto tx, auto ty) {
    return fwd_v<decltype(tx), decltype(ty)>(a, pl, vec, s);
  });
}

extern "C" size_t nf_adaln_bwd_workspace(int64_t M, int64_t N, int64_t T) {
  if (M <= 0 || N <= 0 || T <= 0 || M % T != 0) return 0;
  return workspace_bytes(make_plan(M, N, T), N);
}

extern "C" int nf_adaln_bwd(const void *dh_up, const void *dout, const void *x,
                            int64_t ld_x, const void *y, int64_t ld_y,
                            const void *gate, int64_t ld_gate,
                            const void *weight, const void *scale,
                            int64_t ld_scale, const float *rstd, void *dx,
                            void *dy, void *dgate, void *dweight, void *dscale,
                            void *dshift, void *workspace,
                            size_t workspace_bytes_given, int64_t M, int64_t N,
                            int64_t T, int dt_x, int dt_y, int dt_gate,
                            int dt_weight, int dt_scale, int dt_shift,
                            void *stream) {
  if (int e = check_shape("nf_adaln_bwd", M, N, T)) return e;
  if (M == 0) return NF_OK;
  if (!x || !y || !gate || !weight || !scale || !rstd || !dx || !dy)
    return set_error(NF_ERR_ARG, "nf_adaln_bwd: null pointer");
  if (ld_x < N || ld_y < N || ld_gate < 0 || ld_scale < 0)
    return set_error(NF_ERR_ARG, "nf_adaln_bwd: bad row stride");
  if (!is_dtype(dt_gate) || !is_dtype(dt_weight) || !is_dtype(dt_scale) ||
      !is_dtype(dt_shift))
    return set_error(NF_ERR_DTYPE, "nf_adaln_bwd: bad conditioning dtype");
  const Plan pl = make_plan(M, N, T);
  const size_t need = workspace_bytes(pl, N);
  if (!workspace || workspace_bytes_given < need)
    return set_error(NF_ERR_WORKSPACE,
                     "nf_adaln_bwd: workspace %zu bytes < required %zu",
                     workspace_bytes_given, need);
  const bool vec = N % 8 == 0 && ld_x % 8 == 0 && ld_y % 8 == 0 &&
                   ld_gate % 8 == 0 && ld_scale % 8 == 0 && aligned16(x) &&
                   aligned16(y) && aligned16(gate) && aligned16(weight) &&
                   aligned16(scale) && aligned16(dx) && aligned16(dy) &&
                   aligned16(workspace) && (!dh_up || aligned16(dh_up)) &&
                   (!dout || aligned16(dout));
  float *partial = static_cast<float *>(workspace);
  float *q = partial + pl.B * pl.J * 3 * N;
  BwdArgs a{dh_up, dout, x, y, gate, weight, scale, rstd, dx, dy, partial,
            ld_x, ld_y, ld_gate, ld_scale, M, T, (int)N, pl.J,
            pl.rows_per_block, dt_gate, dt_weight, dt_scale};
  hipStream_t s = static_cast<hipStream_t>(stream);
  int e = dispatch_xy(dt_x, dt_y, "nf_adaln_bwd", [&](auto tx, auto ty) {
    return bwd_v<decltype(tx), decltype(ty)>(a, pl, vec, s);
  });
  if (e) return e;
  if (!dgate && !dscale && !dshift && !dweight) return NF_OK;
  ReduceArgs r{partial, weight, scale, dgate, dscale, dshift,
               dweight ? q : nullptr, ld_scale, (int)N, pl.J, (int)pl.B,
               dt_weight, dt_scale, dt_gate, dt_shift};
  dim3 g1((unsigned)((N + kRedCols - 1) / kRedCols), (unsigned)pl.B);
  adaln_reduce_samples<<<g1, kRedCols * kRedSplit, 0, s>>>(r);
  if ((e = check_launch("nf_adaln_bwd(reduce_samples)"))) return e;
  if (dweight) {
    adaln_reduce_weight<<<(unsigned)((N + 255) / 256), 256, 0, s>>>(
        q, dweight, dt_weight, (int)N, (int)pl.B);
    if ((e = check_launch("nf_adaln_bwd(reduce_weight)"))) return e;
  }
  return NF_OK;
}
