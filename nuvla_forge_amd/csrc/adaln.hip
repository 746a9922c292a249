// adaLN seam C entry points and the fixed-order partial reductions.  The
// forward/backward row kernels live in adaln_impl.h and are instantiated per
// (x, y) element-type pair in adaln_inst_*.hip.
#include <atomic>
#include <mutex>

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
// fixed-order reduction of the partial rows
// ---------------------------------------------------------------------------
struct ReduceArgs {
  const float *partial;  // [B * J, 3, N]
  const void *weight;
  const void *scale;
  void *dgate;
  void *dscale;
  void *dshift;
  void *dweight;
  int64_t ld_scale;
  int N, J, B;
  int dt_weight, dt_scale, dt_gate, dt_shift;
};

constexpr int kRcCols = 8;                     // columns per block
constexpr int kRcThreads = 1024;
constexpr int kRcQ = kRcThreads / kRcCols;     // threads per column (128)
constexpr int kRcSlots = 1024;                 // partial rows staged per round

// One block per 8-column slice.  A round stages the partial rows of up to
// 128 whole samples (<= 1024 rows) in LDS with one wave of loads (24 per
// thread at most); S = 128 / samples threads per (sample, column) each sum
// every S-th of the sample's J rows, one thread per (sample, column) adds the
// S results, and one thread per column folds the samples into dweight.  All
// orders are fixed, so the sums are bit-reproducible.
__global__ __launch_bounds__(kRcThreads) void adaln_reduce_kernel(ReduceArgs p) {
  __shared__ float buf[3][kRcSlots][kRcCols];
  __shared__ float part[3][kRcQ][kRcCols];
  __shared__ float qbuf[kRcQ][kRcCols];
  const int c = threadIdx.x % kRcCols;
  const int q = threadIdx.x / kRcCols;
  // Workgroups are dealt to the 8 XCDs round-robin (block i -> XCD i % 8) and
  // each XCD has its own L2.  Give every XCD a contiguous range of column
  // slices, so the four 32-byte slices of a 128-byte line are read by one L2
  // instead of four (bijection of [0, gridDim.x)).
  const int nblk = gridDim.x, xcd = blockIdx.x % 8, loc = blockIdx.x / 8;
  const int qx = nblk / 8, rx = nblk % 8;
  const int slice = xcd * qx + (xcd < rx ? xcd : rx) + loc;
  const int col = slice * kRcCols + c;
  const bool cv = col < p.N;
  const int64_t N = p.N;
  int per_round = kRcSlots / p.J;  // J <= 1024 by construction of the plan
  if (per_round > kRcQ) per_round = kRcQ;
  if (per_round < 1) per_round = 1;
  float dw = 0.f;
  for (int b0 = 0; b0 < p.B; b0 += per_round) {
    const int nb = p.B - b0 < per_round ? p.B - b0 : per_round;
    const int nslots = nb * p.J;
    const int64_t slot0 = (int64_t)b0 * p.J;
    for (int s = q; s < nslots; s += kRcQ) {
      const float *src = p.partial + (slot0 + s) * 3 * N + col;
      buf[0][s][c] = cv ? src[0] : 0.f;
      buf[1][s][c] = cv ? src[N] : 0.f;
      buf[2][s][c] = cv ? src[2 * N] : 0.f;
    }
    // the (sample, column) threads' weight and scale, loaded now so their
    // latency overlaps the partial-row loads instead of following the sums
    float wcol = 0.f, scol = 0.f;
    if (q < nb && cv) {
      float t8[8];
      if (p.dscale) {
        load8_dyn<false>(p.weight, p.dt_weight, col, 1, t8);
        wcol = t8[0];
      }
      if (p.dweight) {
        load8_dyn<false>(p.scale, p.dt_scale, (int64_t)(b0 + q) * p.ld_scale + col, 1, t8);
        scol = t8[0];
      }
    }
    __syncthreads();
    const int S = kRcQ / nb;  // splits per sample, >= 1
    {
      const int sb = q / S, sp = q % S;
      float A = 0.f, Sh = 0.f, G = 0.f;
      if (sb < nb) {
        for (int jj = sp; jj < p.J; jj += S) {
          A += buf[0][sb * p.J + jj][c];
          Sh += buf[1][sb * p.J + jj][c];
          G += buf[2][sb * p.J + jj][c];
        }
      }
      part[0][q][c] = A;
      part[1][q][c] = Sh;
      part[2][q][c] = G;
    }
    __syncthreads();
    if (q < nb) {
      float A = 0.f, Sh = 0.f, G = 0.f;
      for (int sp = 0; sp < S; ++sp) {
        A += part[0][q * S + sp][c];
        Sh += part[1][q * S + sp][c];
        G += part[2][q * S + sp][c];
      }
      float qv = 0.f;
      if (cv) {
        const int64_t b = b0 + q;
        const int64_t o = b * N + col;
        if (p.dgate) store_dyn(p.dgate, p.dt_gate, o, G);
        if (p.dshift) store_dyn(p.dshift, p.dt_shift, o, Sh);
        if (p.dscale) store_dyn(p.dscale, p.dt_scale, o, wcol * A);
        if (p.dweight) qv = (1.f + scol) * A;
      }
      qbuf[q][c] = qv;
    }
    __syncthreads();
    if (q == 0)
      for (int sb = 0; sb < nb; ++sb) dw += qbuf[sb][c];
    __syncthreads();
  }
  if (q == 0 && cv && p.dweight) store_dyn(p.dweight, p.dt_weight, col, dw);
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
  const Plan pl = make_plan(M, N, T);
  FwdArgs a{x, y, gate, weight, scale, shift, h, out, rstd,
            ld_x, ld_y, ld_gate, ld_scale, ld_shift, M, T, (int)N, pl.fwd_rpg, eps,
            dt_gate, dt_weight, dt_scale, dt_shift};
  hipStream_t s = static_cast<hipStream_t>(stream);
  return dispatch_xy(dt_x, dt_y, "nf_adaln_fwd", [&](auto tx, auto ty) {
    return fwd_v<decltype(tx), decltype(ty)>(a, pl, vec, s);
  });
}

extern "C" size_t nf_adaln_bwd_workspace(int64_t M, int64_t N, int64_t T) {
  if (M <= 0 || N <= 0 || T <= 0 || M % T != 0 || N > kMaxN || M > ((int64_t)1 << 40) / N)
    return 0;
  return workspace_bytes(make_plan(M, N, T), N);
}

extern "C" int nf_adaln_bwd(const void *dh_up, const void *dout, const void *x,
                            int64_t ld_x, const void *y, int64_t ld_y,
                            const void *gate, int64_t ld_gate,
                            const void *weight, const void *scale,
                            int64_t ld_scale, const float *rstd, void *dx,
                            void *dy, void *workspace,
                            size_t workspace_bytes_given, int64_t M, int64_t N,
                            int64_t T, int dt_x, int dt_y, int dt_gate,
                            int dt_weight, int dt_scale, void *stream) {
  if (int e = check_shape("nf_adaln_bwd", M, N, T)) return e;
  if (M == 0) return NF_OK;
  if (!x || !y || !gate || !weight || !scale || !rstd || !dx || !dy)
    return set_error(NF_ERR_ARG, "nf_adaln_bwd: null pointer");
  if (ld_x < N || ld_y < N || ld_gate < 0 || ld_scale < 0)
    return set_error(NF_ERR_ARG, "nf_adaln_bwd: bad row stride");
  if (!is_dtype(dt_gate) || !is_dtype(dt_weight) || !is_dtype(dt_scale))
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
  BwdArgs a{dh_up, dout, x, y, gate, weight, scale, rstd, dx, dy,
            static_cast<float *>(workspace), ld_x, ld_y, ld_gate, ld_scale,
            M, T, (int)N, pl.J, pl.rows_per_block, dt_gate, dt_weight, dt_scale};
  hipStream_t s = static_cast<hipStream_t>(stream);
  return dispatch_xy(dt_x, dt_y, "nf_adaln_bwd", [&](auto tx, auto ty) {
    return bwd_v<decltype(tx), decltype(ty)>(a, pl, vec, s);
  });
}

extern "C" int nf_adaln_bwd_reduce(void *workspace,
                                   size_t workspace_bytes_given,
                                   const void *weight, const void *scale,
                                   int64_t ld_scale, void *dgate, void *dweight,
                                   void *dscale, void *dshift, int64_t M,
                                   int64_t N, int64_t T, int dt_gate,
                                   int dt_weight, int dt_scale, int dt_shift,
                                   void *stream) {
  if (int e = check_shape("nf_adaln_bwd_reduce", M, N, T)) return e;
  if (!dgate && !dscale && !dshift && !dweight) return NF_OK;
  if (!weight || !scale)
    return set_error(NF_ERR_ARG, "nf_adaln_bwd_reduce: null pointer");
  if (ld_scale < 0) return set_error(NF_ERR_ARG, "nf_adaln_bwd_reduce: bad row stride");
  if (!is_dtype(dt_gate) || !is_dtype(dt_weight) || !is_dtype(dt_scale) ||
      !is_dtype(dt_shift))
    return set_error(NF_ERR_DTYPE, "nf_adaln_bwd_reduce: bad dtype");
  const Plan pl = make_plan(M, N, T);
  if (M > 0) {
    const size_t need = workspace_bytes(pl, N);
    if (!workspace || workspace_bytes_given < need)
      return set_error(NF_ERR_WORKSPACE,
                       "nf_adaln_bwd_reduce: workspace %zu bytes < required %zu",
                       workspace_bytes_given, need);
  }
  // M == 0: no sample, every sum is empty; the kernel writes dweight = 0
  ReduceArgs r{static_cast<const float *>(workspace), weight, scale, dgate, dscale, dshift,
               dweight, ld_scale, (int)N, M > 0 ? pl.J : 1, M > 0 ? (int)pl.B : 0,
               dt_weight, dt_scale, dt_gate, dt_shift};
  hipStream_t s = static_cast<hipStream_t>(stream);
  adaln_reduce_kernel<<<(unsigned)((N + kRcCols - 1) / kRcCols), kRcThreads, 0, s>>>(r);
  return check_launch("nf_adaln_bwd_reduce");
}

// ---------------------------------------------------------------------------
// The backward with no caller workspace: the partial rows live in `scratch`,
// a module-scope device array of NF_ADALN_SCRATCH_BYTES.  Every GPU the
// library runs on holds its own copy (allocated when the code object is
// loaded on that device, released at process exit).  In host code the name
// `scratch` is only a stand-in for the symbol, not a device address: the
// device address comes from hipGetSymbolAddress with that device current,
// once per device, and only that address reaches the kernels.
// ---------------------------------------------------------------------------
namespace {
constexpr size_t kScratchBytes = NF_ADALN_SCRATCH_BYTES;
__device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

constexpr int kMaxDevices = 64;
std::atomic<void *> g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mu;

// This device's copy of `scratch` (the current device's).
int scratch_of_current_device(void **out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess)
    return set_error(NF_ERR_LAUNCH, "nf_adaln_bwd_noalloc: hipGetDevice failed: %s",
                     hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return set_error(NF_ERR_ARG, "nf_adaln_bwd_noalloc: device %d beyond %d", dev, kMaxDevices);
  void *p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (!p) {
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess || !p)
        return set_error(NF_ERR_LAUNCH,
                         "nf_adaln_bwd_noalloc: hipGetSymbolAddress(scratch) failed on device "
                         "%d: %s", dev, hipGetErrorString(e));
      g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return NF_OK;
}
}  // namespace

extern "C" int nf_adaln_bwd_noalloc(const void *dh_up, const void *dout, const void *x,
                                    int64_t ld_x, const void *y, int64_t ld_y,
                                    const void *gate, int64_t ld_gate, const void *weight,
                                    const void *scale, int64_t ld_scale, const float *rstd,
                                    void *dx, void *dy, void *dgate, void *dweight,
                                    void *dscale, void *dshift, int64_t M, int64_t N,
                                    int64_t T, int dt_x, int dt_y, int dt_gate, int dt_weight,
                                    int dt_scale, int dt_shift, void *stream) {
  if (int e = check_shape("nf_adaln_bwd_noalloc", M, N, T)) return e;
  if (M == 0)  // no rows: the row part is empty, the reductions write dweight = 0
    return nf_adaln_bwd_reduce(nullptr, 0, weight, scale, ld_scale, dgate, dweight, dscale,
                               dshift, M, N, T, dt_gate, dt_weight, dt_scale, dt_shift, stream);
  const size_t need = workspace_bytes(make_plan(M, N, T), N);
  if (need > kScratchBytes)
    return set_error(NF_ERR_WORKSPACE,
                     "nf_adaln_bwd_noalloc: M=%lld N=%lld T=%lld needs %zu bytes of partial "
                     "rows, more than the %zu-byte static buffer (use nf_adaln_bwd with a "
                     "workspace)", (long long)M, (long long)N, (long long)T, need,
                     kScratchBytes);
  void *ws = nullptr;
  if (int e = scratch_of_current_device(&ws)) return e;
  // every partial row the reduction reads is written by the row kernel first
  // (one full [3, N] row per block), so nothing in the buffer needs clearing
  if (int e = nf_adaln_bwd(dh_up, dout, x, ld_x, y, ld_y, gate, ld_gate, weight, scale,
                           ld_scale, rstd, dx, dy, ws, kScratchBytes, M, N, T, dt_x, dt_y,
                           dt_gate, dt_weight, dt_scale, stream))
    return e;
  return nf_adaln_bwd_reduce(ws, kScratchBytes, weight, scale, ld_scale, dgate, dweight, dscale,
                             dshift, M, N, T, dt_gate, dt_weight, dt_scale, dt_shift, stream);
}
