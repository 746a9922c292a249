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
  int ublocks;    // dgate/dshift/dscale blocks per sample: ceil(3N / 256)
  int gps_w;      // dweight blocks: row groups per sample (a power of two <= 32)
  int dw_blocks;  // dweight blocks: one per 32-column slice, or 0 without dweight
};

constexpr int kRcLanes = 8;                    // 16-byte lanes per slice row
constexpr int kRcCols = 4 * kRcLanes;          // columns per slice (one 128-byte line)
constexpr int kRcThreads = 256;
constexpr int kRcGroups = kRcThreads / kRcLanes;  // row groups per block (32)

// Four consecutive fp32 columns of a partial row; columns at or past N read
// as zero.  VEC: N % 4 == 0 and a 16-byte aligned workspace, so a 4-column
// vector is wholly inside or wholly outside the row.
template <bool VEC>
__device__ __forceinline__ float4 load_cols4(const float *row, int col, int N) {
  if constexpr (VEC) {
    if (col < N) return *reinterpret_cast<const float4 *>(row + col);
    return make_float4(0.f, 0.f, 0.f, 0.f);
  } else {
    float4 v;
    v.x = col < N ? row[col] : 0.f;
    v.y = col + 1 < N ? row[col + 1] : 0.f;
    v.z = col + 2 < N ? row[col + 2] : 0.f;
    v.w = col + 3 < N ? row[col + 3] : 0.f;
    return v;
  }
}
__device__ __forceinline__ void add4(float4 &a, const float4 &b) {
  a.x += b.x; a.y += b.y; a.z += b.z; a.w += b.w;
}
__device__ __forceinline__ void put4(float *dst, const float4 &v) {
  dst[0] = v.x; dst[1] = v.y; dst[2] = v.z; dst[3] = v.w;
}

// Sum of rows k, k + gps, ... (< J) of `base` (row pitch 3N floats, part
// `part` of each row), four columns from `col`.  The loads of up to kRcBatch
// rows are all issued before the first add, so a thread waits for one memory
// round trip per batch, not one per row; the adds run in row order.
constexpr int kRcBatch = 8;
constexpr int kRcRowBatch = 16;  // rows loaded per round trip by a dgate/dshift/dscale thread
template <bool VEC>
__device__ __forceinline__ float4 sum_rows(const float *base, int64_t N3, int k, int gps, int J,
                                           int col, int N) {
  float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int j0 = k; j0 < J; j0 += kRcBatch * gps) {
    float4 v[kRcBatch];
#pragma unroll
    for (int u = 0; u < kRcBatch; ++u) {
      const int j = j0 + u * gps;
      v[u] = j < J ? load_cols4<VEC>(base + j * N3, col, N) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int u = 0; u < kRcBatch; ++u)
      if (j0 + u * gps < J) add4(a, v[u]);
  }
  return a;
}

// Partner exchanges between the row groups of a wavefront: group g holds
// lanes [8g, 8g + 8) of the block, so group g ^ 1, g ^ 2, g ^ 4 sits at lane
// offset 8, 16, 32.  xor 8: DPP row_ror:8 (a rotation by half of a 16-lane
// row); xor 16: ds_swizzle in bit-mask mode (xor mask 16 inside 32 lanes);
// xor 32: ds_bpermute.
__device__ __forceinline__ float xor_lanes8(float v) { return dpp<0x128>(v); }
__device__ __forceinline__ float xor_lanes16(float v) {
  return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F));
}
__device__ __forceinline__ float xor_lanes32(float v) { return __shfl_xor(v, 32); }

// Adds the values of the `gps` consecutive row groups that share a sample
// (gps a power of two, groups aligned to it) inside the wavefront, up to the
// 8 groups a wavefront holds: afterwards the first group of each sample (of
// each wavefront, for gps > 8) holds the total.  The addition tree is fixed
// by gps.
template <int NV>
__device__ __forceinline__ void combine_groups(float (&v)[NV], int gps) {
  if (gps >= 2) {
#pragma unroll
    for (int i = 0; i < NV; ++i) v[i] += xor_lanes8(v[i]);
  }
  if (gps >= 4) {
#pragma unroll
    for (int i = 0; i < NV; ++i) v[i] += xor_lanes16(v[i]);
  }
  if (gps >= 8) {
#pragma unroll
    for (int i = 0; i < NV; ++i) v[i] += xor_lanes32(v[i]);
  }
}

// Four consecutive entries of a [*, N] conditioning row (runtime dtype),
// entries at or past N read as zero.
__device__ __forceinline__ void load_cond4(const void *p, int dt, int64_t row_off, int col, int N,
                                           float (&v)[4]) {
  float t8[8];
  const int valid = N - col < 4 ? N - col : 4;
  load8_dyn<false>(p, dt, row_off + col, valid < 0 ? 0 : valid, t8);
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = t8[i];
}

// One entry of a conditioning tensor (runtime dtype).
__device__ __forceinline__ float load_cond1(const void *p, int dt, int64_t off) {
  float t8[8];
  load8_dyn<false>(p, dt, off, 1, t8);
  return t8[0];
}

// Sum of the per-wavefront totals red[w0 .. w0 + wps) (wps <= 4) of one
// entry: the reads are issued together, then added in order.
__device__ __forceinline__ float sum_waves(const float *first, int stride, int wps) {
  float x[4];
#pragma unroll
  for (int ww = 0; ww < 4; ++ww) x[ww] = ww < wps ? first[ww * stride] : 0.f;
  float s = x[0];
#pragma unroll
  for (int ww = 1; ww < 4; ++ww)
    if (ww < wps) s += x[ww];
  return s;
}

// Two kinds of 256-thread blocks:
//  * blocks [0, dw_blocks), one per 32-column slice when dweight is asked
//    for: dweight = sum_b (1 + scale_b) A_b.  Each thread loads 16 bytes of
//    a partial row at a time (8 lanes per slice row, 32 row groups per
//    block, 8 per wavefront); up to 32 / gps_w samples per round, each
//    sample's J rows of A split over gps_w groups (a power of two): group k
//    sums rows k, k + gps_w, ... in order, the groups' sums are added by a
//    fixed tree of cross-lane exchanges inside each wavefront and, where a
//    sample spans several wavefronts (gps_w > 8), the wavefront totals in
//    order through LDS; the samples are added in order.
//  * the rest, ublocks per sample: one thread per entry of the sample's
//    [3, N] partial rows (dscale = weight * A, dshift, dgate), adding its J
//    rows in order, 16 loads in flight at a time; no LDS, no barrier.
// Every order is fixed by the launch shape, so the sums are bit-reproducible.
// The weight and scale values a thread needs are loaded before the partial
// rows, so their latency hides under those loads; a kernel this small is
// bound by its chains of dependent memory and LDS accesses, not its bytes.
template <bool VEC>
__global__ __launch_bounds__(kRcThreads) void adaln_reduce_kernel(ReduceArgs p) {
  constexpr int kWaves = kRcThreads / kWave;        // 4
  constexpr int kGroupsPerWave = kWave / kRcLanes;  // 8
  __shared__ float red[kWaves][3][kRcCols];
  __shared__ float qbuf[kRcGroups][kRcCols];
  const int t = threadIdx.x;
  const int lane = t % kRcLanes, g = t / kRcLanes, w = t / kWave;
  const int N = p.N, J = p.J;
  const int64_t N3 = 3 * (int64_t)N;
  const int blk = blockIdx.x;
  if (blk < p.dw_blocks) {
    const int slice = blk;
    const int col = slice * kRcCols + 4 * lane;
    const int gps = p.gps_w, per_round = kRcGroups / gps;
    const int sb = g / gps, k = g % gps;
    // gps > 8: thread t < per_round * 32 finishes (sample t / 32, column t % 32)
    const int fs = t / kRcCols, fc = t % kRcCols, fcc = slice * kRcCols + fc;
    float dw = 0.f;
    for (int b0 = 0; b0 < p.B; b0 += per_round) {
      const int nb = p.B - b0 < per_round ? p.B - b0 : per_round;
      const bool live = sb < nb;
      float sc[4] = {0.f, 0.f, 0.f, 0.f};
      if (gps <= kGroupsPerWave) {
        if (live && k == 0)
          load_cond4(p.scale, p.dt_scale, (int64_t)(b0 + sb) * p.ld_scale, col, N, sc);
      } else if (fs < nb && fcc < N) {
        sc[0] = load_cond1(p.scale, p.dt_scale, (int64_t)(b0 + fs) * p.ld_scale + fcc);
      }
      float v[4] = {0.f, 0.f, 0.f, 0.f};
      if (live) {
        const float4 a =
            sum_rows<VEC>(p.partial + ((int64_t)(b0 + sb) * J) * N3, N3, k, gps, J, col, N);
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
      }
      combine_groups(v, gps);
      if (gps > kGroupsPerWave) {
        if (g % kGroupsPerWave == 0) put4(&red[w][0][4 * lane], make_float4(v[0], v[1], v[2], v[3]));
        __syncthreads();
        const int wps = gps / kGroupsPerWave;
        if (fs < nb) qbuf[fs][fc] = (1.f + sc[0]) * sum_waves(&red[fs * wps][0][fc], 3 * kRcCols, wps);
      } else if (live && k == 0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) qbuf[sb][4 * lane + i] = (1.f + sc[i]) * v[i];
      }
      __syncthreads();
      if (t < kRcCols) {
#pragma unroll 8
        for (int s2 = 0; s2 < nb; ++s2) dw += qbuf[s2][t];
      }
      __syncthreads();
    }
    const int cc = slice * kRcCols + t;
    if (t < kRcCols && cc < N) store_dyn(p.dweight, p.dt_weight, cc, dw);
    return;
  }
  // dgate / dshift / dscale: thread t of block (b, ub) owns entry
  // u = 256 ub + t of sample b's [3, N] partial rows (kind u / N: 0 A,
  // 1 shift, 2 gate; column u % N) and adds its J rows in order.
  const int k0 = blk - p.dw_blocks;
  const int b = k0 / p.ublocks;
  const int u = (k0 % p.ublocks) * kRcThreads + t;
  if (u >= 3 * N) return;
  const int q = (u >= N) + (u >= 2 * N);
  const int c = u - q * N;
  void *out = q == 0 ? p.dscale : (q == 1 ? p.dshift : p.dgate);
  if (!out) return;
  const int dt = q == 0 ? p.dt_scale : (q == 1 ? p.dt_shift : p.dt_gate);
  const float wc = q == 0 ? load_cond1(p.weight, p.dt_weight, c) : 1.f;
  const float *base = p.partial + ((int64_t)b * J) * N3 + u;
  float acc = 0.f;
  for (int j0 = 0; j0 < J; j0 += kRcRowBatch) {
    float x[kRcRowBatch];
#pragma unroll
    for (int i = 0; i < kRcRowBatch; ++i) x[i] = j0 + i < J ? base[(int64_t)(j0 + i) * N3] : 0.f;
#pragma unroll
    for (int i = 0; i < kRcRowBatch; ++i)
      if (j0 + i < J) acc += x[i];
  }
  store_dyn(out, dt, (int64_t)b * N + c, wc * acc);
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
  // with no rows there is no sample: nothing is read, dweight becomes 0
  if (M > 0 && (!weight || !scale))
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
  const int J = M > 0 ? pl.J : 1;
  const int B = M > 0 ? (int)pl.B : 0;
  const int slices = (int)((N + kRcCols - 1) / kRcCols);
  // dweight: the smallest power-of-two group count per sample that lets one
  // round hold every sample (at most 32 per round)
  int gps_w = kRcGroups;
  while (gps_w > 1 && (kRcGroups / gps_w) < B) gps_w /= 2;
  const int dw_blocks = dweight ? slices : 0;
  const int ublocks = (int)((3 * N + kRcThreads - 1) / kRcThreads);
  const int64_t sample_blocks = (dgate || dscale || dshift) ? (int64_t)B * ublocks : 0;
  const int64_t grid = dw_blocks + sample_blocks;
  if (grid == 0) return NF_OK;
  if (grid > INT32_MAX) return set_error(NF_ERR_ARG, "nf_adaln_bwd_reduce: too many blocks");
  ReduceArgs r{static_cast<const float *>(workspace), weight, scale, dgate, dscale, dshift,
               dweight, ld_scale, (int)N, J, B, dt_weight, dt_scale, dt_gate, dt_shift,
               ublocks, gps_w, dw_blocks};
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool vec = N % 4 == 0 && (M == 0 || aligned16(workspace));
  if (vec)
    adaln_reduce_kernel<true><<<(unsigned)grid, kRcThreads, 0, s>>>(r);
  else
    adaln_reduce_kernel<false><<<(unsigned)grid, kRcThreads, 0, s>>>(r);
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
