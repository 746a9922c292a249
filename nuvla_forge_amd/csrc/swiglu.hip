// SwiGLU forward/backward: flat elementwise HBM-streaming kernels.
//
// Each thread owns UNROLL 8-element chunks spaced one block-width apart, so a
// wavefront's loads for one unroll step are 64 consecutive 16-byte vectors
// (bf16/f16) or 32-byte pairs (f32): fully coalesced 128-bit accesses.  All
// loads of a thread are issued before any math.  Math is fp32 with one
// rounding at the store; the backward recomputes the sigmoid from `a`.
//
// Stores carry the non-temporal hint (outputs are not re-read by the kernel;
// bf16 fwd+bwd [8192, 4096] 76.5 us against 78.8, [65536, 5632] 950 against
// 962 us); loads take it when the launch streams more input than the
// Infinity Cache holds (nt_loads_for: the stress shape's fwd+bwd 884 us).
//
// Launch shape: one-wavefront blocks with one chunk per thread, the most
// blocks and the fewest registers per wave, so the dispatcher keeps every CU
// full of short-lived waves.  Swept over blocks of 64-1024 threads and 1-8
// chunks per thread, fwd+bwd: bf16 [8192, 4096] 78.7 us (85% of 8 TB/s)
// against 90.8 us for 256 threads x 4 chunks; the [65536, 5632] stress chain
// 1.466 ms against 1.553 ms.
#include "nf_device.h"

namespace nf {
namespace {

constexpr int kBlock = 64;
constexpr int kUnroll = 1;

template <typename T, bool VEC, bool NTL>
__global__ __launch_bounds__(kBlock) void swiglu_fwd_kernel(
    const T *__restrict__ a, const T *__restrict__ b, T *__restrict__ out,
    int64_t n) {
  const int64_t nchunks = (n + 7) >> 3;
  const int64_t first = (int64_t)blockIdx.x * (kBlock * kUnroll) + threadIdx.x;
  float av[kUnroll][8], bv[kUnroll][8];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t c = first + (int64_t)u * kBlock;
    if (c < nchunks) {
      const int64_t rem = n - c * 8;
      const int valid = rem >= 8 ? 8 : (int)rem;
      load8_stream<T, VEC, NTL>(a + c * 8, valid, av[u]);
      load8_stream<T, VEC, NTL>(b + c * 8, valid, bv[u]);
    }
  }
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t c = first + (int64_t)u * kBlock;
    if (c < nchunks) {
      const int64_t rem = n - c * 8;
      const int valid = rem >= 8 ? 8 : (int)rem;
      float o[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float x = av[u][i];
        o[i] = x * sigmoid(x) * bv[u][i];
      }
      store8_hint<T, VEC, true>(out + c * 8, valid, o);
    }
  }
}

template <typename T, bool VEC, bool NTL>
__global__ __launch_bounds__(kBlock) void swiglu_bwd_kernel(
    const T *__restrict__ dout, const T *__restrict__ a,
    const T *__restrict__ b, T *__restrict__ da, T *__restrict__ db,
    int64_t n) {
  const int64_t nchunks = (n + 7) >> 3;
  const int64_t first = (int64_t)blockIdx.x * (kBlock * kUnroll) + threadIdx.x;
  float gv[kUnroll][8], av[kUnroll][8], bv[kUnroll][8];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t c = first + (int64_t)u * kBlock;
    if (c < nchunks) {
      const int64_t rem = n - c * 8;
      const int valid = rem >= 8 ? 8 : (int)rem;
      load8_stream<T, VEC, NTL>(dout + c * 8, valid, gv[u]);
      load8_stream<T, VEC, NTL>(a + c * 8, valid, av[u]);
      load8_stream<T, VEC, NTL>(b + c * 8, valid, bv[u]);
    }
  }
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t c = first + (int64_t)u * kBlock;
    if (c < nchunks) {
      const int64_t rem = n - c * 8;
      const int valid = rem >= 8 ? 8 : (int)rem;
      float ga[8], gb[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float x = av[u][i];
        const float s = sigmoid(x);
        const float g = gv[u][i];
        ga[i] = g * bv[u][i] * (s * (1.f + x * (1.f - s)));
        gb[i] = g * (x * s);
      }
      store8_hint<T, VEC, true>(da + c * 8, valid, ga);
      store8_hint<T, VEC, true>(db + c * 8, valid, gb);
    }
  }
}

inline unsigned grid_for(int64_t n) {
  const int64_t nchunks = (n + 7) >> 3;
  return (unsigned)((nchunks + kBlock * kUnroll - 1) / (kBlock * kUnroll));
}

template <typename T>
int launch_fwd(const void *a, const void *b, void *out, int64_t n,
               hipStream_t s) {
  const bool vec = aligned16(a) && aligned16(b) && aligned16(out);
  const unsigned g = grid_for(n);
  if (vec && nt_loads_for(2 * n * (int64_t)sizeof(T)))
    swiglu_fwd_kernel<T, true, true><<<g, kBlock, 0, s>>>(
        (const T *)a, (const T *)b, (T *)out, n);
  else if (vec)
    swiglu_fwd_kernel<T, true, false><<<g, kBlock, 0, s>>>(
        (const T *)a, (const T *)b, (T *)out, n);
  else
    swiglu_fwd_kernel<T, false, false><<<g, kBlock, 0, s>>>(
        (const T *)a, (const T *)b, (T *)out, n);
  return check_launch("nf_swiglu_fwd");
}

template <typename T>
int launch_bwd(const void *dout, const void *a, const void *b, void *da,
               void *db, int64_t n, hipStream_t s) {
  const bool vec = aligned16(dout) && aligned16(a) && aligned16(b) &&
                   aligned16(da) && aligned16(db);
  const unsigned g = grid_for(n);
  if (vec && nt_loads_for(3 * n * (int64_t)sizeof(T)))
    swiglu_bwd_kernel<T, true, true><<<g, kBlock, 0, s>>>(
        (const T *)dout, (const T *)a, (const T *)b, (T *)da, (T *)db, n);
  else if (vec)
    swiglu_bwd_kernel<T, true, false><<<g, kBlock, 0, s>>>(
        (const T *)dout, (const T *)a, (const T *)b, (T *)da, (T *)db, n);
  else
    swiglu_bwd_kernel<T, false, false><<<g, kBlock, 0, s>>>(
        (const T *)dout, (const T *)a, (const T *)b, (T *)da, (T *)db, n);
  return check_launch("nf_swiglu_bwd");
}

}  // namespace
}  // namespace nf

using namespace nf;

extern "C" int nf_swiglu_fwd(const void *a, const void *b, void *out,
                             int64_t n, int dtype, void *stream) {
  if (n < 0) return set_error(NF_ERR_ARG, "nf_swiglu_fwd: n=%lld < 0", (long long)n);
  if (n == 0) return NF_OK;
  if (!a || !b || !out) return set_error(NF_ERR_ARG, "nf_swiglu_fwd: null pointer");
  if ((n + 7) / 8 > (int64_t)0x7fffffff * kBlock * kUnroll)
    return set_error(NF_ERR_ARG, "nf_swiglu_fwd: n too large");
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case NF_DTYPE_F32: return launch_fwd<float>(a, b, out, n, s);
    case NF_DTYPE_BF16: return launch_fwd<bf16>(a, b, out, n, s);
    case NF_DTYPE_F16: return launch_fwd<f16>(a, b, out, n, s);
  }
  return set_error(NF_ERR_DTYPE, "nf_swiglu_fwd: unsupported dtype %d", dtype);
}

extern "C" int nf_swiglu_bwd(const void *dout, const void *a, const void *b,
                             void *da, void *db, int64_t n, int dtype,
                             void *stream) {
  if (n < 0) return set_error(NF_ERR_ARG, "nf_swiglu_bwd: n=%lld < 0", (long long)n);
  if (n == 0) return NF_OK;
  if (!dout || !a || !b || !da || !db)
    return set_error(NF_ERR_ARG, "nf_swiglu_bwd: null pointer");
  if ((n + 7) / 8 > (int64_t)0x7fffffff * kBlock * kUnroll)
    return set_error(NF_ERR_ARG, "nf_swiglu_bwd: n too large");
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case NF_DTYPE_F32: return launch_bwd<float>(dout, a, b, da, db, n, s);
    case NF_DTYPE_BF16: return launch_bwd<bf16>(dout, a, b, da, db, n, s);
    case NF_DTYPE_F16: return launch_bwd<f16>(dout, a, b, da, db, n, s);
  }
  return set_error(NF_ERR_DTYPE, "nf_swiglu_bwd: unsupported dtype %d", dtype);
}
