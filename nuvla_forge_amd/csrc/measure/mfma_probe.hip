// MFMA ceiling for the cross entropy's products: every block of 256 threads
// (one wavefront per SIMD, the register budget of one wavefront) holds the
// operands of a 128 x 128 wavefront tile of bf16 products in registers --
// read once from `ops`, or zero -- and issues `iters` rounds of products
// with no memory access in the loop: v_mfma_f32_16x16x32_bf16 (form 0, the
// GEMM core's: 64 per round, 8 x 8 products of 32-wide k) or
// v_mfma_f32_32x32x16_bf16 (form 1: 32 per round, two 16-wide k-groups of
// 4 x 4), the same flops per round.  It is the matrix rate the chip
// sustains on that data, with no LDS, cache or HBM traffic competing for the
// power budget: bench.py times it on random bf16 operands (the data of a real
// product) and on zeros, and reads each block's shader clock from its
// stamps, so that the GEMM kernels can be set against what the MFMA pipes
// reach on this box.  A measurement aid only; no op of the library calls it.
#include "../gemm_core.h"
#include "../../../include/nuvla_forge_measure.h"

namespace nf {
namespace {

constexpr int kProbeThreads = 256;

// The thread's operand vectors: A from vectors {0..3, 8..11}, B from
// {4..7, 12..15} of `ops` (vector v of thread t at v * 256 + t).
__device__ __forceinline__ void probe_operands(const u32x4 *ops, int t, u32x4 (&a)[8],
                                               u32x4 (&b)[8]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int v = (i / 4) * 8 + i % 4;
    a[i] = ops ? ops[v * kProbeThreads + t] : u32x4{0u, 0u, 0u, 0u};
    b[i] = ops ? ops[(v + 4) * kProbeThreads + t] : u32x4{0u, 0u, 0u, 0u};
  }
}

template <int FORM>
__global__ __launch_bounds__(kProbeThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
void mfma_probe_kernel(const u32x4 *ops, int64_t iters, float *out, uint64_t *stamps) {
  const uint64_t c0 = __builtin_readcyclecounter();
  const uint64_t r0 = __builtin_amdgcn_s_memrealtime();
  const int t = threadIdx.x;
  u32x4 a[8], b[8];
  probe_operands(ops, t, a, b);
  float sum = 0.f;
  if constexpr (FORM == 0) {
    gemm::floatx4 acc[8][8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[i][j][r] = 0.f;
    for (int64_t it = 0; it < iters; ++it) {
#pragma unroll
      for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              __builtin_bit_cast(gemm::bf16x8, a[i]), __builtin_bit_cast(gemm::bf16x8, b[j]),
              acc[i][j], 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) sum += acc[i][j][r];
  } else {
    gemm::floatx16 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
    for (int64_t it = 0; it < iters; ++it) {
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            gemm::mfma_slab<bf16>(a[4 * s + i], b[4 * s + j], acc[i][j]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) sum += acc[i][j][r];
  }
  out[(int64_t)blockIdx.x * kProbeThreads + t] = sum;
  if (stamps && t == 0) {
    const uint64_t c1 = __builtin_readcyclecounter();
    const uint64_t r1 = __builtin_amdgcn_s_memrealtime();
    uint64_t *p = stamps + (int64_t)blockIdx.x * 4;
    p[0] = c0;
    p[1] = c1;
    p[2] = r0;
    p[3] = r1;
  }
}

}  // namespace
}  // namespace nf

using namespace nf;

extern "C" int nf_mfma_probe(const void *ops, int64_t iters, int64_t blocks, int form,
                             float *out, uint64_t *stamps, void *stream) {
  if (iters < 0 || iters > (int64_t(1) << 30))
    return set_error(NF_ERR_ARG, "nf_mfma_probe: iters = %lld outside [0, 2^30]",
                     (long long)iters);
  if (blocks < 1 || blocks > (int64_t(1) << 20))
    return set_error(NF_ERR_ARG, "nf_mfma_probe: blocks = %lld outside [1, 2^20]",
                     (long long)blocks);
  if (form != 0 && form != 1)
    return set_error(NF_ERR_ARG, "nf_mfma_probe: form = %d is neither 0 nor 1", form);
  if (!out) return set_error(NF_ERR_ARG, "nf_mfma_probe: out is null");
  if (ops && !aligned16(ops))
    return set_error(NF_ERR_ARG, "nf_mfma_probe: ops is not 16-byte aligned");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (form == 0)
    mfma_probe_kernel<0><<<(unsigned)blocks, kProbeThreads, 0, s>>>(
        static_cast<const u32x4 *>(ops), iters, out, stamps);
  else
    mfma_probe_kernel<1><<<(unsigned)blocks, kProbeThreads, 0, s>>>(
        static_cast<const u32x4 *>(ops), iters, out, stamps);
  return check_launch("nf_mfma_probe");
}
