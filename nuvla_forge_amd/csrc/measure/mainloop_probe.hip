// What the GEMM core's mainloop instruction mix costs the matrix pipes, one
// ingredient at a time.  Blocks of 512 threads, two wavefronts per SIMD as in
// the GEMM core; each wavefront issues 32 v_mfma_f32_16x16x32_bf16 per 32-wide
// k-group on 128 fp32 accumulators (a 128 x 64 wavefront tile), two k-groups
// per iteration, `iters` iterations:
//   mode 1: operands held in registers, no memory access in the loop;
//   mode 2: each k-group's 8 A + 4 B operand vectors read from LDS
//           (ds_read_b128), the next k-group's reads interleaved with the
//           current k-group's products, as in the GEMM core;
//   mode 3: mode 2 plus 8 direct-to-LDS copies (1 KB each) per wavefront per
//           iteration into a second LDS region, waited for one iteration
//           later: the GEMM's 64 KB stage per block, from a 1 MiB region of
//           `src` that stays in the L2;
//   mode 4: mode 3 plus one s_barrier per iteration;
//   mode 5: mode 4 with the copies walking 32 streams over 64 MiB of `src`
//           (block b takes stream b % 32, so the blocks sharing a stream sit
//           on one XCD and share its L2, as tiles sharing an operand panel
//           do), a footprint beyond the L2s.
// The operand data (from `ops`) is random bf16, so the products toggle as a
// real GEMM's do.  A measurement aid only; no op of the library calls it.
#include "../gemm_core.h"
#include "../../../include/nuvla_forge_measure.h"

namespace nf {
namespace {

constexpr int kMlThreads = 512;
constexpr int kMlOperandBytes = 65536;   // LDS operand region
constexpr int kMlCopyBytes = 65536;      // LDS region the copies land in
constexpr uint32_t kMlL2Span = 1u << 20;
constexpr uint32_t kMlStreamSpan = 64u << 20;
constexpr int kMlStreams = 32;

__device__ __forceinline__ void ml_products(const u32x4 (&a)[8], const u32x4 (&b)[4],
                                            gemm::floatx4 (&acc)[8][4]) {
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
          __builtin_bit_cast(gemm::bf16x8, a[i]), __builtin_bit_cast(gemm::bf16x8, b[j]),
          acc[i][j], 0, 0, 0);
}

// wavefront w's k-group g: 12 vectors of 1 KB, vector v at 1 KB slot
// (24 w + 12 g + v) mod 64 of the operand region, lane l at byte 16 l
__device__ __forceinline__ void ml_read(const char *lds, int w, int g, u32x4 (&a)[8],
                                        u32x4 (&b)[4]) {
  const int l = threadIdx.x & 63;
#pragma unroll
  for (int i = 0; i < 8; ++i)
    a[i] = *reinterpret_cast<const u32x4 *>(lds + (((24 * w + 12 * g + i) & 63) << 10) + 16 * l);
#pragma unroll
  for (int j = 0; j < 4; ++j)
    b[j] = *reinterpret_cast<const u32x4 *>(lds + (((24 * w + 12 * g + 8 + j) & 63) << 10) + 16 * l);
}

// 32 products and 12 reads: 2 products, then (1 read, 2 products) x 12, then 6
__device__ __forceinline__ void ml_interleave() {
  __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
#pragma unroll
  for (int r = 0; r < 12; ++r) {
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
  }
  __builtin_amdgcn_sched_group_barrier(0x008, 6, 0);
}

template <int MODE>
__global__ __launch_bounds__(kMlThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void mainloop_probe_kernel(const u32x4 *ops, const u32x4 *src, int64_t iters, float *out,
                           uint64_t *stamps) {
  __shared__ __attribute__((aligned(16))) char lds[kMlOperandBytes + kMlCopyBytes];
  const uint64_t c0 = __builtin_readcyclecounter();
  const uint64_t r0 = __builtin_amdgcn_s_memrealtime();
  const int t = threadIdx.x, w = t >> 6, l = t & 63;
#pragma unroll
  for (int k = 0; k < kMlOperandBytes / 16 / kMlThreads; ++k)
    reinterpret_cast<u32x4 *>(lds)[k * kMlThreads + t] = ops[k * kMlThreads + t];
  __syncthreads();
  gemm::floatx4 acc[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = gemm::floatx4{0.f, 0.f, 0.f, 0.f};
  u32x4 a0[8], b0[4], a1[8], b1[4];
  if constexpr (MODE == 1) {
#pragma unroll
    for (int i = 0; i < 8; ++i) a0[i] = ops[i * kMlThreads + t];
#pragma unroll
    for (int j = 0; j < 4; ++j) b0[j] = ops[(8 + j) * kMlThreads + t];
    for (int64_t it = 0; it < iters; ++it) {
      ml_products(a0, b0, acc);
      ml_products(a0, b0, acc);
    }
  } else {
    constexpr uint32_t kSpan = MODE == 5 ? kMlStreamSpan : kMlL2Span;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<u32x4 *>(src), (short)0, (int)kSpan, 0x00020000);
    char *copies = lds + kMlOperandBytes + w * (kMlCopyBytes / 8);
    ml_read(lds, w, 0, a0, b0);
    for (int64_t it = 0; it < iters; ++it) {
      ml_read(lds, w, 1, a1, b1);
      ml_products(a0, b0, acc);
      ml_interleave();
      if constexpr (MODE >= 3) {
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          // 1 KB chunk index within the span, then this lane's 16 bytes
          const uint64_t chunk = MODE == 5
              ? ((uint64_t)(blockIdx.x % kMlStreams) * (uint64_t)iters + (uint64_t)it) * 64 + 8 * w + c
              : (uint64_t)it * 8 + c;
          const uint32_t off = (uint32_t)((chunk * 1024 + 16 * l) & (kSpan - 1));
          __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (gemm::lds_ptr_t)(copies + c * 1024), 16,
                                                   off, 0, 0, 0);
        }
      }
      ml_read(lds, w, 0, a0, b0);
      ml_products(a1, b1, acc);
      ml_interleave();
      // the previous iteration's 8 copies have landed (this one's in flight)
      if constexpr (MODE >= 3) __builtin_amdgcn_s_waitcnt(8 | (7 << 4) | (15 << 8));
      if constexpr (MODE >= 4) __builtin_amdgcn_s_barrier();
    }
    if constexpr (MODE >= 3) __builtin_amdgcn_s_waitcnt(0 | (7 << 4) | (15 << 8));
  }
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) sum += acc[i][j][r];
  out[(int64_t)blockIdx.x * kMlThreads + t] = sum;
  if (stamps && t == 0) {
    uint64_t *p = stamps + (int64_t)blockIdx.x * 4;
    p[0] = c0;
    p[1] = __builtin_readcyclecounter();
    p[2] = r0;
    p[3] = __builtin_amdgcn_s_memrealtime();
  }
}

}  // namespace
}  // namespace nf

using namespace nf;

extern "C" int nf_mainloop_probe(int mode, const void *ops, const void *src, size_t src_bytes,
                                 int64_t iters, int64_t blocks, float *out, uint64_t *stamps,
                                 void *stream) {
  if (mode < 1 || mode > 5) return set_error(NF_ERR_ARG, "nf_mainloop_probe: mode %d outside 1-5", mode);
  if (iters < 0 || iters > (int64_t(1) << 30))
    return set_error(NF_ERR_ARG, "nf_mainloop_probe: iters = %lld outside [0, 2^30]",
                     (long long)iters);
  if (blocks < 1 || blocks > (int64_t(1) << 20))
    return set_error(NF_ERR_ARG, "nf_mainloop_probe: blocks = %lld outside [1, 2^20]",
                     (long long)blocks);
  if (!ops || !out) return set_error(NF_ERR_ARG, "nf_mainloop_probe: null ops or out");
  if (!aligned16(ops)) return set_error(NF_ERR_ARG, "nf_mainloop_probe: ops is not 16-byte aligned");
  const size_t need = mode == 5 ? kMlStreamSpan : (mode >= 3 ? kMlL2Span : 0);
  if (need && (!src || src_bytes < need || !aligned16(src)))
    return set_error(NF_ERR_ARG, "nf_mainloop_probe: mode %d needs a 16-byte aligned src of "
                     "%zu bytes (given %zu)", mode, need, src_bytes);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const unsigned g = (unsigned)blocks;
  const u32x4 *o = static_cast<const u32x4 *>(ops), *sr = static_cast<const u32x4 *>(src);
  switch (mode) {
    case 1: mainloop_probe_kernel<1><<<g, kMlThreads, 0, s>>>(o, sr, iters, out, stamps); break;
    case 2: mainloop_probe_kernel<2><<<g, kMlThreads, 0, s>>>(o, sr, iters, out, stamps); break;
    case 3: mainloop_probe_kernel<3><<<g, kMlThreads, 0, s>>>(o, sr, iters, out, stamps); break;
    case 4: mainloop_probe_kernel<4><<<g, kMlThreads, 0, s>>>(o, sr, iters, out, stamps); break;
    default: mainloop_probe_kernel<5><<<g, kMlThreads, 0, s>>>(o, sr, iters, out, stamps); break;
  }
  return check_launch("nf_mainloop_probe");
}
