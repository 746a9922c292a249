// Streaming ceiling for the row kernels: a grid-stride loop that reads R
// arrays and writes W arrays of 16-byte vectors with no dependency between
// its accesses (no row reduction, no LDS, no barrier), two vectors per thread
// per pass with all their loads issued first, non-temporal stores like the
// row kernels', and non-temporal loads under the row kernels' rule
// (nt_loads_for: more input than the Infinity Cache holds), up to 8192
// blocks (the best of 2048 / 4096 / 8192 blocks, one or two vectors per
// pass, plain or non-temporal stores on the cfg2 and cfg5 sizes).  bench.py
// times it on the adaLN step's traffic shapes (forward: 2 reads + 2 writes;
// backward: 4 reads + 2 writes) so that
// each row kernel can be set against what plain streaming reaches on the
// same box, the same bytes and the same cache state.  A measurement aid
// only; no op of the library calls it.
#include "../nf_device.h"
#include "../../../include/nuvla_forge_measure.h"

namespace nf {
namespace {

constexpr int kStreamThreads = 256;
constexpr int kStreamMaxBlocks = 8192;
constexpr int kStreamUnroll = 2;  // vectors per thread per pass, all loads issued first

struct StreamArgs {
  const u32x4 *in[4];
  u32x4 *out[2];
  int64_t n;  // 16-byte vectors per array
};

template <int R, int W, bool NTL>
__global__ __launch_bounds__(kStreamThreads) void stream_probe_kernel(StreamArgs a) {
  constexpr int U = kStreamUnroll;
  const int64_t stride = (int64_t)gridDim.x * kStreamThreads * U;
  for (int64_t i0 = (int64_t)blockIdx.x * kStreamThreads * U + threadIdx.x; i0 < a.n;
       i0 += stride) {
    u32x4 v[U][R];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t i = i0 + (int64_t)u * kStreamThreads;
#pragma unroll
      for (int r = 0; r < R; ++r)
        v[u][r] = i < a.n ? stream_load16<NTL>(&a.in[r][i]) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t i = i0 + (int64_t)u * kStreamThreads;
      if (i >= a.n) break;
      u32x4 s = v[u][0];
#pragma unroll
      for (int r = 1; r < R; ++r) s ^= v[u][r];
#pragma unroll
      for (int w = 0; w < W; ++w) __builtin_nontemporal_store(s + (unsigned)w, &a.out[w][i]);
    }
  }
}

// A read-only pass over in[0] (the (1, 0) form): every vector is loaded and
// folded into a per-thread xor; the store that keeps the loads alive fires
// only for a marker value, so the pass writes nothing in practice (at most
// out[0][0]).  Used to evict the caches before a cold-cache measurement.
__global__ __launch_bounds__(kStreamThreads) void stream_read_kernel(StreamArgs a) {
  constexpr int U = kStreamUnroll;
  const int64_t stride = (int64_t)gridDim.x * kStreamThreads * U;
  u32x4 s = {0u, 0u, 0u, 0u};
  for (int64_t i0 = (int64_t)blockIdx.x * kStreamThreads * U + threadIdx.x; i0 < a.n;
       i0 += stride) {
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t i = i0 + (int64_t)u * kStreamThreads;
      v[u] = i < a.n ? a.in[0][i] : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < U; ++u) s ^= v[u];
  }
  if (s.x == 0x9e3779b9u && s.y == 0x7f4a7c15u && s.z == 0x85ebca6bu && s.w == 0xc2b2ae35u)
    a.out[0][0] = s;
}

}  // namespace
}  // namespace nf

using namespace nf;

extern "C" int nf_stream_probe(int reads, int writes, const void *in0, const void *in1,
                               const void *in2, const void *in3, void *out0, void *out1,
                               int64_t n16, void *stream) {
  if (n16 < 0) return set_error(NF_ERR_ARG, "nf_stream_probe: n16 = %lld < 0", (long long)n16);
  const bool rw_ok = (reads == 1 && writes <= 1) || (reads == 2 && writes == 2) ||
                     (reads == 4 && writes == 2);
  if (!rw_ok)
    return set_error(NF_ERR_ARG, "nf_stream_probe: (reads, writes) = (%d, %d) is not one of "
                     "(1, 0), (1, 1), (2, 2), (4, 2)", reads, writes);
  if (n16 == 0) return NF_OK;
  const void *in[4] = {in0, in1, in2, in3};
  void *out[2] = {out0, out1};
  StreamArgs a{};
  for (int r = 0; r < reads; ++r) {
    if (!in[r] || !aligned16(in[r])) return set_error(NF_ERR_ARG, "nf_stream_probe: input %d is "
                                                      "null or not 16-byte aligned", r);
    a.in[r] = static_cast<const u32x4 *>(in[r]);
  }
  for (int w = 0; w < (writes > 0 ? writes : 1); ++w) {
    if (!out[w] || !aligned16(out[w])) return set_error(NF_ERR_ARG, "nf_stream_probe: output %d "
                                                        "is null or not 16-byte aligned", w);
    a.out[w] = static_cast<u32x4 *>(out[w]);
  }
  a.n = n16;
  int64_t blocks = (n16 + kStreamThreads * kStreamUnroll - 1) / (kStreamThreads * kStreamUnroll);
  if (blocks > kStreamMaxBlocks) blocks = kStreamMaxBlocks;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool ntl = nt_loads_for((int64_t)reads * n16 * 16);
  if (writes == 0)  // plain loads: an evicting pass must allocate in the caches
    stream_read_kernel<<<(unsigned)blocks, kStreamThreads, 0, s>>>(a);
  else if (reads == 1)
    ntl ? stream_probe_kernel<1, 1, true><<<(unsigned)blocks, kStreamThreads, 0, s>>>(a)
        : stream_probe_kernel<1, 1, false><<<(unsigned)blocks, kStreamThreads, 0, s>>>(a);
  else if (reads == 2)
    ntl ? stream_probe_kernel<2, 2, true><<<(unsigned)blocks, kStreamThreads, 0, s>>>(a)
        : stream_probe_kernel<2, 2, false><<<(unsigned)blocks, kStreamThreads, 0, s>>>(a);
  else
    ntl ? stream_probe_kernel<4, 2, true><<<(unsigned)blocks, kStreamThreads, 0, s>>>(a)
        : stream_probe_kernel<4, 2, false><<<(unsigned)blocks, kStreamThreads, 0, s>>>(a);
  return check_launch("nf_stream_probe");
}
