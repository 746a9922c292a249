/*
 * nuvla_forge_measure.h -- measurement aids and a test hook, built into
 * nuvla_forge_amd/libnf_measure.so beside the product library
 * (libnf_hip.so, include/nuvla_forge_hip.h).  None of these has a
 * counterpart in the reference, and no op of the product calls them: the
 * benchmark sets the product kernels against the two probes, and the tests
 * drive the MFMA GEMM core through nf_gemm_nt and nf_gemm_nn.
 *
 * Same conventions as the product ABI: device pointers, int64_t sizes, a
 * hipStream_t as `void *`, NF_OK or a negative status, and the failure text
 * in the product library's nf_last_error() (this library reports through
 * it; libnf_measure.so links libnf_hip.so).
 */
#ifndef NUVLA_FORGE_MEASURE_H
#define NUVLA_FORGE_MEASURE_H

#include "nuvla_forge_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------------
 * Test hook with no counterpart in the reference: C[M, N] (fp32, row stride
 * ldc) = A[M, K] @ B[N, K]^T with the MFMA core the cross entropy uses.
 * A and B are row-major with unit-stride K, type `dtype` (bf16 or f32).
 * ---------------------------------------------------------------------- */
int nf_gemm_nt(const void *A, int64_t lda, const void *B, int64_t ldb,
               float *C, int64_t ldc, int64_t M, int64_t N, int64_t K,
               int dtype, void *stream);

/* ------------------------------------------------------------------------
 * Test hook with no counterpart in the reference: C += A[M, K] @ B[N, K]^T
 * for bf16 A, B and fp32 C (ldc >= N), the accumulator preloaded from C
 * before the K loop: the path of a product accumulated onto an earlier one.
 * ---------------------------------------------------------------------- */
int nf_gemm_nt_acc(const void *A, int64_t lda, const void *B, int64_t ldb, float *C,
                   int64_t ldc, int64_t M, int64_t N, int64_t K, void *stream);

/* ------------------------------------------------------------------------
 * Test hook with no counterpart in the reference: C = A[M, K] @ B[K, N]
 * (bf16 A and B, fp32 C) through the MFMA core's N-major-B path: A
 * row-major with unit-stride K, B row-major with unit-stride N (ldb >= N;
 * columns up to ldb are read).  With lda, K and ldb multiples of 8, 16-byte
 * aligned operands each under 2 GiB, the operands go global -> LDS by the
 * buffer unit; otherwise through registers.  C[m, n] is stored at
 * C[m * ldc + n], or at C[n * ldc + m] when c_transposed is nonzero.
 * ---------------------------------------------------------------------- */
int nf_gemm_nn(const void *A, int64_t lda, const void *B, int64_t ldb,
               float *C, int64_t ldc, int64_t M, int64_t N, int64_t K,
               int c_transposed, void *stream);

/* ------------------------------------------------------------------------
 * Measurement aid with no counterpart in the reference: the streaming
 * ceiling bench.py sets the row kernels against.  Reads `reads` arrays
 * (in0..in3) and writes `writes` arrays (out0, out1) of n16 16-byte vectors
 * each, (reads, writes) one of (1, 1), (2, 2), (4, 2); out_w[i] = (in0[i]
 * xor ... xor in_{reads-1}[i]) + w in every 32-bit lane.  (1, 0) is a
 * read-only pass over in0 that writes at most one vector, out0[0] (only for
 * a marker value): a cache-evicting pass for cold-cache measurements.
 * Pointers unused by the (reads, writes) pair may be null; the others must
 * be 16-byte aligned.
 * ---------------------------------------------------------------------- */
int nf_stream_probe(int reads, int writes, const void *in0, const void *in1,
                    const void *in2, const void *in3, void *out0, void *out1,
                    int64_t n16, void *stream);

/* ------------------------------------------------------------------------
 * Measurement aid with no counterpart in the reference: the MFMA ceiling
 * bench.py sets the cross entropy's products against.  `blocks` blocks of
 * 256 threads each issue iters * 256 bf16 v_mfma_f32_16x16x32 products
 * (form 0, the GEMM core's; 2 * 16 * 16 * 32 flops each) or iters * 128
 * v_mfma_f32_32x32x16 products (form 1; 2 * 32 * 32 * 16 flops each) on
 * operands held in registers, with no memory access in the loop.  ops:
 * 16 * 256 16-byte vectors (vector v of thread t at index v * 256 + t; A
 * operands from vectors 0-3 and 8-11, B from 4-7 and 12-15; every block
 * reads the same ones), or NULL for zero operands.  out[b * 256 + t] = the
 * sum of thread t's 256 accumulators in block b (blocks * 256 floats).
 * stamps (NULL or blocks * 4 values): per block, the shader clock counter
 * at start and end, then the 100 MHz real-time counter at start and end.
 * ---------------------------------------------------------------------- */
int nf_mfma_probe(const void *ops, int64_t iters, int64_t blocks, int form, float *out,
                  uint64_t *stamps, void *stream);

/* ------------------------------------------------------------------------
 * The GEMM core's mainloop instruction mix, one ingredient at a time: what
 * each costs the matrix pipes (and the power-limited clock).  `blocks`
 * blocks of 512 threads (two wavefronts per SIMD), each wavefront issuing
 * iters * 64 v_mfma_f32_16x16x32_bf16 products (2 * 16 * 16 * 32 flops each)
 * on 128 accumulators:
 *   mode 1  operands in registers, no memory access in the loop;
 *   mode 2  + the operands read from LDS, 12 ds_read_b128 per 32 products,
 *           interleaved with the products as the GEMM core does;
 *   mode 3  + 8 direct-to-LDS copies of 1 KB per wavefront per iteration
 *           (the GEMM's 64 KB stage per block) from the first 1 MiB of src
 *           (L2-resident), waited for one iteration later;
 *   mode 4  + one s_barrier per iteration;
 *   mode 5  mode 4 with the copies walking 32 streams over 64 MiB of src
 *           (blocks b and b + 32 k share stream b % 32 and one XCD's L2).
 * ops: 12 * 512 16-byte vectors of bf16 operands (random data toggles the
 * multipliers as a real product does).  src: 16-byte aligned, at least
 * 1 MiB for modes 3-4 and 64 MiB for mode 5 (may be NULL for modes 1-2).
 * out[b * 512 + t] = the sum of thread t's accumulators in block b; stamps
 * (NULL or blocks * 4): per block the shader clock counter at start and end,
 * then the 100 MHz real-time counter at start and end.
 * ---------------------------------------------------------------------- */
int nf_mainloop_probe(int mode, const void *ops, const void *src, size_t src_bytes,
                      int64_t iters, int64_t blocks, float *out, uint64_t *stamps,
                      void *stream);

#ifdef __cplusplus
}
#endif

#endif /* NUVLA_FORGE_MEASURE_H */
