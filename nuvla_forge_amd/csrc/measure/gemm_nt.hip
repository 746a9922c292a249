// Test hook for the MFMA GEMM core (no counterpart in the reference): a plain
// C = A B^T through the same mainloop, store epilogue and launch helpers the
// cross entropy's products use, so tests can check the MFMA lane layouts and
// the ragged-edge handling at arbitrary sizes.  Built into libnf_measure.so,
// not the product library.
#include "../gemm_store.h"
#include "../../../include/nuvla_forge_measure.h"

using namespace nf;
using namespace nf::gemm;

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

extern "C" int nf_gemm_nt_acc(const void *A, int64_t lda, const void *B, int64_t ldb, float *C,
                              int64_t ldc, int64_t M, int64_t N, int64_t K, void *stream) {
  if (M < 0 || N < 0 || K < 0) return set_error(NF_ERR_ARG, "nf_gemm_nt_acc: negative size");
  if (M > 0x7fffffffLL || N > 0x7fffffffLL || K > 0x7fffffffLL)
    return set_error(NF_ERR_ARG, "nf_gemm_nt_acc: a size exceeds int32");
  if (M == 0 || N == 0) return NF_OK;
  if (!A || !B || !C) return set_error(NF_ERR_ARG, "nf_gemm_nt_acc: null pointer");
  if (lda < K || ldb < K || ldc < N)
    return set_error(NF_ERR_ARG, "nf_gemm_nt_acc: bad leading dim");
  if (((M + 255) / 256) * ((N + 255) / 256) > 0x7fffffffLL)
    return set_error(NF_ERR_ARG, "nf_gemm_nt_acc: grid too large");
  using C16 = MainCfg<bf16>;
  // C as its own preload: every element is read and written by one thread
  auto j = make_job<C16>((const bf16 *)A, lda, (const bf16 *)B, ldb, C, C, NF_DTYPE_F32, nullptr,
                         ldc, M, N, K);
  j.ldcin = ldc;
  const GemmJob<bf16> none{};
  return launch_gemm_store<C16>(j, none, static_cast<hipStream_t>(stream));
}

extern "C" int nf_gemm_nn(const void *A, int64_t lda, const void *B, int64_t ldb, float *C,
                          int64_t ldc, int64_t M, int64_t N, int64_t K, int c_transposed,
                          void *stream) {
  if (M < 0 || N < 0 || K < 0) return set_error(NF_ERR_ARG, "nf_gemm_nn: negative size");
  if (M > 0x7fffffffLL || N > 0x7fffffffLL || K > 0x7fffffffLL)
    return set_error(NF_ERR_ARG, "nf_gemm_nn: a size exceeds int32");
  if (M == 0 || N == 0) return NF_OK;
  if (!A || !B || !C) return set_error(NF_ERR_ARG, "nf_gemm_nn: null pointer");
  if (lda < K || ldb < N || ldc < (c_transposed ? M : N))
    return set_error(NF_ERR_ARG, "nf_gemm_nn: bad leading dim");
  if (((M + 255) / 256) * ((N + 255) / 256) > 0x7fffffffLL)
    return set_error(NF_ERR_ARG, "nf_gemm_nn: grid too large");
  using C16 = MainCfg<bf16>;
  auto j = make_job<C16>((const bf16 *)A, lda, (const bf16 *)B, ldb, nullptr, C, NF_DTYPE_F32,
                         nullptr, ldc, M, N, K);
  j.bt = 1;
  j.ct = c_transposed ? 1 : 0;
  const GemmJob<bf16> none{};
  return launch_gemm_store<C16>(j, none, static_cast<hipStream_t>(stream));
}
