/* Drives libnf_hip.so through its C ABI alone -- no Python, no torch: what a
 * C or C++ host of the kernels links against (include/nuvla_forge_hip.h).
 * Checks the ABI version, an argument error with its message, the SwiGLU
 * forward and backward and the adaLN forward (fp32) against host arithmetic
 * in double, on a stream of its own.  Prints "c abi smoke OK" and exits 0 on
 * success. */
#include <hip/hip_runtime_api.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#include "nuvla_forge_hip.h"

#define CHECK_HIP(x)                                                   \
  do {                                                                 \
    if ((x) != hipSuccess) {                                           \
      fprintf(stderr, "FAIL %s: %s\n", #x, hipGetErrorString(x));      \
      return 1;                                                        \
    }                                                                  \
  } while (0)

#define CHECK_NF(x)                                                    \
  do {                                                                 \
    int rc_ = (x);                                                     \
    if (rc_ != NF_OK) {                                                \
      fprintf(stderr, "FAIL %s: %d %s\n", #x, rc_, nf_last_error());  \
      return 1;                                                        \
    }                                                                  \
  } while (0)

static uint32_t lcg = 12345u;
static float uniform(float lo, float hi) {
  lcg = lcg * 1664525u + 1013904223u;
  return lo + (hi - lo) * (float)(lcg >> 8) / 16777216.0f;
}

/* norm-wise relative error max|got - want| / max|want| */
static double rel_err(const float *got, const double *want, int64_t n) {
  double num = 0.0, den = 0.0;
  for (int64_t i = 0; i < n; ++i) {
    const double d = fabs((double)got[i] - want[i]);
    if (d > num) num = d;
    if (fabs(want[i]) > den) den = fabs(want[i]);
  }
  return den > 0.0 ? num / den : num;
}

static int to_device(void **dst, const float *src, int64_t n) {
  if (hipMalloc(dst, (size_t)n * sizeof(float)) != hipSuccess) return 1;
  return hipMemcpy(*dst, src, (size_t)n * sizeof(float), hipMemcpyHostToDevice) != hipSuccess;
}

int main(void) {
  if (nf_abi_version() != NF_ABI_VERSION) {
    fprintf(stderr, "FAIL abi version %d\n", nf_abi_version());
    return 1;
  }
  /* an argument error is a status and a message, before any launch */
  if (nf_swiglu_fwd(NULL, NULL, NULL, 8, NF_DTYPE_F32, NULL) != NF_ERR_ARG ||
      nf_last_error()[0] == '\0') {
    fprintf(stderr, "FAIL null-pointer check\n");
    return 1;
  }
  hipStream_t s;
  CHECK_HIP(hipStreamCreate(&s));

  /* SwiGLU, fp32, n = 1000 */
  const int64_t n = 1000;
  float *a = malloc(n * sizeof(float)), *b = malloc(n * sizeof(float));
  float *g = malloc(n * sizeof(float)), *o = malloc(n * sizeof(float));
  float *ga = malloc(n * sizeof(float)), *gb = malloc(n * sizeof(float));
  double *want = malloc(3 * n * sizeof(double));
  for (int64_t i = 0; i < n; ++i) {
    a[i] = uniform(-6.f, 6.f);
    b[i] = uniform(-2.f, 2.f);
    g[i] = uniform(-1.f, 1.f);
  }
  void *da, *db, *dg, *dout, *dga, *dgb;
  if (to_device(&da, a, n) || to_device(&db, b, n) || to_device(&dg, g, n)) {
    fprintf(stderr, "FAIL device copies\n");
    return 1;
  }
  CHECK_HIP(hipMalloc(&dout, n * sizeof(float)));
  CHECK_HIP(hipMalloc(&dga, n * sizeof(float)));
  CHECK_HIP(hipMalloc(&dgb, n * sizeof(float)));
  CHECK_NF(nf_swiglu_fwd(da, db, dout, n, NF_DTYPE_F32, (void *)s));
  CHECK_NF(nf_swiglu_bwd(dg, da, db, dga, dgb, n, NF_DTYPE_F32, (void *)s));
  CHECK_HIP(hipStreamSynchronize(s));
  CHECK_HIP(hipMemcpy(o, dout, n * sizeof(float), hipMemcpyDeviceToHost));
  CHECK_HIP(hipMemcpy(ga, dga, n * sizeof(float), hipMemcpyDeviceToHost));
  CHECK_HIP(hipMemcpy(gb, dgb, n * sizeof(float), hipMemcpyDeviceToHost));
  for (int64_t i = 0; i < n; ++i) {
    const double sg = 1.0 / (1.0 + exp(-(double)a[i]));
    want[i] = a[i] * sg * b[i];
    want[n + i] = g[i] * b[i] * sg * (1.0 + a[i] * (1.0 - sg));
    want[2 * n + i] = g[i] * a[i] * sg;
  }
  const double e_out = rel_err(o, want, n), e_da = rel_err(ga, want + n, n),
               e_db = rel_err(gb, want + 2 * n, n);
  if (!(e_out <= 1e-5 && e_da <= 1e-5 && e_db <= 1e-5)) {
    fprintf(stderr, "FAIL swiglu rel err %g %g %g\n", e_out, e_da, e_db);
    return 1;
  }

  /* adaLN forward, fp32, B = 2 samples of T = 4 rows, N = 64 */
  enum { B = 2, T = 4, N = 64, M = B * T };
  static float x[M * N], y[M * N], gate[B * N], w[N], sc[B * N], sh[B * N];
  static float h[M * N], out[M * N], rstd[M];
  static double hw[M * N], ow[M * N];
  for (int i = 0; i < M * N; ++i) {
    x[i] = uniform(-2.f, 2.f);
    y[i] = uniform(-2.f, 2.f);
  }
  for (int i = 0; i < B * N; ++i) {
    gate[i] = uniform(-0.3f, 0.3f);
    sc[i] = uniform(-0.3f, 0.3f);
    sh[i] = uniform(-0.3f, 0.3f);
  }
  for (int i = 0; i < N; ++i) w[i] = uniform(0.9f, 1.1f);
  void *dx, *dy, *dgt, *dw, *dsc, *dsh, *dh, *dout2, *drstd;
  if (to_device(&dx, x, M * N) || to_device(&dy, y, M * N) || to_device(&dgt, gate, B * N) ||
      to_device(&dw, w, N) || to_device(&dsc, sc, B * N) || to_device(&dsh, sh, B * N)) {
    fprintf(stderr, "FAIL device copies\n");
    return 1;
  }
  CHECK_HIP(hipMalloc(&dh, sizeof(h)));
  CHECK_HIP(hipMalloc(&dout2, sizeof(out)));
  CHECK_HIP(hipMalloc(&drstd, sizeof(rstd)));
  CHECK_NF(nf_adaln_fwd(dx, N, dy, N, dgt, N, dw, dsc, N, dsh, N, dh, dout2, (float *)drstd, M,
                        N, T, 1e-6f, NF_DTYPE_F32, NF_DTYPE_F32, NF_DTYPE_F32, NF_DTYPE_F32,
                        NF_DTYPE_F32, NF_DTYPE_F32, (void *)s));
  CHECK_HIP(hipStreamSynchronize(s));
  CHECK_HIP(hipMemcpy(h, dh, sizeof(h), hipMemcpyDeviceToHost));
  CHECK_HIP(hipMemcpy(out, dout2, sizeof(out), hipMemcpyDeviceToHost));
  for (int m = 0; m < M; ++m) {
    const int bs = m / T;
    double ss = 0.0;
    for (int c = 0; c < N; ++c) {
      const double v = (double)x[m * N + c] + (double)gate[bs * N + c] * y[m * N + c];
      hw[m * N + c] = v;
      ss += v * v;
    }
    const double r = 1.0 / sqrt(ss / N + 1e-6);
    for (int c = 0; c < N; ++c)
      ow[m * N + c] = hw[m * N + c] * r * w[c] * (1.0 + sc[bs * N + c]) + sh[bs * N + c];
  }
  const double e_h = rel_err(h, hw, M * N), e_o = rel_err(out, ow, M * N);
  if (!(e_h <= 1e-5 && e_o <= 1e-5)) {
    fprintf(stderr, "FAIL adaln rel err %g %g\n", e_h, e_o);
    return 1;
  }
  void *bufs[] = {da, db, dg, dout, dga, dgb, dx, dy, dgt, dw, dsc, dsh, dh, dout2, drstd};
  for (size_t i = 0; i < sizeof(bufs) / sizeof(bufs[0]); ++i) CHECK_HIP(hipFree(bufs[i]));
  CHECK_HIP(hipStreamDestroy(s));
  free(a); free(b); free(g); free(o); free(ga); free(gb); free(want);
  printf("c abi smoke OK (swiglu %.1e %.1e %.1e, adaln %.1e %.1e)\n", e_out, e_da, e_db, e_h,
         e_o);
  return 0;
}
