/*
 * capi_check.c -- the C ABI (include/rl_triton_amd.h) from a plain C11 program: no Python
 * and no torch in the process, only the HIP runtime and librl_triton_amd.so.  It calls GAE,
 * V-trace and the look-back prefix sum on seeded inputs in device memory it allocates
 * itself, and checks each result against the float64 CPU oracle (oracle/rlk_oracle.c, the
 * test suite's checker) with the GPU suite's tolerances.  Exit 0 and "capi_check ok" on
 * success.  Built by __graft_entry__.build(); run by tests/test_gpu_capi_c.py.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <hip/hip_runtime_api.h>

#include "rl_triton_amd.h"

/* the oracle (oracle/rlk_oracle.c) */
int orc_gae(int64_t E, int64_t T, const float *r, const float *val, const float *term,
            const float *trunc, const float *boot, int boot_mode, double gamma, double lambda,
            double *out);
int orc_vtrace(int64_t E, int64_t T, const float *lpt, const float *lpb, const float *val,
               const float *r, const float *term, const float *trunc, const float *boot,
               int boot_mode, double gamma, double rho_bar, double c_bar, double *targets,
               double *adv);
int orc_prefix_sum(int64_t E, int64_t T, const float *x, const float *dones, const float *seed,
                   int ends_at, double *out);

#define HIP_CHECK(call)                                                               \
  do {                                                                                \
    hipError_t e_ = (call);                                                           \
    if (e_ != hipSuccess) {                                                           \
      fprintf(stderr, "%s:%d %s: %s\n", __FILE__, __LINE__, #call, hipGetErrorString(e_)); \
      exit(2);                                                                        \
    }                                                                                 \
  } while (0)

static uint64_t rng = 0x9E3779B97F4A7C15ull;
static double uniform(void) { /* xorshift64*, [0, 1) */
  rng ^= rng >> 12;
  rng ^= rng << 25;
  rng ^= rng >> 27;
  return (double)((rng * 0x2545F4914F6CDD1Dull) >> 11) * (1.0 / 9007199254740992.0);
}
static float normal(void) { /* Box-Muller */
  double u = uniform(), v = uniform();
  return (float)(sqrt(-2.0 * log(u + 1e-300)) * cos(6.283185307179586 * v));
}
static float *host(int64_t n) {
  float *p = (float *)calloc((size_t)n, sizeof(float));
  if (!p) exit(3);
  return p;
}
static float *dev_copy(const float *h, int64_t n) {
  void *d = NULL;
  HIP_CHECK(hipMalloc(&d, (size_t)n * sizeof(float)));
  HIP_CHECK(hipMemcpy(d, h, (size_t)n * sizeof(float), hipMemcpyHostToDevice));
  return (float *)d;
}
static float *dev_empty(int64_t n) {
  void *d = NULL;
  HIP_CHECK(hipMalloc(&d, (size_t)n * sizeof(float)));
  return (float *)d;
}
/* max |got - want| against atol * max(1, max|want|) + rtol * |want| */
static int compare(const char *what, const float *dgot, const double *want, int64_t n,
                   double rtol, double atol) {
  float *got = host(n);
  HIP_CHECK(hipMemcpy(got, dgot, (size_t)n * sizeof(float), hipMemcpyDeviceToHost));
  double scale = 1.0, err = 0.0;
  for (int64_t i = 0; i < n; ++i) scale = fmax(scale, fabs(want[i]));
  int bad = 0;
  for (int64_t i = 0; i < n; ++i) {
    double d = fabs((double)got[i] - want[i]);
    err = fmax(err, d);
    if (!(d <= atol * scale + rtol * fabs(want[i]))) bad = 1;
  }
  printf("%-34s max abs err %.3e (atol %.2e)%s\n", what, err, atol * scale, bad ? "  FAILED" : "");
  free(got);
  return bad;
}

static int check_gae(hipStream_t st, int64_t E, int64_t T) {
  const int64_t n = E * T;
  float *r = host(n), *v = host(n), *te = host(n), *tr = host(n), *bv = host(n);
  for (int64_t i = 0; i < n; ++i) {
    r[i] = normal();
    v[i] = normal();
    te[i] = uniform() < 0.02 ? 1.f : 0.f;
    tr[i] = (te[i] == 0.f && uniform() < 0.01) ? 1.f : 0.f;
    bv[i] = (tr[i] == 1.f || i % T == T - 1) ? normal() : 0.f;
  }
  float *dr = dev_copy(r, n), *dv = dev_copy(v, n), *dte = dev_copy(te, n), *dtr = dev_copy(tr, n);
  float *dbv = dev_copy(bv, n), *dout = dev_empty(n);
  const int st_code = rlk_gae(dr, dv, dte, dtr, dbv, RLK_BOOT_FULL, dout, E, T, 0.99f, 0.95f, NULL, 0, st);
  if (st_code != RLK_OK) {
    printf("rlk_gae: %s\n", rlk_status_string(st_code));
    return 1;
  }
  HIP_CHECK(hipStreamSynchronize(st));
  double *want = (double *)calloc((size_t)n, sizeof(double));
  orc_gae(E, T, r, v, te, tr, bv, RLK_BOOT_FULL, 0.99, 0.95, want);
  char what[64];
  snprintf(what, sizeof what, "rlk_gae [%lld,%lld]", (long long)E, (long long)T);
  const int bad = compare(what, dout, want, n, 1e-5, 1e-5);
  hipFree(dr), hipFree(dv), hipFree(dte), hipFree(dtr), hipFree(dbv), hipFree(dout);
  free(r), free(v), free(te), free(tr), free(bv), free(want);
  return bad;
}

static int check_vtrace(hipStream_t st, int64_t E, int64_t T) {
  const int64_t n = E * T;
  float *lpt = host(n), *lpb = host(n), *v = host(n), *r = host(n), *te = host(n), *lv = host(E);
  for (int64_t i = 0; i < n; ++i) {
    lpt[i] = 0.5f * normal();
    lpb[i] = 0.5f * normal();
    v[i] = normal();
    r[i] = normal();
    te[i] = uniform() < 0.01 ? 1.f : 0.f;
  }
  for (int64_t e = 0; e < E; ++e) lv[e] = normal();
  float *d[6] = {dev_copy(lpt, n), dev_copy(lpb, n), dev_copy(v, n), dev_copy(r, n), dev_copy(te, n),
                 dev_copy(lv, E)};
  float *tg = dev_empty(n), *ad = dev_empty(n);
  const int st_code = rlk_vtrace(d[0], d[1], d[2], d[3], d[4], NULL, d[5], RLK_BOOT_ROW, tg, ad, E, T,
                                 0.99f, 1.f, 1.f, NULL, 0, st);
  if (st_code != RLK_OK) {
    printf("rlk_vtrace: %s\n", rlk_status_string(st_code));
    return 1;
  }
  HIP_CHECK(hipStreamSynchronize(st));
  double *wt = (double *)calloc((size_t)n, sizeof(double)), *wa = (double *)calloc((size_t)n, sizeof(double));
  orc_vtrace(E, T, lpt, lpb, v, r, te, NULL, lv, RLK_BOOT_ROW, 0.99, 1.0, 1.0, wt, wa);
  char what[64];
  snprintf(what, sizeof what, "rlk_vtrace [%lld,%lld] targets", (long long)E, (long long)T);
  int bad = compare(what, tg, wt, n, 1e-5, 1e-5);
  snprintf(what, sizeof what, "rlk_vtrace [%lld,%lld] advantages", (long long)E, (long long)T);
  bad |= compare(what, ad, wa, n, 1e-5, 1e-5);
  for (int i = 0; i < 6; ++i) hipFree(d[i]);
  hipFree(tg), hipFree(ad);
  free(lpt), free(lpb), free(v), free(r), free(te), free(lv), free(wt), free(wa);
  return bad;
}

/* rows longer than 2048 steps: the look-back path and its caller-provided workspace */
static int check_prefix_sum(hipStream_t st, int64_t E, int64_t T) {
  const int64_t n = E * T;
  float *x = host(n), *dn = host(n);
  int64_t run = 0, longest = 0;
  for (int64_t i = 0; i < n; ++i) {
    x[i] = normal();
    dn[i] = uniform() < 1e-3 ? 1.f : 0.f;
    run = (dn[i] == 1.f || i % T == 0) ? 1 : run + 1;
    if (run > longest) longest = run;
  }
  float *dx = dev_copy(x, n), *dd = dev_copy(dn, n), *dout = dev_empty(n);
  const size_t wsb = rlk_workspace_bytes(E, T);
  void *ws = NULL;
  HIP_CHECK(hipMalloc(&ws, wsb));
  HIP_CHECK(hipMemsetAsync(ws, 0, wsb, st)); /* zero once, before the first use */
  double *want = (double *)calloc((size_t)n, sizeof(double));
  orc_prefix_sum(E, T, x, dn, NULL, 1, want);
  int bad = 0;
  for (int rep = 0; rep < 3; ++rep) { /* the workspace is left ready for the next call */
    const int st_code = rlk_prefix_sum(dx, dd, NULL, dout, E, T, 1, ws, wsb, st);
    if (st_code != RLK_OK) {
      printf("rlk_prefix_sum: %s\n", rlk_status_string(st_code));
      return 1;
    }
    HIP_CHECK(hipStreamSynchronize(st));
    char what[64];
    snprintf(what, sizeof what, "rlk_prefix_sum [%lld,%lld] call %d", (long long)E, (long long)T, rep + 1);
    bad |= compare(what, dout, want, n, 1e-5, 1e-5 * sqrt(fmax((double)longest, 128.0) / 128.0));
  }
  uint64_t flag = 1;
  HIP_CHECK(hipMemcpy(&flag, (char *)ws + 3 * sizeof(uint64_t), sizeof flag, hipMemcpyDeviceToHost));
  if (flag != 0) {
    printf("workspace error flag set\n");
    bad = 1;
  }
  hipFree(dx), hipFree(dd), hipFree(dout), hipFree(ws);
  free(x), free(dn), free(want);
  return bad;
}

int main(void) {
  int ndev = 0;
  HIP_CHECK(hipGetDeviceCount(&ndev));
  if (ndev < 1) {
    printf("no GPU\n");
    return 2;
  }
  HIP_CHECK(hipSetDevice(0));
  printf("librl_triton_amd %d, %s\n", rlk_version(), rlk_status_string(RLK_OK));
  hipStream_t st;
  HIP_CHECK(hipStreamCreate(&st));
  int bad = 0;
  bad |= check_gae(st, 256, 128);     /* aligned quads */
  bad |= check_gae(st, 64, 333);      /* element-aligned quads */
  bad |= check_vtrace(st, 16, 1000);
  bad |= check_prefix_sum(st, 2, 70001);
  HIP_CHECK(hipStreamDestroy(st));
  printf(bad ? "capi_check FAILED\n" : "capi_check ok\n");
  return bad;
}
